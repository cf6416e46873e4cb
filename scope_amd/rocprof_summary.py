"""Summaries of rocprofv3 CSV output for the attention hot path.

Two inputs are understood:

* ``--stats DIR``: a ``--kernel-trace --stats --output-format csv`` run
  (``*_kernel_stats.csv``) -> per-kernel calls / average / total time;
* ``--pmc DIR``: a ``--pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE ...`` run ->
  per-kernel MFMA busy fraction = busy cycles summed over SIMDs /
  (elapsed cycles x SIMDs), where GRBM_GUI_ACTIVE counts elapsed cycles once
  per XCD (SIMD and XCD counts from the run's agent_info.csv), plus the
  instruction mix and the LDS bank-conflict rate when those counters are there;
* ``--fetch DIR --write DIR``: two ``--pmc FETCH_SIZE`` and ``--pmc WRITE_SIZE``
  runs (``*_counter_collection.csv``) of ``bench.py --copy-probe-mib N``.  The
  plain device copy of known size in the same run calibrates each counter:
  factor = copied bytes / counter bytes, applied to every kernel.

``python -m scope_amd.rocprof_summary --stats D [--fetch F --write W --copy-bytes B] [--json OUT]``
prints a markdown table and optionally writes the per-kernel traffic as JSON
(read by bench.py to fill ``roofline.traffic``).
"""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import json
import os
import sys

KERNELS = ("attn_fwd_kernel", "attn_fwd_kernel(lse)", "attn_fwd_kernel(mass)", "attn_bwd_dq2_kernel",
           "attn_bwd_dq16_kernel", "attn_bwd_dq_kernel", "attn_bwd_dkv16_kernel", "attn_bwd_dkv_kernel", "bwd_reduce_kernel", "block_means_kernel", "ptr_logits_kernel", "ptr_score_kernel",
           "stats_kernel", "tr_fill_kernel", "tr_sort_kernel", "tr_count_kernel", "swa_count_kernel",
           "swa_rows_kernel", "swa_pad_kernel", "coeff_fwd_kernel", "coeff_bwd_kernel", "coeff_reg_kernel",
           "probe_mfma_kernel", "probe_copy_kernel")
COPY = "copyBuffer"
FWD_KINDS = {"0": "", "1": "(lse)", "2": "(mass)"}


def _base(name: str) -> str:
    """The kernel's name without namespace and template arguments (the
    forward's kind as a suffix), or the tail of an unknown name."""
    if "attn_fwd_kernel<" in name:
        args = name.split("attn_fwd_kernel<", 1)[1].split(">", 1)[0].split(",")
        kind = args[2].strip() if len(args) > 2 else "0"
        return "attn_fwd_kernel" + FWD_KINDS.get(kind, "")
    for k in KERNELS + (COPY,):
        if "(" not in k and k in name:
            return k
    name = name.replace("(anonymous namespace)::", "")
    return name.split("(")[0][-60:]


def _short(name: str) -> str:
    """_base, with the block size and bias mode of an attention kernel
    (``attn_bwd_dkv16_kernel<256,1>``): one run can hold several instances
    (the headline layer and the reference's default layer)."""
    b = _base(name)
    if not b.startswith("attn_"):
        return b
    stem = b.split("(")[0]
    if stem + "<" not in name:
        return b
    args = [a.strip() for a in name.split(stem + "<", 1)[1].split(">", 1)[0].split(",")]
    return f"{stem}<{','.join(args[:2])}>" + b[len(stem):]


def _order(k: str) -> tuple[int, str]:
    b = k.split("<")[0] + (k.split(">", 1)[1] if ">" in k else "")
    return (KERNELS.index(b) if b in KERNELS else len(KERNELS), k)


def _csv(dir_: str, suffix: str) -> list[dict]:
    files = glob.glob(os.path.join(dir_, "**", f"*{suffix}"), recursive=True)
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {dir_}")
    rows: list[dict] = []
    for f in files:
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    return rows


def kernel_stats(dir_: str) -> list[tuple[str, int, float, float]]:
    out = []
    for r in _csv(dir_, "_kernel_stats.csv"):
        out.append((_short(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3, float(r["TotalDurationNs"]) / 1e6))
    return sorted(out, key=lambda t: -t[3])


def counter_means(dir_: str, counter: str) -> dict[str, tuple[float, int]]:
    acc: dict[str, list[float]] = collections.defaultdict(list)
    for r in _csv(dir_, "_counter_collection.csv"):
        if r["Counter_Name"] == counter:
            acc[_short(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: (sum(v) / len(v), len(v)) for k, v in acc.items()}


def topology(dir_: str) -> tuple[int, int]:
    """(SIMDs, XCDs) of the GPU agent."""
    for r in _csv(dir_, "_agent_info.csv"):
        if r.get("Agent_Type", "").upper().find("GPU") >= 0:
            return int(r["Simd_Count"]), int(r["Num_Xcc"])
    raise ValueError("no GPU agent in agent_info")


def pmc_table(dir_: str) -> list[str]:
    simds, xcds = topology(dir_)
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for r in _csv(dir_, "_counter_collection.csv"):
        acc[_short(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    lines = [f"SIMDs {simds}, XCDs {xcds}; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs)", "",
             "| kernel | MFMA busy | VALU / MFMA instr | LDS instr / MFMA | LDS bank conflict / LDS active | wait / wave cycles |",
             "|---|---|---|---|---|---|"]
    for k in sorted(acc, key=_order):
        if _order(k)[0] == len(KERNELS):
            continue
        m = {c: sum(v) / len(v) for c, v in acc[k].items()}
        if "SQ_VALU_MFMA_BUSY_CYCLES" not in m or not m.get("GRBM_GUI_ACTIVE"):
            continue
        busy = m["SQ_VALU_MFMA_BUSY_CYCLES"] / (m["GRBM_GUI_ACTIVE"] / xcds * simds)
        mf = m.get("SQ_INSTS_MFMA", 0.0)
        f = lambda x: f"{x:.2f}" if x == x else "-"
        valu = m.get("SQ_INSTS_VALU", float("nan")) / mf if mf else float("nan")
        lds = m.get("SQ_INSTS_LDS", float("nan")) / mf if mf else float("nan")
        conf = m.get("SQ_LDS_BANK_CONFLICT", float("nan")) / m["SQ_LDS_IDX_ACTIVE"] if m.get("SQ_LDS_IDX_ACTIVE") else float("nan")
        wait = m.get("SQ_WAIT_ANY", float("nan")) / m["SQ_WAVE_CYCLES"] if m.get("SQ_WAVE_CYCLES") else float("nan")
        lines.append(f"| {k} | {100 * busy:.1f}% | {f(valu)} | {f(lds)} | {f(conf)} | {f(wait)} |")
    return lines


def copy_factor(dir_: str, counter: str, copy_bytes: int) -> float:
    """copied bytes / counter bytes of the largest copy dispatch."""
    best = 0.0
    for r in _csv(dir_, "_counter_collection.csv"):
        if r["Counter_Name"] == counter and COPY in r["Kernel_Name"]:
            best = max(best, float(r["Counter_Value"]) * 1024.0)
    if best <= 0:
        raise ValueError(f"no copy dispatch with {counter} in {dir_}")
    return copy_bytes / best


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--stats")
    ap.add_argument("--pmc")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-bytes", type=int, default=256 << 20)
    ap.add_argument("--json")
    args = ap.parse_args(argv)
    if args.stats:
        print("| kernel | calls | avg µs | total ms |\n|---|---|---|---|")
        for name, calls, avg, tot in kernel_stats(args.stats):
            print(f"| {name} | {calls} | {avg:.1f} | {tot:.2f} |")
    if args.pmc:
        print()
        print("\n".join(pmc_table(args.pmc)))
    if args.fetch and args.write:
        ff = copy_factor(args.fetch, "FETCH_SIZE", args.copy_bytes)
        wf = copy_factor(args.write, "WRITE_SIZE", args.copy_bytes)
        fetch = counter_means(args.fetch, "FETCH_SIZE")
        write = counter_means(args.write, "WRITE_SIZE")
        print(f"\ncalibration (copy of {args.copy_bytes} B): FETCH_SIZE x{ff:.4f}, WRITE_SIZE x{wf:.4f}\n")
        print("| kernel | FETCH KiB | WRITE KiB | HBM bytes per launch (calibrated) |\n|---|---|---|---|")
        out = {"copy_bytes": args.copy_bytes, "fetch_factor": ff, "write_factor": wf, "kernels": {}}
        for k in sorted(set(fetch) & set(write), key=lambda k: -(fetch[k][0] + write[k][0])):
            if k == COPY:
                continue
            b = fetch[k][0] * 1024 * ff + write[k][0] * 1024 * wf
            out["kernels"][k] = dict(fetch_kib=fetch[k][0], write_kib=write[k][0], bytes=b)
            print(f"| {k} | {fetch[k][0]:.0f} | {write[k][0]:.0f} | {b / 1e9:.3f} GB |")
        if args.json:
            with open(args.json, "w") as fh:
                json.dump(out, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Golden fixtures and the loaders the tests use to read them."""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def load_cases(fname: str) -> dict[str, dict]:
    """Group ``<case>__<key>`` arrays of a fixture file into per-case dicts."""
    z = np.load(os.path.join(HERE, fname), allow_pickle=False)
    out: dict[str, dict] = {}
    for key in z.files:
        case, field = key.split("__", 1)
        v = z[key]
        out.setdefault(case, {})[field] = v.item() if v.ndim == 0 else v
    return out


def load_flat(fname: str) -> dict:
    z = np.load(os.path.join(HERE, fname), allow_pickle=False)
    return {k: (z[k].item() if z[k].ndim == 0 else z[k]) for k in z.files}


def pointer_case_args(c: dict) -> dict:
    """Keyword arguments of ``oracle.pointer.pointer_mask_reference`` for a
    recorded reference case (after the call-site overrides)."""
    H, T, bs, M = int(c["H"]), int(c["T"]), int(c["bs"]), int(c["M"])
    local = c["cfg_build_local_blocks"] if c["cfg_build_local_blocks"] >= 0 else c["cfg_pointer_local_blocks"]
    half = c["cfg_build_ptr_half_blocks"] if c["cfg_build_ptr_half_blocks"] >= 0 else c["cfg_pointer_half_blocks"]
    budget = c["cfg_build_budget_blocks"] if c["cfg_build_budget_blocks"] >= 0 else c["cfg_pointer_budget_blocks"]
    gact = c["cfg_build_global_blocks"] if c["cfg_build_global_blocks"] >= 0 else c["cfg_global_active"]
    p = max(0, int(half))
    k = int(c["cfg_gumbel_topk_k"])
    if k <= 0 or k > M:
        k = M
    gumbel_active = bool(c["training"]) and bool(c["cfg_gumbel_topk"]) and p > 0 and k < M
    return dict(bs=bs, M=M, local_blocks=int(local), ptr_half_blocks=int(half),
                global_blocks_cfg=int(c["cfg_pointer_global_blocks"]), global_active=int(gact),
                budget_blocks=int(budget), budget_is_total=bool(c["cfg_pointer_budget_is_total"]),
                budget_temp=float(c["cfg_pointer_budget_temp"]), radius_mode=str(c["cfg_pointer_radius_mode"]),
                doc_clamp=bool(c["cfg_pointer_doc_clamp"]), mask_active=bool(c["cfg_mask_active"]),
                half_active=int(c["cfg_half_active"]), reset_active=bool(c["cfg_reset_active"]),
                reset_len=int(c["cfg_reset_len_active"]), gumbel_active=gumbel_active, gumbel_k=k,
                gumbel_tau=float(c["cfg_gumbel_topk_tau"]), eps=float(c["cfg_eps"]))


def pointer_case_reps(c: dict) -> tuple[np.ndarray, np.ndarray]:
    """Representatives [H,QB,M] of a recorded case."""
    from oracle.pointer import representatives

    if c["rep_mode"] == "last":
        return c["delta_rep"].astype(np.float32), c["budget_rep"].astype(np.float32)
    bs = int(c["bs"])
    return (representatives(c["delta_star"], bs, "mean"), representatives(c["budget_logits"], bs, "mean"))

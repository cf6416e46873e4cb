"""Benchmark of the SCOPE attention hot path on one MI355X.

One step = one pass of the hot path over one synthetic batch:
doc starts -> block means -> pointer selection (block-mean q·k + Gumbel top-k
under the budget) -> mask statistics -> q-list transpose -> block-sparse
attention forward -> backward (dq, dk, dv and the spectral coefficient
gradients).  Inputs are resident in HBM before the timed region.

Workload (long-context prefill, one layer): B=1, H=8, T=131072, D=128 bf16,
block 256 (512 blocks), window 2, 2 doc-local global blocks, pointer budget 8
(sweep {2,4,8} with --sweep), 8 spectral bands ω_k = π·2^-k over block
offsets with coefficients q·W_b (W_b ~ N(0, 0.02) [D,16]), documents starting
at seeded positions (~1 per 8192 tokens), a planted needle (a key block equal
to 3 × a query block's mean query, ≥ 64 blocks back), seeded in-kernel Gumbel
noise, dO ~ N(0,1).

value = active-block TFLOP/s = (F_fwd + F_bwd) / step time, with
F_fwd = 4·bs²·D·N_act, F_bwd = 10·bs²·D·N_act, N_act = Σ kv_num_blocks.

The million-token layer (T=1048576, 4096 blocks of 256, window 2, one global
block, budget 8, one document, no needle) is the same workload with
``--T 1048576 --n-global 1 --docs 1 --no-needle``.

``--workload swa`` times instead a layer without the pointer mask: the long
sliding-window mask (scoped_medium.py:535-576, window 14 blocks of 128 = the
reference's final 1792-token window) built from the document ids, the q-list
transpose and the attention forward and backward without a bias, at
T=65536, H=8, D=128 (the training shape).

``--workload coeff`` times the coefficient head of SpectralBias.forward after
its MLP (model/attn_bias.py:419-506, M=8 peaks, K=8 bands, regularisers on)
forward and backward at T=131072, H=8: the fused kernels against the same
module's torch steps on the same GPU.

``--workload teacher`` times the teacher's block mass (scoped_medium.py:
1799-1819: dense document-causal attention with the token-offset band term
and slope, probabilities summed per q-block and key block) at the teacher's
length T=4096 (8 heads, bs 128) and at T=65536.

``--workload train`` times the training-shape layer: T=65536, H=8, D=128,
block 128 (512 blocks), window 4, 1 global block, pointer budget 4, one
document, seeded in-kernel Gumbel noise, no needle, the same spectral bias,
with the soft pointer weights on (``--soft-temp``, default 4): each pick's
weight log σ(z/τ_w) enters its tile's scores, and the backward carries their
gradient through the block means into dq and dk (pointer backward timed as
its own phase).  ``--soft-temp`` also turns the weights on for the default
workload.

``--workload ref`` times the reference's default layer path (its defaults:
T=16384, bs 128, K=6 token-offset bands with slope as in qk_aug, reference-mode
lists with local 8, half 4, M 8, budget 64 in total, temperature 0.5): the
coefficient head, the reference-mode mask, the attention and the whole
backward; ``--T 65536`` for the training shape.

The default line also carries, timed after the headline with their own
events: ``reference_default_layer`` (the ``--workload ref`` figures below at
T=16384), and in ``cpu_baseline`` the oracle's attention on a bounded sample,
the reference's own CPU path at config 1, and ``pointer_and_stats``: the
oracle's block-scoring selection and mask statistics (kernels 1 and 3) on the
host at config 1 and at this workload, beside the GPU time of the same two
phases.

``--workload decode`` runs the 16-layer decoder (d_model 1024, 8 heads of
128, MLP 4096 ReLU², vocabulary 50304, bf16, random weights): a prefill of
131072 seeded uniform-random tokens, then 256 greedy decode steps with the
pointer lists (window 4 blocks of 128, budget 4, 1 global) reselected at every
new q-block (the steps inside a block replay one captured HIP graph).
value = decode tokens/s; the prefill time is reported beside it.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "SCOPE attn fwd+bwd active-block TFLOP/s & tokens/s at T=128k, 1 MI355X"
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--budget", type=int, default=8)
    ap.add_argument("--T", type=int, default=131072)
    ap.add_argument("--H", type=int, default=8)
    ap.add_argument("--bs", type=int, default=256)
    ap.add_argument("--window", type=int, default=2)
    ap.add_argument("--n-global", type=int, default=2)
    ap.add_argument("--sweep", action="store_true", help="also time budgets 2 and 4")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ref-layer", action="store_true",
                    help="leave the reference's default layer out of the default line (profiles of the headline "
                         "kernels alone)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--workload", choices=["pointer", "train", "swa", "coeff", "teacher", "decode", "ref"],
                    default="pointer")
    ap.add_argument("--soft-temp", type=float, default=0.0,
                    help="soft pointer weights log σ(z/τ) on the picks (0: default, off except --workload train: 4; < 0: off)")
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--docs", type=int, default=0,
                    help="documents at seeded positions (0: one per 8192 tokens; the training shape: 1)")
    ap.add_argument("--no-needle", action="store_true", help="no planted needle block")
    ap.add_argument("--swa-window", type=int, default=14, help="long-mask window in blocks (--workload swa)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, one plain device copy of this many MiB (calibrates HBM byte counters)")
    return ap.parse_args()


def make_inputs(H, T, D, bs, seed=0, n_docs=None, needle=True):
    import torch

    g = torch.Generator().manual_seed(seed)
    q = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16)
    k = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16)
    v = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16)
    dout = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16)
    n_docs = max(1, T // 8192) if n_docs is None else n_docs
    cuts = torch.randperm(T - 1, generator=g)[: n_docs - 1] + 1
    flag = torch.zeros(T, dtype=torch.int64)
    flag[cuts] = 1
    docs = flag.cumsum(0).to(torch.int32)
    NB = T // bs
    # planted needle: key block kb = 3 × mean query of block qb, at a seeded
    # distance of at least 64 blocks (pointer candidates are document-local,
    # so both sit in the longest document: qb its last whole block, kb clear
    # of its global blocks; when the document is shorter than 64 + 4 blocks,
    # as far back as it allows)
    bd = docs[::bs]  # document of each block's first token
    starts = [0] + [b for b in range(1, NB) if bd[b] != bd[b - 1]] + [NB]
    # whole blocks of document i: from its first block whose first token is in it
    spans = [(starts[i], starts[i + 1] - 1) for i in range(len(starts) - 1)]
    fb, lb = max(spans, key=lambda sp: sp[1] - sp[0])
    qb_n = lb - 1  # block lb may hold the next document's first tokens
    room = qb_n - (fb + 3)  # farthest distance that stays clear of the document's global blocks
    if room >= 64:  # seeded distance of at least 64 blocks
        dist = 64 + int(torch.randint(0, room - 64 + 1, (1,), generator=g))
    else:
        dist = max(4, room)
    kb_n = qb_n - dist
    if needle:
        mq = q[0, :, qb_n * bs:(qb_n + 1) * bs].float().mean(dim=1)
        k[0, :, kb_n * bs:(kb_n + 1) * bs] = (3.0 * mq[:, None, :]).to(torch.bfloat16)
    W = torch.randn((D, 16), generator=g) * 0.02
    c = q.float() @ W
    coeff_cos, coeff_sin = c[..., :8].contiguous(), c[..., 8:].contiguous()
    omegas = torch.tensor([math.pi * 2.0 ** (-i) for i in range(8)], dtype=torch.float32)
    return dict(q=q, k=k, v=v, dout=dout, docs=docs, coeff_cos=coeff_cos, coeff_sin=coeff_sin, omegas=omegas,
                needle=(qb_n, kb_n) if needle else None)


PRIOR_SCALE = 0.5


def radius_prior(NB: int, scale: float):
    """Radius prior of the block-scoring logits over the block distance
    r = qb - kb: prior[r] = -scale·ln(1 + r), a power-law preference for
    nearer blocks (the reference spreads its pointer offsets Δ* over a
    log-spaced range, model/attn_bias.py:220-226)."""
    import torch

    return -scale * torch.log1p(torch.arange(NB, dtype=torch.float32))


class EventSets:
    """One set of start/end events per recorded step, so that the recorded
    steps run back to back, as in the timed region (no synchronisation
    between them: a phase at the start of a step does not absorb the host's
    launch latency), and are read after one synchronisation."""

    def __init__(self, names):
        self.names = list(names)
        self.sets: list = []
        self.n = 0

    def next(self):
        import torch

        if self.n == len(self.sets):
            self.sets.append({p: (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                              for p in self.names})
        ev = self.sets[self.n]
        self.n += 1
        return ev

    def drain(self):
        used, self.n = self.sets[:self.n], 0
        return used


class Step:
    """The hot path on GPU-resident inputs; phase events on the current stream."""

    def __init__(self, inp, *, bs, window, n_global, budget, seed=1234, soft_temp=0.0, prior_scale=PRIOR_SCALE):
        import torch

        from scope_amd import ops
        from scope_amd.attention import spectral_table

        self.t = {k_: (v_.cuda() if torch.is_tensor(v_) else v_) for k_, v_ in inp.items()}
        self.bs, self.window, self.n_global, self.budget, self.seed = bs, window, n_global, budget, seed
        self.H, self.T = self.t["q"].shape[1], self.t["q"].shape[2]
        self.NB = self.T // bs
        self.prior = radius_prior(self.NB, prior_scale).cuda() if prior_scale > 0 else None
        self.table = spectral_table(self.t["omegas"], self.T, bs, "block")
        self.ops = ops
        self.soft_temp = float(soft_temp)
        self.phases = ["pointer", "stats", "transpose", "attn_fwd", "attn_bwd_dq", "attn_bwd_dkv", "attn_bwd_aux"]
        if self.soft_temp > 0:
            self.phases.append("pointer_bwd")
        # "_aux": the span of the kv-major kernels; "_means": the block means alone
        self.evs = EventSets(self.phases + ["_aux", "_means"])
        self.acc = {p: 0.0 for p in self.phases}
        self.means_ms = 0.0

    def __call__(self, record=False):
        ops, t, bs = self.ops, self.t, self.bs
        ev = self.evs.next() if record else None

        def mark(p, i):
            if record:
                ev[p][i].record()

        mark("pointer", 0)
        # block means with the document starts folded in (the per-block phase
        # rides on the block-means pass, then the scan)
        mark("_means", 0)
        qbar, kbar, ds_ptr, ds_local, ds_tok_end = ops.block_means_docs(t["q"], t["k"], t["docs"], bs)
        mark("_means", 1)
        ls = bs / math.sqrt(t["q"].shape[-1])
        kv_num, kv_idx, picks = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=self.NB, H=self.H,
                                                   window=self.window, n_global=self.n_global, budget=self.budget,
                                                   qbar=qbar, kbar=kbar, prior=self.prior, temp=1.0, logit_scale=ls,
                                                   noise="counter", seed=self.seed)
        soft = self.soft_temp > 0
        pb = None
        if soft:
            pb = ops.pointer_pair_bias(kv_num, kv_idx, picks, bs=bs, window=self.window, n_global=self.n_global,
                                       soft_temp=self.soft_temp, qbar=qbar, kbar=kbar, prior=self.prior,
                                       logit_scale=ls, check=False)
        mark("pointer", 1)
        mark("stats", 0)
        counts, values = ops.mask_stats(H=self.H, QB=self.NB, bs=bs, kv_num=kv_num, picks=picks, ds_ptr=ds_ptr,
                                        ds_local=ds_local, maxkv_bins=kv_idx.shape[-1] + 1,
                                        bs_local_blocks=self.window)
        mark("stats", 1)
        mark("transpose", 0)
        q_off, q_list = ops.transpose_blocks(kv_num, kv_idx, self.NB, check=False)
        mark("transpose", 1)
        mark("attn_fwd", 0)
        out, lse = ops.attn_fwd(t["q"], t["k"], t["v"], kv_num, kv_idx, t["docs"], ds_tok_end, bs=bs, scale=0.12,
                                beta=0.5, bias_mode="block", table=self.table, coeff_cos=t["coeff_cos"],
                                coeff_sin=t["coeff_sin"], pair_bias=pb, check=False)
        mark("attn_fwd", 1)
        # attn_bwd_dkv is the dK/dV kernel alone; attn_bwd_aux its plan and reduce kernels

        def hook(phase):
            if phase == "dq":
                mark("attn_bwd_dq", 0)
            elif phase == "plan":
                mark("attn_bwd_dq", 1)
                mark("attn_bwd_aux", 0)
            elif phase == "dkv":
                mark("_aux", 0)
                mark("attn_bwd_dkv", 0)
            elif phase == "reduce":
                mark("attn_bwd_dkv", 1)
                mark("_aux", 1)
            else:
                mark("attn_bwd_aux", 1)

        grads = ops.attn_bwd(t["q"], t["k"], t["v"], out, t["dout"], lse, kv_num, kv_idx, q_off, q_list, t["docs"],
                             ds_tok_end, bs=bs, scale=0.12, beta=0.5, bias_mode="block", table=self.table,
                             coeff_cos=t["coeff_cos"], coeff_sin=t["coeff_sin"], phase_hook=hook, pair_bias=pb,
                             need_pair_grad=soft, check=False)
        if soft:
            mark("pointer_bwd", 0)
            ops.pointer_bwd(qbar, kbar, kv_num, kv_idx, q_off, q_list, pb, grads["dpair_bias"], grads["dq"],
                            grads["dk"], bs=bs, logit_scale=ls, soft_temp=self.soft_temp, check=False)
            mark("pointer_bwd", 1)
        self.last = dict(kv_num=kv_num, kv_idx=kv_idx, picks=picks, counts=counts, values=values, out=out, lse=lse,
                         grads=grads, q_off=q_off, q_list=q_list, ds_tok_end=ds_tok_end, pair_bias=pb)

    def collect(self):
        for ev in self.evs.drain():
            for p in self.phases:
                self.acc[p] += ev[p][0].elapsed_time(ev[p][1])
            # the aux span brackets the dK/dV kernel: remove it
            self.acc["attn_bwd_aux"] -= ev["_aux"][0].elapsed_time(ev["_aux"][1])
            self.means_ms += ev["_means"][0].elapsed_time(ev["_means"][1])


class SwaStep:
    """A layer without the pointer mask: sliding-window lists, transpose,
    attention forward and backward (no bias)."""

    def __init__(self, inp, *, bs, window):
        import torch

        from scope_amd import ops

        self.t = {k_: (v_.cuda() if torch.is_tensor(v_) else v_) for k_, v_ in inp.items()}
        self.bs, self.window, self.ops = bs, window, ops
        self.H, self.T = self.t["q"].shape[1], self.t["q"].shape[2]
        self.NB = self.T // bs
        self.phases = ["swa_mask", "transpose", "attn_fwd", "attn_bwd"]
        self.evs = EventSets(self.phases)
        self.acc = {p: 0.0 for p in self.phases}

    def __call__(self, record=False):
        ops, t, bs = self.ops, self.t, self.bs
        ev = self.evs.next() if record else None

        def mark(p, i):
            if record:
                ev[p][i].record()

        mark("swa_mask", 0)
        r = ops.swa_blockmask(t["docs"], bs, self.window)
        _, _, ds_tok_end = ops.doc_starts(t["docs"], bs)
        kv_num = r["long"][0].expand(self.H, -1).contiguous()
        kv_idx = r["long"][1].expand(self.H, -1, -1).contiguous()
        mark("swa_mask", 1)
        mark("transpose", 0)
        q_off, q_list = ops.transpose_blocks(kv_num, kv_idx, self.NB, check=False)
        mark("transpose", 1)
        mark("attn_fwd", 0)
        out, lse = ops.attn_fwd(t["q"], t["k"], t["v"], kv_num, kv_idx, t["docs"], ds_tok_end, bs=bs, scale=0.12,
                                bias_mode="none", check=False)
        mark("attn_fwd", 1)
        mark("attn_bwd", 0)
        grads = ops.attn_bwd(t["q"], t["k"], t["v"], out, t["dout"], lse, kv_num, kv_idx, q_off, q_list, t["docs"],
                             ds_tok_end, bs=bs, scale=0.12, bias_mode="none", check=False)
        mark("attn_bwd", 1)
        self.last = dict(kv_num=kv_num, kv_idx=kv_idx, out=out, lse=lse, grads=grads)

    def collect(self):
        for ev in self.evs.drain():
            for p in self.phases:
                self.acc[p] += ev[p][0].elapsed_time(ev[p][1])


def main_swa(args):
    import torch

    H, T, D, bs = args.H, args.T, 128, args.bs
    inp = make_inputs(H, T, D, bs)
    step = SwaStep(inp, bs=bs, window=args.swa_window)
    step()
    torch.cuda.synchronize()
    n_act = int(step.last["kv_num"].sum())
    F_fwd, F_bwd = 4.0 * bs * bs * D * n_act, 10.0 * bs * bs * D * n_act
    t_step = time_region(step, args.steps, args.warmup)
    time_steps(step, args.steps, 0)
    ph = {p: step.acc[p] / args.steps for p in step.phases}
    fwd_tf = F_fwd / (ph["attn_fwd"] / 1e3) / 1e12
    res = {
        "metric": "SWA attn fwd+bwd active-block TFLOP/s (layer without the pointer mask), 1 MI355X",
        "value": round((F_fwd + F_bwd) / t_step / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "one attention layer fwd+bwd over the long sliding-window mask (mask build + "
                               "transpose + attention, no bias)", "B": 1, "H": H, "T": T, "D": D, "block": bs,
                   "window_blocks": args.swa_window, "docs": max(1, T // 8192)},
        "tokens_per_s": round(T / t_step, 1),
        "n_act": n_act,
        "breakdown_ms": {p: round(v_, 4) for p, v_ in ph.items()},
        "attn_fwd_tflops": round(fwd_tf, 2),
        "attn_bwd_tflops": round(F_bwd / (ph["attn_bwd"] / 1e3) / 1e12, 2),
        "roofline": dict(bound="mfma", kernel="attn_fwd_kernel", achieved=round(fwd_tf, 2), peak=PEAK_BF16_TFLOPS,
                         unit="TFLOP/s", frac=round(fwd_tf / PEAK_BF16_TFLOPS, 4), traffic=None),
    }
    print(json.dumps(res))


def main_coeff(args):
    import torch

    from scope_amd import SpectralBias, ops

    H, T, M, K = args.H, args.T, 8, 8
    sb = SpectralBias(head_dim=128, num_heads=H, L_train=T, M=M, K=K).cuda().train()
    g = torch.Generator(device="cuda").manual_seed(0)
    Y = 5 * M + 1
    y = (torch.randn((1, H, T, Y), generator=g, device="cuda") * 2).to(torch.bfloat16)
    _, _, cm, sm = sb._get_trig_tables(T, y.device)
    prm = sb._head_params(T)
    names = ("coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width")
    o = ops.coeff_head_fwd(y, prm, sb.omegas, sb.log_omegas, cm, sm)
    grads = {n: torch.randn(o[n].shape, generator=g, device="cuda") for n in names}
    g_reg = torch.ones((), device="cuda")

    def fused():
        r = ops.coeff_head_fwd(y, prm, sb.omegas, sb.log_omegas, cm, sm)
        ops.coeff_head_bwd(y, prm, sb.omegas, sb.log_omegas, cm, sm, grads, g_reg, r["reg"])

    t_fused = time_region(fused, args.steps, args.warmup)
    rows = H * T
    # algorithmic bytes: fwd reads y (bf16) and writes the outputs (fp32); bwd reads y and the
    # upstream gradients of the outputs and writes dy (bf16)
    out_b = (2 * K + 4 + 3 * M) * 4
    bytes_ = rows * (Y * 2 + out_b + Y * 2 + out_b + Y * 2)
    ach = bytes_ / t_fused / 1e9
    res = {
        "metric": "coefficient head (after the MLP) fwd+bwd rows/s, 1 MI355X",
        "value": round(rows / t_fused, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_fused * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "SpectralBias coefficient head after the MLP, fwd+bwd with regularisers", "B": 1,
                   "H": H, "T": T, "M": M, "K": K, "y_dtype": "bf16"},
        "roofline": dict(bound="hbm", kernel="coeff_fwd_kernel+coeff_bwd_kernel", achieved=round(ach, 1),
                         peak=PEAK_HBM_GBS, unit="GB/s", frac=round(ach / PEAK_HBM_GBS, 4), traffic=None,
                         bytes_per_step=bytes_),
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_coeff(sb, names, args.cpu_seconds)
    print(json.dumps(res))


def cpu_baseline_coeff(sb, names, seconds: float):
    """The reference's coefficient-head steps after the MLP (the oracle's
    torch ops, model/attn_bias.py:419-506) forward + autograd backward with
    the regularisers on the host cores, over a bounded sample: batches of
    4096 rows per head of random MLP outputs, until `seconds` are spent."""
    import copy

    import torch

    from oracle.coeff_head import coeff_head_forward

    torch.set_num_threads(os.cpu_count() or 1)
    cpu = copy.deepcopy(sb).cpu().float().train()
    H, M, L = cpu.num_heads, cpu.M, 4096
    Y = 5 * M + (1 if cpu.use_slope else 0)
    g = torch.Generator().manual_seed(0)
    q = torch.zeros((1, H, L, cpu.head_dim))
    done, t_used = 0, 0.0
    while t_used < seconds:
        y = (torch.randn((1, H, L, Y), generator=g) * 2).requires_grad_()
        cpu._mlp_forward = lambda _q, y=y: y  # the head alone, like the timed kernels
        t0 = time.perf_counter()
        out = coeff_head_forward(cpu, q)
        loss = sum(out[i].sum() for i in range(len(names))) + out[11]
        loss.backward()
        t_used += time.perf_counter() - t0
        done += H * L
    return dict(value=round(done / t_used, 1), unit="rows/s", cores=torch.get_num_threads(), kind="port",
                sample=f"oracle coefficient head after the MLP (torch fp32 on CPU) fwd+bwd with regularisers "
                       f"over {done} rows ({t_used:.1f} s)", cpu_model=cpu_model())


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def main_teacher(args):
    import torch

    import scope_amd

    H, D, bs, K = args.H, 128, 128, 8
    lines = {}
    for T in (4096, 65536):
        inp = make_inputs(H, T, D, bs)
        q, k, docs = inp["q"].cuda(), inp["k"].cuda(), inp["docs"].cuda()
        g = torch.Generator().manual_seed(7)
        sp = scope_amd.SpectralTerms(coeff_cos=(torch.randn((1, H, T, K), generator=g) * 0.3).cuda(),
                                     coeff_sin=(torch.randn((1, H, T, K), generator=g) * 0.3).cuda(),
                                     omegas=torch.logspace(-5.0, -1.3, K).cuda(), offset="token", beta=0.5,
                                     slope=(torch.randn((1, H, T), generator=g) * 0.002).cuda(), use_slope=True)

        def step():
            scope_amd.attention.teacher_block_mass(q, k, docs, scale=0.12, spectral=sp, block_size=bs)

        t = time_region(step, args.steps, args.warmup)
        # active tiles of the dense document-causal lists: Σ_qb (qb - first + 1)
        from scope_amd import ops

        _, ds_local, _ = ops.doc_starts(docs, bs)
        nb = T // bs
        n_act = H * int((torch.arange(nb, device="cuda") - ds_local + 1).sum())
        flops = 2 * (2.0 * bs * bs * D) * n_act  # two passes of S = q·k^T over every listed tile
        lines[str(T)] = dict(ms=round(t * 1e3, 4), n_act=n_act, tflops=round(flops / t / 1e12, 2))
    res = {
        "metric": "teacher block mass (dense document-causal attention probabilities per block) TFLOP/s, 1 MI355X",
        "value": lines["4096"]["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": lines["4096"]["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "teacher block mass (LSE pass + mass pass, token band term + slope)", "B": 1, "H": H,
                   "T": 4096, "D": D, "block": bs, "bands": K},
        "by_length": lines,
        "roofline": dict(bound="mfma", kernel="attn_fwd_kernel (lse + mass)", achieved=lines["65536"]["tflops"],
                         peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                         frac=round(lines["65536"]["tflops"] / PEAK_BF16_TFLOPS, 4), traffic=None, at_T=65536),
    }
    print(json.dumps(res))


def main_decode(args):
    import torch

    from scope_amd.decode import DecoderConfig, ScopeDecoder

    T0 = args.T if args.T != 131072 or args.bs != 256 else 131072
    n = args.decode_steps
    cfg = DecoderConfig()
    m = ScopeDecoder(cfg, max_len=T0 + ((n + cfg.block_size) // cfg.block_size) * cfg.block_size, device="cuda",
                     seed=0)
    g = torch.Generator().manual_seed(0)
    toks = torch.randint(0, cfg.vocab_size, (T0 + 1,), generator=g)
    # warm-up on a short prompt (kernels, allocator), then the measured run
    w = ScopeDecoder(cfg, max_len=1024, device="cuda", seed=1)
    w.prefill(toks[:512])
    w.generate(8, int(toks[512]))
    del w
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = m.prefill(toks[:T0])
    torch.cuda.synchronize()
    t_pre = time.perf_counter() - t0
    first = int(logits[:cfg.vocab_size].argmax())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = m.generate(n, first)
    torch.cuda.synchronize()
    t_dec = time.perf_counter() - t0
    res = {
        "metric": "SCOPE decoder greedy decode tokens/s after a 131072-token prefill (16 layers), 1 MI355X",
        "value": round(n / t_dec, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": 8,
        "ms_per_step": round(t_dec / n * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "16-layer decoder: prefill + greedy token loop", "layers": cfg.num_layers,
                   "d_model": cfg.model_dim, "H": cfg.num_heads, "D": cfg.head_dim, "mlp": 4 * cfg.model_dim,
                   "vocab": cfg.vocab_padded, "prefill_tokens": T0, "decode_steps": n, "block": cfg.block_size,
                   "window": cfg.window, "budget": cfg.budget, "global": cfg.n_global},
        "prefill_ms": round(t_pre * 1e3, 2),
        "prefill_tokens_per_s": round(T0 / t_pre, 1),
        "generated_head": out[:8].tolist(),
    }
    print(json.dumps(res))


def main_ref(args):
    """The reference's default layer path as its own bench line (see ref_layer)."""
    print(json.dumps(ref_layer(args.H, args.T if args.T != 131072 else 16384, args.steps, args.warmup)))


def ref_layer(H: int, T: int, steps: int, warmup: int) -> dict:
    """The reference's default layer path (scoped_medium.py:334-466 with the
    defaults of :692-727): SpectralBias.forward (MLP + coefficient head, K=6
    bands, M=8 peaks), build_pointer_blockmask in reference mode (local 8,
    half 4, budget 64 in total, temperature 0.5, "pi" radii, no global
    blocks), the attention with the qk_aug terms (token offsets, slope, no
    gate) and the whole backward, through scope_attention / SpectralBias as
    the reference would call them.  Timed with events around `steps`
    back-to-back steps after `warmup`."""
    import torch

    from scope_amd import SpectralBias, SpectralTerms, scope_attention

    D, bs = 128, 128
    inp = make_inputs(H, T, D, bs, needle=False)
    q, k, v, dout, docs = (inp[n].cuda() for n in ("q", "k", "v", "dout", "docs"))
    sb = SpectralBias(head_dim=D, num_heads=H, L_train=4096, K=6, M=8, use_pointer_mask=True,
                      pointer_local_blocks=8, pointer_half_blocks=4, pointer_budget_blocks=64,
                      pointer_budget_is_total=True, pointer_budget_temp=0.5, pointer_radius_mode="pi",
                      pointer_global_blocks=0).cuda().train()
    sb.set_delta_star_max_active(max_tokens=T - 1)
    g = torch.Generator(device="cuda").manual_seed(0)
    with torch.no_grad():  # a spread of pointer offsets (the reference zero-initialises the head's last layer)
        for p_ in sb.mlp.parameters():
            p_.copy_(torch.randn(p_.shape, generator=g, device="cuda") * 0.05)
    one = torch.ones((), device="cuda")

    def layer(q_, k_, v_):
        out = sb(q_, docs=docs)
        bm = sb.build_pointer_blockmask(docs=docs, delta_star=out[4], pi=out[5], budget_logits=out[6], block_size=bs)
        sp = SpectralTerms(coeff_cos=out[0], coeff_sin=out[1], omegas=sb.omegas, offset="token", beta=sb.beta,
                           slope=out[2], use_slope=True)
        return scope_attention(q_, k_, v_, block_mask=bm, scale=0.12, spectral=sp), out[11], bm

    params = list(sb.parameters())

    def step():
        for p_ in params:  # a training step's zero_grad(set_to_none=True): no accumulation adds
            p_.grad = None
        qd, kd, vd = (x.detach().requires_grad_() for x in (q, k, v))
        y, reg, _ = layer(qd, kd, vd)
        torch.autograd.backward([y, reg], [dout, one])

    with torch.no_grad():
        _, _, bm = layer(q, k, v)
    n_act = int(bm.kv_num_blocks.sum())
    maxkv = bm.maxkv
    t_step = time_region(step, steps, warmup)
    # the attention alone on the same lists and terms
    qd, kd, vd = (x.detach().requires_grad_() for x in (q, k, v))
    with torch.no_grad():
        out = sb(q, docs=docs)
    sp = SpectralTerms(coeff_cos=out[0], coeff_sin=out[1], omegas=sb.omegas, offset="token", beta=sb.beta,
                       slope=out[2], use_slope=True)

    def attn_fwd_only():
        with torch.no_grad():
            scope_attention(q, k, v, block_mask=bm, scale=0.12, spectral=sp)

    def attn_fwd_bwd():
        qd.grad = kd.grad = vd.grad = None  # no gradient accumulation adds in the timed region
        y = scope_attention(qd, kd, vd, block_mask=bm, scale=0.12, spectral=sp)
        y.backward(dout)

    t_fwd = time_region(attn_fwd_only, steps, warmup)
    t_attn = time_region(attn_fwd_bwd, steps, warmup)
    graph = graph_step_time(layer, q, k, v, dout, one, steps, params)
    F_fwd, F_bwd = 4.0 * bs * bs * D * n_act, 10.0 * bs * bs * D * n_act
    res = {
        "metric": "SCOPE layer fwd+bwd on the reference's default path (qk_aug terms, reference-mode lists) "
                  "active-block TFLOP/s, 1 MI355X",
        "value": round((F_fwd + F_bwd) / t_step / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(t_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "reference default layer: coefficient head + reference-mode pointer mask + attention "
                               "(token offsets, K=6, slope, no gate) fwd+bwd", "B": 1, "H": H, "T": T, "D": D,
                   "block": bs, "local": 8, "half": 4, "M": 8, "budget_total": 64, "budget_temp": 0.5,
                   "global": 0, "maxkv": maxkv, "docs": max(1, T // 8192)},
        "tokens_per_s": round(T / t_step, 1),
        "n_act": n_act,
        "attn_fwd_ms": round(t_fwd * 1e3, 4),
        "attn_fwd_tflops": round(F_fwd / t_fwd / 1e12, 2),
        "attn_fwd_bwd_ms": round(t_attn * 1e3, 4),
        # the same step replayed from one captured HIP graph: no host launch
        # overhead (eager, the ~45 launches of the module path can outrun a slow
        # host's Python); equal to eager bit for bit on every replay checked
        "graph_ms_per_step": graph["ms"], "graph_tflops": (round((F_fwd + F_bwd) / graph["ms"] / 1e9, 2)
                                                          if graph["ms"] else None),
        "graph_check": graph["check"],
        "attn_fwd_bwd_tflops": round((F_fwd + F_bwd) / t_attn / 1e12, 2),
        "roofline": dict(bound="mfma", kernel="attention fwd+bwd (token mode)",
                         achieved=round((F_fwd + F_bwd) / t_attn / 1e12, 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                         frac=round((F_fwd + F_bwd) / t_attn / 1e12 / PEAK_BF16_TFLOPS, 4), traffic=None),
    }
    return res


def graph_step_time(layer, q, k, v, dout, one, steps: int, params=()) -> dict:
    """ms per fwd+bwd step of `layer` replayed from a captured HIP graph, and
    whether each checked replay's output equals an eager step's bit for bit."""
    import torch

    qs, ks, vs = (x.detach().clone().requires_grad_() for x in (q, k, v))

    def body():
        # fresh gradients each step, as the eager step's fresh leaves get
        # (accumulating into .grad would add three q-sized sums per step)
        qs.grad = ks.grad = vs.grad = None
        for p_ in params:
            p_.grad = None
        y, reg, _ = layer(qs, ks, vs)
        torch.autograd.backward([y, reg], [dout, one])
        return y

    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                body()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y_g = body()
        with torch.no_grad():
            y_e = layer(q, k, v)[0]
        ok = True
        for _ in range(3):  # replays with eager work and synchronisations between them
            g.replay()
            torch.cuda.synchronize()
            ok = ok and bool(torch.equal(y_g, y_e))
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return dict(ms=round(e0.elapsed_time(e1) / steps, 4), check="equal to eager" if ok else "DIFFERS from eager")
    except Exception as ex:  # capture not possible here: report why, keep the eager numbers
        return dict(ms=None, check=f"not captured: {type(ex).__name__}: {ex}"[:200])


def graph_time_layer(step, steps: int) -> dict:
    """ms per step of the headline step replayed from one captured HIP graph
    (no host launches between the ~40 kernels), and whether every checked
    replay's lists, output, LSE and gradients equal an eager step's bit for
    bit."""
    import torch

    keys = ("kv_num", "kv_idx", "out", "lse")
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        cap = dict(step.last)
        step()  # eager, fresh tensors
        torch.cuda.synchronize()
        ref = dict(step.last)

        def same():
            a = [cap[k_] for k_ in keys] + [cap["grads"][n_] for n_ in ("dq", "dk", "dv")]
            b = [ref[k_] for k_ in keys] + [ref["grads"][n_] for n_ in ("dq", "dk", "dv")]
            return all(bool(torch.equal(x, y)) for x, y in zip(a, b))

        ok = True
        for _ in range(3):  # replays with eager work and synchronisations between them
            g.replay()
            torch.cuda.synchronize()
            ok = ok and same()
            step()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return dict(ms=round(e0.elapsed_time(e1) / steps, 4), check="equal to eager" if ok else "DIFFERS from eager")
    except Exception as ex:  # capture not possible here: report why, keep the eager numbers
        return dict(ms=None, check=f"not captured: {type(ex).__name__}: {ex}"[:200])


def time_steps(step, steps, warmup):
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(record=True)  # back to back, as in the timed region
    torch.cuda.synchronize()
    step.collect()
    return (time.perf_counter() - t0) / steps


def time_region(step, steps, warmup):
    """Whole-step time with events bracketing exactly `steps` back-to-back steps."""
    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps / 1000.0


def measured_traffic(kernel: str, H: int, T: int, bs: int, budget: int):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary of
    this workload (FETCH_SIZE + WRITE_SIZE, each scaled by a calibration copy),
    or (None, None) when no summary for this exact workload is present."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_T{T}_H{H}_bs{bs}_b{budget}.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as fh:
        data = json.load(fh)
    kernels = data.get("kernels", {})
    k = kernels.get(kernel) or kernels.get(kernel.split("<")[0])
    if not k:
        return None, None
    return int(k["bytes"]), os.path.relpath(path, ROOT)


def cpu_baseline(inp, step, seconds: float, bs: int):
    """The oracle's block-sparse attention fwd+bwd (torch fp32, all host
    threads) on a bounded sample of q-blocks of head 0 with their real lists."""
    import torch

    from oracle import attention as OA

    torch.set_num_threads(os.cpu_count() or 1)
    kv_num = step.last["kv_num"].cpu()
    kv_idx = step.last["kv_idx"].cpu()
    pb = step.last.get("pair_bias")
    pb = None if pb is None else pb.float().cpu()
    docs = inp["docs"]
    H, T, D = inp["q"].shape[1:]
    QB = T // bs
    q, k, v = (inp[n][0].float() for n in ("q", "k", "v"))
    dout = inp["dout"][0].float()
    cc, cs, om = inp["coeff_cos"][0].float(), inp["coeff_sin"][0].float(), inp["omegas"].float()
    done_tiles, t_used, n_rows = 0, 0.0, 0
    i = 0
    while t_used < seconds and i < H * QB:
        h, qb = (i * 7) % H, (QB - 1 - (i * 37) % QB)  # spread the sample over heads and the sequence
        i += 1
        qq = q[h:h + 1].clone().requires_grad_()
        kk = k[h:h + 1].clone().requires_grad_()
        vv = v[h:h + 1].clone().requires_grad_()
        t0 = time.perf_counter()
        res = OA.attention_blocksparse(qq, kk, vv, kv_num[h:h + 1], kv_idx[h:h + 1], docs, bs=bs, scale=0.12,
                                       beta=0.5, bias_mode="block", coeff_cos=cc[h:h + 1], coeff_sin=cs[h:h + 1],
                                       omegas=om, heads=[0], qblocks=[qb],
                                       pair_bias=None if pb is None else pb[h:h + 1])
        o, _ = res[(0, qb)]
        o.backward(dout[h, qb * bs:(qb + 1) * bs])
        t_used += time.perf_counter() - t0
        done_tiles += int(kv_num[h, qb])
        n_rows += 1
    flops = 14.0 * bs * bs * D * done_tiles
    return dict(value=flops / t_used / 1e12, unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                sample=f"oracle block-sparse attention fwd+bwd (torch fp32 on CPU) for {n_rows} (head, q-block) "
                       f"rows of the same mask ({done_tiles} active {bs}x{bs} tiles, {t_used:.1f} s)",
                seconds=round(t_used, 2), cpu_count=os.cpu_count(), cpu_model=cpu_model())


def cpu_pointer_stats(configs, seconds: float) -> dict:
    """Kernels 1 and 3 on the host: the oracle's block-scoring selection
    (block means, logits bs/√D·q̄·k̄ + radius prior, counter Gumbel noise,
    top-budget picks, union and pack; oracle/pointer.py) and its mask
    statistics (oracle/stats.py:blockscore_stats), numpy on the host cores,
    repeated until `seconds` per config are used; beside them the GPU time of
    the same two phases on the same inputs (doc starts + block means +
    selection; the statistics kernel), events around `reps` launches.
    configs: (name, inputs, bs, window, n_global, budget)."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_info

    from oracle import pointer as OP
    from oracle import stats as OS
    from scope_amd import ops

    out = {}
    for name, inp, bs, W, G, B in configs:
        q, k, docs = inp["q"][0].float().numpy(), inp["k"][0].float().numpy(), inp["docs"].numpy()
        H, T, D = q.shape
        NB = T // bs
        prior = radius_prior(NB, PRIOR_SCALE)
        hh, qq, kk = np.meshgrid(np.arange(H), np.arange(NB), np.arange(NB), indexing="ij")

        def kernel1():
            lg = OP.pointer_logits(OP.block_means(q, bs), OP.block_means(k, bs), logit_scale=bs / math.sqrt(D),
                                   prior=prior.double().numpy()).astype(np.float32)
            g = OP.gumbel_from_u(OP.counter_uniform(1234, hh, qq, kk))
            return OP.pointer_select_blockscore(lg, docs, bs=bs, window=W, n_global=G, budget=B, gumbel=g)

        n1 = n3 = 0
        t1 = t3 = 0.0
        while t1 + t3 < seconds:
            t0 = time.perf_counter()
            sel = kernel1()
            t1 += time.perf_counter() - t0
            n1 += 1
            t0 = time.perf_counter()
            OS.blockscore_stats(sel["kv_num"], sel["picks"], sel["ds_ptr"], sel["ds_local"], maxkv=sel["maxkv"],
                                local_blocks=W)
            t3 += time.perf_counter() - t0
            n3 += 1
        gq, gk, gd = (inp[n].cuda() for n in ("q", "k", "docs"))
        gprior = prior.cuda()
        res = {}

        def gpu_k1():
            ds_ptr, ds_local, _ = ops.doc_starts(gd, bs)
            qbar, kbar = ops.block_means(gq, gk, bs)
            res["sel"] = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=W, n_global=G, budget=B,
                                            qbar=qbar, kbar=kbar, prior=gprior, temp=1.0,
                                            logit_scale=bs / math.sqrt(D), noise="counter", seed=1234)
            res["ds"] = (ds_ptr, ds_local)

        gpu_k1()
        kv_num, kv_idx, picks = res["sel"]
        ds_ptr, ds_local = res["ds"]

        def gpu_k3():
            ops.mask_stats(H=H, QB=NB, bs=bs, kv_num=kv_num, picks=picks, ds_ptr=ds_ptr, ds_local=ds_local,
                           maxkv_bins=kv_idx.shape[-1] + 1, bs_local_blocks=W)

        g1 = time_region(gpu_k1, 20, 3)
        g3 = time_region(gpu_k3, 20, 3)
        out[name] = dict(H=H, T=T, block=bs, window=W, n_global=G, budget=B,
                         cpu_select_ms=round(t1 / n1 * 1e3, 3), cpu_stats_ms=round(t3 / n3 * 1e3, 3),
                         cpu_calls=n1, cpu_seconds=round(t1 + t3, 2),
                         gpu_select_ms=round(g1 * 1e3, 4), gpu_stats_ms=round(g3 * 1e3, 4),
                         select_speedup=round(t1 / n1 / g1, 1), stats_speedup=round(t3 / n3 / g3, 1))
    blas = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
    return dict(kind="port", unit="ms per call", configs=out, cores=blas[0] if blas else 1,
                cores_note="numpy: the logit products on the BLAS threads, the rest on one thread",
                cpu_count=os.cpu_count(), cpu_model=cpu_model())


def c1_lists(inp, bs: int, window: int, n_global: int, budget: int, seed: int):
    """The config-1 lists from the oracle's block-scoring selection: fp64
    block means, logits bs/√D·q̄·k̄ + radius prior, counter Gumbel noise (τ=1)."""
    import numpy as np

    from oracle import pointer as OP

    q, k, docs = inp["q"][0].float().numpy(), inp["k"][0].float().numpy(), inp["docs"].numpy()
    H, T, D = q.shape
    NB = T // bs
    lg = OP.pointer_logits(OP.block_means(q, bs), OP.block_means(k, bs), logit_scale=bs / math.sqrt(D),
                           prior=radius_prior(NB, PRIOR_SCALE).double().numpy()).astype(np.float32)
    hh, qq, kk = np.meshgrid(np.arange(H), np.arange(NB), np.arange(NB), indexing="ij")
    g = OP.gumbel_from_u(OP.counter_uniform(seed, hh, qq, kk))
    sel = OP.pointer_select_blockscore(lg, docs, bs=bs, window=window, n_global=n_global, budget=budget, gumbel=g)
    return sel["kv_num"], sel["packed"]


def cpu_reference_path_c1(seconds: float):
    """The reference's own CPU path (its eager FlexAttention fallback,
    scoped_medium.py:37-38) at config 1: B=1, H=6, T=4096, D=128, bs=128,
    window 3, global 1, budget 2, block-offset spectral bias with 8 bands,
    forward only.  Eager flex_attention on the host cores in fp32, with the
    block lists restated inside mask_mod (eager FlexAttention evaluates
    mask_mod on every score and ignores kv_indices) together with
    document_causal (model/attn_bias.py:674-679), and the band term as
    score_mod; then dense masked SDPA in fp32 with an explicit bias.  The GPU
    forward of the same layer and lists is timed beside them."""
    import numpy as np
    import torch
    import torch.nn.functional as F
    from torch.nn.attention.flex_attention import create_block_mask, flex_attention

    from scope_amd import ops
    from scope_amd.attention import spectral_table

    torch.set_num_threads(os.cpu_count() or 1)
    H, T, D, bs, W, G, B = 6, 4096, 128, 128, 3, 1, 2
    NB = T // bs
    inp = make_inputs(H, T, D, bs, n_docs=1, needle=False)
    kv_num, kv_idx = c1_lists(inp, bs, W, G, B, seed=1234)
    n_act = int(kv_num.sum())
    flops = 4.0 * bs * bs * D * n_act
    q, k, v = (inp[n][0].float() for n in ("q", "k", "v"))
    cc, cs = inp["coeff_cos"][0].float(), inp["coeff_sin"][0].float()
    om = inp["omegas"].float()
    blk = torch.zeros((H, NB, NB), dtype=torch.bool)
    for h in range(H):
        for qb in range(NB):
            blk[h, qb, torch.from_numpy(kv_idx[h, qb, :kv_num[h, qb]]).long()] = True
    docs_l = inp["docs"].long()
    rr = torch.arange(NB, dtype=torch.float32)
    cosR, sinR = torch.cos(om[:, None] * rr[None]), torch.sin(om[:, None] * rr[None])  # [K, NB]

    def mask_mod(b, h, qi, ki):
        return blk[h, qi // bs, ki // bs] & (qi >= ki) & (docs_l[qi] == docs_l[ki])

    CC, CS = cc[None], cs[None]

    def score_mod(score, b, h, q_idx, kv_idx_):  # the shape of scoped_medium.py:425-457, block offsets
        qi = q_idx.to(torch.long).reshape(-1)
        ki = kv_idx_.to(torch.long).reshape(-1)
        r = (qi[:, None] // bs - ki[None, :] // bs).clamp(min=0)
        A, Bc = CC[b, h, qi], CS[b, h, qi]
        bias = score.new_zeros(r.shape, dtype=torch.float32)
        for kx in range(cc.shape[-1]):
            bias = bias + A[:, kx:kx + 1] * cosR[kx, r] + Bc[:, kx:kx + 1] * sinR[kx, r]
        return score + 0.5 * bias.reshape_as(score).to(score.dtype)

    def flex_step():
        bm = create_block_mask(mask_mod, None, H, T, T, device="cpu", BLOCK_SIZE=bs)
        return flex_attention(q[None], k[None], v[None], block_mask=bm, score_mod=score_mod, scale=0.12)

    def sdpa_step():
        i = torch.arange(T)
        allowed = blk.repeat_interleave(bs, 1).repeat_interleave(bs, 2) & ((i[:, None] >= i[None, :]) &
                                                                           (docs_l[:, None] == docs_l[None, :]))
        r = (i[:, None] // bs - i[None, :] // bs).clamp(min=0)
        bias = torch.zeros((H, T, T))
        for kx in range(cc.shape[-1]):
            bias += cc[:, :, kx, None] * cosR[kx][r][None] + cs[:, :, kx, None] * sinR[kx][r][None]
        mask = torch.where(allowed, 0.5 * bias, torch.tensor(float("-inf")))
        return F.scaled_dot_product_attention(q[None], k[None], v[None], attn_mask=mask[None], scale=0.12)

    def timed(fn):
        ts = []
        while not ts or (sum(ts) < seconds / 2 and len(ts) < 5):
            t0 = time.perf_counter()
            out = fn()
            ts.append(time.perf_counter() - t0)
        return min(ts), len(ts), out

    t_flex, n_flex, o_flex = timed(flex_step)
    t_sdpa, n_sdpa, o_sdpa = timed(sdpa_step)
    # the GPU forward of the same layer and lists
    dev = torch.device("cuda")
    gq, gk, gv = (inp[n].to(dev) for n in ("q", "k", "v"))
    docs_d = inp["docs"].to(dev)
    _, _, ds_tok_end = ops.doc_starts(docs_d, bs)
    kn, ki = torch.from_numpy(kv_num).to(dev), torch.from_numpy(kv_idx).to(dev)
    tab = spectral_table(inp["omegas"].to(dev), T, bs, "block")
    gcc, gcs = inp["coeff_cos"].to(dev), inp["coeff_sin"].to(dev)

    def gpu_fwd():
        ops.attn_fwd(gq, gk, gv, kn, ki, docs_d, ds_tok_end, bs=bs, scale=0.12, beta=0.5, bias_mode="block",
                     table=tab, coeff_cos=gcc, coeff_sin=gcs, check=False)

    t_gpu = time_region(gpu_fwd, 20, 3)
    o_gpu, _ = ops.attn_fwd(gq, gk, gv, kn, ki, docs_d, ds_tok_end, bs=bs, scale=0.12, beta=0.5, bias_mode="block",
                            table=tab, coeff_cos=gcc, coeff_sin=gcs, check=False)
    o_gpu = o_gpu.float().cpu()[0]
    return dict(workload="config 1: B=1, H=6, T=4096, D=128, bs=128, window 3, global 1, budget 2, "
                         "block-offset bias (8 bands), forward only, fp32 on the host",
                n_act=n_act, flops_fwd=flops, cores=torch.get_num_threads(), cpu_count=os.cpu_count(),
                cpu_model=cpu_model(),
                eager_flex_attention=dict(ms=round(t_flex * 1e3, 1), tflops=round(flops / t_flex / 1e12, 5),
                                          runs=n_flex, kind="reference",
                                          source="torch eager flex_attention (the reference's fallback, "
                                                 "scoped_medium.py:37-38) with restated mask_mod/score_mod"),
                dense_sdpa=dict(ms=round(t_sdpa * 1e3, 1), tflops=round(flops / t_sdpa / 1e12, 5), runs=n_sdpa,
                                kind="reference", source="F.scaled_dot_product_attention fp32 with a dense "
                                                         "bias + mask (built inside the timed call)"),
                gpu_fwd_ms=round(t_gpu * 1e3, 4), gpu_tflops=round(flops / t_gpu / 1e12, 2),
                gpu_speedup_vs_eager_flex=round(t_flex / t_gpu, 1),
                max_abs_diff=dict(flex_vs_sdpa=round(float((o_flex[0] - o_sdpa[0]).abs().max()), 6),
                                  gpu_vs_flex=round(float((o_gpu - o_flex[0]).abs().max()), 6)))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU: the SCOPE hot path is sharded by head across GPUs "
                                   "(no exchange inside the layer), multi-GPU runs are out of scope",
                          "n_gpus": args.gpus}))
        sys.exit(1)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.workload == "decode":
        main_decode(args)
        return
    if args.workload == "ref":
        main_ref(args)
        return
    if args.workload == "teacher":
        main_teacher(args)
        return
    if args.workload == "coeff":
        main_coeff(args)
        return
    if args.workload == "swa":
        if args.T == 131072 and args.bs == 256:  # the pointer workload's defaults -> the training shape
            args.T, args.bs = 65536, 128
        main_swa(args)
        return
    train = args.workload == "train"
    if train and (args.T, args.bs, args.window, args.n_global, args.budget) == (131072, 256, 2, 2, 8):
        # the pointer workload's defaults -> the training shape
        args.T, args.bs, args.window, args.n_global, args.budget = 65536, 128, 4, 1, 4
    soft = args.soft_temp if args.soft_temp != 0 else (4.0 if train else 0.0)  # < 0: off
    H, T, D, bs = args.H, args.T, 128, args.bs
    n_docs = args.docs if args.docs > 0 else (1 if train else max(1, T // 8192))
    inp = make_inputs(H, T, D, bs, n_docs=n_docs, needle=not (train or args.no_needle))
    print(f"inputs ready: H={H} T={T} bs={bs} docs={n_docs}", file=sys.stderr, flush=True)
    step = Step(inp, bs=bs, window=args.window, n_global=args.n_global, budget=args.budget, soft_temp=soft)
    step()
    torch.cuda.synchronize()
    n_act = int(step.last["kv_num"].sum())
    F_fwd = 4.0 * bs * bs * D * n_act
    F_bwd = 10.0 * bs * bs * D * n_act

    t_step = time_region(step, args.steps, args.warmup)
    time_steps(step, args.steps, 0)  # per-phase breakdown (events around each phase)
    ph = {p: step.acc[p] / args.steps for p in step.phases}

    # Algorithmic FLOPs per kernel: the forward does 2 GEMMs (4·bs²·D per tile);
    # of the backward's 5 GEMMs (10·bs²·D) the q-major pass owns S, dP, dQ
    # (6·bs²·D) and the kv-major pass dK, dV (4·bs²·D); its S/dP recompute is
    # not counted.
    per_kernel = {"attn_fwd": (F_fwd, "attn_fwd_kernel"),
                  "attn_bwd_dq": (6.0 * bs * bs * D * n_act, "attn_bwd_dq2_kernel" if bs == 256 else "attn_bwd_dq_kernel"),
                  "attn_bwd_dkv": (4.0 * bs * bs * D * n_act, "attn_bwd_dkv16_kernel")}
    dom = max(per_kernel, key=lambda p: ph[p])
    flops, kname = per_kernel[dom]
    achieved = flops / (ph[dom] / 1e3) / 1e12
    # the instance of this block size in the block-offset bias mode (1)
    traffic, tsrc = measured_traffic(f"{kname}<{bs},1>", H, T, bs, args.budget)
    roofline = dict(bound="mfma", kernel=kname, achieved=round(achieved, 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                    frac=round(achieved / PEAK_BF16_TFLOPS, 4), traffic=traffic, traffic_source=tsrc,
                    flops_per_launch=flops, launch_ms=round(ph[dom], 4))
    # what the kernel executes: the kv-major pass also recomputes S and dP
    executed = 8.0 * bs * bs * D * n_act if dom == "attn_bwd_dkv" else flops
    roofline["executed_flops_per_launch"] = executed
    roofline["executed_achieved"] = round(executed / (ph[dom] / 1e3) / 1e12, 2)
    # the pointer path is HBM-bound: q and k read once (bf16), the document ids,
    # and the compact lists written (the byte count of the workload definition)
    maxkv = int(step.last["kv_idx"].shape[-1])
    ptr_bytes = 2 * H * T * D * 2 + T * 8 + H * (T // bs) * (1 + maxkv) * 4
    means_ms = step.means_ms / args.steps
    pointer = dict(bound="hbm", unit="GB/s", peak=PEAK_HBM_GBS, bytes=ptr_bytes,
                   phase_ms=round(ph["pointer"], 4), phase_achieved=round(ptr_bytes / (ph["pointer"] / 1e3) / 1e9, 1),
                   phase_frac=round(ptr_bytes / (ph["pointer"] / 1e3) / 1e9 / PEAK_HBM_GBS, 4),
                   block_means_ms=round(means_ms, 4),
                   block_means_achieved=round(2 * H * T * D * 2 / (means_ms / 1e3) / 1e9, 1),
                   block_means_frac=round(2 * H * T * D * 2 / (means_ms / 1e3) / 1e9 / PEAK_HBM_GBS, 4))
    needle_sel = None
    if inp.get("needle") is not None:
        qb_n, kb_n = inp["needle"]
        picks = step.last["picks"]
        needle_sel = dict(q_block=qb_n, key_block=kb_n, distance_blocks=qb_n - kb_n,
                          selected_heads=int((picks[:, qb_n] == kb_n).any(dim=-1).sum().item()), heads=H)
    workload = ("training-shape layer, one SCOPE layer fwd+bwd (pointer select + stats + block-sparse attention "
                "+ soft pointer weights and their backward)") if train else (
        "long-context prefill, one SCOPE layer fwd+bwd (pointer select + stats + block-sparse attention)")
    res = {
        "metric": ("SCOPE attn fwd+bwd active-block TFLOP/s & tokens/s at T=64k with soft pointer weights, 1 MI355X"
                   if train else METRIC),
        "value": round((F_fwd + F_bwd) / t_step / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "B": 1, "H": H, "T": T, "D": D, "block": bs,
                   "window": args.window, "global": args.n_global, "budget": args.budget, "bands": 8,
                   "bias": "block offsets", "docs": n_docs,
                   "soft_pointer_temp": soft if soft > 0 else None},
        "tokens_per_s": round(T / t_step, 1),
        "n_act": n_act,
        "flops_fwd": F_fwd,
        "flops_bwd": F_bwd,
        "attn_fwd_tflops": round(F_fwd / (ph["attn_fwd"] / 1e3) / 1e12, 2),
        "attn_bwd_tflops": round(F_bwd / ((ph["attn_bwd_dq"] + ph["attn_bwd_dkv"] + ph["attn_bwd_aux"]) / 1e3) / 1e12,
                                 2),
        "breakdown_ms": {p: round(v_, 4) for p, v_ in ph.items()},
        "needle": needle_sel,
        "pointer_bwd_ms": round(ph["pointer_bwd"], 4) if soft > 0 else None,
        "roofline": roofline,
        "pointer_roofline": pointer,
    }
    # the same step replayed from one captured HIP graph (an extra: `value`
    # stays the eager step's)
    graph = graph_time_layer(step, args.steps)
    res["graph_ms_per_step"] = graph["ms"]
    res["graph_tflops"] = round((F_fwd + F_bwd) / graph["ms"] / 1e9, 2) if graph["ms"] else None
    res["graph_check"] = graph["check"]
    if args.sweep:
        sweep = {}
        for b in (2, 4):
            st = Step(inp, bs=bs, window=args.window, n_global=args.n_global, budget=b, soft_temp=soft)
            st()
            torch.cuda.synchronize()
            na = int(st.last["kv_num"].sum())
            ts = time_region(st, args.steps, args.warmup)
            sweep[str(b)] = dict(value=round(14.0 * bs * bs * D * na / ts / 1e12, 2), ms_per_step=round(ts * 1e3, 3),
                                 n_act=na)
        res["budget_sweep"] = sweep
    # measured ceilings next to the vendor figures used as `peak`
    mp = step.ops.measure_peaks("cuda")
    res["measured_peaks"] = mp
    roofline["peak_measured"] = mp["mfma_bf16_tflops"]
    roofline["frac_of_measured"] = round(achieved / mp["mfma_bf16_tflops"], 4)
    # the MFMA rate on random operands, at the clock the power limit leaves
    roofline["peak_measured_random"] = mp["mfma_bf16_tflops_random"]
    roofline["executed_frac_of_measured_random"] = round(roofline["executed_achieved"] / mp["mfma_bf16_tflops_random"],
                                                         4)
    pointer["peak_measured"] = mp["hbm_copy_gbs"]
    pointer["block_means_frac_of_measured"] = round(pointer["block_means_achieved"] / mp["hbm_copy_gbs"], 4)
    if not train and (H, T, bs) == (8, 131072, 256) and not args.no_ref_layer:
        # the reference's default layer (T=16384, bs 128, token offsets, reference-mode
        # lists), timed after the headline with its own events and steps
        res["reference_default_layer"] = ref_layer(8, 16384, args.steps, args.warmup)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(inp, step, args.cpu_seconds, bs)
        if not train:
            res["cpu_baseline"]["reference_path_c1"] = cpu_reference_path_c1(args.cpu_seconds)
            c1 = make_inputs(6, 4096, D, 128, n_docs=1, needle=False)
            res["cpu_baseline"]["pointer_and_stats"] = cpu_pointer_stats(
                [("config 1: H=6, T=4096, bs 128, window 3, global 1, budget 2", c1, 128, 3, 1, 2),
                 (f"this workload: H={H}, T={T}, bs {bs}, window {args.window}, global {args.n_global}, "
                  f"budget {args.budget}", inp, bs, args.window, args.n_global, args.budget)],
                min(args.cpu_seconds, 10.0))
    if args.copy_probe_mib > 0:
        src = torch.ones(args.copy_probe_mib << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        res["copy_probe_bytes"] = src.numel() * 4
    print(json.dumps(res))


if __name__ == "__main__":
    main()

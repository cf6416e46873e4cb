"""torch-facing wrappers of the C ABI: allocate outputs with torch's caching
allocator on the inputs' device, pass raw device pointers and the current
stream, raise ``ScopeLibraryError`` on failure.  Every function here requires
GPU tensors; there is no CPU path.
"""
from __future__ import annotations

import ctypes as C
import threading

import torch

from . import _lib
from ._lib import PTR_LOGITS_SCRATCH, AttnParams, PtrRefParams, PtrScoreParams, StatsParams, query

BIAS_MODES = {"none": 0, "block": 1, "token": 2}
GATE_KINDS = {"none": 0, "softplus": 1, "relu": 2}

# counts layout (include/scope_amd.h SCOPE_ST_*)
ST_DELTA_TOKENS, ST_DELTA_BLOCKS, ST_CENTER = 0, 16, 31
ST_DOCSTART, ST_OUTSIDE, ST_BLOCK0, ST_BLOCK0_EXCL, ST_N_CENTRES, ST_N_CENTRES_EXCL = 46, 47, 48, 49, 50, 51
ST_PTR_DIST, ST_BS_OUTSIDE, ST_BS_BLOCK0, ST_BS_BLOCK0_EXCL, ST_BS_DOCSTART, ST_BS_N, ST_BS_N_EXCL = (
    52, 67, 68, 69, 70, 71, 72)
ST_RADIUS0, ST_N_RADIUS, ST_FIXED = 73, 74, 75
SV_NAMES = ["pi_entropy_mean", "ptr_docstart_frac", "ptr_outside_local_frac", "ptr_block0_frac",
            "ptr_block0_frac_excl", "ptr_radius0_frac", "bs_ptr_outside_local_frac", "bs_ptr_block0_frac",
            "bs_ptr_block0_frac_excl", "bs_ptr_docstart_frac"]


# Tensors whose pointers _p handed out, held until the next call() returns.
_held = threading.local()


def _p(t: torch.Tensor | None):
    """Device pointer of t for a library call.  t stays referenced until the
    next ``call`` returns: a dtype or layout copy made inside an argument list
    (``_p(_i32(x))``) would otherwise go back to torch's caching allocator
    before the launch, and a later copy in the same argument list could be
    given its memory, so the kernel would read one operand in place of
    another.  (Argument lists must not themselves run a ``call``.)"""
    if t is None:
        return None
    held = getattr(_held, "ts", None)
    if held is None:
        held = _held.ts = []
    held.append(t)
    return C.c_void_p(t.data_ptr())


def call(name: str, *args) -> None:
    """``_lib.call`` (raise on a non-zero status), then release the tensors
    held for the arguments: the launch is on the stream by then, so torch's
    allocator hands their memory to later work on that stream only after it."""
    try:
        _lib.call(name, *args)
    finally:
        held = getattr(_held, "ts", None)
        if held:
            held.clear()


def _stream(dev: torch.device):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _gpu(name: str, *ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{name}: tensors must live on the GPU (got {t.device}); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{name}: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise RuntimeError(f"{name}: no GPU tensor given")
    return dev


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int32 and t.is_contiguous()) else t.to(torch.int32).contiguous()


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
    return None if t is None else (t if (t.dtype == torch.float32 and t.is_contiguous()) else t.float().contiguous())


def _bhtd(name: str, x: torch.Tensor):
    """[1,H,T,D] or [H,T,D] with unit last stride -> (H, T, D, stride_h, stride_t)."""
    if x.dim() == 4:
        if x.shape[0] != 1:
            raise RuntimeError(f"{name}: batch size must be 1 (got {x.shape[0]})")
        _, H, T, D = x.shape
        sh, st, sd = x.stride(1), x.stride(2), x.stride(3)
    elif x.dim() == 3:
        H, T, D = x.shape
        sh, st, sd = x.stride()
    else:
        raise RuntimeError(f"{name}: expected [1,H,T,D] or [H,T,D], got {tuple(x.shape)}")
    if sd != 1:
        raise RuntimeError(f"{name}: last dimension must be contiguous")
    return H, T, D, sh, st


# ---------------------------------------------------------------------------
def doc_starts(docs: torch.Tensor, bs: int, *, doc_clamp: bool = True, reset_len: int = 0):
    """(ds_ptr, ds_local, ds_tok_end) int32 [QB] (model/attn_bias.py:688-709)."""
    dev = _gpu("doc_starts", docs)
    docs = _i32(docs.reshape(-1))
    T = docs.numel()
    if T % bs:
        raise RuntimeError(f"doc_starts: T={T} not a multiple of bs={bs}")
    NB = T // bs
    out = [torch.empty(NB, dtype=torch.int32, device=dev) for _ in range(3)]
    call("scope_doc_starts", _p(docs), T, int(bs), int(bool(doc_clamp)), int(max(0, reset_len)), _p(out[0]),
         _p(out[1]), _p(out[2]), _stream(dev))
    return out[0], out[1], out[2]


def pointer_mask_ref(delta_star: torch.Tensor, budget_logits: torch.Tensor, ds_ptr: torch.Tensor,
                     ds_local: torch.Tensor, *, bs: int, local_blocks: int, ptr_half_blocks: int,
                     global_blocks_cfg: int, global_active: int, radius_mode: str, budget_rem: int,
                     budget_temp: float, mask_active: bool, half_active: int, rep_mode: str = "last",
                     gumbel_k: int = 0, gumbel_tau: float = 1.0, gumbel_u: torch.Tensor | None = None,
                     eps: float = 1e-9):
    """Reference-mode pointer mask -> (kv_num [H,QB], kv_idx [H,QB,MAXKV], radius, centre)."""
    dev = _gpu("pointer_mask_ref", delta_star, budget_logits, ds_ptr, ds_local, gumbel_u)
    ds4 = delta_star.float() if delta_star.dtype != torch.float32 else delta_star
    bl4 = budget_logits.float() if budget_logits.dtype != torch.float32 else budget_logits
    if ds4.dim() == 4:
        ds4, bl4 = ds4[0], bl4[0]
    if ds4.stride() != bl4.stride() or ds4.stride(-1) != 1:
        ds4, bl4 = ds4.contiguous(), bl4.contiguous()
    H, T, M = ds4.shape
    prm = PtrRefParams(H=H, M=M, bs=bs, T=T, stride_h=ds4.stride(0), stride_t=ds4.stride(1),
                       rep_mean=int(rep_mode == "mean"), local_blocks=int(local_blocks),
                       ptr_half_blocks=int(ptr_half_blocks), global_blocks_cfg=int(global_blocks_cfg),
                       global_active=int(global_active), radius_mode_pi=int(radius_mode == "pi"),
                       budget_rem=int(budget_rem), budget_temp=float(max(budget_temp, 1e-6)),
                       mask_active=int(bool(mask_active)), half_active=int(half_active), gumbel_k=int(gumbel_k),
                       gumbel_tau=float(max(gumbel_tau, 1e-6)), eps=float(eps))
    L = query("scope_ptr_ref_maxkv", C.byref(prm))
    QB = T // bs
    kv_num = torch.empty((H, QB), dtype=torch.int32, device=dev)
    kv_idx = torch.empty((H, QB, L), dtype=torch.int32, device=dev)
    radius = torch.empty((H, QB, M), dtype=torch.int32, device=dev)
    centre = torch.empty((H, QB, M), dtype=torch.int32, device=dev)
    gu = _f32(gumbel_u) if gumbel_k > 0 else None
    call("scope_pointer_mask_ref", C.byref(prm), _p(ds4), _p(bl4), _p(gu), _p(_i32(ds_ptr)), _p(_i32(ds_local)),
         _p(kv_num), _p(kv_idx), _p(radius), _p(centre), _stream(dev))
    return kv_num, kv_idx, radius, centre


def block_means(q: torch.Tensor, k: torch.Tensor, bs: int):
    """Block means q̄, k̄ [H, NB, D] fp32 of bf16 q, k."""
    dev = _gpu("block_means", q, k)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise RuntimeError("block_means: q and k must be bfloat16")
    H, T, D, qsh, qst = _bhtd("block_means q", q)
    _, _, _, ksh, kst = _bhtd("block_means k", k)
    NB = T // bs
    qbar = torch.empty((H, NB, D), dtype=torch.float32, device=dev)
    kbar = torch.empty((H, NB, D), dtype=torch.float32, device=dev)
    call("scope_block_means", _p(q), _p(k), H, T, D, bs, qsh, qst, ksh, kst, _p(qbar), _p(kbar), _stream(dev))
    return qbar, kbar


def block_means_docs(q: torch.Tensor, k: torch.Tensor, docs: torch.Tensor, bs: int, *, doc_clamp: bool = True,
                     reset_len: int = 0):
    """``block_means`` and ``doc_starts`` in one call with one launch fewer
    (``scope_block_means_docs``) -> (q̄, k̄, ds_ptr, ds_local, ds_tok_end)."""
    dev = _gpu("block_means_docs", q, k, docs)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise RuntimeError("block_means_docs: q and k must be bfloat16")
    H, T, D, qsh, qst = _bhtd("block_means_docs q", q)
    _, Tk, _, ksh, kst = _bhtd("block_means_docs k", k)
    docs = _i32(docs.reshape(-1))
    if Tk != T or docs.numel() != T:
        raise RuntimeError(f"block_means_docs: q has {T} tokens, k {Tk}, docs {docs.numel()}")
    if T % bs:
        raise RuntimeError(f"block_means_docs: T={T} not a multiple of bs={bs}")
    NB = T // bs
    qbar = torch.empty((H, NB, D), dtype=torch.float32, device=dev)
    kbar = torch.empty((H, NB, D), dtype=torch.float32, device=dev)
    ds = [torch.empty(NB, dtype=torch.int32, device=dev) for _ in range(3)]
    call("scope_block_means_docs", _p(q), _p(k), _p(docs), H, T, D, bs, qsh, qst, ksh, kst, int(bool(doc_clamp)),
         int(max(0, reset_len)), _p(qbar), _p(kbar), _p(ds[0]), _p(ds[1]), _p(ds[2]), _stream(dev))
    return qbar, kbar, ds[0], ds[1], ds[2]


def pointer_select(ds_ptr: torch.Tensor, ds_local: torch.Tensor, *, bs: int, NB: int, H: int, window: int,
                   n_global: int, budget: int, qbar: torch.Tensor | None = None, kbar: torch.Tensor | None = None,
                   logits_in: torch.Tensor | None = None, prior: torch.Tensor | None = None, temp: float = 1.0,
                   logit_scale: float = 1.0, noise: str = "none", gumbel_u: torch.Tensor | None = None,
                   seed: int = 0, eps: float = 1e-9, return_logits: bool = False):
    """Block-scoring selection -> (kv_num [H,QB], kv_idx [H,QB,W+budget+G], picks [H,QB,budget][, logits])."""
    dev = _gpu("pointer_select", ds_ptr, ds_local, qbar, kbar, logits_in, prior, gumbel_u)
    noise_mode = {"none": 0, "uniform": 1, "counter": 2}[noise]
    D = qbar.shape[-1] if qbar is not None else 128
    pstride = 0
    if prior is not None:
        prior = _f32(prior)
        pstride = NB if prior.dim() == 2 else 0
    prm = PtrScoreParams(H=H, NB=NB, D=D, bs=bs, window=window, n_global=n_global, budget=budget,
                         temp=float(temp), logit_scale=float(logit_scale), noise_mode=noise_mode,
                         seed=int(seed) & 0xFFFFFFFFFFFFFFFF, eps=float(eps), prior_head_stride=pstride)
    L = min(window, NB) + budget + min(n_global, NB)
    kv_num = torch.empty((H, NB), dtype=torch.int32, device=dev)
    kv_idx = torch.empty((H, NB, L), dtype=torch.int32, device=dev)
    picks = torch.empty((H, NB, max(budget, 1)), dtype=torch.int32, device=dev)
    # from LOGITS_GEMM_NB blocks on (D = 128) the library computes the logits on
    # MFMA into the logits buffer before the selection reads them: give it one
    gemm = logits_in is None and qbar is not None and D == 128 and NB >= LOGITS_GEMM_NB
    logits = torch.empty((H, NB, NB), dtype=torch.float32, device=dev) if (return_logits or gemm) else None
    # a buffer only the library reads: its non-candidate entries are not set to -inf
    prm.flags = PTR_LOGITS_SCRATCH if (gemm and not return_logits) else 0
    call("scope_pointer_select", C.byref(prm), _p(_f32(qbar)), _p(_f32(kbar)), _p(_f32(logits_in)), _p(prior),
         _p(_f32(gumbel_u) if noise_mode == 1 else None), _p(_i32(ds_ptr)), _p(_i32(ds_local)), _p(kv_num),
         _p(kv_idx), _p(picks), _p(logits), _stream(dev))
    picks = picks[..., :budget]
    return (kv_num, kv_idx, picks, logits) if return_logits else (kv_num, kv_idx, picks)


LOGITS_GEMM_NB = 1024  # pointer.hip kLogitsGemmNB


def pointer_pair_bias(kv_num: torch.Tensor, kv_idx: torch.Tensor, picks: torch.Tensor, *, bs: int, window: int,
                      n_global: int, soft_temp: float, qbar: torch.Tensor | None = None,
                      kbar: torch.Tensor | None = None, logits_in: torch.Tensor | None = None,
                      prior: torch.Tensor | None = None, logit_scale: float = 1.0,
                      check: bool = True) -> torch.Tensor:
    """Soft pointer weights as a per-list-entry score bias [H,QB,L] (log σ(z/τ_w)
    on the pick entries, 0 elsewhere), aligned with kv_idx.  ``check``:
    validate the lists first (``check_lists``)."""
    dev = _gpu("pointer_pair_bias", kv_num, kv_idx, picks, qbar, kbar, logits_in, prior)
    if check:
        check_lists(kv_num, kv_idx, kv_num.shape[-1], who="pointer_pair_bias")
    H, NB = kv_num.shape[-2], kv_num.shape[-1]
    L = kv_idx.shape[-1]
    budget = picks.shape[-1]
    D = qbar.shape[-1] if qbar is not None else 128
    pstride = 0
    if prior is not None:
        prior = _f32(prior)
        pstride = NB if prior.dim() == 2 else 0
    prm = PtrScoreParams(H=H, NB=NB, D=D, bs=bs, window=window, n_global=n_global, budget=budget, temp=1.0,
                         logit_scale=float(logit_scale), noise_mode=0, seed=0, eps=1e-9, prior_head_stride=pstride)
    if min(window, NB) + budget + min(n_global, NB) != L:
        raise RuntimeError("pointer_pair_bias: kv_idx width does not match window + budget + global")
    out = torch.empty((H, NB, L), dtype=torch.float32, device=dev)
    call("scope_pointer_pair_bias", C.byref(prm), float(soft_temp), _p(_f32(qbar)), _p(_f32(kbar)),
         _p(_f32(logits_in)), _p(prior), _p(_i32(kv_num.reshape(H, NB))), _p(_i32(kv_idx.reshape(H, NB, L))),
         _p(_i32(picks.reshape(H, NB, budget))), _p(out), _stream(dev))
    return out


def pointer_bwd(qbar: torch.Tensor, kbar: torch.Tensor, kv_num: torch.Tensor, kv_idx: torch.Tensor,
                q_off: torch.Tensor, q_list: torch.Tensor, pair_bias: torch.Tensor, dpair_bias: torch.Tensor,
                dq: torch.Tensor, dk: torch.Tensor, *, bs: int, logit_scale: float, soft_temp: float,
                check: bool = True) -> None:
    """Add the soft pointer weights' gradient path (through the block means)
    to dq and dk [1,H,T,D] bf16 in place.  ``check``: validate kv_num /
    kv_idx first (``check_lists``); q_off / q_list must be their transpose."""
    from ._lib import PtrBwdParams

    dev = _gpu("pointer_bwd", qbar, kbar, kv_num, kv_idx, q_off, q_list, pair_bias, dpair_bias, dq, dk)
    if check:
        check_lists(kv_num, kv_idx, qbar.shape[1], who="pointer_bwd")
    H, NB, D = qbar.shape
    L = kv_idx.shape[-1]
    _, _, _, qsh, qst = _bhtd("pointer_bwd dq", dq)
    _, _, _, ksh, kst = _bhtd("pointer_bwd dk", dk)
    prm = PtrBwdParams(H=H, NB=NB, D=D, bs=int(bs), maxkv=L, logit_scale=float(logit_scale),
                       soft_temp=float(soft_temp), q_sh=qsh, q_st=qst, k_sh=ksh, k_st=kst)
    ws = torch.empty(max(16, query("scope_pointer_bwd_workspace_bytes", C.byref(prm))), dtype=torch.uint8,
                     device=dev)
    call("scope_pointer_bwd", C.byref(prm), _p(_f32(qbar)), _p(_f32(kbar)), _p(_i32(kv_num.reshape(H, NB))),
         _p(_i32(kv_idx.reshape(H, NB, L))), _p(_i32(q_off)), _p(_i32(q_list)), _p(_f32(pair_bias)),
         _p(_f32(dpair_bias)), _p(dq), _p(dk), _p(ws), _stream(dev))


def _check_lists_host(kn: torch.Tensor, ki: torch.Tensor, NB: int, causal: bool) -> list[int]:
    """The counters of scope_check_lists, in torch on the host."""
    H, QB, maxkv = ki.shape
    kn, ki = kn.long(), ki.long()
    bad_num = (kn < 0) | (kn > maxkv)
    e = torch.arange(maxkv)
    used = (e[None, None] < kn[..., None]) & ~bad_num[..., None]
    oor = used & ((ki < 0) | (ki >= NB))
    late = used & ~oor & (ki > torch.arange(QB)[None, :, None]) if causal else torch.zeros_like(used)
    ok = used & ~oor & ~late
    srt = torch.where(ok, ki, NB + e).sort(dim=-1).values  # unused slots get distinct values >= NB
    dup = ((srt[..., 1:] == srt[..., :-1]) & (srt[..., 1:] < NB)).sum(-1)
    row_bad = (bad_num | oor.any(-1) | late.any(-1) | (dup > 0)).flatten()
    first = int(torch.nonzero(row_bad)[0, 0]) if bool(row_bad.any()) else 2 ** 31 - 1
    return [int(bad_num.sum()), int(oor.sum()), int(late.sum()), int(dup.sum()), first]


def check_lists(kv_num: torch.Tensor, kv_idx: torch.Tensor, NB: int, *, causal: bool = True,
                who: str = "check_lists") -> None:
    """Raise ``RuntimeError`` unless every row (h, qb) of the compact lists
    kv_num [.., H, QB] / kv_idx [.., H, QB, MAXKV] holds 0 <= kv_num <= MAXKV
    distinct key blocks in [0, NB), each <= qb when ``causal`` — what the
    reference's pack guarantees (model/attn_bias.py:825-837) and every kernel
    here relies on.  GPU tensors: ``scope_check_lists`` and a host read of its
    counters (skipped under graph capture, where nothing may synchronise);
    CPU tensors: the same rules in torch."""
    H, QB = int(kv_num.shape[-2]), int(kv_num.shape[-1])
    maxkv = int(kv_idx.shape[-1])
    if kv_num.numel() != H * QB or kv_idx.numel() != H * QB * maxkv:
        raise RuntimeError(f"{who}: kv_num {tuple(kv_num.shape)} and kv_indices {tuple(kv_idx.shape)} do not match")
    if kv_num.is_cuda or kv_idx.is_cuda:
        dev = _gpu(who, kv_num, kv_idx)
        if torch.cuda.is_current_stream_capturing():
            return
        res = torch.empty(5, dtype=torch.int32, device=dev)
        call("scope_check_lists", _p(_i32(kv_num.reshape(H, QB))), _p(_i32(kv_idx.reshape(H, QB, maxkv))), H, QB,
             int(NB), maxkv, int(bool(causal)), _p(res), _stream(dev))
        r = res.tolist()
    else:
        r = _check_lists_host(kv_num.reshape(H, QB), kv_idx.reshape(H, QB, maxkv), int(NB), bool(causal))
    if any(r[:4]):
        h, qb = divmod(int(r[4]), QB)
        raise RuntimeError(f"{who}: malformed block lists: {r[0]} rows with kv_num outside [0, {maxkv}], {r[1]} "
                           f"entries outside [0, {NB}), {r[2]} entries after their q-block, {r[3]} repeated "
                           f"entries (first bad row: head {h}, q-block {qb})")


def transpose_blocks(kv_num: torch.Tensor, kv_idx: torch.Tensor, NB: int, tail: int | None = None, *,
                     check: bool = True):
    """q lists (CSR): q_off [H, NB+1], q_list [H, QB*MAXKV].  Entries of a
    head's q_list past q_off[h, NB] are -1 (the kernels set them), or ``tail``.
    ``check``: validate the lists first (``check_lists``, one host read);
    the library's own callers pass lists its builders made and skip it."""
    dev = _gpu("transpose_blocks", kv_num, kv_idx)
    if check:
        check_lists(kv_num, kv_idx, NB, who="transpose_blocks")
    kv_num = _i32(kv_num.reshape(kv_num.shape[-2], kv_num.shape[-1]))
    H, QB = kv_num.shape
    kv_idx = _i32(kv_idx.reshape(H, QB, kv_idx.shape[-1]))
    maxkv = kv_idx.shape[-1]
    q_off = torch.empty((H, NB + 1), dtype=torch.int32, device=dev)
    q_list = torch.empty((H, QB * maxkv), dtype=torch.int32, device=dev)
    ws = torch.empty(max(1, query("scope_transpose_workspace_bytes", H, NB)), dtype=torch.uint8, device=dev)
    call("scope_transpose_blocks", _p(kv_num), _p(kv_idx), H, QB, NB, maxkv, _p(q_off), _p(q_list), _p(ws),
         _stream(dev))
    if tail is not None and int(tail) != -1:
        q_list.masked_fill_(q_list == -1, int(tail))
    return q_off, q_list


NOALLOC_MAX_HNB = 262144  # include/scope_amd.h SCOPE_NOALLOC_MAX_HNB


def transpose_blocks_noalloc(kv_num: torch.Tensor, kv_idx: torch.Tensor, q_off: torch.Tensor,
                             q_list: torch.Tensor) -> None:
    """``transpose_blocks`` into caller-provided q_off [H, NB+1] / q_list
    [H, QB*MAXKV] int32 without any device allocation by the library (its
    cursors sit in a static device array: H*NB <= 262144; calls that overlap
    on one device race).  kv_num / kv_idx must already be contiguous int32."""
    dev = _gpu("transpose_blocks_noalloc", kv_num, kv_idx, q_off, q_list)
    for n_, t in (("kv_num", kv_num), ("kv_idx", kv_idx), ("q_off", q_off), ("q_list", q_list)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise RuntimeError(f"transpose_blocks_noalloc: {n_} must be a contiguous int32 tensor")
    H, QB = kv_num.shape[-2], kv_num.shape[-1]
    maxkv = kv_idx.shape[-1]
    NB = q_off.shape[-1] - 1
    if q_off.numel() != H * (NB + 1) or q_list.numel() != H * QB * maxkv or kv_idx.numel() != H * QB * maxkv:
        raise RuntimeError("transpose_blocks_noalloc: q_off [H, NB+1], q_list [H, QB*MAXKV] do not match the lists")
    call("scope_transpose_blocks_noalloc", _p(kv_num), _p(kv_idx), H, QB, NB, maxkv, _p(q_off), _p(q_list),
         _stream(dev))


def _coeff_prm(y: torch.Tensor, prm: dict):
    from ._lib import CoeffParams

    Y = y.shape[-1]
    rows = y.numel() // Y
    c = CoeffParams(M=int(prm["M"]), K=int(prm["K"]), rows=rows, L=int(prm["L"]), y_cols=Y, y_stride=Y,
                    y_bf16=int(y.dtype == torch.bfloat16), use_slope=int(bool(prm["use_slope"])),
                    subtract_b0=int(bool(prm["subtract_b0"])), training=int(bool(prm["training"])),
                    delta_cap=float(prm["delta_cap"]), logw_min=float(prm["logw_min"]),
                    logw_max=float(prm["logw_max"]), c_scale=float(prm["c_scale"]),
                    width_min=float(prm["width_min"]), width_max=float(prm["width_max"]), eps=float(prm["eps"]),
                    lambda_omega=float(prm["lambda_omega"]), lambda_entropy=float(prm["lambda_entropy"]),
                    lambda_zero_mean=float(prm["lambda_zero_mean"]),
                    lambda_delta_edge=float(prm["lambda_delta_edge"]), entropy_floor=float(prm["entropy_floor"]),
                    delta_edge_eps=float(prm["delta_edge_eps"]))
    return c, rows


def coeff_head_fwd(y: torch.Tensor, prm: dict, omegas: torch.Tensor, log_omegas: torch.Tensor,
                   cos_mean: torch.Tensor | None, sin_mean: torch.Tensor | None) -> dict:
    """Fused coefficient head (model/attn_bias.py:419-506) on the MLP output
    y [..., 5M (+1)] (fp32 or bf16): the nine per-row outputs, shaped like y's
    leading dimensions, and ``reg`` [6] (total, omega, entropy, delta_edge,
    zero_mean, mean b̄) when ``prm["training"]``."""
    dev = _gpu("coeff_head_fwd", y, omegas, log_omegas)
    if y.dtype not in (torch.float32, torch.bfloat16):
        y = y.float()
    y = y.contiguous()
    c, rows = _coeff_prm(y, prm)
    lead = tuple(y.shape[:-1])
    M, K = c.M, c.K
    f = dict(dtype=torch.float32, device=dev)
    out = dict(coeff_cos=torch.empty(lead + (K,), **f), coeff_sin=torch.empty(lead + (K,), **f),
               slope=torch.empty(lead, **f), b0=torch.empty(lead, **f), delta_star=torch.empty(lead + (M,), **f),
               pi=torch.empty(lead + (M,), **f), budget_logits=torch.empty(lead + (M,), **f),
               delta_main=torch.empty(lead, **f), width=torch.empty(lead, **f))
    # the regulariser kernel writes all six values when training; otherwise they are zero
    reg = torch.empty(6, **f) if prm["training"] else torch.zeros(6, **f)
    ws = torch.empty(max(1, int(query("scope_coeff_head_workspace_bytes", C.byref(c)))), dtype=torch.uint8,
                     device=dev)
    call("scope_coeff_head_fwd", C.byref(c), _p(y), _p(_f32(omegas)), _p(_f32(log_omegas)), _p(_f32(cos_mean)),
         _p(_f32(sin_mean)), *(_p(out[n]) for n in ("coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi",
                                                     "budget_logits", "delta_main", "width")),
         _p(reg), _p(ws), _stream(dev))
    out["reg"] = reg
    return out


def _row_layout(x: torch.Tensor):
    """(rows, seg, segment stride, row stride) of x's rows (its last dimension
    is the row, unit stride): a 2-D [R, C] tensor, or [..., S, T, C] with
    size-1 leading dimensions (segments S of T rows, e.g. the heads of a
    [1, H, T, D] view).  None when x has neither form."""
    if x.stride(-1) != 1:
        return None
    shape, strides = list(x.shape[:-1]), list(x.stride()[:-1])
    while len(shape) > 2 and shape[0] == 1:
        shape.pop(0)
        strides.pop(0)
    if len(shape) == 1:
        return shape[0], shape[0], 0, strides[0]
    if len(shape) == 2:
        return shape[0] * shape[1], shape[1], strides[0], strides[1]
    return None


WGRAD_SHAPES = {(64, 128), (64, 256), (128, 128), (128, 256), (256, 64), (256, 128)}


def linear_wgrad_takes(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Whether ``linear_wgrad`` takes a [..., M] and b [..., N] as they are:
    bf16, (M, N) one of WGRAD_SHAPES, and rows (and every segment of rows of
    a strided operand) a multiple of 64 (scope_linear_wgrad's limits)."""
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16 or (a.shape[-1], b.shape[-1]) not in WGRAD_SHAPES:
        return False
    rows = a.numel() // max(1, a.shape[-1])
    if rows == 0 or rows % 64 or b.numel() // max(1, b.shape[-1]) != rows:
        return False
    for x in (a, b):
        lx = _row_layout(x)
        if lx is not None and (lx[1] % 64 or lx[3] % 8 or (lx[1] != lx[0] and lx[2] % 8) or x.data_ptr() % 16):
            return False
    return True


def linear_wgrad(a: torch.Tensor, b: torch.Tensor, *, round_bf16: bool = True, want_db: bool = True):
    """dw [M, N] = Σ_r a[r]^T b[r] and db [M] = Σ_r a[r] over the rows of a
    [..., M] and b [..., N] (bf16, the same rows): the weight and bias
    gradients of a linear layer with output gradient a and input b
    (model/attn_bias.py:271-276; autograd of F.linear).  fp32 results,
    rounded to bf16 first with ``round_bf16``; db is None without
    ``want_db``."""
    dev = _gpu("linear_wgrad", a, b)
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise RuntimeError("linear_wgrad: a and b must be bf16")
    M, N = a.shape[-1], b.shape[-1]
    la, lb = _row_layout(a), _row_layout(b)
    if la is None:  # copied to one segment of rows
        a = a.contiguous().reshape(-1, M)
        la = _row_layout(a)
    if lb is None:
        b = b.contiguous().reshape(-1, N)
        lb = _row_layout(b)
    if la[0] != lb[0]:
        raise RuntimeError(f"linear_wgrad: {la[0]} rows of a against {lb[0]} rows of b")
    rows = la[0]
    # one segment length for both: an operand with one row stride takes the other's segments
    segs = {l[1] for l in (la, lb) if l[1] != rows}
    if len(segs) > 1:
        raise RuntimeError(f"linear_wgrad: segments of {sorted(segs)} rows in a and b")
    seg = segs.pop() if segs else rows

    def strides(l):
        return (l[2], l[3]) if l[1] == seg else (seg * l[3], l[3])

    a_ss, a_rs = strides(la)
    b_ss, b_rs = strides(lb)
    prm = _lib.WgradParams(rows=rows, seg=seg, M=M, N=N, a_ss=a_ss, a_rs=a_rs, b_ss=b_ss, b_rs=b_rs,
                           round_bf16=int(bool(round_bf16)))
    dw = torch.empty((M, N), dtype=torch.float32, device=dev)
    db = torch.empty(M, dtype=torch.float32, device=dev) if want_db else None
    ws = torch.empty(max(16, int(query("scope_linear_wgrad_workspace_bytes", C.byref(prm)))), dtype=torch.uint8,
                     device=dev)
    call("scope_linear_wgrad", C.byref(prm), _p(a), _p(b), _p(dw), _p(db), _p(ws), _stream(dev))
    return dw, db


def _mlp_params(q: torch.Tensor, w2: torch.Tensor):
    lq = _row_layout(q)
    if lq is None:  # e.g. [B, H, L, D] with B > 1: copied to one segment of rows
        q = q.contiguous().reshape(-1, q.shape[-1])
        lq = _row_layout(q)
    rows, seg, ss, rs = lq
    if seg == rows:
        ss = 0
    return q, _lib.MlpParams(rows=rows, seg=seg, q_ss=ss, q_rs=rs, D=q.shape[-1], H=256, O=w2.shape[0])


def coeff_mlp_fused(q: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> bool:
    """Whether the fused MLP kernels take these operands: bf16 rows of 128, fp32
    contiguous weights [256][128] and [O][256] with O <= 64, rows (and the
    segments of a [1, H, T, 128] view) a multiple of 32 (otherwise the
    operator runs the reference's torch steps)."""
    if not (q.dtype == torch.bfloat16 and q.shape[-1] == 128 and w1.dtype == torch.float32
            and w2.dtype == torch.float32 and tuple(w1.shape) == (256, 128) and w2.dim() == 2
            and w2.shape[1] == 256 and 1 <= w2.shape[0] <= 64 and q.numel() // 128 % 32 == 0 and q.numel() > 0):
        return False
    lq = _row_layout(q)
    return lq is None or lq[1] % 32 == 0  # no row layout: the operands are copied to one segment


def coeff_mlp_fwd(q: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor,
                  b2: torch.Tensor) -> torch.Tensor:
    """y [..., O] = W2·SiLU(W1·q + b1) + b2 on bf16 rows of q [..., 128] with the
    fp32 weights rounded to bf16 (model/attn_bias.py:271-276, 380-386)."""
    dev = _gpu("coeff_mlp_fwd", q, w1, b1, w2, b2)
    w1, b1, w2, b2 = (t.contiguous() for t in (w1, b1, w2, b2))
    qc, prm = _mlp_params(q, w2)
    y = torch.empty(q.shape[:-1] + (w2.shape[0],), dtype=q.dtype, device=dev)
    call("scope_coeff_mlp_fwd", C.byref(prm), _p(qc), _p(w1), _p(b1), _p(w2), _p(b2), _p(y), _stream(dev))
    return y


def coeff_mlp_bwd(q: torch.Tensor, gy: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor,
                  b2: torch.Tensor, *, intermediates: bool = True):
    """The row-wise part of the MLP's backward: (dq [..., 128], dz1 [..., 256],
    x1 [..., 256], gy padded to [..., 64]), bf16, from the output gradient gy
    [..., O]; z1 and x1 are recomputed from q.  Without ``intermediates``,
    dz1 and x1 are not written and come back as None."""
    dev = _gpu("coeff_mlp_bwd", q, gy, w1, b1, w2, b2)
    w1, b1, w2, b2 = (t.contiguous() for t in (w1, b1, w2, b2))
    qc, prm = _mlp_params(q, w2)
    gy = gy.to(q.dtype).contiguous()
    lead = q.shape[:-1]
    dq = torch.empty(lead + (128,), dtype=q.dtype, device=dev)
    dz1 = torch.empty(lead + (256,), dtype=q.dtype, device=dev) if intermediates else None
    x1 = torch.empty(lead + (256,), dtype=q.dtype, device=dev) if intermediates else None
    gyp = torch.empty(lead + (64,), dtype=q.dtype, device=dev)
    call("scope_coeff_mlp_bwd", C.byref(prm), _p(qc), _p(gy), _p(w1), _p(b1), _p(w2), _p(b2), _p(dq), _p(dz1),
         _p(x1), _p(gyp), _stream(dev))
    return dq, dz1, x1, gyp


def coeff_mlp_wgrad_fused(q: torch.Tensor) -> bool:
    """Whether scope_coeff_mlp_wgrad takes q's row layout (segments of a
    multiple of 128 rows)."""
    lq = _row_layout(q)
    return lq is not None and lq[1] % 128 == 0


def coeff_mlp_wgrad(q: torch.Tensor, gyp: torch.Tensor, w1: torch.Tensor, b1: torch.Tensor, w2: torch.Tensor):
    """The MLP's weight and bias gradients (dw1 [256][128], db1 [256], dw2
    [O][256], db2 [O]), fp32 values of the bf16 weight copies' gradients
    rounded to bf16, from q and the padded output gradient gyp [..., 64]
    (coeff_mlp_bwd's fourth output); z1, x1 and dz1 are recomputed per tile
    and never stored."""
    dev = _gpu("coeff_mlp_wgrad", q, gyp, w1, b1, w2)
    w1, b1, w2 = (t.contiguous() for t in (w1, b1, w2))
    qc, prm = _mlp_params(q, w2)
    if prm.seg % 128:
        raise RuntimeError(f"coeff_mlp_wgrad: segments of {prm.seg} rows (a multiple of 128 is needed)")
    gyp = gyp.contiguous()
    if gyp.dtype != torch.bfloat16 or gyp.shape[-1] != 64 or gyp.numel() != prm.rows * 64:
        raise RuntimeError("coeff_mlp_wgrad: gyp must be bf16 [..., 64] with q's rows")
    O = w2.shape[0]
    dw1 = torch.empty((256, 128), dtype=torch.float32, device=dev)
    db1 = torch.empty(256, dtype=torch.float32, device=dev)
    dw2 = torch.empty((64, 256), dtype=torch.float32, device=dev)
    db2 = torch.empty(64, dtype=torch.float32, device=dev)
    ws = torch.empty(max(16, int(query("scope_coeff_mlp_wgrad_workspace_bytes", C.byref(prm)))), dtype=torch.uint8,
                     device=dev)
    call("scope_coeff_mlp_wgrad", C.byref(prm), _p(qc), _p(gyp), _p(w1), _p(b1), _p(w2), _p(dw1), _p(db1), _p(dw2),
         _p(db2), _p(ws), _stream(dev))
    return dw1, db1, dw2[:O], db2[:O]


def coeff_head_bwd(y: torch.Tensor, prm: dict, omegas: torch.Tensor, log_omegas: torch.Tensor,
                   cos_mean: torch.Tensor | None, sin_mean: torch.Tensor | None, grads: dict,
                   g_reg: torch.Tensor | None = None, reg: torch.Tensor | None = None) -> torch.Tensor:
    """dy (y's dtype and shape) from the upstream gradients of the outputs
    (``grads[name]``, missing = zero) and of reg[0] (``g_reg``)."""
    dev = _gpu("coeff_head_bwd", y, omegas, log_omegas)
    if y.dtype not in (torch.float32, torch.bfloat16):
        y = y.float()
    y = y.contiguous()
    c, rows = _coeff_prm(y, prm)
    dy = torch.empty_like(y)
    g = [_f32(grads.get(n)) for n in ("coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits",
                                       "delta_main", "width")]
    gr = None if g_reg is None else _f32(g_reg.reshape(1))
    call("scope_coeff_head_bwd", C.byref(c), _p(y), _p(_f32(omegas)), _p(_f32(log_omegas)), _p(_f32(cos_mean)),
         _p(_f32(sin_mean)), *(_p(x) for x in g), _p(gr), _p(reg), _p(dy), _stream(dev))
    return dy


def swa_blockmask(docs: torch.Tensor, bs: int, window_blocks: int, *, export: bool = False) -> dict:
    """Sliding-window block lists of the long (W) and short (W // 2) masks
    (scoped_medium.py:535-576) from int document ids [T].

    Returns ``counts`` [6, NB] (n_partial, n_full, then the BlockMask counts
    kv_num_blocks / full_kv_num_blocks of the long and the short mask),
    ``long`` / ``short`` = (kv_num [NB], kv_idx [NB, width]) compact lists,
    and, with ``export``, the ordered rows ``partial_idx`` / ``full_idx``
    [NB, NB] of dense_to_ordered."""
    dev = _gpu("swa_blockmask", docs)
    docs = _i32(docs.reshape(-1))
    T = docs.numel()
    if T % bs:
        raise RuntimeError(f"swa_blockmask: T={T} not a multiple of bs={bs}")
    NB = T // bs
    W = int(window_blocks)
    wl, ws = query("scope_swa_width", T, int(bs), W), query("scope_swa_width", T, int(bs), W // 2)
    counts = torch.empty((6, NB), dtype=torch.int32, device=dev)
    pidx = torch.empty((NB, NB), dtype=torch.int32, device=dev) if export else None
    fidx = torch.empty((NB, NB), dtype=torch.int32, device=dev) if export else None
    kvl = torch.empty(NB, dtype=torch.int32, device=dev)
    kil = torch.empty((NB, wl), dtype=torch.int32, device=dev)
    kvs = torch.empty(NB, dtype=torch.int32, device=dev)
    kis = torch.empty((NB, ws), dtype=torch.int32, device=dev)
    call("scope_swa_blockmask", _p(docs), T, int(bs), W, _p(counts), _p(pidx), _p(fidx), _p(kvl), _p(kil), _p(kvs),
         _p(kis), _stream(dev))
    return dict(counts=counts, partial_idx=pidx, full_idx=fidx, long=(kvl, kil), short=(kvs, kis))


def mask_stats(*, H: int, QB: int, bs: int, M: int = 0, delta_star: torch.Tensor | None = None,
               pi: torch.Tensor | None = None, rep_mode: str = "last", has_docs: bool = False,
               docstart_enabled: bool = False, local_blocks_cfg: int = 1, eps: float = 1e-9,
               ds_ptr_fwd: torch.Tensor | None = None, ds_local_fwd: torch.Tensor | None = None,
               kv_num: torch.Tensor | None = None, radius: torch.Tensor | None = None, maxkv_bins: int = 1,
               radius_bins: int = 1, extra_bins: int = 1, picks: torch.Tensor | None = None,
               ds_ptr: torch.Tensor | None = None, ds_local: torch.Tensor | None = None,
               bs_local_blocks: int = 1):
    """Fused statistics -> (counts int32, values fp32 [SCOPE_SV_COUNT])."""
    dev = _gpu("mask_stats", delta_star, pi, kv_num, radius, picks)
    sh = st = 0
    T = QB * bs
    if delta_star is not None:
        d3, p3 = (delta_star[0], pi[0]) if delta_star.dim() == 4 else (delta_star, pi)
        d3, p3 = _f32(d3), _f32(p3)
        sh, st = d3.stride(0), d3.stride(1)
        M = d3.shape[-1]
    else:
        d3 = p3 = None
    budget = picks.shape[-1] if picks is not None else 0
    prm = StatsParams(H=H, QB=QB, bs=bs, M=M, T=T, stride_h=sh, stride_t=st, rep_mean=int(rep_mode == "mean"),
                      has_docs=int(has_docs), docstart_enabled=int(docstart_enabled),
                      local_blocks_cfg=int(local_blocks_cfg), eps=float(eps), maxkv_bins=int(maxkv_bins),
                      radius_bins=int(radius_bins), extra_bins=int(extra_bins), budget=int(budget),
                      bs_local_blocks=int(bs_local_blocks))
    n = query("scope_stats_counts_len", C.byref(prm))
    counts = torch.empty(n, dtype=torch.int32, device=dev)
    values = torch.zeros(len(SV_NAMES), dtype=torch.float32, device=dev)
    ws = torch.empty(max(4, query("scope_stats_workspace_bytes", C.byref(prm))), dtype=torch.uint8, device=dev)
    call("scope_mask_stats", C.byref(prm), _p(d3), _p(p3), _p(_i32(ds_ptr_fwd) if ds_ptr_fwd is not None else None),
         _p(_i32(ds_local_fwd) if ds_local_fwd is not None else None),
         _p(_i32(kv_num) if kv_num is not None else None), _p(_i32(radius) if radius is not None else None),
         _p(_i32(picks.contiguous()) if picks is not None else None),
         _p(_i32(ds_ptr) if ds_ptr is not None else None), _p(_i32(ds_local) if ds_local is not None else None),
         _p(counts), _p(values), _p(ws), _stream(dev))
    return counts, values


def unpack_counts(counts: torch.Tensor, maxkv_bins: int, radius_bins: int) -> dict:
    c = counts
    out = dict(delta_tokens_hist=c[ST_DELTA_TOKENS:ST_DELTA_TOKENS + 16],
               delta_blocks_hist=c[ST_DELTA_BLOCKS:ST_DELTA_BLOCKS + 15],
               ptr_center_hist=c[ST_CENTER:ST_CENTER + 15],
               ptr_dist_hist=c[ST_PTR_DIST:ST_PTR_DIST + 15],
               kv_unique_hist=c[ST_FIXED:ST_FIXED + maxkv_bins],
               ptr_radius_hist=c[ST_FIXED + maxkv_bins:ST_FIXED + maxkv_bins + radius_bins],
               ptr_extra_sum_hist=c[ST_FIXED + maxkv_bins + radius_bins:])
    for name, i in (("docstart", ST_DOCSTART), ("outside", ST_OUTSIDE), ("block0", ST_BLOCK0),
                    ("block0_excl", ST_BLOCK0_EXCL), ("n_centres", ST_N_CENTRES), ("bs_outside", ST_BS_OUTSIDE),
                    ("bs_block0", ST_BS_BLOCK0), ("bs_block0_excl", ST_BS_BLOCK0_EXCL),
                    ("bs_docstart", ST_BS_DOCSTART), ("bs_n", ST_BS_N), ("bs_n_excl", ST_BS_N_EXCL),
                    ("radius0", ST_RADIUS0), ("n_radius", ST_N_RADIUS)):
        out[name] = c[i]
    return out


def spectral_table(omegas: torch.Tensor, T: int, bs: int, mode: str) -> torch.Tensor:
    """cos/sin(ω_k r) tables (model/attn_bias.py:326-340 restated per block or token)."""
    dev = _gpu("spectral_table", omegas)
    m = BIAS_MODES[mode]
    om = _f32(omegas.reshape(-1))
    K = om.numel()
    nbytes = query("scope_spectral_table_bytes", m, T, bs)
    tab = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    call("scope_spectral_table", m, _p(om), K, T, bs, _p(tab), _stream(dev))
    return tab


def _attn_params(q, k, v, out, *, bs, maxkv, scale, beta, bias_mode, K, use_slope, subtract_b0, gate_kind,
                 ramp_lambda, tau) -> AttnParams:
    H, T, D, qsh, qst = _bhtd("attention q", q)
    _, _, _, ksh, kst = _bhtd("attention k", k)
    _, _, _, vsh, vst = _bhtd("attention v", v)
    _, _, _, osh, ost = _bhtd("attention out", out)
    if not (q.shape == k.shape == v.shape):
        raise RuntimeError(f"attention: q, k, v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    for n_, x in (("q", q), ("k", k), ("v", v)):
        if x.dtype != torch.bfloat16:
            raise RuntimeError(f"attention: {n_} must be bfloat16 (got {x.dtype})")
    return AttnParams(H=H, D=D, bs=bs, maxkv=maxkv, T=T, scale=float(scale), beta=float(beta),
                      bias_mode=int(bias_mode), K=int(K), use_slope=int(bool(use_slope)),
                      subtract_b0=int(bool(subtract_b0)), gate_kind=int(gate_kind), ramp_lambda=float(ramp_lambda),
                      tau=float(tau), q_sh=qsh, q_st=qst, k_sh=ksh, k_st=kst, v_sh=vsh, v_st=vst, o_sh=osh, o_st=ost)


def _pair_bias(pair_bias, kv_idx3):
    if pair_bias is None:
        return None
    pb = _f32(pair_bias.reshape(kv_idx3.shape))
    return pb


def empty_like_layout(x: torch.Tensor) -> torch.Tensor:
    """New tensor with x's shape and memory order (like FlexAttention's output)."""
    return torch.empty_like(x)


def attn_fwd(q, k, v, kv_num, kv_idx, docs, ds_tok_end, *, bs: int, scale: float, beta: float = 0.5,
             bias_mode: str = "none", table=None, coeff_cos=None, coeff_sin=None, b0=None, slope=None,
             delta_main=None, width=None, use_slope=False, subtract_b0=False, gate_kind="none",
             ramp_lambda=0.0, tau=64.0, out=None, pair_bias=None, check: bool = True):
    """Block-sparse attention forward -> (out like q, lse [1,H,T] fp32, natural log).
    ``pair_bias`` [H,QB,MAXKV] (aligned with kv_idx) is added to every score of
    each listed tile.  ``check``: validate the lists first (``check_lists``)."""
    dev = _gpu("attn_fwd", q, k, v, kv_num, kv_idx, docs, ds_tok_end, pair_bias)
    if check:
        check_lists(kv_num, kv_idx, q.shape[-2] // bs, who="attn_fwd")
    out = empty_like_layout(q) if out is None else out
    kv_idx3 = _i32(kv_idx.reshape(-1, kv_idx.shape[-2], kv_idx.shape[-1]))
    m = BIAS_MODES[bias_mode]
    K = coeff_cos.shape[-1] if (m and coeff_cos is not None) else 0
    prm = _attn_params(q, k, v, out, bs=bs, maxkv=kv_idx3.shape[-1], scale=scale, beta=beta, bias_mode=m, K=K,
                       use_slope=use_slope, subtract_b0=subtract_b0, gate_kind=GATE_KINDS[gate_kind],
                       ramp_lambda=ramp_lambda, tau=tau)
    H, T = prm.H, prm.T
    pb = _pair_bias(pair_bias, kv_idx3)
    prm.pair_bias = _p(pb)
    lse = torch.empty((1, H, T), dtype=torch.float32, device=dev)
    call("scope_attn_fwd", C.byref(prm), _p(q), _p(k), _p(v), _p(_i32(kv_num)), _p(kv_idx3),
         _p(_i32(docs.reshape(-1))), _p(_i32(ds_tok_end)), _p(table), _p(_f32(coeff_cos)), _p(_f32(coeff_sin)),
         _p(_f32(b0)), _p(_f32(slope)), _p(_f32(delta_main)), _p(_f32(width)), _p(out), _p(lse), _stream(dev))
    return out, lse


def attn_block_mass(q, k, kv_num, kv_idx, docs, ds_tok_end, *, bs: int, scale: float, beta: float = 0.5,
                    bias_mode: str = "none", table=None, coeff_cos=None, coeff_sin=None, b0=None, slope=None,
                    delta_main=None, width=None, use_slope=False, subtract_b0=False, gate_kind="none",
                    ramp_lambda=0.0, tau=64.0, check: bool = True):
    """Attention probability mass per (head, q-block, listed key block),
    summed over the q-block's rows -> (mass [H, QB, NB] fp32, lse [1,H,T]).
    ``check``: validate the lists first (``check_lists``)."""
    dev = _gpu("attn_block_mass", q, k, kv_num, kv_idx, docs, ds_tok_end)
    if check:
        check_lists(kv_num, kv_idx, q.shape[-2] // bs, who="attn_block_mass")
    kv_idx3 = _i32(kv_idx.reshape(-1, kv_idx.shape[-2], kv_idx.shape[-1]))
    m = BIAS_MODES[bias_mode]
    K = coeff_cos.shape[-1] if (m and coeff_cos is not None) else 0
    prm = _attn_params(q, k, k, q, bs=bs, maxkv=kv_idx3.shape[-1], scale=scale, beta=beta, bias_mode=m, K=K,
                       use_slope=use_slope, subtract_b0=subtract_b0, gate_kind=GATE_KINDS[gate_kind],
                       ramp_lambda=ramp_lambda, tau=tau)
    H, T = prm.H, prm.T
    NB = T // bs
    lse = torch.empty((1, H, T), dtype=torch.float32, device=dev)
    mass = torch.zeros((H, NB, NB), dtype=torch.float32, device=dev)
    call("scope_attn_block_mass", C.byref(prm), _p(q), _p(k), _p(_i32(kv_num)), _p(kv_idx3),
         _p(_i32(docs.reshape(-1))), _p(_i32(ds_tok_end)), _p(table), _p(_f32(coeff_cos)), _p(_f32(coeff_sin)),
         _p(_f32(b0)), _p(_f32(slope)), _p(_f32(delta_main)), _p(_f32(width)), _p(lse), _p(mass), _stream(dev))
    return mass, lse


def decode_attn(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_num: torch.Tensor,
                kv_idx: torch.Tensor, docs: torch.Tensor, t: int | torch.Tensor, *, bs: int, scale: float,
                workspace: torch.Tensor | None = None, check: bool = True):
    """Attention of the token at position t: q [H, D] bf16 against the cache
    k_cache / v_cache [H, T_cap, D] over the listed blocks kv_idx [H, maxkv]
    (kv_num [H]) -> (out [H, D] bf16, lse [H] natural log).  ``t`` is an int,
    or a one-element int64 tensor on the device that the kernel reads (no host
    sync; what a captured decode step needs).  ``check``: validate the list
    first (distinct blocks of the cache; ``check_lists``, skipped under capture)."""
    from ._lib import DecodeParams

    dev = _gpu("decode_attn", q, k_cache, v_cache, kv_num, kv_idx, docs)
    if check:
        check_lists(kv_num.reshape(-1, 1), kv_idx.reshape(kv_idx.shape[0], 1, -1), k_cache.shape[1] // bs,
                    causal=False, who="decode_attn")
    if q.dim() != 2 or k_cache.dim() != 3 or v_cache.dim() != 3:
        raise RuntimeError("decode_attn: q [H, D], caches [H, T_cap, D]")
    for n_, x in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        if x.dtype != torch.bfloat16 or x.stride(-1) != 1:
            raise RuntimeError(f"decode_attn: {n_} must be bfloat16 with a unit last stride")
    H, D = q.shape
    T_cap = k_cache.shape[1]
    kv_idx = _i32(kv_idx)
    t_dev = t if isinstance(t, torch.Tensor) else None
    if t_dev is not None and (t_dev.dtype != torch.int64 or t_dev.numel() != 1 or t_dev.device != q.device):
        raise RuntimeError("decode_attn: a tensor position must be one int64 element on the device of q")
    prm = DecodeParams(H=H, D=D, bs=int(bs), maxkv=kv_idx.shape[-1], T_cap=T_cap, t=0 if t_dev is not None else int(t),
                       scale=float(scale),
                       q_sh=q.stride(0), k_sh=k_cache.stride(0), k_st=k_cache.stride(1), v_sh=v_cache.stride(0),
                       v_st=v_cache.stride(1), o_sh=D)
    need = int(query("scope_decode_workspace_bytes", C.byref(prm)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    out = torch.empty((H, D), dtype=torch.bfloat16, device=dev)
    lse = torch.empty(H, dtype=torch.float32, device=dev)
    tail = (_p(q), _p(k_cache), _p(v_cache), _p(_i32(kv_num)), _p(kv_idx), _p(_i32(docs.reshape(-1))), _p(workspace),
            _p(out), _p(lse), _stream(dev))
    if t_dev is not None:
        call("scope_decode_attn_at", C.byref(prm), _p(t_dev), *tail)
    else:
        call("scope_decode_attn", C.byref(prm), *tail)
    return out, lse


def decode_attn_glue(qkv: torch.Tensor, ve: torch.Tensor | None, t_dev: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, kv_num: torch.Tensor,
                     kv_idx: torch.Tensor, docs: torch.Tensor, *, heads: int, va: float, vb: float, bs: int,
                     scale: float, workspace: torch.Tensor | None = None, eps: float | None = None,
                     want_q: bool = False, check: bool = True):
    """``decoder_qkv_glue`` of one token (qkv [3·heads·D] bf16) fused into
    ``decode_attn`` at the device position t_dev: k and v go to cache row t
    and the attention uses them.  Returns (out [heads, D] bf16, lse [heads],
    q [heads, D] bf16 or None).  ``check`` as in ``decode_attn``."""
    from ._lib import DecodeParams

    dev = _gpu("decode_attn_glue", qkv, ve, t_dev, cos, sin, k_cache, v_cache, kv_num, kv_idx, docs)
    if check:
        check_lists(kv_num.reshape(-1, 1), kv_idx.reshape(kv_idx.shape[0], 1, -1), k_cache.shape[1] // bs,
                    causal=False, who="decode_attn_glue")
    D = k_cache.shape[-1]
    if qkv.dtype != torch.bfloat16 or not qkv.is_contiguous() or qkv.numel() != 3 * heads * D:
        raise RuntimeError("decode_attn_glue: qkv must be a contiguous bfloat16 [3*heads*D]")
    if ve is not None and (ve.dtype != torch.bfloat16 or not ve.is_contiguous() or ve.numel() != heads * D):
        raise RuntimeError("decode_attn_glue: ve must be a contiguous bfloat16 [heads*D]")
    if t_dev.dtype != torch.int64 or t_dev.numel() != 1:
        raise RuntimeError("decode_attn_glue: t_dev must be one int64 element")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.stride(-1) != 1 \
            or sin.stride() != cos.stride() or cos.shape[-1] != D // 2:
        raise RuntimeError("decode_attn_glue: cos/sin must be float32 [rows, D/2] with the same strides")
    for n_, x in (("k_cache", k_cache), ("v_cache", v_cache)):
        if x.dtype != torch.bfloat16 or x.dim() != 3 or x.shape[0] != heads or x.stride(-1) != 1:
            raise RuntimeError(f"decode_attn_glue: {n_} must be bfloat16 [heads, T_cap, D] with a unit last stride")
    kv_idx = _i32(kv_idx)
    prm = DecodeParams(H=heads, D=D, bs=int(bs), maxkv=kv_idx.shape[-1], T_cap=k_cache.shape[1], t=0,
                       scale=float(scale), q_sh=D, k_sh=k_cache.stride(0), k_st=k_cache.stride(1),
                       v_sh=v_cache.stride(0), v_st=v_cache.stride(1), o_sh=D)
    need = int(query("scope_decode_workspace_bytes", C.byref(prm)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    out = torch.empty((heads, D), dtype=torch.bfloat16, device=dev)
    lse = torch.empty(heads, dtype=torch.float32, device=dev)
    q = torch.empty((heads, D), dtype=torch.bfloat16, device=dev) if want_q else None
    e = torch.finfo(torch.float32).eps if eps is None else float(eps)
    call("scope_decode_attn_glue_at", C.byref(prm), _p(t_dev), _p(qkv), _p(ve), float(va), float(vb), e, _p(cos),
         _p(sin), cos.shape[0], cos.stride(0), _p(k_cache), _p(v_cache), _p(_i32(kv_num)), _p(kv_idx),
         _p(_i32(docs.reshape(-1))), _p(workspace), _p(out), _p(lse), _p(q), _stream(dev))
    return out, lse, q


def decoder_qkv_glue(qkv: torch.Tensor, ve: torch.Tensor | None, pos: torch.Tensor, cos: torch.Tensor,
                     sin: torch.Tensor, *, heads: int, va: float, vb: float, k_out: torch.Tensor | None = None,
                     v_out: torch.Tensor | None = None, eps: float | None = None):
    """The decoder attention layer's glue (scoped_medium.py:339-345): qkv
    [T, 3·heads·D] bf16 -> q [T, heads, D] (RMS-normed, rotated at pos [T]);
    k and v (normed + rotated / va·v + vb·ve) go to rows pos of the caches
    k_out / v_out [heads, rows, D], or, without caches, are returned as
    [T, heads, D] tensors.  Returns (q, k, v) with k, v the caches or the
    new tensors."""
    dev = _gpu("decoder_qkv_glue", qkv, ve, pos, cos, sin, k_out, v_out)
    T = qkv.shape[0]
    D = qkv.shape[-1] // (3 * heads)
    if qkv.dtype != torch.bfloat16 or not qkv.is_contiguous() or qkv.shape[-1] != 3 * heads * D:
        raise RuntimeError("decoder_qkv_glue: qkv must be a contiguous bfloat16 [T, 3*heads*D]")
    if ve is not None and (ve.dtype != torch.bfloat16 or not ve.is_contiguous() or ve.numel() != T * heads * D):
        raise RuntimeError("decoder_qkv_glue: ve must be a contiguous bfloat16 [T, heads*D]")
    if pos.dtype != torch.int64 or pos.numel() != T or not pos.is_contiguous():
        raise RuntimeError("decoder_qkv_glue: pos must be a contiguous int64 [T]")
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape != sin.shape or cos.stride(-1) != 1 \
            or sin.stride() != cos.stride() or cos.shape[-1] != D // 2:
        raise RuntimeError("decoder_qkv_glue: cos/sin must be float32 [rows, D/2] with the same strides")
    q = torch.empty((T, heads, D), dtype=torch.bfloat16, device=dev)
    at_pos = k_out is not None
    if at_pos:
        if v_out is None or k_out.shape != v_out.shape or k_out.dtype != torch.bfloat16 or v_out.dtype != torch.bfloat16 \
                or k_out.stride(-1) != 1 or v_out.stride(-1) != 1 or k_out.shape[0] != heads or k_out.shape[-1] != D:
            raise RuntimeError("decoder_qkv_glue: caches must be bfloat16 [heads, rows, D] with a unit last stride")
        kt, vt, rows = k_out, v_out, k_out.shape[1]
        strides = (kt.stride(0), kt.stride(1), vt.stride(0), vt.stride(1))
    else:
        kt = torch.empty((T, heads, D), dtype=torch.bfloat16, device=dev)
        vt = torch.empty((T, heads, D), dtype=torch.bfloat16, device=dev)
        rows = T
        strides = (D, heads * D, D, heads * D)  # head stride, row stride of a [T, heads, D] tensor
    # F.rms_norm's default eps for bf16 inputs is the epsilon of its fp32 compute type
    e = torch.finfo(torch.float32).eps if eps is None else float(eps)
    call("scope_decoder_qkv_glue", T, heads, D, rows, e, float(va), float(vb), _p(qkv), _p(ve), _p(pos), _p(cos),
         _p(sin), cos.shape[0], cos.stride(0), _p(q), _p(kt), _p(vt), *strides, 1 if at_pos else 0, _stream(dev))
    return q, kt, vt


GEMV_EPI = {"plain": 0, "relu2": 1, "resid": 2, "logit": 3}


def decoder_gemv(x: torch.Tensor, w: torch.Tensor, *, norm: bool = False, epi: str = "plain",
                 res: torch.Tensor | None = None, addx: torch.Tensor | None = None, eps: float | None = None):
    """One row-vector product of the decoder's token step with what surrounds
    it: x [K] bf16 (plus addx [K], the U-net skip, when given), optionally
    RMS-normed, times W [N, K] bf16, then the epilogue: "plain" -> bf16 [N],
    "relu2" -> relu(z)² bf16, "resid" -> res + z bf16 (res [N]), "logit" ->
    30·σ(z / 7.5) fp32.  With addx it returns (y, x + addx), else y."""
    dev = _gpu("decoder_gemv", x, w, res, addx)
    K = x.numel()
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise RuntimeError("decoder_gemv: x must be a contiguous bfloat16 row")
    if w.dtype != torch.bfloat16 or w.dim() != 2 or w.shape[1] != K or w.stride(1) != 1:
        raise RuntimeError(f"decoder_gemv: w must be bfloat16 [N, {K}] with a unit column stride")
    if epi not in GEMV_EPI:
        raise ValueError(f"decoder_gemv: epi must be one of {sorted(GEMV_EPI)}")
    N = w.shape[0]
    if (epi == "resid") != (res is not None):
        raise ValueError("decoder_gemv: res is given exactly with epi='resid'")
    if res is not None and (res.dtype != torch.bfloat16 or res.numel() != N or not res.is_contiguous()):
        raise RuntimeError(f"decoder_gemv: res must be a contiguous bfloat16 [{N}]")
    if addx is not None and (addx.dtype != torch.bfloat16 or addx.numel() != K or not addx.is_contiguous()):
        raise RuntimeError(f"decoder_gemv: addx must be a contiguous bfloat16 [{K}]")
    out = torch.empty(N, dtype=torch.float32 if epi == "logit" else torch.bfloat16, device=dev)
    xout = torch.empty(K, dtype=torch.bfloat16, device=dev) if addx is not None else None
    # F.rms_norm's default eps for bf16 inputs is the epsilon of its fp32 compute type
    e = torch.finfo(torch.float32).eps if eps is None else float(eps)
    call("scope_decoder_gemv", N, K, w.stride(0), 1 if norm else 0, e, GEMV_EPI[epi], _p(x), _p(addx), _p(xout),
         _p(w), _p(res), _p(out), _stream(dev))
    return (out, xout) if addx is not None else out


def argmax(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Index of the largest element of a contiguous fp32 vector (the first on
    ties, as torch.argmax; NaN never chosen), as an int64 [1] tensor on the
    device (``out`` when given)."""
    dev = _gpu("argmax", x, out)
    if x.dtype != torch.float32 or not x.is_contiguous() or x.numel() < 1:
        raise RuntimeError("argmax: x must be a non-empty contiguous float32 tensor")
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=dev)
    elif out.dtype != torch.int64 or out.numel() != 1:
        raise RuntimeError("argmax: out must be one int64 element")
    call("scope_argmax_f32", _p(x), x.numel(), _p(out), _stream(dev))
    return out


def decoder_step_prologue(tok: torch.Tensor, t_dev: torch.Tensor, tokens: torch.Tensor, docs: torch.Tensor,
                          embed: torch.Tensor, value_embeds, *, eot: int, eps: float | None = None):
    """The start of a decoder token step at the position t_dev (int64 [1] on
    the device): tokens[t] = tok, docs[t] = docs[t-1] + (tok == eot), and
    returns (x0 [dm] = F.rms_norm(embed[tok]) bf16, ve [len(value_embeds), dm]
    bf16 rows of the value-embedding tables, or None without tables)."""
    dev = _gpu("decoder_step_prologue", tok, t_dev, tokens, docs, embed, *value_embeds)
    if tok.dtype != torch.int64 or tok.numel() != 1 or t_dev.dtype != torch.int64 or t_dev.numel() != 1:
        raise RuntimeError("decoder_step_prologue: tok and t_dev must be one int64 element each")
    if tokens.dtype != torch.int64 or docs.dtype != torch.int32 or tokens.numel() != docs.numel() \
            or not tokens.is_contiguous() or not docs.is_contiguous():
        raise RuntimeError("decoder_step_prologue: tokens int64 [T_cap] and docs int32 [T_cap], contiguous")
    if len(value_embeds) > 3:
        raise ValueError("decoder_step_prologue: at most 3 value-embedding tables")
    V, dm = embed.shape
    for tb in (embed, *value_embeds):
        if tb.dtype != torch.bfloat16 or not tb.is_contiguous() or tb.shape != (V, dm):
            raise RuntimeError(f"decoder_step_prologue: embedding tables must be contiguous bfloat16 [{V}, {dm}]")
    x0 = torch.empty(dm, dtype=torch.bfloat16, device=dev)
    ve = torch.empty((len(value_embeds), dm), dtype=torch.bfloat16, device=dev) if value_embeds else None
    tabs = list(value_embeds) + [None] * (3 - len(value_embeds))
    e = torch.finfo(torch.float32).eps if eps is None else float(eps)
    call("scope_decoder_step_prologue", _p(tok), _p(t_dev), tokens.numel(), V, dm, e, int(eot), _p(tokens),
         _p(docs), _p(embed), *(_p(x) for x in tabs), _p(x0), _p(ve), _stream(dev))
    return x0, ve


def attn_bwd(q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list, docs, ds_tok_end, *, bs: int, scale: float,
             beta: float = 0.5, bias_mode: str = "none", table=None, coeff_cos=None, coeff_sin=None, b0=None,
             slope=None, delta_main=None, width=None, use_slope=False, subtract_b0=False, gate_kind="none",
             ramp_lambda=0.0, tau=64.0, need_coeff_grads: bool = True, phase_hook=None, pair_bias=None,
             need_pair_grad: bool = False, check: bool = True):
    """Block-sparse attention backward -> dict of gradients.  With
    ``phase_hook`` the phases (q-major dQ pass; kv-major plan, dK/dV kernel
    and reduce) are launched separately and the hook is called before, between
    and after them with the phase name ("dq", "plan", "dkv", "reduce", "end")
    (used for per-kernel timing).  ``check``: validate kv_num / kv_idx first
    (``check_lists``); q_off / q_list must be their transpose."""
    dev = _gpu("attn_bwd", q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list)
    if check:
        check_lists(kv_num, kv_idx, q.shape[-2] // bs, who="attn_bwd")
    kv_idx3 = _i32(kv_idx.reshape(-1, kv_idx.shape[-2], kv_idx.shape[-1]))
    m = BIAS_MODES[bias_mode]
    K = coeff_cos.shape[-1] if (m and coeff_cos is not None) else 0
    dq, dk, dv = empty_like_layout(q), empty_like_layout(k), empty_like_layout(v)
    prm = _attn_params(q, k, v, dq, bs=bs, maxkv=kv_idx3.shape[-1], scale=scale, beta=beta, bias_mode=m, K=K,
                       use_slope=use_slope, subtract_b0=subtract_b0, gate_kind=GATE_KINDS[gate_kind],
                       ramp_lambda=ramp_lambda, tau=tau)
    for name, a_, b_ in (("k", k, dk), ("v", v, dv), ("out", out, dout)):
        if a_.stride() != b_.stride():
            raise RuntimeError(f"attn_bwd: {name} and its gradient must share strides")
    if dout.stride() != q.stride() or out.stride() != q.stride():
        raise RuntimeError("attn_bwd: out and dout must share q's strides")
    H, T = prm.H, prm.T
    z = dict(dtype=torch.float32, device=dev)
    pb = _pair_bias(pair_bias, kv_idx3)
    dpb = torch.empty(kv_idx3.shape, **z) if need_pair_grad else None
    prm.pair_bias = _p(pb)
    prm.dpair_bias = _p(dpb)
    dcc = torch.empty((1, H, T, K), **z) if (m and need_coeff_grads) else None
    dcs = torch.empty((1, H, T, K), **z) if (m and need_coeff_grads) else None
    tok = m == 2 and need_coeff_grads
    db0 = torch.empty((1, H, T), **z) if (tok and subtract_b0) else None
    dsl = torch.empty((1, H, T), **z) if (tok and use_slope) else None
    gate = tok and GATE_KINDS[gate_kind] != 0
    ddm = torch.empty((1, H, T), **z) if gate else None
    dwd = torch.empty((1, H, T), **z) if gate else None
    ws = torch.empty(max(16, query("scope_attn_bwd_workspace_bytes", C.byref(prm))), dtype=torch.uint8, device=dev)
    # the converted inputs as locals: with phase_hook the same pointers serve four calls
    ins = (_f32(lse), _i32(kv_num), kv_idx3, _i32(q_off), _i32(q_list), _i32(docs.reshape(-1)), _i32(ds_tok_end),
           table, _f32(coeff_cos), _f32(coeff_sin), _f32(b0), _f32(slope), _f32(delta_main), _f32(width))
    args = (_p(q), _p(k), _p(v), _p(out), _p(dout), *(_p(t) for t in ins), _p(dq), _p(dk), _p(dv), _p(dcc), _p(dcs),
            _p(db0), _p(dsl), _p(ddm), _p(dwd), _p(ws), _stream(dev))
    if phase_hook is None:
        call("scope_attn_bwd", C.byref(prm), *args)
    else:
        phase_hook("dq")
        call("scope_attn_bwd_phase", C.byref(prm), 1, *args)
        phase_hook("plan")
        call("scope_attn_bwd_phase", C.byref(prm), 4, *args)
        phase_hook("dkv")
        call("scope_attn_bwd_phase", C.byref(prm), 8, *args)
        phase_hook("reduce")
        call("scope_attn_bwd_phase", C.byref(prm), 16, *args)
        phase_hook("end")
    return dict(dq=dq, dk=dk, dv=dv, dcoeff_cos=dcc, dcoeff_sin=dcs, db0=db0, dslope=dsl, ddelta_main=ddm,
                dwidth=dwd, dpair_bias=dpb)


def measure_peaks(device: torch.device | str = "cuda", *, mfma_iters: int = 16384, copy_mib: int = 1024,
                  repeats: int = 5) -> dict:
    """Measured ceilings on this GPU: bf16 dense MFMA TFLOP/s (independent
    32x32x16 chains on every SIMD) on constant operands and on random bf16
    operands in [-1, 1) (which draw the power attention's operands draw, so
    the power limit lowers the clock), and HBM copy GB/s (2 x bytes per
    copy).  The best of `repeats` timed launches is reported."""
    dev = torch.device(device)
    _gpu("measure_peaks", torch.empty(1, device=dev))
    lib = _lib.load()
    st = _stream(dev)
    props = torch.cuda.get_device_properties(dev)
    blocks = props.multi_processor_count * 2  # 8 wavefronts per CU: 2 per SIMD
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flops = lib.scope_probe_mfma_flops(blocks, mfma_iters)
    g = torch.Generator(device=dev).manual_seed(7)
    ops_rnd = (torch.rand((blocks * 256, 16, 8), generator=g, device=dev) * 2 - 1).to(torch.bfloat16)
    src = torch.ones(copy_mib << 18, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    nbytes = src.numel() * 4

    def best(fn):
        fn()
        ts = []
        for _ in range(repeats):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize(dev)
            ts.append(e0.elapsed_time(e1) / 1e3)
        return min(ts)

    t_mfma = best(lambda: call("scope_probe_mfma", _p(out), blocks, mfma_iters, st))
    it8 = max(8, mfma_iters // 8 * 8)  # the data probe's steps come in groups of 8
    t_data = best(lambda: call("scope_probe_mfma_data", _p(ops_rnd), _p(out), blocks, it8, st))
    t_copy = best(lambda: call("scope_probe_copy", _p(src), _p(dst), nbytes, st))
    return dict(mfma_bf16_tflops=round(flops / t_mfma / 1e12, 1),
                mfma_bf16_tflops_random=round(lib.scope_probe_mfma_flops(blocks, it8) / t_data / 1e12, 1),
                hbm_copy_gbs=round(2 * nbytes / t_copy / 1e9, 1),
                mfma_probe=f"{blocks} workgroups x 4 wavefronts x 4 chains x {mfma_iters} steps",
                copy_probe=f"{copy_mib} MiB copy (read + write)")

"""The C ABI registered as torch operators: ``torch.ops.scope.*``.

Each operator is a ``torch.library.custom_op`` whose implementation calls the
gfx950 library through ``scope_amd.ops`` (device pointers, the current
stream); a ``register_fake`` shape function lets it trace under FakeTensor,
``torch.compile`` (fullgraph) and AOT autograd without a graph break, and the
differentiable ones carry ``register_autograd`` backward formulas.  This is
the pattern of the reference's own native operator (scoped_medium.py:74-154:
``torch.library.custom_op`` + ``register_fake`` + an autograd formula), and
it is how the drop-in runs inside the reference's compiled model
(scoped_medium.py:2332-2338).

Operators (schemas are the decorated signatures below):

* ``scope::doc_starts``, ``scope::pointer_mask_ref`` — build_pointer_blockmask
  (model/attn_bias.py:623-873), reference mode;
* ``scope::block_means`` (or ``scope::block_means_docs``, with the document
  starts folded in), ``scope::pointer_select`` — block-scoring selection;
* ``scope::soft_pointer_bias`` (+ autograd via ``scope::soft_pointer_bwd``),
  ``scope::pair_bias_from_logits``;
* ``scope::transpose_blocks`` — BlockMask.from_kv_blocks' q lists
  (torch:nn/attention/flex_attention.py:399-441);
* ``scope::mask_stats`` — the debug statistics (model/attn_bias.py:510-600,
  839-849);
* ``scope::spectral_table`` — _get_trig_tables (model/attn_bias.py:326-340);
* ``scope::attn_fwd`` (+ autograd via ``scope::attn_bwd``) — the FlexAttention
  calls (scoped_medium.py:422, 459-466, 470-476) with the spectral score_mod;
* ``scope::coeff_head_fwd`` (+ autograd via ``scope::coeff_head_bwd``) — the
  coefficient head of SpectralBias.forward after its MLP (model/attn_bias.py:
  419-506);
* ``scope::coeff_mlp`` (+ autograd: ``scope::coeff_mlp_bwd_wgrad``, the
  row-wise backward and the weight and bias gradients on the fused kernels;
  for row layouts those do not take, ``scope::coeff_mlp_bwd`` and
  ``scope::linear_wgrad``) — the head's shared MLP (model/attn_bias.py:271-276,
  380-386).

Optional outputs that an operator cannot return as None (a gradient that is
not asked for) are returned as empty tensors.
"""
import functools
from typing import Optional, Sequence

import torch
import torch.nn.functional as F
from torch import Tensor

from . import ops

_NS = "scope"
_I32, _F32 = torch.int32, torch.float32
_HEAD_NAMES = ("coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width")


def _none(dev: torch.device) -> Tensor:
    """The empty stand-in of an absent optional output."""
    return torch.empty(0, dtype=_F32, device=dev)


def _bht(x: Tensor):
    """(H, T, D) of a [1,H,T,D] or [H,T,D] tensor."""
    return (x.shape[1], x.shape[2], x.shape[3]) if x.dim() == 4 else (x.shape[0], x.shape[1], x.shape[2])


def seed_to_signed(seed: int) -> int:
    """A 64-bit seed as the signed int64 an operator schema carries."""
    seed &= 0xFFFFFFFFFFFFFFFF
    return seed - (1 << 64) if seed >= (1 << 63) else seed


# ---------------------------------------------------------------------------
# document starts
@torch.library.custom_op(f"{_NS}::doc_starts", mutates_args=())
def doc_starts(docs: Tensor, bs: int, doc_clamp: bool, reset_len: int) -> tuple[Tensor, Tensor, Tensor]:
    return ops.doc_starts(docs, bs, doc_clamp=doc_clamp, reset_len=reset_len)


@doc_starts.register_fake
def _(docs, bs, doc_clamp, reset_len):
    NB = docs.numel() // bs
    return tuple(docs.new_empty(NB, dtype=_I32) for _ in range(3))


# ---------------------------------------------------------------------------
# reference-mode pointer mask
def ref_maxkv(T: int, bs: int, M: int, local_blocks: int, ptr_half_blocks: int, global_blocks_cfg: int) -> int:
    """MAXKV of the reference-mode list (scope_ptr_ref_maxkv):
    local + (p > 0 ? M(2p+1) : M) + min(G, NB) (model/attn_bias.py:250)."""
    NB = T // bs
    local = min(max(1, local_blocks), NB)
    npk = M * (2 * ptr_half_blocks + 1) if ptr_half_blocks > 0 else M
    return local + npk + min(max(global_blocks_cfg, 0), NB)


@torch.library.custom_op(f"{_NS}::pointer_mask_ref", mutates_args=())
def pointer_mask_ref(delta_star: Tensor, budget_logits: Tensor, ds_ptr: Tensor, ds_local: Tensor,
                     gumbel_u: Optional[Tensor], bs: int, local_blocks: int, ptr_half_blocks: int,
                     global_blocks_cfg: int, global_active: int, radius_pi: bool, budget_rem: int, budget_temp: float,
                     mask_active: bool, half_active: int, rep_mean: bool, gumbel_k: int, gumbel_tau: float,
                     eps: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return ops.pointer_mask_ref(delta_star, budget_logits, ds_ptr, ds_local, bs=bs, local_blocks=local_blocks,
                                ptr_half_blocks=ptr_half_blocks, global_blocks_cfg=global_blocks_cfg,
                                global_active=global_active, radius_mode="pi" if radius_pi else "fixed",
                                budget_rem=budget_rem, budget_temp=budget_temp, mask_active=mask_active,
                                half_active=half_active, rep_mode="mean" if rep_mean else "last",
                                gumbel_k=gumbel_k, gumbel_tau=gumbel_tau, gumbel_u=gumbel_u, eps=eps)


@pointer_mask_ref.register_fake
def _(delta_star, budget_logits, ds_ptr, ds_local, gumbel_u, bs, local_blocks, ptr_half_blocks, global_blocks_cfg,
      global_active, radius_pi, budget_rem, budget_temp, mask_active, half_active, rep_mean, gumbel_k, gumbel_tau,
      eps):
    H, T, M = delta_star.shape[-3], delta_star.shape[-2], delta_star.shape[-1]
    QB = T // bs
    L = ref_maxkv(T, bs, M, local_blocks, ptr_half_blocks, global_blocks_cfg)
    e = delta_star.new_empty
    return e((H, QB), dtype=_I32), e((H, QB, L), dtype=_I32), e((H, QB, M), dtype=_I32), e((H, QB, M), dtype=_I32)


# ---------------------------------------------------------------------------
# block-scoring selection
@torch.library.custom_op(f"{_NS}::block_means", mutates_args=())
def block_means(q: Tensor, k: Tensor, bs: int) -> tuple[Tensor, Tensor]:
    return ops.block_means(q, k, bs)


@block_means.register_fake
def _(q, k, bs):
    H, T, D = _bht(q)
    return q.new_empty((H, T // bs, D), dtype=_F32), q.new_empty((H, T // bs, D), dtype=_F32)


@torch.library.custom_op(f"{_NS}::block_means_docs", mutates_args=())
def block_means_docs(q: Tensor, k: Tensor, docs: Tensor, bs: int, doc_clamp: bool,
                     reset_len: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return ops.block_means_docs(q, k, docs, bs, doc_clamp=doc_clamp, reset_len=reset_len)


@block_means_docs.register_fake
def _(q, k, docs, bs, doc_clamp, reset_len):
    H, T, D = _bht(q)
    NB = T // bs
    means = tuple(q.new_empty((H, NB, D), dtype=_F32) for _ in range(2))
    return means + tuple(docs.new_empty(NB, dtype=_I32) for _ in range(3))


@torch.library.custom_op(f"{_NS}::pointer_select", mutates_args=())
def pointer_select(ds_ptr: Tensor, ds_local: Tensor, qbar: Optional[Tensor], kbar: Optional[Tensor],
                   logits_in: Optional[Tensor], prior: Optional[Tensor], gumbel_u: Optional[Tensor], bs: int, NB: int,
                   H: int, window: int, n_global: int, budget: int, temp: float, logit_scale: float, noise_mode: int,
                   seed: int, eps: float, return_logits: bool) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    noise = {0: "none", 1: "uniform", 2: "counter"}[noise_mode]
    r = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=window, n_global=n_global, budget=budget,
                           qbar=qbar, kbar=kbar, logits_in=logits_in, prior=prior, temp=temp,
                           logit_scale=logit_scale, noise=noise, gumbel_u=gumbel_u, seed=seed & 0xFFFFFFFFFFFFFFFF,
                           eps=eps, return_logits=return_logits)
    kv_num, kv_idx, picks = r[0], r[1], r[2].contiguous() if budget == 0 else r[2]
    logits = r[3] if return_logits else _none(ds_ptr.device)
    return kv_num, kv_idx, picks, logits


@pointer_select.register_fake
def _(ds_ptr, ds_local, qbar, kbar, logits_in, prior, gumbel_u, bs, NB, H, window, n_global, budget, temp,
      logit_scale, noise_mode, seed, eps, return_logits):
    L = min(window, NB) + budget + min(n_global, NB)
    e = ds_ptr.new_empty
    return (e((H, NB), dtype=_I32), e((H, NB, L), dtype=_I32), e((H, NB, budget), dtype=_I32),
            e((H, NB, NB) if return_logits else (0,), dtype=_F32))


# ---------------------------------------------------------------------------
# soft pointer weights (no reference counterpart: the reference selects under
# torch.no_grad, model/attn_bias.py:623)
@torch.library.custom_op(f"{_NS}::soft_pointer_bias", mutates_args=())
def soft_pointer_bias(q: Tensor, k: Tensor, kv_num: Tensor, kv_idx: Tensor, picks: Tensor, prior: Optional[Tensor],
                      bs: int, window: int, n_global: int, logit_scale: float,
                      soft_temp: float) -> tuple[Tensor, Tensor, Tensor]:
    """(pair_bias [H,QB,L], q̄, k̄): b = log σ(z/τ_w) on the picks, z from the
    block means of q, k; q̄, k̄ are returned for the backward."""
    qbar, kbar = ops.block_means(q, k, bs)
    pb = ops.pointer_pair_bias(kv_num, kv_idx, picks, bs=bs, window=window, n_global=n_global, soft_temp=soft_temp,
                               qbar=qbar, kbar=kbar, prior=prior, logit_scale=logit_scale, check=False)
    return pb, qbar, kbar


@soft_pointer_bias.register_fake
def _(q, k, kv_num, kv_idx, picks, prior, bs, window, n_global, logit_scale, soft_temp):
    H, T, D = _bht(q)
    return (kv_idx.new_empty(kv_idx.shape, dtype=_F32), q.new_empty((H, T // bs, D), dtype=_F32),
            q.new_empty((H, T // bs, D), dtype=_F32))


@torch.library.custom_op(f"{_NS}::pair_bias_from_logits", mutates_args=())
def pair_bias_from_logits(kv_num: Tensor, kv_idx: Tensor, picks: Tensor, logits: Tensor, bs: int, window: int,
                          n_global: int, soft_temp: float) -> Tensor:
    """The soft weights of the picks from given logits [H,QB,NB] (constants:
    no gradient)."""
    return ops.pointer_pair_bias(kv_num, kv_idx, picks, bs=bs, window=window, n_global=n_global,
                                 soft_temp=soft_temp, logits_in=logits, check=False)


@pair_bias_from_logits.register_fake
def _(kv_num, kv_idx, picks, logits, bs, window, n_global, soft_temp):
    return kv_idx.new_empty(kv_idx.shape, dtype=_F32)


@torch.library.custom_op(f"{_NS}::soft_pointer_bwd", mutates_args=())
def soft_pointer_bwd(qbar: Tensor, kbar: Tensor, kv_num: Tensor, kv_idx: Tensor, q_off: Tensor, q_list: Tensor,
                     pair_bias: Tensor, dpair_bias: Tensor, q_like: Tensor, k_like: Tensor, bs: int,
                     logit_scale: float, soft_temp: float) -> tuple[Tensor, Tensor]:
    """(dq, dk) bf16 with q_like's / k_like's shape and strides: the soft
    weights' gradient through the block means."""
    dq = torch.empty_like(q_like, dtype=torch.bfloat16).zero_()
    dk = torch.empty_like(k_like, dtype=torch.bfloat16).zero_()
    ops.pointer_bwd(qbar, kbar, kv_num, kv_idx, q_off, q_list, pair_bias, dpair_bias.contiguous(), dq, dk, bs=bs,
                    logit_scale=logit_scale, soft_temp=soft_temp, check=False)
    return dq, dk


@soft_pointer_bwd.register_fake
def _(qbar, kbar, kv_num, kv_idx, q_off, q_list, pair_bias, dpair_bias, q_like, k_like, bs, logit_scale, soft_temp):
    return torch.empty_like(q_like, dtype=torch.bfloat16), torch.empty_like(k_like, dtype=torch.bfloat16)


def _soft_setup(ctx, inputs, output):
    q, k, kv_num, kv_idx, picks, prior, bs, window, n_global, logit_scale, soft_temp = inputs
    pb, qbar, kbar = output
    ctx.save_for_backward(q, k, kv_num, kv_idx, pb, qbar, kbar)
    ctx.bs, ctx.logit_scale, ctx.soft_temp = bs, logit_scale, soft_temp
    ctx.mark_non_differentiable(qbar, kbar)
    ctx.set_materialize_grads(False)  # an output's unused gradient stays None (no zero tensors)


def _soft_backward(ctx, dpb, _dq, _dk):
    if dpb is None:
        return (None,) * 11
    q, k, kv_num, kv_idx, pb, qbar, kbar = ctx.saved_tensors
    q_off, q_list = transpose_blocks(kv_num, kv_idx, kv_num.shape[-1])
    dq, dk = soft_pointer_bwd(qbar, kbar, kv_num, kv_idx, q_off, q_list, pb, dpb, q, k, ctx.bs, ctx.logit_scale,
                              ctx.soft_temp)
    return dq, dk, None, None, None, None, None, None, None, None, None


soft_pointer_bias.register_autograd(_soft_backward, setup_context=_soft_setup)


# ---------------------------------------------------------------------------
# transposed lists
@torch.library.custom_op(f"{_NS}::transpose_blocks", mutates_args=())
def transpose_blocks(kv_num: Tensor, kv_idx: Tensor, NB: int) -> tuple[Tensor, Tensor]:
    """(q_off [H, NB+1], q_list [H, QB*MAXKV]); a head's entries past
    q_off[h, NB] are -1."""
    return ops.transpose_blocks(kv_num, kv_idx, NB, tail=-1, check=False)


@transpose_blocks.register_fake
def _(kv_num, kv_idx, NB):
    H, QB = kv_num.shape[-2], kv_num.shape[-1]
    return kv_num.new_empty((H, NB + 1), dtype=_I32), kv_num.new_empty((H, QB * kv_idx.shape[-1]), dtype=_I32)


# ---------------------------------------------------------------------------
# statistics
@torch.library.custom_op(f"{_NS}::mask_stats", mutates_args=())
def mask_stats(delta_star: Optional[Tensor], pi: Optional[Tensor], ds_ptr_fwd: Optional[Tensor],
               ds_local_fwd: Optional[Tensor], kv_num: Optional[Tensor], radius: Optional[Tensor],
               picks: Optional[Tensor], ds_ptr: Optional[Tensor], ds_local: Optional[Tensor], H: int, QB: int,
               bs: int, M: int, rep_mean: bool, has_docs: bool, docstart_enabled: bool, local_blocks_cfg: int,
               eps: float, maxkv_bins: int, radius_bins: int, extra_bins: int,
               bs_local_blocks: int) -> tuple[Tensor, Tensor]:
    return ops.mask_stats(H=H, QB=QB, bs=bs, M=M, delta_star=delta_star, pi=pi,
                          rep_mode="mean" if rep_mean else "last", has_docs=has_docs,
                          docstart_enabled=docstart_enabled, local_blocks_cfg=local_blocks_cfg, eps=eps,
                          ds_ptr_fwd=ds_ptr_fwd, ds_local_fwd=ds_local_fwd, kv_num=kv_num, radius=radius,
                          maxkv_bins=maxkv_bins, radius_bins=radius_bins, extra_bins=extra_bins, picks=picks,
                          ds_ptr=ds_ptr, ds_local=ds_local, bs_local_blocks=bs_local_blocks)


@mask_stats.register_fake
def _(delta_star, pi, ds_ptr_fwd, ds_local_fwd, kv_num, radius, picks, ds_ptr, ds_local, H, QB, bs, M, rep_mean,
      has_docs, docstart_enabled, local_blocks_cfg, eps, maxkv_bins, radius_bins, extra_bins, bs_local_blocks):
    like = next(t for t in (delta_star, kv_num, radius, picks) if t is not None)
    n = ops.ST_FIXED + maxkv_bins + radius_bins + extra_bins
    return like.new_empty(n, dtype=_I32), like.new_empty(len(ops.SV_NAMES), dtype=_F32)


# ---------------------------------------------------------------------------
# spectral tables
def table_bytes(mode: int, T: int, bs: int) -> int:
    """scope_spectral_table_bytes: [NB][16] fp32 (block) or [T][32] bf16 (token)."""
    return (T // bs) * 16 * 4 if mode == 1 else (T * 32 * 2 if mode == 2 else 0)


@torch.library.custom_op(f"{_NS}::spectral_table", mutates_args=())
def spectral_table(omegas: Tensor, T: int, bs: int, mode: int) -> Tensor:
    return ops.spectral_table(omegas, T, bs, {1: "block", 2: "token"}[mode])


@spectral_table.register_fake
def _(omegas, T, bs, mode):
    return omegas.new_empty(table_bytes(mode, T, bs), dtype=torch.uint8)


# ---------------------------------------------------------------------------
# attention forward / backward
_GATES = ("none", "softplus", "relu")
_MODES = ("none", "block", "token")


@torch.library.custom_op(f"{_NS}::attn_fwd", mutates_args=())
def attn_fwd(q: Tensor, k: Tensor, v: Tensor, kv_num: Tensor, kv_idx: Tensor, docs: Tensor, ds_tok_end: Tensor,
             q_off: Tensor, q_list: Tensor, table: Optional[Tensor], coeff_cos: Optional[Tensor],
             coeff_sin: Optional[Tensor], b0: Optional[Tensor], slope: Optional[Tensor], delta_main: Optional[Tensor],
             width: Optional[Tensor], pair_bias: Optional[Tensor], bs: int, scale: float, beta: float, bias_mode: int,
             use_slope: bool, subtract_b0: bool, gate_kind: int, ramp_lambda: float,
             tau: float) -> tuple[Tensor, Tensor]:
    """(out like q, lse [1,H,T] natural log).  q_off / q_list (the transposed
    lists) are not read here; they are inputs so that the backward finds
    them (empty tensors when no gradient will be taken)."""
    return ops.attn_fwd(q, k, v, kv_num, kv_idx, docs, ds_tok_end, bs=bs, scale=scale, beta=beta,
                        bias_mode=_MODES[bias_mode], table=table, coeff_cos=coeff_cos, coeff_sin=coeff_sin, b0=b0,
                        slope=slope, delta_main=delta_main, width=width, use_slope=use_slope,
                        subtract_b0=subtract_b0, gate_kind=_GATES[gate_kind], ramp_lambda=ramp_lambda, tau=tau,
                        pair_bias=pair_bias, check=False)


@attn_fwd.register_fake
def _(q, k, v, kv_num, kv_idx, docs, ds_tok_end, q_off, q_list, table, coeff_cos, coeff_sin, b0, slope, delta_main,
      width, pair_bias, bs, scale, beta, bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda, tau):
    H, T, _ = _bht(q)
    return torch.empty_like(q), q.new_empty((1, H, T), dtype=_F32)


def bwd_outputs_present(bias_mode: int, K: int, need_coeff_grads: bool, use_slope: bool, subtract_b0: bool,
                        gate_kind: int, need_pair_grad: bool) -> dict:
    """Which gradients scope_attn_bwd writes (the rest come back empty)."""
    coeff = bias_mode != 0 and K > 0 and need_coeff_grads
    tok = bias_mode == 2 and need_coeff_grads
    gate = tok and gate_kind != 0
    return dict(dcoeff_cos=coeff, dcoeff_sin=coeff, db0=tok and subtract_b0, dslope=tok and use_slope,
                ddelta_main=gate, dwidth=gate, dpair_bias=need_pair_grad)


_BWD_NAMES = ("dcoeff_cos", "dcoeff_sin", "db0", "dslope", "ddelta_main", "dwidth", "dpair_bias")


@torch.library.custom_op(f"{_NS}::attn_bwd", mutates_args=())
def attn_bwd(q: Tensor, k: Tensor, v: Tensor, out: Tensor, dout: Tensor, lse: Tensor, kv_num: Tensor,
             kv_idx: Tensor, q_off: Tensor, q_list: Tensor, docs: Tensor, ds_tok_end: Tensor, table: Optional[Tensor],
             coeff_cos: Optional[Tensor], coeff_sin: Optional[Tensor], b0: Optional[Tensor], slope: Optional[Tensor],
             delta_main: Optional[Tensor], width: Optional[Tensor], pair_bias: Optional[Tensor], bs: int,
             scale: float, beta: float, bias_mode: int, use_slope: bool, subtract_b0: bool, gate_kind: int,
             ramp_lambda: float, tau: float, need_coeff_grads: bool,
             need_pair_grad: bool) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                            Tensor]:
    """(dq, dk, dv, dcoeff_cos, dcoeff_sin, db0, dslope, ddelta_main, dwidth,
    dpair_bias); the gradients not computed come back as empty tensors."""
    if dout.stride() != q.stride():
        dout = torch.empty_like(q).copy_(dout)
    if out.stride() != q.stride():
        out = torch.empty_like(q).copy_(out)
    g = ops.attn_bwd(q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list, docs, ds_tok_end, bs=bs, scale=scale,
                     beta=beta, bias_mode=_MODES[bias_mode], table=table, coeff_cos=coeff_cos, coeff_sin=coeff_sin,
                     b0=b0, slope=slope, delta_main=delta_main, width=width, use_slope=use_slope,
                     subtract_b0=subtract_b0, gate_kind=_GATES[gate_kind], ramp_lambda=ramp_lambda, tau=tau,
                     need_coeff_grads=need_coeff_grads, pair_bias=pair_bias, need_pair_grad=need_pair_grad, check=False)
    rest = tuple(_none(q.device) if g[n] is None else g[n] for n in _BWD_NAMES)
    return (g["dq"], g["dk"], g["dv"]) + rest


@attn_bwd.register_fake
def _(q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list, docs, ds_tok_end, table, coeff_cos, coeff_sin, b0,
      slope, delta_main, width, pair_bias, bs, scale, beta, bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda,
      tau, need_coeff_grads, need_pair_grad):
    H, T, _ = _bht(q)
    K = coeff_cos.shape[-1] if coeff_cos is not None else 0
    pres = bwd_outputs_present(bias_mode, K, need_coeff_grads, use_slope, subtract_b0, gate_kind, need_pair_grad)
    e = q.new_empty
    shapes = dict(dcoeff_cos=(1, H, T, K), dcoeff_sin=(1, H, T, K), db0=(1, H, T), dslope=(1, H, T),
                  ddelta_main=(1, H, T), dwidth=(1, H, T), dpair_bias=tuple(kv_idx.shape[-3:]))
    rest = tuple(e(shapes[n] if pres[n] else (0,), dtype=_F32) for n in _BWD_NAMES)
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)) + rest


def _attn_setup(ctx, inputs, output):
    (q, k, v, kv_num, kv_idx, docs, ds_tok_end, q_off, q_list, table, cc, cs, b0, slope, dm, wd, pb, bs, scale, beta,
     bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda, tau) = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, kv_num, kv_idx, docs, ds_tok_end, q_off, q_list, table, cc, cs, b0,
                          slope, dm, wd, pb)
    ctx.cfg = (bs, scale, beta, bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda, tau)
    ctx.mark_non_differentiable(lse)
    ctx.set_materialize_grads(False)  # lse's gradient stays None (no zero tensor)


def _attn_backward(ctx, dout, _dlse):
    if dout is None:
        return (None,) * 26
    (q, k, v, out, lse, kv_num, kv_idx, docs, ds_tok_end, q_off, q_list, table, cc, cs, b0, slope, dm, wd,
     pb) = ctx.saved_tensors
    bs, scale, beta, bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda, tau = ctx.cfg
    if q_off.numel() == 0:  # the forward ran without the transposed lists
        q_off, q_list = transpose_blocks(kv_num, kv_idx, q.shape[-2] // bs)
    need = ctx.needs_input_grad
    need_c = bias_mode != 0 and any(need[10:16])
    need_p = pb is not None and need[16]
    g = attn_bwd(q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list, docs, ds_tok_end, table, cc, cs, b0, slope,
                 dm, wd, pb, bs, scale, beta, bias_mode, use_slope, subtract_b0, gate_kind, ramp_lambda, tau, need_c,
                 need_p)
    dq, dk, dv = g[:3]
    rest = tuple(None if (x is None or gr.numel() == 0) else gr.reshape(x.shape)
                 for x, gr in zip((cc, cs, b0, slope, dm, wd, pb), g[3:]))
    return (dq, dk, dv, None, None, None, None, None, None, None) + rest + (None,) * 9


attn_fwd.register_autograd(_attn_backward, setup_context=_attn_setup)


# ---------------------------------------------------------------------------
# coefficient head after the MLP
_IPRM = ("M", "K", "L", "use_slope", "subtract_b0", "training")
_FPRM = ("delta_cap", "logw_min", "logw_max", "c_scale", "width_min", "width_max", "eps", "lambda_omega",
         "lambda_entropy", "lambda_zero_mean", "lambda_delta_edge", "entropy_floor", "delta_edge_eps")


def pack_head_params(prm: dict) -> tuple[list[int], list[float]]:
    return [int(prm[n]) for n in _IPRM], [float(prm[n]) for n in _FPRM]


def _unpack(iprm: Sequence[int], fprm: Sequence[float]) -> dict:
    d = {n: int(x) for n, x in zip(_IPRM, iprm)}
    d.update({n: float(x) for n, x in zip(_FPRM, fprm)})
    for n in ("use_slope", "subtract_b0", "training"):
        d[n] = bool(d[n])
    return d


@torch.library.custom_op(f"{_NS}::coeff_head_fwd", mutates_args=())
def coeff_head_fwd(y: Tensor, omegas: Tensor, log_omegas: Tensor, cos_mean: Optional[Tensor],
                   sin_mean: Optional[Tensor], iprm: list[int],
                   fprm: list[float]) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor,
                                               Tensor]:
    """The nine per-row outputs of the head (_HEAD_NAMES order) and reg [6]."""
    o = ops.coeff_head_fwd(y, _unpack(iprm, fprm), omegas, log_omegas, cos_mean, sin_mean)
    return tuple(o[n] for n in _HEAD_NAMES) + (o["reg"],)


@coeff_head_fwd.register_fake
def _(y, omegas, log_omegas, cos_mean, sin_mean, iprm, fprm):
    M, K = int(iprm[0]), int(iprm[1])
    lead = tuple(y.shape[:-1])
    e = y.new_empty
    shp = dict(coeff_cos=lead + (K,), coeff_sin=lead + (K,), slope=lead, b0=lead, delta_star=lead + (M,),
               pi=lead + (M,), budget_logits=lead + (M,), delta_main=lead, width=lead)
    return tuple(e(shp[n], dtype=_F32) for n in _HEAD_NAMES) + (e(6, dtype=_F32),)


@torch.library.custom_op(f"{_NS}::coeff_head_bwd", mutates_args=())
def coeff_head_bwd(y: Tensor, omegas: Tensor, log_omegas: Tensor, cos_mean: Optional[Tensor],
                   sin_mean: Optional[Tensor], grads: list[Optional[Tensor]], g_reg: Optional[Tensor], reg: Tensor,
                   iprm: list[int], fprm: list[float]) -> Tensor:
    """dy (y's dtype and shape) from the upstream gradients of the nine
    outputs (None = zero) and of reg[0]."""
    g = {n: x for n, x in zip(_HEAD_NAMES, grads) if x is not None}
    return ops.coeff_head_bwd(y, _unpack(iprm, fprm), omegas, log_omegas, cos_mean, sin_mean, g, g_reg, reg)


@coeff_head_bwd.register_fake
def _(y, omegas, log_omegas, cos_mean, sin_mean, grads, g_reg, reg, iprm, fprm):
    return torch.empty_like(y, memory_format=torch.contiguous_format)


def _head_setup(ctx, inputs, output):
    y, omegas, log_omegas, cos_mean, sin_mean, iprm, fprm = inputs
    ctx.save_for_backward(y, omegas, log_omegas, cos_mean, sin_mean, output[-1])
    ctx.iprm, ctx.fprm = list(iprm), list(fprm)
    ctx.set_materialize_grads(False)  # the unused outputs' gradients stay None (the kernel skips them)


def _head_backward(ctx, *g):
    y, omegas, log_omegas, cos_mean, sin_mean, reg = ctx.saved_tensors
    g_reg = g[len(_HEAD_NAMES)]
    dy = coeff_head_bwd(y, omegas, log_omegas, cos_mean, sin_mean, list(g[:len(_HEAD_NAMES)]),
                        None if g_reg is None else g_reg[:1], reg, ctx.iprm, ctx.fprm)
    return dy, None, None, None, None, None, None


coeff_head_fwd.register_autograd(_head_backward, setup_context=_head_setup)


# ---------------------------------------------------------------------------
# The head's MLP (model/attn_bias.py:271-276, applied at :380-398)
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_NS}::linear_wgrad", mutates_args=())
def linear_wgrad(a: Tensor, b: Tensor, round_bf16: bool) -> tuple[Tensor, Tensor]:
    """dw [M, N] = Σ_r a[r]^T b[r], db [M] = Σ_r a[r] over the bf16 rows of
    a [..., M] and b [..., N] (fp32, rounded to bf16 with ``round_bf16``)."""
    return ops.linear_wgrad(a, b, round_bf16=round_bf16)


@linear_wgrad.register_fake
def _(a, b, round_bf16):
    return a.new_empty((a.shape[-1], b.shape[-1]), dtype=_F32), a.new_empty(a.shape[-1], dtype=_F32)


@torch.library.custom_op(f"{_NS}::coeff_mlp_bwd", mutates_args=())
def coeff_mlp_bwd(q: Tensor, gy: Tensor, w1: Tensor, b1: Tensor, w2: Tensor,
                  b2: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """The row-wise backward of the fused MLP: (dq, dz1, x1, gy padded to 64
    columns), bf16, with z1 and x1 recomputed from q."""
    return ops.coeff_mlp_bwd(q, gy, w1, b1, w2, b2)


@coeff_mlp_bwd.register_fake
def _(q, gy, w1, b1, w2, b2):
    lead = tuple(q.shape[:-1])
    return (q.new_empty(lead + (q.shape[-1],)), q.new_empty(lead + (w1.shape[0],)), q.new_empty(lead + (w1.shape[0],)),
            q.new_empty(lead + (64,)))


@torch.library.custom_op(f"{_NS}::coeff_mlp_bwd_wgrad", mutates_args=())
def coeff_mlp_bwd_wgrad(q: Tensor, gy: Tensor, w1: Tensor, b1: Tensor, w2: Tensor,
                        b2: Tensor) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """The whole MLP backward on the fused kernels: (dq bf16, dw1, db1, dw2,
    db2 fp32), the weight and bias gradients from q and the padded output
    gradient with z1, x1 and dz1 recomputed per tile (never stored)."""
    dq, _, _, gyp = ops.coeff_mlp_bwd(q, gy, w1, b1, w2, b2, intermediates=False)
    return (dq,) + ops.coeff_mlp_wgrad(q, gyp, w1, b1, w2)


@coeff_mlp_bwd_wgrad.register_fake
def _(q, gy, w1, b1, w2, b2):
    O = w2.shape[0]
    f = functools.partial(q.new_empty, dtype=_F32)
    return (q.new_empty(tuple(q.shape[:-1]) + (q.shape[-1],)), f((w1.shape[0], w1.shape[1])), f((w1.shape[0],)),
            f((O, w2.shape[1])), f((O,)))


@torch.library.custom_op(f"{_NS}::coeff_mlp", mutates_args=())
def coeff_mlp(q: Tensor, w1: Tensor, b1: Tensor, w2: Tensor, b2: Tensor) -> Tensor:
    """The head's shared MLP on q [..., D]: y = Linear(w2, b2)(SiLU(Linear(w1,
    b1)(q))) with the weights cast to q's dtype (model/attn_bias.py:380-386).
    bf16 rows of 128 with fp32 weights (the reference's default) run one fused
    kernel; other dtypes and shapes the reference's torch steps."""
    ops._gpu("coeff_mlp", q, w1, b1, w2, b2)
    if ops.coeff_mlp_fused(q, w1, w2):
        return ops.coeff_mlp_fwd(q, w1, b1, w2, b2)
    dt = q.dtype
    return F.linear(F.silu(F.linear(q, w1.to(dt), b1.to(dt))), w2.to(dt), b2.to(dt))


@coeff_mlp.register_fake
def _(q, w1, b1, w2, b2):
    return q.new_empty(tuple(q.shape[:-1]) + (w2.shape[0],))


def _mlp_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)
    ctx.set_materialize_grads(False)


def _wgrad(a: Tensor, b: Tensor) -> tuple[Tensor, Tensor]:
    """Weight and bias gradient of a linear layer (output gradient a, input b):
    the split-row kernel where it takes the operands (bf16, the output columns
    padded to 64, 128 or 256, a supported (M, N), rows a multiple of 64),
    else the product autograd of F.linear computes (in the operands' dtype,
    bf16 results rounded, as autograd rounds them)."""
    M = a.shape[-1]
    Mp = 64 if M <= 64 else (128 if M <= 128 else 256)
    if a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16 and M <= 256:
        ap = F.pad(a.reshape(-1, M), (0, Mp - M)) if Mp != M else a  # pad the output columns
        if ops.linear_wgrad_takes(ap, b):
            dw, db = linear_wgrad(ap, b, True)
            return dw[:M], db[:M]
    a2, b2 = a.reshape(-1, M), b.reshape(-1, b.shape[-1])
    return a2.t().matmul(b2).float(), a2.sum(0).float()


def _mlp_backward(ctx, gy):
    """Autograd of the two F.linear and the SiLU (the reference's backward):
    dx1 = gy·W2, dz1 = SiLU'(z1)·dx1, dq = dz1·W1 with z1 and x1 recomputed.
    The forward's fused case with segments of a multiple of 128 rows runs
    two fused kernels (dq; the weight and bias gradients, recomputing z1, x1
    and dz1 per tile); other fused cases write x1 and dz1 for the split-row
    weight-gradient kernel where it takes them (rows and segments a multiple
    of 64), else for the product autograd computes; the rest take the torch
    steps.  The weights' gradients are those of their bf16 copies (rounded to
    bf16), in the weights' dtype."""
    if gy is None:
        return None, None, None, None, None
    q, w1, b1, w2, b2 = ctx.saved_tensors
    dt = q.dtype
    O = w2.shape[0]
    if ops.coeff_mlp_fused(q, w1, w2) and ops.coeff_mlp_wgrad_fused(q):
        dq, dw1, db1, dw2, db2 = coeff_mlp_bwd_wgrad(q, gy, w1, b1, w2, b2)
        if not ctx.needs_input_grad[0]:
            dq = None
        return dq, dw1.to(w1.dtype), db1.to(b1.dtype), dw2.to(w2.dtype), db2.to(b2.dtype)
    if ops.coeff_mlp_fused(q, w1, w2):
        dq, dz1, x1, gyp = coeff_mlp_bwd(q, gy, w1, b1, w2, b2)
        dw2, db2 = _wgrad(gyp, x1)  # gyp: gy padded to 64 columns with zeros
        dw2, db2 = dw2[:O], db2[:O]
        if not ctx.needs_input_grad[0]:
            dq = None
    else:
        gy = gy.to(dt)
        z1 = F.linear(q, w1.to(dt), b1.to(dt))
        x1 = F.silu(z1)
        dz1 = torch.ops.aten.silu_backward(gy.matmul(w2.to(dt)), z1)
        dw2, db2 = _wgrad(gy, x1)
        dq = dz1.matmul(w1.to(dt)) if ctx.needs_input_grad[0] else None
    dw1, db1 = _wgrad(dz1, q)
    return dq, dw1.to(w1.dtype), db1.to(b1.dtype), dw2.to(w2.dtype), db2.to(b2.dtype)


coeff_mlp.register_autograd(_mlp_backward, setup_context=_mlp_setup)

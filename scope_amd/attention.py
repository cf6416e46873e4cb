"""``scope_attention``: the drop-in for the FlexAttention calls of
``CausalSelfAttention.forward`` (scoped_medium.py:422, 459-466, 470-476).

The reference passes a Python ``score_mod`` closure over the spectral
coefficients (scoped_medium.py:425-457); here the same terms are passed as
tensors in a ``SpectralTerms`` record and evaluated inside the HIP kernels.
Gradients flow to q, k, v and to every coefficient tensor that requires grad,
like FlexAttention's captured-buffer gradients.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops
from .blockmask import ScopeBlockMask


@dataclass
class SpectralTerms:
    """Inputs of the spectral bias (per query row).

    ``offset="token"`` is the reference's score_mod (Δ = max(i-j, 0)):
        Σ_k A_k cos(ω_k Δ) + B_k sin(ω_k Δ) - b0·[subtract_b0] + slope·Δ·[use_slope]
        - ramp_lambda·gate((|Δ - delta_main| - width)/tau)
    ``offset="block"`` uses the block offset r = qb - kb instead and only the
    band term.  The score becomes ``scale·q·k + beta·bias``.
    """
    coeff_cos: torch.Tensor          # [1,H,T,K]
    coeff_sin: torch.Tensor          # [1,H,T,K]
    omegas: torch.Tensor             # [K]
    offset: str = "token"
    beta: float = 0.5
    b0: torch.Tensor | None = None   # [1,H,T]
    slope: torch.Tensor | None = None
    delta_main: torch.Tensor | None = None
    width: torch.Tensor | None = None
    use_slope: bool = False
    subtract_b0: bool = False
    gate_kind: str = "none"
    ramp_lambda: float = 0.0
    tau: float = 64.0


_TABLES: dict = {}


def spectral_table(omegas: torch.Tensor, T: int, bs: int, mode: str) -> torch.Tensor:
    """Cached cos/sin table (the analogue of SpectralBias._get_trig_tables)."""
    key = (omegas.data_ptr(), omegas._version, omegas.device, T, bs, mode)
    tab = _TABLES.get(key)
    if tab is None:
        if len(_TABLES) > 16:
            _TABLES.clear()
        tab = ops.spectral_table(omegas, T, bs, mode)
        _TABLES[key] = tab
    return tab


def _kwargs(sp: SpectralTerms | None, bm: ScopeBlockMask):
    if sp is None:
        return dict(bias_mode="none")
    T = bm.seq_len
    return dict(bias_mode=sp.offset, beta=sp.beta, table=spectral_table(sp.omegas, T, bm.BLOCK_SIZE, sp.offset),
                use_slope=sp.use_slope and sp.offset == "token",
                subtract_b0=sp.subtract_b0 and sp.offset == "token",
                gate_kind=sp.gate_kind if sp.offset == "token" else "none", ramp_lambda=sp.ramp_lambda, tau=sp.tau)


class _ScopeAttnFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, cc, cs, b0, slope, dm, wd, pb, bm: ScopeBlockMask, sp: SpectralTerms | None,
                scale: float):
        kw = _kwargs(sp, bm)
        out, lse = ops.attn_fwd(q, k, v, bm.kv_num_blocks[0], bm.kv_indices[0], bm.docs, bm.ds_tok_end,
                                bs=bm.BLOCK_SIZE, scale=scale, coeff_cos=cc, coeff_sin=cs, b0=b0, slope=slope,
                                delta_main=dm, width=wd, pair_bias=pb, **kw)
        ctx.save_for_backward(q, k, v, out, lse, cc, cs, b0, slope, dm, wd, pb)
        ctx.bm, ctx.sp, ctx.scale = bm, sp, scale
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, out, lse, cc, cs, b0, slope, dm, wd, pb = ctx.saved_tensors
        bm, sp = ctx.bm, ctx.sp
        kw = _kwargs(sp, bm)
        q_off, q_list = bm.q_lists()
        dout = dout if dout.stride() == q.stride() else _match(dout, q)
        out_m = out if out.stride() == q.stride() else _match(out, q)
        need_c = sp is not None and any(ctx.needs_input_grad[3:9])
        need_p = pb is not None and ctx.needs_input_grad[9]
        g = ops.attn_bwd(q, k, v, out_m, dout, lse, bm.kv_num_blocks[0], bm.kv_indices[0], q_off, q_list, bm.docs,
                         bm.ds_tok_end, bs=bm.BLOCK_SIZE, scale=ctx.scale, coeff_cos=cc, coeff_sin=cs, b0=b0,
                         slope=slope, delta_main=dm, width=wd, need_coeff_grads=need_c, pair_bias=pb,
                         need_pair_grad=need_p, **kw)
        dpb = g["dpair_bias"].reshape(pb.shape) if need_p else None
        return (g["dq"], g["dk"], g["dv"], g["dcoeff_cos"], g["dcoeff_sin"], g["db0"], g["dslope"],
                g["ddelta_main"], g["dwidth"], dpb, None, None, None)


class _SoftPointerFn(torch.autograd.Function):
    """Soft weights of the block-scoring picks as a per-list-entry score
    bias: b = log σ(z/τ_w), z = logit_scale·q̄·k̄ + prior (noise-free), on the
    pick entries (scope_pointer_pair_bias).  Backward: the block-mean chain
    into q and k (scope_pointer_bwd).  No reference counterpart: the
    reference's selection runs under torch.no_grad (model/attn_bias.py:623)."""

    @staticmethod
    def forward(ctx, q, k, bm: ScopeBlockMask, window: int, n_global: int, logit_scale: float, soft_temp: float,
                prior):
        bs = bm.BLOCK_SIZE
        qbar, kbar = ops.block_means(q, k, bs)
        picks = bm.extras["picks"]
        pb = ops.pointer_pair_bias(bm.kv_num_blocks[0], bm.kv_indices[0], picks, bs=bs, window=window,
                                   n_global=n_global, soft_temp=soft_temp, qbar=qbar, kbar=kbar, prior=prior,
                                   logit_scale=logit_scale)
        ctx.save_for_backward(qbar, kbar, pb)
        ctx.bm, ctx.logit_scale, ctx.soft_temp = bm, logit_scale, soft_temp
        ctx.q_like, ctx.k_like = (q.shape, q.stride()), (k.shape, k.stride())
        return pb

    @staticmethod
    def backward(ctx, dpb):
        qbar, kbar, pb = ctx.saved_tensors
        bm = ctx.bm
        q_off, q_list = bm.q_lists()
        dq = torch.empty_strided(*ctx.q_like, dtype=torch.bfloat16, device=pb.device).zero_()
        dk = torch.empty_strided(*ctx.k_like, dtype=torch.bfloat16, device=pb.device).zero_()
        ops.pointer_bwd(qbar, kbar, bm.kv_num_blocks[0], bm.kv_indices[0], q_off, q_list, pb, dpb.contiguous(), dq,
                        dk, bs=bm.BLOCK_SIZE, logit_scale=ctx.logit_scale, soft_temp=ctx.soft_temp)
        return dq, dk, None, None, None, None, None, None


def soft_pointer_bias(q: torch.Tensor, k: torch.Tensor, block_mask: ScopeBlockMask, *, window: int, n_global: int,
                      logit_scale: float, soft_temp: float, prior: torch.Tensor | None = None) -> torch.Tensor:
    """Differentiable soft weights [H,QB,MAXKV] of a block-scoring mask's
    picks (q, k the tensors the mask was selected from)."""
    return _SoftPointerFn.apply(q, k, block_mask, int(window), int(n_global), float(logit_scale),
                                float(soft_temp), prior)


def _match(x: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    y = torch.empty_like(like)
    y.copy_(x)
    return y


def scope_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block_mask: ScopeBlockMask,
                    scale: float, spectral: SpectralTerms | None = None, return_lse: bool = False):
    """Block-sparse attention over ``block_mask`` with the document-causal
    mask and the optional spectral bias.  q, k, v: [1,H,T,D] bf16 (any
    head/token strides, unit last stride).  Returns out [1,H,T,D] (and
    lse [1,H,T], natural log, if ``return_lse``).  A mask built with soft
    pointer weights carries them in ``extras["pair_bias"]``; they are added
    to the listed tiles' scores and receive gradients."""
    sp = spectral
    cc = cs = b0 = sl = dm = wd = None
    if sp is not None:
        cc, cs = sp.coeff_cos, sp.coeff_sin
        if sp.offset == "token":
            b0 = sp.b0 if sp.subtract_b0 else None
            sl = sp.slope if sp.use_slope else None
            if sp.gate_kind != "none":
                dm, wd = sp.delta_main, sp.width
    pb = block_mask.extras.get("pair_bias")
    out, lse = _ScopeAttnFn.apply(q, k, v, cc, cs, b0, sl, dm, wd, pb, block_mask, sp, float(scale))
    return (out, lse) if return_lse else out


def teacher_block_mass(q: torch.Tensor, k: torch.Tensor, docs: torch.Tensor, *, scale: float,
                       spectral: SpectralTerms | None = None, block_size: int = 128) -> torch.Tensor:
    """The teacher's block mass (scoped_medium.py:1799-1819): for every head,
    q-block qb and key block kb, the softmax probability mass of the dense
    document-causal attention summed over the q-block's rows and the key
    block's keys -> [H, NB, NB] fp32.  The reference builds the same scores
    from bf16 q / k and augmented q_pos / k_pos features (the band term and
    slope of ``spectral``, offset="token"); here the bias is evaluated as in
    ``scope_attention``.  q, k: [1,H,T,D] bf16 (the teacher's selected heads)."""
    from .blockmask import ScopeBlockMask  # noqa: F401  (same mask conventions)

    T = q.shape[-2]
    bs = block_size
    NB = T // bs
    docs = docs.reshape(-1).to(torch.int32).contiguous()
    _, ds_local, ds_tok_end = ops.doc_starts(docs, bs)
    # dense document-causal list: key blocks from the q-block's first document start to the diagonal
    qb = torch.arange(NB, device=q.device, dtype=torch.int32)
    first = ds_local.to(torch.int32)
    kv_num = (qb - first + 1)[None].expand(q.shape[1], -1).contiguous()
    kv_idx = torch.minimum(first[:, None] + torch.arange(NB, device=q.device, dtype=torch.int32)[None],
                           qb[:, None])[None].expand(q.shape[1], -1, -1).contiguous()
    kw = dict(bias_mode="none")
    if spectral is not None:
        if spectral.offset != "token":
            raise ValueError("teacher_block_mass: the teacher's bias uses token offsets")
        kw = dict(bias_mode="token", beta=spectral.beta, table=spectral_table(spectral.omegas, T, bs, "token"),
                  coeff_cos=spectral.coeff_cos, coeff_sin=spectral.coeff_sin,
                  slope=spectral.slope if spectral.use_slope else None, use_slope=spectral.use_slope)
    mass, _ = ops.attn_block_mass(q, k, kv_num, kv_idx, docs, ds_tok_end, bs=bs, scale=scale, **kw)
    return mass

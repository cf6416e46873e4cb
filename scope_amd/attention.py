"""``scope_attention``: the drop-in for the FlexAttention calls of
``CausalSelfAttention.forward`` (scoped_medium.py:422, 459-466, 470-476).

The reference passes a Python ``score_mod`` closure over the spectral
coefficients (scoped_medium.py:425-457); here the same terms are passed as
tensors in a ``SpectralTerms`` record and evaluated inside the HIP kernels.
Gradients flow to q, k, v and to every coefficient tensor that requires grad,
like FlexAttention's captured-buffer gradients.
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch
from torch._subclasses.fake_tensor import FakeTensor

from . import library, ops
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
_MODE = {"none": 0, "block": 1, "token": 2}
_GATE = {"none": 0, "softplus": 1, "relu": 2}


def spectral_table(omegas: torch.Tensor, T: int, bs: int, mode: str) -> torch.Tensor:
    """cos/sin table (the analogue of SpectralBias._get_trig_tables), cached
    per (ω, T, bs, mode) in eager mode and rebuilt in compiled graphs."""
    if torch.compiler.is_compiling() or isinstance(omegas, FakeTensor):  # traced: no cache keyed on pointers
        return library.spectral_table(omegas, T, bs, _MODE[mode])
    # the entry also holds a weak reference to the ω tensor it was built
    # from: a new tensor that the allocator placed at a freed one's address
    # (a per-call .to(device) copy, another module's ω) is not that tensor
    key = (omegas.data_ptr(), omegas._version, omegas.device, T, bs, mode)
    hit = _TABLES.get(key)
    if hit is not None and hit[0]() is omegas:
        return hit[1]
    if len(_TABLES) > 16:
        _TABLES.clear()
    tab = library.spectral_table(omegas, T, bs, _MODE[mode])
    _TABLES[key] = (weakref.ref(omegas), tab)
    return tab


def soft_pointer_bias(q: torch.Tensor, k: torch.Tensor, block_mask: ScopeBlockMask, *, window: int, n_global: int,
                      logit_scale: float, soft_temp: float, prior: torch.Tensor | None = None) -> torch.Tensor:
    """Differentiable soft weights [H,QB,MAXKV] of a block-scoring mask's
    picks (q, k the tensors the mask was selected from): b = log σ(z/τ_w),
    z = logit_scale·q̄·k̄ + prior (noise-free), on the pick entries; the
    backward carries the block-mean chain into q and k.  No reference
    counterpart: the reference's selection runs under torch.no_grad
    (model/attn_bias.py:623)."""
    pb, _, _ = library.soft_pointer_bias(q, k, block_mask.kv_num_blocks[0], block_mask.kv_indices[0],
                                         block_mask.extras["picks"], prior, block_mask.BLOCK_SIZE, int(window),
                                         int(n_global), float(logit_scale), float(soft_temp))
    return pb


def scope_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block_mask: ScopeBlockMask,
                    scale: float, spectral: SpectralTerms | None = None, return_lse: bool = False):
    """Block-sparse attention over ``block_mask`` with the document-causal
    mask and the optional spectral bias.  q, k, v: [1,H,T,D] bf16 (any
    head/token strides, unit last stride).  Returns out [1,H,T,D] (and
    lse [1,H,T], natural log, if ``return_lse``).  A mask built with soft
    pointer weights carries them in ``extras["pair_bias"]``; they are added
    to the listed tiles' scores and receive gradients.  Runs the
    ``scope::attn_fwd`` operator (its autograd formula is ``scope::attn_bwd``),
    so it traces under torch.compile without a graph break."""
    bm, sp = block_mask, spectral
    bs = bm.BLOCK_SIZE
    cc = cs = b0 = sl = dm = wd = table = None
    mode, gate, beta, use_slope, sub_b0, lam, tau = 0, 0, 0.5, False, False, 0.0, 64.0
    if sp is not None:
        cc, cs = sp.coeff_cos, sp.coeff_sin
        mode, beta, lam, tau = _MODE[sp.offset], float(sp.beta), float(sp.ramp_lambda), float(sp.tau)
        table = spectral_table(sp.omegas, bm.seq_len, bs, sp.offset)
        if sp.offset == "token":
            use_slope, sub_b0, gate = bool(sp.use_slope), bool(sp.subtract_b0), _GATE[sp.gate_kind]
            b0 = sp.b0 if sub_b0 else None
            sl = sp.slope if use_slope else None
            if gate:
                dm, wd = sp.delta_main, sp.width
    pb = bm.extras.get("pair_bias")
    kv_num, kv_idx = bm.kv_num_blocks[0], bm.kv_indices[0]
    grad = torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                           for t in (q, k, v, cc, cs, b0, sl, dm, wd, pb))
    if grad:
        q_off, q_list = bm.q_lists()
    else:  # no backward: the transposed lists are not needed
        q_off = q_list = kv_num.new_empty(0)
    out, lse = library.attn_fwd(q, k, v, kv_num, kv_idx, bm.docs, bm.ds_tok_end, q_off, q_list, table, cc, cs, b0,
                                sl, dm, wd, pb, bs, float(scale), beta, mode, use_slope, sub_b0, gate, lam, tau)
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
    mass, _ = ops.attn_block_mass(q, k, kv_num, kv_idx, docs, ds_tok_end, bs=bs, scale=scale, **kw, check=False)
    return mass

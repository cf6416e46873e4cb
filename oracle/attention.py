"""CPU oracle: block-sparse attention with the SCOPE spectral bias.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  torch on the CPU.

Semantics (FlexAttention with a ``score_mod`` and a ``BlockMask``):

    s_ij  = scale · q_i·k_j + β · bias_ij          (scoped_medium.py:425-457)
    allowed_ij = kb(j) ∈ list(h, qb(i))  ∧  j ≤ i  ∧  docs[i] == docs[j]
                 (model/attn_bias.py:674-679; the block list is applied
                 explicitly, because eager FlexAttention ignores it)
    out_i = Σ_j softmax_j(s_i·, allowed) v_j,   lse_i = logsumexp_j s_ij
    rows with no allowed key give out = 0 and lse = -inf
    (torch:_higher_order_ops/flex_attention.py:250-258)

Bias modes:

* token (the reference's ``score_mod``, scoped_medium.py:425-457), Δ = max(i-j, 0):
      Σ_k A_k(i) cos(ω_k Δ) + B_k(i) sin(ω_k Δ)  - b0(i)·[subtract_b0]
      + slope(i)·Δ·[use_slope] - λ·gate((|Δ - Δmain(i)| - width(i))/τ)
  with gate = softplus | relu | none.  The reference evaluates cos/sin from
  bf16 tables (model/attn_bias.py:336-337); the oracle uses exact fp64.
* block (the block-offset bias of the benchmark workloads), r = qb(i) - kb(j):
      Σ_k A_k(i) cos(ω_k r) + B_k(i) sin(ω_k r)

Parity pins (tests/test_oracle_attention.py): torch's own eager
``flex_attention`` (library code) with a restated ``mask_mod`` that includes
block membership and a restated ``score_mod``; the qk_aug identity of
scoped_medium.py:380-423 (equal up to the gate and a row constant);
``torch.autograd.gradcheck`` of the fp64 function; the block-sparse variant
against the dense one.
"""
from __future__ import annotations

import math

import torch

GATES = {"none": 0, "softplus": 1, "relu": 2}


def allowed_mask(kv_num, kv_idx, docs, bs: int, T: int) -> torch.Tensor:
    """Dense [H,T,T] bool mask: block membership ∧ causal ∧ same document."""
    kv_num = torch.as_tensor(kv_num)
    kv_idx = torch.as_tensor(kv_idx)
    docs = torch.as_tensor(docs).long()
    H, QB = kv_num.shape
    NB = T // bs
    blk = torch.zeros((H, QB, NB), dtype=torch.bool)
    for h in range(H):
        for qb in range(QB):
            n = int(kv_num[h, qb])
            blk[h, qb, kv_idx[h, qb, :n].long()] = True
    dense = blk.repeat_interleave(bs, dim=1).repeat_interleave(bs, dim=2)
    i = torch.arange(T)
    causal = i[:, None] >= i[None, :]
    same = docs[:, None] == docs[None, :]
    return dense & (causal & same)[None]


def bias_block(coeff_cos, coeff_sin, omegas, bs: int, rows=None, cols=None) -> torch.Tensor:
    """[H,T,K] coefficients -> [H,len(rows),len(cols)] block-offset bias."""
    H, T, K = coeff_cos.shape
    rows = torch.arange(T) if rows is None else rows
    cols = torch.arange(T) if cols is None else cols
    r = (rows[:, None] // bs - cols[None, :] // bs).to(coeff_cos.dtype)  # [R,C]
    w = omegas.to(coeff_cos.dtype)
    ph = w[:, None, None] * r[None]  # [K,R,C]
    A = coeff_cos[:, rows, :]
    B = coeff_sin[:, rows, :]
    return torch.einsum("hrk,krc->hrc", A, torch.cos(ph)) + torch.einsum("hrk,krc->hrc", B, torch.sin(ph))


def bias_token(coeff_cos, coeff_sin, omegas, *, b0=None, slope=None, delta_main=None, width=None,
               gate: str = "none", ramp_lambda: float = 0.0, tau: float = 64.0, rows=None, cols=None
               ) -> torch.Tensor:
    """Token-offset bias (the reference's score_mod body) -> [H,R,C]."""
    H, T, K = coeff_cos.shape
    rows = torch.arange(T) if rows is None else rows
    cols = torch.arange(T) if cols is None else cols
    delta = (rows[:, None] - cols[None, :]).clamp(min=0).to(coeff_cos.dtype)  # [R,C]
    w = omegas.to(coeff_cos.dtype)
    ph = w[:, None, None] * delta[None]
    A = coeff_cos[:, rows, :]
    B = coeff_sin[:, rows, :]
    bias = torch.einsum("hrk,krc->hrc", A, torch.cos(ph)) + torch.einsum("hrk,krc->hrc", B, torch.sin(ph))
    if b0 is not None:
        bias = bias - b0[:, rows][:, :, None]
    if slope is not None:
        bias = bias + slope[:, rows][:, :, None] * delta[None]
    if gate != "none" and ramp_lambda > 0:
        x = ((delta[None] - delta_main[:, rows][:, :, None]).abs() - width[:, rows][:, :, None]) / tau
        g = torch.relu(x) if gate == "relu" else torch.nn.functional.softplus(x)
        bias = bias - ramp_lambda * g
    return bias


def attention_dense(q, k, v, allowed, bias=None, *, scale: float, beta: float = 0.5, extra=None):
    """q,k,v [H,T,D]; allowed [H,T,T] bool; bias [H,T,T] or None (scaled by
    beta); extra [H,T,T] or None (added as is) -> (out [H,T,D], lse [H,T])."""
    s = scale * torch.einsum("hid,hjd->hij", q, k)
    if bias is not None:
        s = s + beta * bias
    if extra is not None:
        s = s + extra
    s = s.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
    p = torch.exp(s - safe[..., None])
    out = torch.einsum("hij,hjd->hid", p, v)
    return out, lse


def attention_blocksparse(q, k, v, kv_num, kv_idx, docs, *, bs: int, scale: float, beta: float = 0.5,
                          bias_mode: str = "none", coeff_cos=None, coeff_sin=None, omegas=None,
                          token_kwargs: dict | None = None, heads=None, qblocks=None, pair_bias=None):
    """Per (h, qb) gather of the listed key blocks; same semantics as
    ``attention_dense`` without a [T,T] tensor.  Returns dicts keyed by
    (h, qb) -> (out [bs,D], lse [bs]) for the requested heads / q-blocks.
    ``pair_bias`` [H,QB,L] (aligned with kv_idx) adds b[h,qb,e] to every
    score of the tile (q-block qb, key block kv_idx[h,qb,e])."""
    H, T, D = q.shape
    docs = torch.as_tensor(docs).long()
    kv_num = torch.as_tensor(kv_num)
    kv_idx = torch.as_tensor(kv_idx)
    heads = range(H) if heads is None else heads
    QB = T // bs
    qblocks = range(QB) if qblocks is None else qblocks
    res = {}
    for h in heads:
        for qb in qblocks:
            n = int(kv_num[h, qb])
            blocks = kv_idx[h, qb, :n].long()
            rows = torch.arange(qb * bs, (qb + 1) * bs)
            cols = (blocks[:, None] * bs + torch.arange(bs)[None]).reshape(-1)
            s = scale * (q[h, rows] @ k[h, cols].T)
            if bias_mode == "block":
                s = s + beta * bias_block(coeff_cos[h:h + 1], coeff_sin[h:h + 1], omegas, bs, rows, cols)[0]
            elif bias_mode == "token":
                tk = dict(token_kwargs or {})
                for key in ("b0", "slope", "delta_main", "width"):
                    if tk.get(key) is not None:
                        tk[key] = tk[key][h:h + 1]
                s = s + beta * bias_token(coeff_cos[h:h + 1], coeff_sin[h:h + 1], omegas, rows=rows, cols=cols, **tk)[0]
            if pair_bias is not None:
                s = s + pair_bias[h, qb, :n].repeat_interleave(bs)[None, :]
            ok = (rows[:, None] >= cols[None, :]) & (docs[rows][:, None] == docs[cols][None, :])
            s = s.masked_fill(~ok, float("-inf"))
            lse = torch.logsumexp(s, dim=-1)
            safe = torch.where(torch.isinf(lse), torch.zeros_like(lse), lse)
            p = torch.exp(s - safe[:, None])
            res[(h, qb)] = (p @ v[h, cols], lse)
    return res


def scope_attention_blocksparse(q, k, v, kv_num, kv_idx, docs, *, bs: int, scale: float, beta: float = 0.5,
                                bias_mode: str = "none", coeff_cos=None, coeff_sin=None, omegas=None,
                                token_kwargs: dict | None = None, pair_bias=None):
    """Differentiable block-sparse reference: (out [H,T,D], lse [H,T]) built
    from the per-(h, q-block) gathers, so autograd gives every gradient
    without a [T,T] tensor."""
    H, T, D = q.shape
    QB = T // bs
    res = attention_blocksparse(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=scale, beta=beta, bias_mode=bias_mode,
                                coeff_cos=coeff_cos, coeff_sin=coeff_sin, omegas=omegas, token_kwargs=token_kwargs,
                                pair_bias=pair_bias)
    out = torch.stack([torch.cat([res[(h, qb)][0] for qb in range(QB)], 0) for h in range(H)], 0)
    lse = torch.stack([torch.cat([res[(h, qb)][1] for qb in range(QB)], 0) for h in range(H)], 0)
    return out, lse


def pair_bias_dense(pair_bias, kv_num, kv_idx, bs: int, T: int):
    """[H,QB,L] per-list-entry bias -> dense [H,T,T] (zero off the lists)."""
    H, QB, L = pair_bias.shape
    NB = T // bs
    blk = torch.zeros((H, QB, NB), dtype=pair_bias.dtype)
    for h in range(H):
        for qb in range(QB):
            n = int(kv_num[h, qb])
            idx = torch.as_tensor(kv_idx[h, qb, :n]).long()
            blk = blk.index_put((torch.full_like(idx, h), torch.full_like(idx, qb), idx), pair_bias[h, qb, :n])
    return blk.repeat_interleave(bs, dim=1).repeat_interleave(bs, dim=2)


def scope_attention_reference(q, k, v, kv_num, kv_idx, docs, *, bs: int, scale: float, beta: float = 0.5,
                              bias_mode: str = "none", coeff_cos=None, coeff_sin=None, omegas=None,
                              token_kwargs: dict | None = None, pair_bias=None):
    """Dense-masked reference with autograd: returns (out, lse)."""
    H, T, D = q.shape
    allowed = allowed_mask(kv_num, kv_idx, docs, bs, T)
    bias = None
    if bias_mode == "block":
        bias = bias_block(coeff_cos, coeff_sin, omegas, bs)
    elif bias_mode == "token":
        bias = bias_token(coeff_cos, coeff_sin, omegas, **(token_kwargs or {}))
    out, lse = attention_dense(q, k, v, allowed, bias, scale=scale, beta=beta,
                               extra=None if pair_bias is None else pair_bias_dense(pair_bias, kv_num, kv_idx, bs, T))
    return out, lse


def block_mass(q, k, docs, *, bs: int, scale: float, beta: float = 0.5, bias_mode: str = "none", coeff_cos=None,
               coeff_sin=None, omegas=None, token_kwargs: dict | None = None, kv_num=None, kv_idx=None):
    """Teacher block mass (scoped_medium.py:1799-1819): for every head, q-block
    qb and key block kb, the softmax probability mass summed over the
    q-block's rows and the key block's keys -> [H, NB, NB].

    Without lists the attention is the dense document-causal one (the
    teacher's); with (kv_num, kv_idx) it is restricted to the listed blocks.
    One q-block at a time, like the reference's loop.  Parity pin
    (tests/test_oracle_attention.py): ``attention_dense`` with V = the one-hot
    key-block indicator gives the same numbers summed over the rows; the
    row-sum invariant Σ_kb mass = bs; the uniform closed form for q = 0."""
    H, T, D = q.shape
    NB = T // bs
    docs = torch.as_tensor(docs).long()
    mass = torch.zeros((H, NB, NB), dtype=q.dtype)
    cols = torch.arange(T)
    for qb in range(NB):
        rows = torch.arange(qb * bs, (qb + 1) * bs)
        s = scale * torch.einsum("hrd,hcd->hrc", q[:, rows], k)
        if bias_mode == "token":
            tk = dict(token_kwargs or {})
            s = s + beta * bias_token(coeff_cos, coeff_sin, omegas, rows=rows, cols=cols, **tk)
        elif bias_mode == "block":
            s = s + beta * bias_block(coeff_cos, coeff_sin, omegas, bs, rows, cols)
        ok = (rows[:, None] >= cols[None, :]) & (docs[rows][:, None] == docs[cols][None, :])
        ok = ok[None].expand(H, -1, -1)
        if kv_num is not None:
            blk = torch.zeros((H, NB), dtype=torch.bool)
            for h in range(H):
                blk[h, torch.as_tensor(kv_idx)[h, qb, :int(kv_num[h, qb])].long()] = True
            ok = ok & blk.repeat_interleave(bs, dim=1)[:, None, :]
        s = s.masked_fill(~ok, float("-inf"))
        lse = torch.logsumexp(s, dim=-1, keepdim=True)
        p = torch.exp(s - torch.where(torch.isinf(lse), torch.zeros_like(lse), lse))
        mass[:, qb] = p.sum(dim=1).reshape(H, NB, bs).sum(dim=-1)
    return mass


def decode_attention(q, k_cache, v_cache, kv_num, kv_idx, docs, t: int, *, bs: int, scale: float):
    """One query at position t (q [H, D]) against the cache [H, T_cap, D] over
    the listed blocks (kv_num [H], kv_idx [H, maxkv]) with the document-causal
    mask -> (out [H, D], lse [H]).  Pinned (tests/test_oracle_attention.py)
    by ``attention_blocksparse``'s row t with the same list."""
    H, T_cap, D = k_cache.shape
    docs = torch.as_tensor(docs).long()
    out = torch.zeros((H, D), dtype=q.dtype)
    lse = torch.full((H,), float("-inf"), dtype=q.dtype)
    for h in range(H):
        blocks = torch.as_tensor(kv_idx)[h, :int(kv_num[h])].long()
        cols = (blocks[:, None] * bs + torch.arange(bs)[None]).reshape(-1)
        cols = cols[(cols <= t)]
        cols = cols[docs[cols] == docs[t]]
        if cols.numel() == 0:
            continue
        s = scale * (k_cache[h, cols] @ q[h])
        lse[h] = torch.logsumexp(s, 0)
        out[h] = torch.softmax(s, 0) @ v_cache[h, cols]
    return out, lse


def flops_active(kv_num, bs: int, D: int) -> tuple[float, float]:
    """(F_fwd, F_bwd) counting every listed tile as a full bs×bs tile."""
    n_act = float(torch.as_tensor(kv_num).sum())
    return 4.0 * bs * bs * D * n_act, 10.0 * bs * bs * D * n_act


def omegas_block(K: int = 8) -> torch.Tensor:
    """ω_k = π·2^-k (block-offset configuration)."""
    return torch.tensor([math.pi * 2.0 ** (-k) for k in range(K)], dtype=torch.float32)


def omegas_logspaced(K: int, L_train: int, L_max: int) -> torch.Tensor:
    """model/attn_bias.py:220-226."""
    w_min = 2 * math.pi / L_max
    w_max = 2 * math.pi / L_train
    return torch.logspace(math.log10(w_min), math.log10(w_max), K, dtype=torch.float32)


def soft_pointer_pair_bias(q, k, kv_num, kv_idx, picks, *, bs: int, logit_scale: float, soft_temp: float,
                           prior=None):
    """Differentiable soft top-k weights of the block-scoring picks (a
    specification of this project): q̄, k̄ = block means of q, k [H,T,D];
    z = logit_scale · q̄·k̄ + prior[qb-kb]; b = log σ(z/τ_w) on the pick
    entries of the packed lists, 0 elsewhere.  Returns b [H,QB,L] with the
    autograd graph back to q and k (the prior is a constant schedule)."""
    H, T, D = q.shape
    NB = T // bs
    qbar = q.reshape(H, NB, bs, D).mean(dim=2)
    kbar = k.reshape(H, NB, bs, D).mean(dim=2)
    kv_idx = torch.as_tensor(kv_idx).long()
    kv_num = torch.as_tensor(kv_num)
    picks = torch.as_tensor(picks).long()
    L = kv_idx.shape[-1]
    hh = torch.arange(H)[:, None, None].expand(H, NB, L)
    qq = torch.arange(NB)[None, :, None].expand(H, NB, L)
    z = logit_scale * (qbar[hh, qq] * kbar[hh, kv_idx.clamp(0, NB - 1)]).sum(-1)
    if prior is not None:
        pr = torch.as_tensor(prior, dtype=z.dtype).reshape(-1, NB).expand(H, NB)
        z = z + pr[hh, (qq - kv_idx).clamp(0, NB - 1)]
    e = torch.arange(L)[None, None, :]
    is_pick = (kv_idx[..., :, None] == picks[..., None, :]).any(-1) & (e < kv_num[..., None])
    return torch.where(is_pick, torch.nn.functional.logsigmoid(z / soft_temp), torch.zeros_like(z))

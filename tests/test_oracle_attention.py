"""CPU: pin the attention oracle against torch's own eager FlexAttention
(library code, with the block list restated inside mask_mod), the qk_aug
identity of scoped_medium.py:380-423, gradcheck and the block-sparse variant."""
from __future__ import annotations

import math
import warnings

import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention as A
from oracle import pointer as P

warnings.filterwarnings("ignore")


def _setup(H=2, T=512, D=32, bs=128, K=6, n_docs=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    docs = torch.zeros(T, dtype=torch.int32)
    if n_docs > 1:
        cuts = torch.randperm(T - 1, generator=g)[: n_docs - 1] + 1
        f = torch.zeros(T, dtype=torch.int64)
        f[cuts] = 1
        docs = f.cumsum(0).to(torch.int32)
    NB = T // bs
    logits = np.random.default_rng(seed).standard_normal((H, NB, NB)).astype(np.float32)
    sel = P.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=1, n_global=1, budget=1)
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    q, k, v = (torch.randn((H, T, D), generator=g, dtype=torch.float64) for _ in range(3))
    cc = torch.randn((H, T, K), generator=g, dtype=torch.float64) * 0.3
    cs = torch.randn((H, T, K), generator=g, dtype=torch.float64) * 0.3
    om = A.omegas_logspaced(K, 128, 4096).double()
    return docs, kv_num, kv_idx, q, k, v, cc, cs, om


def _flex(q, k, v, kv_num, kv_idx, docs, bs, score_mod):
    from torch.nn.attention.flex_attention import create_block_mask, flex_attention

    H, T, _ = q.shape
    NB = T // bs
    blk = torch.zeros((H, NB, NB), dtype=torch.bool)
    for h in range(H):
        for qb in range(NB):
            blk[h, qb, kv_idx[h, qb, :kv_num[h, qb]].long()] = True
    docs_l = docs.long()

    def mask_mod(b, h, qi, ki):  # document_causal (model/attn_bias.py:674-679) ∧ block membership
        return blk[h, qi // bs, ki // bs] & (qi >= ki) & (docs_l[qi] == docs_l[ki])

    bm = create_block_mask(mask_mod, None, H, T, T, device="cpu", BLOCK_SIZE=bs)
    o, lse = flex_attention(q[None], k[None], v[None], block_mask=bm, score_mod=score_mod, scale=0.12,
                            return_lse=True)
    return o[0], lse[0]


def test_token_mode_matches_eager_flex_attention():
    """The reference's score_mod (scoped_medium.py:425-457) restated for
    torch's eager FlexAttention vs the oracle, every term on."""
    docs, kv_num, kv_idx, q, k, v, cc, cs, om = _setup()
    H, T, K = cc.shape
    bs = 128
    b0 = cc.sum(-1)
    g = torch.Generator().manual_seed(3)
    slope = torch.randn((H, T), generator=g, dtype=torch.float64) * 0.01
    dm = torch.rand((H, T), generator=g, dtype=torch.float64) * 100
    wd = 32 + torch.rand((H, T), generator=g, dtype=torch.float64) * 100
    Dd = torch.arange(T, dtype=torch.float64)
    cosT, sinT = torch.cos(om[:, None] * Dd[None]), torch.sin(om[:, None] * Dd[None])
    CC, CS, B0, SL, DM, WD = cc[None], cs[None], b0[None], slope[None], dm[None], wd[None]

    def score_mod(score, b, h, q_idx, kv_idx):
        qq = q_idx.to(torch.long).reshape(-1)
        kk = kv_idx.to(torch.long).reshape(-1)
        delta = (qq[:, None] - kk[None, :]).clamp(min=0)
        Aa, Bb = CC[b, h, qq], CS[b, h, qq]
        bias = score.new_zeros(delta.shape, dtype=torch.float64)
        for kx in range(K):
            bias = bias + Aa[:, kx:kx + 1] * cosT[kx, delta] + Bb[:, kx:kx + 1] * sinT[kx, delta]
        df = delta.to(bias.dtype)
        bias = bias - B0[b, h, qq][:, None] + SL[b, h, qq][:, None] * df
        x = ((df - DM[b, h, qq][:, None]).abs() - WD[b, h, qq][:, None]) / 64.0
        bias = bias - 0.2 * F.softplus(x)
        return score + 0.5 * bias.reshape_as(score).to(score.dtype)

    o_ref, l_ref = _flex(q, k, v, kv_num, kv_idx, docs, bs, score_mod)
    tk = dict(b0=b0, slope=slope, delta_main=dm, width=wd, gate="softplus", ramp_lambda=0.2, tau=64.0)
    o, l = A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=0.12, beta=0.5, bias_mode="token",
                                       coeff_cos=cc, coeff_sin=cs, omegas=om, token_kwargs=tk)
    assert (o - o_ref).abs().max() < 1e-12
    assert (l - l_ref).abs().max() < 1e-12


def test_block_mode_matches_eager_flex_attention():
    docs, kv_num, kv_idx, q, k, v, cc, cs, om = _setup(seed=1)
    bs, K = 128, cc.shape[-1]
    om = torch.tensor([math.pi * 2.0 ** (-i) for i in range(K)], dtype=torch.float64)
    CC, CS = cc[None], cs[None]

    NB = q.shape[1] // bs
    rr = torch.arange(NB, dtype=torch.float64)
    cosR, sinR = torch.cos(om[:, None] * rr[None]), torch.sin(om[:, None] * rr[None])  # [K, NB]

    def score_mod(score, b, h, q_idx, kv_idx):
        qq = q_idx.to(torch.long).reshape(-1)
        kk = kv_idx.to(torch.long).reshape(-1)
        r = (qq[:, None] // bs - kk[None, :] // bs).clamp(min=0)
        Aa, Bb = CC[b, h, qq], CS[b, h, qq]
        bias = score.new_zeros(r.shape, dtype=torch.float64)
        for kx in range(K):
            bias = bias + Aa[:, kx:kx + 1] * cosR[kx, r] + Bb[:, kx:kx + 1] * sinR[kx, r]
        return score + 0.5 * bias.reshape_as(score).to(score.dtype)

    o_ref, l_ref = _flex(q, k, v, kv_num, kv_idx, docs, bs, score_mod)
    o, l = A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=0.12, beta=0.5, bias_mode="block",
                                       coeff_cos=cc, coeff_sin=cs, omegas=om)
    assert (o - o_ref).abs().max() < 1e-12
    assert (l - l_ref).abs().max() < 1e-12


def test_qk_aug_identity():
    """scoped_medium.py:380-423: concatenating [Qcos, Qsin, -slope]·s to q and
    [cos ωj, sin ωj, j]·s to k reproduces the token-mode bias without the gate,
    up to a per-row constant (softmax-invariant)."""
    docs, kv_num, kv_idx, q, k, v, cc, cs, om = _setup(seed=2)
    H, T, K = cc.shape
    g = torch.Generator().manual_seed(4)
    slope = torch.randn((H, T), generator=g, dtype=torch.float64) * 0.01
    s = math.sqrt(0.5 / 0.12)
    pos = torch.arange(T, dtype=torch.float64)
    cos_t, sin_t = torch.cos(pos[:, None] * om[None]), torch.sin(pos[:, None] * om[None])  # [T,K]
    Qcos = cc * cos_t + cs * sin_t
    Qsin = cc * sin_t - cs * cos_t
    q_aug = torch.cat([q, torch.cat([Qcos, Qsin, -slope[..., None]], -1) * s], -1)
    k_aug = torch.cat([k, torch.cat([cos_t, sin_t, pos[:, None]], -1).expand(H, T, 2 * K + 1) * s], -1)
    o_aug, _ = A.scope_attention_reference(q_aug, k_aug, v, kv_num, kv_idx, docs, bs=128, scale=0.12)
    o, _ = A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=128, scale=0.12, beta=0.5, bias_mode="token",
                                       coeff_cos=cc, coeff_sin=cs, omegas=om,
                                       token_kwargs=dict(b0=cc.sum(-1), slope=slope))
    assert (o - o_aug).abs().max() < 1e-9


def test_blocksparse_equals_dense():
    docs, kv_num, kv_idx, q, k, v, cc, cs, om = _setup(seed=5, n_docs=3)
    o, l = A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=128, scale=0.12, beta=0.5, bias_mode="block",
                                       coeff_cos=cc, coeff_sin=cs, omegas=om)
    res = A.attention_blocksparse(q, k, v, kv_num, kv_idx, docs, bs=128, scale=0.12, beta=0.5, bias_mode="block",
                                  coeff_cos=cc, coeff_sin=cs, omegas=om)
    for (h, qb), (ob, lb) in res.items():
        assert (ob - o[h, qb * 128:(qb + 1) * 128]).abs().max() < 1e-12
        assert (lb - l[h, qb * 128:(qb + 1) * 128]).abs().max() < 1e-12


def test_fully_masked_rows_give_zero_and_neg_inf():
    """torch:_higher_order_ops/flex_attention.py:250-258 semantics."""
    T, bs = 64, 32
    q = torch.randn((1, T, 8), dtype=torch.float64)
    docs = torch.zeros(T, dtype=torch.int32)
    kv_num = torch.tensor([[1, 1]], dtype=torch.int32)
    kv_idx = torch.tensor([[[1], [1]]], dtype=torch.int32)  # block 0 lists only the future block 1
    o, l = A.scope_attention_reference(q, q, q, kv_num, kv_idx, docs, bs=bs, scale=0.12)
    assert torch.all(o[0, :bs] == 0) and torch.all(torch.isneginf(l[0, :bs]))


def test_gradcheck_token_and_block_modes():
    H, T, D, bs, K = 1, 64, 4, 16, 3
    g = torch.Generator().manual_seed(6)
    docs = torch.zeros(T, dtype=torch.int32)
    docs[40:] = 1
    kv_num = torch.tensor([[1, 2, 3, 2]], dtype=torch.int32)
    kv_idx = torch.tensor([[[0, 0, 0], [0, 1, 1], [0, 1, 2], [2, 3, 3]]], dtype=torch.int32)
    mk = lambda *s: torch.randn(s, generator=g, dtype=torch.float64).requires_grad_()  # noqa: E731
    q, k, v = mk(H, T, D), mk(H, T, D), mk(H, T, D)
    cc, cs = mk(H, T, K), mk(H, T, K)
    om = A.omegas_logspaced(K, 16, 256).double()
    sl, dm, wd = mk(H, T), (torch.rand((H, T), generator=g, dtype=torch.float64) * 20).requires_grad_(), \
        (5 + torch.rand((H, T), generator=g, dtype=torch.float64) * 10).requires_grad_()

    def f_tok(q, k, v, cc, cs, sl, dm, wd):
        tk = dict(b0=cc.sum(-1), slope=sl * 0.01, delta_main=dm, width=wd, gate="softplus", ramp_lambda=0.2, tau=8.0)
        return A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=0.3, beta=0.5,
                                           bias_mode="token", coeff_cos=cc, coeff_sin=cs, omegas=om,
                                           token_kwargs=tk)[0]

    def f_blk(q, k, v, cc, cs):
        return A.scope_attention_reference(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=0.3, beta=0.5,
                                           bias_mode="block", coeff_cos=cc, coeff_sin=cs, omegas=om)[0]

    assert torch.autograd.gradcheck(f_tok, (q, k, v, cc, cs, sl, dm, wd), eps=1e-6, atol=1e-5)
    assert torch.autograd.gradcheck(f_blk, (q, k, v, cc, cs), eps=1e-6, atol=1e-5)


def test_block_mass_pins():
    """oracle.attention.block_mass: (1) the dense attention with V = the
    one-hot key-block indicator, summed over the q-block's rows; (2) every
    row's probabilities sum to 1; (3) q = 0 without a bias gives the uniform
    closed form (visible keys of a row in kb / visible keys of the row)."""
    H, T, D, bs = 2, 256, 16, 32
    NB = T // bs
    g = torch.Generator().manual_seed(4)
    docs = torch.zeros(T, dtype=torch.long)
    docs[70:] = 1
    docs[161:] = 2
    q, k = (torch.randn((H, T, D), generator=g, dtype=torch.float64) for _ in range(2))
    K = 4
    cc = torch.randn((H, T, K), generator=g, dtype=torch.float64) * 0.3
    cs = torch.randn((H, T, K), generator=g, dtype=torch.float64) * 0.3
    om = A.omegas_logspaced(K, 64, 4096).double()
    sl = torch.randn((H, T), generator=g, dtype=torch.float64) * 0.01
    tk = dict(slope=sl)
    m = A.block_mass(q, k, docs, bs=bs, scale=0.2, bias_mode="token", coeff_cos=cc, coeff_sin=cs, omegas=om,
                     token_kwargs=tk)
    i = torch.arange(T)
    allowed = ((i[:, None] >= i[None, :]) & (docs[:, None] == docs[None, :]))[None].expand(H, -1, -1)
    onehot = torch.nn.functional.one_hot(i // bs, NB).double()[None].expand(H, -1, -1)
    bias = A.bias_token(cc, cs, om, **tk)
    out, _ = A.attention_dense(q, k, onehot, allowed, bias, scale=0.2)
    want = out.reshape(H, NB, bs, NB).sum(dim=2)
    assert torch.allclose(m, want, atol=1e-12)
    assert torch.allclose(m.sum(-1), torch.full((H, NB), float(bs), dtype=torch.float64), atol=1e-10)
    mu = A.block_mass(torch.zeros_like(q), k, docs, bs=bs, scale=0.2)
    vis = allowed[0].double()
    closed = (vis / vis.sum(-1, keepdim=True)).reshape(NB, bs, NB, bs).sum(dim=(1, 3))
    assert torch.allclose(mu[0], closed, atol=1e-12) and torch.allclose(mu[1], closed, atol=1e-12)


def test_decode_attention_is_a_row_of_the_blocksparse_oracle():
    H, T, D, bs = 2, 256, 16, 32
    NB = T // bs
    g = torch.Generator().manual_seed(8)
    docs = torch.zeros(T, dtype=torch.long)
    docs[100:] = 1
    q, k, v = (torch.randn((H, T, D), generator=g, dtype=torch.float64) for _ in range(3))
    for t in (0, 99, 100, 131, 255):
        qb = t // bs
        kv_idx = torch.zeros((H, NB, 4), dtype=torch.int32)
        kv_num = torch.zeros((H, NB), dtype=torch.int32)
        lists = [sorted({qb, max(qb - 1, 0), 0}), sorted({qb, max(qb - 2, 0)})]
        for h in range(H):
            kv_num[h, qb] = len(lists[h])
            kv_idx[h, qb, :len(lists[h])] = torch.tensor(lists[h])
        res = A.attention_blocksparse(q, k, v, kv_num, kv_idx, docs, bs=bs, scale=0.3, qblocks=[qb])
        o, l = A.decode_attention(q[:, t], k, v, kv_num[:, qb], kv_idx[:, qb], docs, t, bs=bs, scale=0.3)
        for h in range(H):
            ro, rl = res[(h, qb)]
            assert torch.allclose(o[h], ro[t % bs], atol=1e-12)
            assert torch.allclose(l[h], rl[t % bs], atol=1e-12)

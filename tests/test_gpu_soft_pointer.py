"""GPU parity of the soft pointer weights (the differentiable inclusion
weight of each block-scoring pick; a specification of this project, pinned
by tests/test_oracle_soft_pointer.py) and of the attention with a
per-list-entry score bias, through the C ABI.

Bars written in every comparison: pair bias 1e-5 abs against the oracle on
the kernel's own fp32 logits and 2e-3 abs against fp64 block means; outputs
and every gradient |got - ref| <= 2e-2 + 1e-2·|ref| elementwise against fp64
autograd (the dpair_bias bar scales with the tile sums: 2e-2·max|ref| abs)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import pointer as OP
from oracle.pointer import doc_start_blocks
from tests.helpers import band_coefficients, docs_with_boundaries, omegas_block, qkv, random_blockscore_mask, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2
SCALE, BETA = 0.12, 0.5


def _mask(kv_num, kv_idx, docs, bs, extras=None):
    from scope_amd.blockmask import ScopeBlockMask

    return ScopeBlockMask(kv_num_blocks=kv_num[None].to(DEV), kv_indices=kv_idx[None].to(DEV), BLOCK_SIZE=bs,
                          docs=docs.to(DEV), ds_tok_end=torch.from_numpy(doc_start_blocks(docs.numpy(), bs)[2]).to(DEV),
                          extras=extras or {})


@pytest.mark.parametrize("H,T,bs,W,G,B,tau", [(2, 4096, 128, 2, 1, 3, 2.0), (3, 8192, 256, 2, 2, 4, 0.7)])
def test_pair_bias_kernel_vs_oracle(H, T, bs, W, G, B, tau):
    from scope_amd import ops

    print(f"pair bias H={H} T={T} bs={bs} B={B} tau={tau}", flush=True)
    q, k, _ = qkv(H, T, seed=3)
    docs = docs_with_boundaries(T, 3, seed=4)
    ds_ptr, ds_local, _ = (torch.from_numpy(x).to(DEV) for x in doc_start_blocks(docs.numpy(), bs))
    NB = T // bs
    qbar, kbar = ops.block_means(q.to(DEV), k.to(DEV), bs)
    prior = torch.linspace(0.3, -0.3, NB)
    ls = bs / math.sqrt(128)
    kv_num, kv_idx, picks, logits = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=W, n_global=G,
                                                       budget=B, qbar=qbar, kbar=kbar, prior=prior.to(DEV),
                                                       logit_scale=ls, return_logits=True)
    pb = ops.pointer_pair_bias(kv_num, kv_idx, picks, bs=bs, window=W, n_global=G, soft_temp=tau, qbar=qbar,
                               kbar=kbar, prior=prior.to(DEV), logit_scale=ls).cpu().numpy()
    kn, ki, pk, lg = (x.cpu().numpy() for x in (kv_num, kv_idx, picks, logits))
    # exact structure and values on the kernel's own fp32 logits
    ref = OP.soft_pair_bias(lg.astype(np.float64), kn, ki, pk, soft_temp=tau)
    assert np.array_equal(pb != 0, ref != 0)
    assert np.abs(pb - ref).max() <= 1e-5, np.abs(pb - ref).max()
    # and on fp64 block means of the same bf16 inputs
    qb64 = OP.block_means(q[0].double().numpy(), bs)
    kb64 = OP.block_means(k[0].double().numpy(), bs)
    lg64 = OP.pointer_logits(qb64, kb64, logit_scale=ls, prior=prior.double().numpy())
    ref64 = OP.soft_pair_bias(lg64, kn, ki, pk, soft_temp=tau)
    assert np.abs(pb - ref64).max() <= 2e-3, np.abs(pb - ref64).max()


CASES = [
    # (H, T, bs, mode, n_docs, W, G, B): the dK/dV kernels of every mode family
    (2, 2048, 128, "none", 2, 2, 1, 3),    # 16-key kernel, bs=128
    (2, 2048, 256, "block", 3, 2, 2, 3),   # 16-key kernel, bs=256, block bias
    (1, 2048, 128, "token", 2, 2, 1, 2),   # 32-key kernel (token mode)
    (2, 4096, 128, "block", 1, 2, 1, 3),   # global block listed by 32 q-blocks: one full dK/dV item
    # (pair bias on q-lists longer than 32: test_gpu_bwd_hot_blocks.py)
]


@pytest.mark.parametrize("H,T,bs,mode,n_docs,W,G,B", CASES)
def test_attention_pair_bias_fwd_bwd_vs_fp64(H, T, bs, mode, n_docs, W, G, B):
    import scope_amd

    print(f"pair-bias attention H={H} T={T} bs={bs} mode={mode}", flush=True)
    q, k, v = qkv(H, T, seed=T + bs + 1)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    docs = docs_with_boundaries(T, n_docs, seed=bs)
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=W, n_global=G, budget=B, seed=T + 1)
    g = torch.Generator().manual_seed(11)
    pb = -3.0 * torch.rand(kv_idx.shape, generator=g, dtype=torch.float64)  # log-weights in [-3, 0]
    pb = torch.where(torch.arange(kv_idx.shape[-1])[None, None] < kv_num[..., None], pb, torch.zeros_like(pb))
    sp_kw = {}
    if mode == "block":
        A_, B_ = band_coefficients(q)
        sp_kw = dict(coeff_cos=A_, coeff_sin=B_, omegas=omegas_block(8))
    elif mode == "token":
        K = 6
        sp_kw = dict(coeff_cos=torch.randn((1, H, T, K), generator=g) * 0.3,
                     coeff_sin=torch.randn((1, H, T, K), generator=g) * 0.3,
                     omegas=OA.omegas_logspaced(K, 1024, 1 << 20))
    # GPU
    pbd = pb.float().to(DEV).requires_grad_()
    bm = _mask(kv_num, kv_idx, docs, bs, dict(pair_bias=pbd))
    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    sp = None
    if mode != "none":
        sp = scope_amd.SpectralTerms(coeff_cos=sp_kw["coeff_cos"].to(DEV), coeff_sin=sp_kw["coeff_sin"].to(DEV),
                                     omegas=sp_kw["omegas"].to(DEV), offset=mode, beta=BETA)
    out, lse = scope_amd.scope_attention(qd, kd, vd, block_mask=bm, scale=SCALE, spectral=sp, return_lse=True)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    # fp64 oracle
    qq, kk, vv = (x[0].double().requires_grad_() for x in (q, k, v))
    pr = pb.clone().requires_grad_()
    kw = dict(bias_mode=mode)
    if mode != "none":
        kw.update(coeff_cos=sp_kw["coeff_cos"][0].double(), coeff_sin=sp_kw["coeff_sin"][0].double(),
                  omegas=sp_kw["omegas"].double())
    ro, rl = OA.scope_attention_blocksparse(qq, kk, vv, kv_num, kv_idx, docs, bs=bs, scale=SCALE, beta=BETA,
                                            pair_bias=pr, **kw)
    ro.backward(dout[0].double())
    for name, gg, rr in (("out", out[0], ro), ("lse", lse[0], rl), ("dq", qd.grad[0], qq.grad),
                         ("dk", kd.grad[0], kk.grad), ("dv", vd.grad[0], vv.grad)):
        ok, worst = tol_check(gg.detach().float().cpu(), rr.detach(), ATOL, RTOL)
        print(f"  {name}: worst ratio {worst:.3f}")
        assert ok, f"{name} violates 2e-2 abs / 1e-2 rel: worst ratio {worst:.3f}"
    dref = pr.grad
    bar = 2e-2 * float(dref.abs().max())
    err = float((pbd.grad.double().cpu() - dref).abs().max())
    print(f"  dpair_bias: max err {err:.4g} (bar {bar:.4g}, max |ref| {float(dref.abs().max()):.3g})")
    assert err <= bar


def _soft_case(H, T, bs, W, G, B, seed):
    q, k, v = qkv(H, T, seed=seed)
    docs = docs_with_boundaries(T, 2, seed=seed + 1)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(seed + 2)).to(torch.bfloat16)
    return q, k, v, docs, dout


@pytest.mark.parametrize("H,T,bs,W,G,B,tau,ls", [(2, 2048, 128, 2, 1, 3, 1.0, 32.0), (2, 4096, 256, 2, 2, 4, 2.0, 48.0)])
def test_soft_pointer_end_to_end_grads_vs_fp64(H, T, bs, W, G, B, tau, ls):
    """mask with soft weights built from q, k -> attention -> backward: the
    gradients of q and k include the pointer path through the block means."""
    import scope_amd

    print(f"soft pointer e2e H={H} T={T} bs={bs} tau={tau}", flush=True)
    q, k, v, docs, dout = _soft_case(H, T, bs, W, G, B, seed=21)
    sb = scope_amd.SpectralBias(head_dim=128, num_heads=H, L_train=T).to(DEV)
    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    prior = torch.linspace(0.2, -0.2, T // bs)
    bm = sb.build_blockscore_mask(qd, kd, docs=docs.to(DEV), block_size=bs, window_blocks=W, global_blocks=G,
                                  budget_blocks=B, noise="none", logit_scale=ls, prior=prior.to(DEV), soft_temp=tau)
    assert bm.extras["pair_bias"].requires_grad
    out = scope_amd.scope_attention(qd, kd, vd, block_mask=bm, scale=SCALE)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    kv_num = bm.kv_num_blocks[0].cpu()
    kv_idx = bm.kv_indices[0].cpu()
    picks = bm.extras["picks"].cpu()
    qq, kk, vv = (x[0].double().requires_grad_() for x in (q, k, v))
    pbr = OA.soft_pointer_pair_bias(qq, kk, kv_num.numpy(), kv_idx.numpy(), picks.numpy(), bs=bs, logit_scale=ls,
                                    soft_temp=tau, prior=prior.double().numpy())
    ok, worst = tol_check(bm.extras["pair_bias"].detach().cpu(), pbr.detach(), 1e-3, 0.0)
    assert ok, f"pair bias worst ratio {worst:.3f}"
    ro, _ = OA.scope_attention_blocksparse(qq, kk, vv, kv_num, kv_idx, docs, bs=bs, scale=SCALE, pair_bias=pbr)
    ro.backward(dout[0].double())
    # the pointer path must matter in this case, or the test pins nothing
    qn, kn = (x[0].double().requires_grad_() for x in (q, k))
    ro2, _ = OA.scope_attention_blocksparse(qn, kn, vv.detach(), kv_num, kv_idx, docs, bs=bs, scale=SCALE,
                                            pair_bias=pbr.detach())
    ro2.backward(dout[0].double())
    path = float((qq.grad - qn.grad).abs().max())
    print(f"  pointer path: max |dq change| {path:.3g} of max |dq| {float(qq.grad.abs().max()):.3g}")
    assert path > 0.05
    for name, gg, rr in (("out", out[0], ro), ("dq", qd.grad[0], qq.grad), ("dk", kd.grad[0], kk.grad),
                         ("dv", vd.grad[0], vv.grad)):
        ok, worst = tol_check(gg.detach().float().cpu(), rr.detach(), ATOL, RTOL)
        print(f"  {name}: worst ratio {worst:.3f}")
        assert ok, f"{name} violates 2e-2 abs / 1e-2 rel: worst ratio {worst:.3f}"


def test_soft_pointer_training_shape_sampled():
    """The 65536-token training layer (H=8, bs=128, window 4, global 1,
    budget 4, block-mode spectral bias) with soft weights: dpair_bias of
    sampled q-blocks against fp64 autograd of those q-blocks, and the pointer
    backward's increments of dq / dk on sampled blocks against the fp64 chain
    rule fed with the kernel's dpair_bias."""
    import scope_amd
    from scope_amd import ops

    H, T, bs, W, G, B, tau = 8, 65536, 128, 4, 1, 4, 4.0
    NB = T // bs
    print(f"soft pointer training shape H={H} T={T}", flush=True)
    q, k, v = qkv(H, T, seed=31)
    docs = torch.zeros(T, dtype=torch.int32)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    A_, B_ = band_coefficients(q)
    sb = scope_amd.SpectralBias(head_dim=128, num_heads=H, L_train=T).to(DEV)
    qd, kd, vd = (x.to(DEV) for x in (q, k, v))
    ls = bs / math.sqrt(128)
    bm = sb.build_blockscore_mask(qd, kd, docs=docs.to(DEV), block_size=bs, window_blocks=W, global_blocks=G,
                                  budget_blocks=B, noise="counter", seed=7, logit_scale=ls, soft_temp=tau)
    pb = bm.extras["pair_bias"].detach()
    kv_num, kv_idx = bm.kv_num_blocks[0], bm.kv_indices[0]
    kw = dict(bias_mode="block", beta=BETA, coeff_cos=A_.to(DEV), coeff_sin=B_.to(DEV),
              table=scope_amd.attention.spectral_table(omegas_block(8).to(DEV), T, bs, "block"))
    out, lse = ops.attn_fwd(qd, kd, vd, kv_num, kv_idx, bm.docs, bm.ds_tok_end, bs=bs, scale=SCALE, pair_bias=pb,
                            **kw)
    q_off, q_list = bm.q_lists()
    g = ops.attn_bwd(qd, kd, vd, out, dout.to(DEV), lse, kv_num, kv_idx, q_off, q_list, bm.docs, bm.ds_tok_end,
                     bs=bs, scale=SCALE, pair_bias=pb, need_pair_grad=True, need_coeff_grads=False, **kw)
    dpair = g["dpair_bias"].cpu()
    assert torch.isfinite(dpair).all()
    kn, ki = kv_num.cpu(), kv_idx.cpu()
    pbc = pb.cpu().double()
    rng = np.random.default_rng(1)
    sample = [(int(rng.integers(H)), int(rng.integers(NB // 2, NB))) for _ in range(3)] + [(0, 0), (H - 1, NB - 1)]
    for h, qb in sample:
        # fp64 autograd of this q-block's attention with a pair-bias leaf
        leaf = pbc.clone().requires_grad_()
        res = OA.attention_blocksparse(q[0].double(), k[0].double(), v[0].double(), kn, ki, docs, bs=bs, scale=SCALE,
                                       beta=BETA, bias_mode="block", coeff_cos=A_[0].double(),
                                       coeff_sin=B_[0].double(), omegas=omegas_block(8).double(), heads=[h],
                                       qblocks=[qb], pair_bias=leaf)
        o, _ = res[(h, qb)]
        (o * dout[0, h, qb * bs:(qb + 1) * bs].double()).sum().backward()
        n = int(kn[h, qb])
        ref = leaf.grad[h, qb, :n]
        err = float((dpair[h, qb, :n].double() - ref).abs().max())
        bar = 2e-2 * float(ref.abs().max()) + 1e-3
        print(f"  dpair (h={h}, qb={qb}): max err {err:.4g}, bar {bar:.4g}")
        assert err <= bar
    # pointer backward increments on zero gradients vs the fp64 chain rule on the kernel's dpair
    qbar, kbar = ops.block_means(qd, kd, bs)
    dq0 = torch.zeros_like(qd)
    dk0 = torch.zeros_like(kd)
    ops.pointer_bwd(qbar, kbar, kv_num, kv_idx, q_off, q_list, pb, g["dpair_bias"], dq0, dk0, bs=bs, logit_scale=ls,
                    soft_temp=tau)
    torch.cuda.synchronize()
    qb64 = torch.from_numpy(OP.block_means(q[0].double().numpy(), bs))
    kb64 = torch.from_numpy(OP.block_means(k[0].double().numpy(), bs))
    dz = dpair.double() * (1.0 - torch.exp(pbc)) / tau
    for h, qb in sample:
        n = int(kn[h, qb])
        dqb = ls * sum(dz[h, qb, e] * kb64[h, int(ki[h, qb, e])] for e in range(n)) / bs
        got = dq0[0, h, qb * bs].double().cpu()
        assert torch.allclose(got, dqb, atol=2e-3, rtol=1e-2), float((got - dqb).abs().max())
        assert torch.equal(dq0[0, h, qb * bs:(qb + 1) * bs].cpu(), dq0[0, h, qb * bs].cpu().expand(bs, -1))
    qo, ql = q_off.cpu(), q_list.cpu()
    for h, kb in sample:
        dkb = torch.zeros(128, dtype=torch.float64)
        for i in range(int(qo[h, kb]), int(qo[h, kb + 1])):
            qb = int(ql[h, i])
            e = int((ki[h, qb, :int(kn[h, qb])] == kb).nonzero()[0])
            dkb += ls * dz[h, qb, e] * qb64[h, qb] / bs
        got = dk0[0, h, kb * bs].double().cpu()
        assert torch.allclose(got, dkb, atol=2e-3, rtol=1e-2), float((got - dkb).abs().max())

"""CPU: pin the oracle of the soft pointer weights (the differentiable
inclusion weight of each block-scoring pick, a specification of this
project) and of the attention with a per-list-entry bias.

Pins: the numpy per-entry loop against the vectorised torch function; the
block-sparse gather against the dense [T,T] formulation; softmax shift
invariance under a bias that is constant over a row's listed tiles;
``torch.autograd.gradcheck`` of the whole chain q, k, v -> out in fp64; and
the chain rule of the pointer path that the HIP backward implements
(dq_i += ls/bs · Σ_e dz_e k̄_e, dk_j += ls/bs · Σ dz q̄, dz = db·(1-e^b)/τ_w)
against autograd."""
from __future__ import annotations

import warnings

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import pointer as P

warnings.filterwarnings("ignore")


def _case(H=2, T=512, D=16, bs=64, window=2, n_global=1, budget=2, n_docs=2, seed=0, ls=None, prior=True):
    g = torch.Generator().manual_seed(seed)
    docs = torch.zeros(T, dtype=torch.int32)
    if n_docs > 1:
        cuts = torch.randperm(T - 1, generator=g)[: n_docs - 1] + 1
        f = torch.zeros(T, dtype=torch.int64)
        f[cuts] = 1
        docs = f.cumsum(0).to(torch.int32)
    q, k, v = (torch.randn((H, T, D), generator=g, dtype=torch.float64) for _ in range(3))
    NB = T // bs
    ls = float(bs / np.sqrt(D)) if ls is None else ls
    pr = np.linspace(0.5, -0.5, NB) if prior else None
    qbar = P.block_means(q.numpy(), bs)
    kbar = P.block_means(k.numpy(), bs)
    logits = P.pointer_logits(qbar, kbar, logit_scale=ls, prior=pr)
    sel = P.pointer_select_blockscore(logits.astype(np.float32), docs.numpy(), bs=bs, window=window,
                                      n_global=n_global, budget=budget)
    return dict(docs=docs, q=q, k=k, v=v, logits=logits, sel=sel, ls=ls, prior=pr, bs=bs)


def test_pair_bias_loop_equals_vectorised():
    c = _case()
    sel = c["sel"]
    ref = P.soft_pair_bias(c["logits"], sel["kv_num"], sel["packed"], sel["picks"], soft_temp=2.0)
    got = A.soft_pointer_pair_bias(c["q"], c["k"], sel["kv_num"], sel["packed"], sel["picks"], bs=c["bs"],
                                   logit_scale=c["ls"], soft_temp=2.0, prior=c["prior"])
    assert np.allclose(got.numpy(), ref, rtol=1e-12, atol=1e-12)
    # exactly the valid picks carry a (strictly negative) bias
    n_picks = int((sel["picks"] >= 0).sum())
    assert int((ref < 0).sum()) == n_picks
    for h in range(ref.shape[0]):
        for qb in range(ref.shape[1]):
            n = int(sel["kv_num"][h, qb])
            assert np.all(ref[h, qb, n:] == 0)
            nz = {int(sel["packed"][h, qb, e]) for e in range(n) if ref[h, qb, e] != 0}
            assert nz == {int(x) for x in sel["picks"][h, qb] if x >= 0}


def test_blocksparse_equals_dense_with_pair_bias():
    c = _case(T=256, bs=32, budget=3, n_docs=3, seed=1)
    sel = c["sel"]
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    pb = torch.from_numpy(np.random.default_rng(2).standard_normal(sel["packed"].shape))
    o1, l1 = A.scope_attention_blocksparse(c["q"], c["k"], c["v"], kv_num, kv_idx, c["docs"], bs=32, scale=0.2,
                                           pair_bias=pb)
    o2, l2 = A.scope_attention_reference(c["q"], c["k"], c["v"], kv_num, kv_idx, c["docs"], bs=32, scale=0.2,
                                         pair_bias=pb)
    assert torch.allclose(o1, o2, atol=1e-12) and torch.allclose(l1, l2, atol=1e-12)
    # the bias changes the output (it is not silently dropped)
    o3, _ = A.scope_attention_blocksparse(c["q"], c["k"], c["v"], kv_num, kv_idx, c["docs"], bs=32, scale=0.2)
    assert (o1 - o3).abs().max() > 1e-3


def test_constant_bias_is_softmax_invariant():
    c = _case(T=256, bs=32, seed=3)
    sel = c["sel"]
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    # the same constant on every listed entry of a q-block shifts each row's scores uniformly
    row_c = torch.from_numpy(np.random.default_rng(4).standard_normal(sel["kv_num"].shape))
    pb = row_c[..., None].expand(*sel["packed"].shape).clone()
    o1, l1 = A.scope_attention_blocksparse(c["q"], c["k"], c["v"], kv_num, kv_idx, c["docs"], bs=32, scale=0.2,
                                           pair_bias=pb)
    o0, l0 = A.scope_attention_blocksparse(c["q"], c["k"], c["v"], kv_num, kv_idx, c["docs"], bs=32, scale=0.2)
    assert torch.allclose(o1, o0, atol=1e-12)
    shift = row_c.repeat_interleave(32, dim=1)
    assert torch.allclose(l1, l0 + shift, atol=1e-12)


def _soft_forward(c, q, k, v, soft_temp):
    sel = c["sel"]
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    pb = A.soft_pointer_pair_bias(q, k, sel["kv_num"], sel["packed"], sel["picks"], bs=c["bs"], logit_scale=c["ls"],
                                  soft_temp=soft_temp, prior=c["prior"])
    out, _ = A.scope_attention_blocksparse(q, k, v, kv_num, kv_idx, c["docs"], bs=c["bs"], scale=0.3,
                                           pair_bias=pb)
    return out


def test_gradcheck_soft_pointer_chain():
    c = _case(H=1, T=64, D=4, bs=16, window=1, n_global=1, budget=1, n_docs=1, seed=5, ls=1.5)
    q, k, v = (x.clone().requires_grad_() for x in (c["q"], c["k"], c["v"]))
    assert torch.autograd.gradcheck(lambda a, b, cc: _soft_forward(c, a, b, cc, 1.5), (q, k, v), eps=1e-6,
                                    atol=1e-6, rtol=1e-5)


def test_pointer_path_chain_rule():
    """autograd of the whole chain = attention gradients at fixed bias + the
    closed-form pointer path fed with d(loss)/d(bias)."""
    c = _case(H=2, T=256, D=16, bs=32, window=2, n_global=1, budget=2, n_docs=2, seed=6)
    tau = 3.0
    sel = c["sel"]
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    g = torch.Generator().manual_seed(7)
    dout = torch.randn(c["q"].shape, generator=g, dtype=torch.float64)
    q, k, v = (x.clone().requires_grad_() for x in (c["q"], c["k"], c["v"]))
    (_soft_forward(c, q, k, v, tau) * dout).sum().backward()
    # attention at a fixed (detached) bias, and the bias gradient db
    pb = A.soft_pointer_pair_bias(c["q"], c["k"], sel["kv_num"], sel["packed"], sel["picks"], bs=32,
                                  logit_scale=c["ls"], soft_temp=tau, prior=c["prior"]).detach().requires_grad_()
    q2, k2, v2 = (x.clone().requires_grad_() for x in (c["q"], c["k"], c["v"]))
    out2, _ = A.scope_attention_blocksparse(q2, k2, v2, kv_num, kv_idx, c["docs"], bs=32, scale=0.3, pair_bias=pb)
    (out2 * dout).sum().backward()
    db = pb.grad
    # pointer path: dz = db·(1 - e^b)/τ, dq̄ = ls Σ_e dz k̄_e, dk̄ = ls Σ dz q̄
    H, T, D = c["q"].shape
    bs, NB = 32, T // 32
    qbar = c["q"].reshape(H, NB, bs, D).mean(2)
    kbar = c["k"].reshape(H, NB, bs, D).mean(2)
    dz = db * (1.0 - torch.exp(pb.detach())) / tau
    dqbar = torch.zeros_like(qbar)
    dkbar = torch.zeros_like(kbar)
    for h in range(H):
        for qb in range(NB):
            for e in range(int(kv_num[h, qb])):
                kb = int(kv_idx[h, qb, e])
                dqbar[h, qb] += c["ls"] * dz[h, qb, e] * kbar[h, kb]
                dkbar[h, kb] += c["ls"] * dz[h, qb, e] * qbar[h, qb]
    dq = q2.grad + dqbar.repeat_interleave(bs, dim=1) / bs
    dk = k2.grad + dkbar.repeat_interleave(bs, dim=1) / bs
    assert torch.allclose(q.grad, dq, atol=1e-10)
    assert torch.allclose(k.grad, dk, atol=1e-10)
    assert torch.allclose(v.grad, v2.grad, atol=1e-12)
    # the pointer path is not negligible in this case
    assert (dq - q2.grad).abs().max() > 1e-4


@pytest.mark.parametrize("tau", [0.5, 4.0])
def test_pair_bias_closed_form_limits(tau):
    # logsigmoid(x) -> 0 for x >> 0 and ~ x for x << 0; the bias only touches picks
    c = _case(seed=8)
    sel = c["sel"]
    logits = c["logits"].copy()
    logits[:] = 1e4
    b = P.soft_pair_bias(logits, sel["kv_num"], sel["packed"], sel["picks"], soft_temp=tau)
    assert np.all(np.abs(b) < 1e-300 + 1e-12)
    logits[:] = -60.0
    b = P.soft_pair_bias(logits, sel["kv_num"], sel["packed"], sel["picks"], soft_temp=tau)
    picks_mask = b != 0
    assert np.allclose(b[picks_mask], -60.0 / tau - np.log1p(np.exp(-60.0 / tau)), rtol=1e-12)

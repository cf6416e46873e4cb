"""GPU: the head's MLP operator (``scope::coeff_mlp``) and the split-row
weight-gradient kernel (``scope_linear_wgrad``) under it.

* ``linear_wgrad``: dw = Σ_r a[r]^T b[r] and db = Σ_r a[r] against fp64 sums
  of the same bf16 rows, for every supported (M, N), with b a strided
  [1, H, T, N] view (rows in head segments, as the transposed q of the
  reference) and a 2-D; the bound is 1e-5 of Σ_r |a||b| (fp32 accumulation
  of exact bf16 products) unrounded, plus half a bf16 ulp rounded.
* ``coeff_mlp`` against autograd of the reference's steps
  (oracle.coeff_head.mlp_forward: F.linear, SiLU, F.linear with the weights
  cast to bf16), at the reference's default shape (D=128, hidden 256, 41
  outputs): y, z1 and x1 bit for bit (the same torch ops), dq within 1e-3 of
  max|dq| (the same BLAS calls; autograd may pick another kernel), and the
  weight and bias gradients within a bf16 ulp plus 1e-5 of Σ|a||b|."""
from __future__ import annotations

import pytest
import torch

from oracle.coeff_head import mlp_forward
from scope_amd import SpectralBias, library, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _bf16_view(H, T, C, g, transposed):
    x = torch.randn((1, T, H, C) if transposed else (1, H, T, C), generator=g, device=DEV).to(torch.bfloat16)
    return x.transpose(1, 2) if transposed else x


def _check_wgrad(dw, db, a, b, rnd):
    a64 = a.reshape(-1, a.shape[-1]).double()
    b64 = b.reshape(-1, b.shape[-1]).double()
    ref, refb = a64.t() @ b64, a64.sum(0)
    bound = 1e-5 * (a64.abs().t() @ b64.abs()) + 1e-30
    boundb = 1e-5 * a64.abs().sum(0) + 1e-30
    if rnd:  # rounding to bf16: half an ulp, 2^-9 relative
        bound = bound + ref.abs() * 2.0 ** -8
        boundb = boundb + refb.abs() * 2.0 ** -8
    err = (dw.double() - ref).abs()
    assert bool((err <= bound).all()), f"dw: worst {float((err / bound).max()):.3f} of the bound"
    errb = (db.double() - refb).abs()
    assert bool((errb <= boundb).all()), f"db: worst {float((errb / boundb).max()):.3f} of the bound"


@pytest.mark.parametrize("M,N", [(64, 128), (64, 256), (128, 128), (128, 256), (256, 64), (256, 128)])
@pytest.mark.parametrize("rnd", [False, True])
def test_linear_wgrad_vs_fp64(M, N, rnd):
    g = torch.Generator(device=DEV).manual_seed(M * 7 + N + int(rnd))
    H, T = 8, 1024
    a = _bf16_view(H, T, M, g, False)
    b = _bf16_view(H, T, N, g, True)  # strided rows: head segments of T rows
    dw, db = ops.linear_wgrad(a, b, round_bf16=rnd)
    torch.cuda.synchronize()
    _check_wgrad(dw, db, a, b, rnd)
    # 2-D operands, a single row stride
    dw2, db2 = ops.linear_wgrad(a.reshape(-1, M), b.contiguous().reshape(-1, N), round_bf16=rnd)
    assert torch.equal(dw2, dw) and torch.equal(db2, db)


def test_linear_wgrad_rejects_bad_shapes():
    a = torch.zeros((100, 64), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros((100, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        ops.linear_wgrad(a, b)
    a = torch.zeros((128, 96), dtype=torch.bfloat16, device=DEV)
    b = torch.zeros((128, 128), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="not supported"):
        ops.linear_wgrad(a, b)


@pytest.mark.parametrize("T", [2048, 16384])
def test_coeff_mlp_matches_reference_autograd(T):
    H, D = 8, 128
    sb = SpectralBias(head_dim=D, num_heads=H, L_train=T, K=6, M=8).to(DEV).train()
    g = torch.Generator(device=DEV).manual_seed(T)
    with torch.no_grad():
        for p_ in sb.mlp.parameters():
            p_.copy_(torch.randn(p_.shape, generator=g, device=DEV) * 0.05)
    q0 = _bf16_view(H, T, D, g, True)
    gy = torch.randn(q0.shape[:-1] + (sb.mlp[2].weight.shape[0],), generator=g, device=DEV).to(torch.bfloat16)
    params = list(sb.mlp.parameters())

    def run(fn):
        q = q0.detach().clone().requires_grad_()
        for p_ in params:
            p_.grad = None
        out = fn(q)
        out.backward(gy)
        torch.cuda.synchronize()
        return out.detach(), q.grad, [p_.grad.clone() for p_ in params]

    fc1, fc2 = sb.mlp[0], sb.mlp[2]
    y_op, dq_op, gw_op = run(lambda q: library.coeff_mlp(q, fc1.weight, fc1.bias, fc2.weight, fc2.bias)[0])
    y_ref, dq_ref, gw_ref = run(lambda q: mlp_forward(sb, q))
    assert torch.equal(y_op, y_ref)
    with torch.no_grad():
        z1, x1 = library.coeff_mlp(q0, fc1.weight, fc1.bias, fc2.weight, fc2.bias)[1:]
        z_ref = torch.nn.functional.linear(q0, fc1.weight.bfloat16(), fc1.bias.bfloat16())
    assert torch.equal(z1, z_ref) and torch.equal(x1, torch.nn.functional.silu(z_ref))
    tol = 1e-3 * float(dq_ref.float().abs().max())
    assert float((dq_op.float() - dq_ref.float()).abs().max()) <= tol
    # the gradients' inputs: gy with x1 (fc2), dz1 with q (fc1)
    dx1 = gy.matmul(fc2.weight.bfloat16())
    dz1 = torch.ops.aten.silu_backward(dx1, z1)
    for got, ref, (a, b) in zip(gw_op, gw_ref, [(dz1, q0), (dz1, None), (gy, x1), (gy, None)]):
        a64 = a.reshape(-1, a.shape[-1]).double()
        if b is None:
            bound = 1e-5 * a64.abs().sum(0)
        else:
            bound = 1e-5 * (a64.abs().t() @ b.reshape(-1, b.shape[-1]).double().abs())
        bound = bound + ref.double().abs() * 2.0 ** -7 + 1e-30
        err = (got.double() - ref.double()).abs()
        assert bool((err <= bound).all()), f"worst {float((err / bound).max()):.3f} of the bound"

"""GPU: the head's MLP operator (``scope::coeff_mlp``) and the split-row
weight-gradient kernel (``scope_linear_wgrad``) under it.

* ``linear_wgrad``: dw = Σ_r a[r]^T b[r] and db = Σ_r a[r] against fp64 sums
  of the same bf16 rows, for every supported (M, N), with b a strided
  [1, H, T, N] view (rows in head segments, as the transposed q of the
  reference) and a 2-D; the bound is 1e-5 of Σ_r |a||b| (fp32 accumulation
  of exact bf16 products) unrounded, plus half a bf16 ulp rounded.
* ``coeff_mlp`` (fused kernels) against autograd of the reference's steps
  (oracle.coeff_head.mlp_forward: F.linear, SiLU, F.linear with the weights
  cast to bf16), at the reference's default shape (D=128, hidden 256, 41
  outputs): y, dq and the weight and bias gradients at least as close to
  fp64 arithmetic on the same bf16 operands as the torch steps are (1.5x
  their error, max and mean); the backward's x1 and dz1 against the torch
  steps but for one-ulp rounding flips; fp32 rows on the torch steps."""
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


def _mlp64(q, w1, b1, w2, b2, gy):
    """fp64 forward and row-wise backward of the MLP from the same bf16 operands
    (the weights rounded to bf16, no intermediate rounding): y, dq, z."""
    q64 = q.reshape(-1, q.shape[-1]).double()
    w1d, b1d, w2d, b2d = (t.bfloat16().double() for t in (w1, b1, w2, b2))
    z = q64 @ w1d.t() + b1d
    s = torch.sigmoid(z)
    y = (z * s) @ w2d.t() + b2d
    dx1 = gy.reshape(-1, gy.shape[-1]).double() @ w2d
    dq = (dx1 * s * (1 + z * (1 - s))) @ w1d
    return y, dq, z


@pytest.mark.parametrize("T", [2048, 16384])
def test_coeff_mlp_matches_reference_autograd(T):
    """The fused forward and backward against autograd of the reference's torch
    steps (F.linear, SiLU, F.linear in bf16): both are compared with fp64
    arithmetic on the same bf16 operands, and the fused kernels must be at
    least as accurate (within 1.5x of the torch steps' error, max and mean) —
    bit equality is not expected, the two sum in different orders and round
    their bf16 intermediates at different boundaries."""
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
    assert ops.coeff_mlp_fused(q0, fc1.weight, fc2.weight)
    y_op, dq_op, gw_op = run(lambda q: library.coeff_mlp(q, fc1.weight, fc1.bias, fc2.weight, fc2.bias))
    y_ref, dq_ref, gw_ref = run(lambda q: mlp_forward(sb, q))
    assert y_op.shape == y_ref.shape and y_op.dtype == y_ref.dtype and dq_op.shape == q0.shape
    y64, dq64, _ = _mlp64(q0, fc1.weight, fc1.bias, fc2.weight, fc2.bias, gy)
    for got, ref, exact in ((y_op, y_ref, y64), (dq_op, dq_ref, dq64)):
        e_got = (got.reshape(exact.shape).double() - exact).abs()
        e_ref = (ref.reshape(exact.shape).double() - exact).abs()
        assert float(e_got.max()) <= 1.5 * float(e_ref.max()) + 1e-6
        assert float(e_got.mean()) <= 1.5 * float(e_ref.mean()) + 1e-7
    # the weight and bias gradients, likewise against fp64 from the same operands
    q64 = q0.reshape(-1, D).double()
    g64 = gy.reshape(-1, gy.shape[-1]).double()
    w1d, b1d, w2d = (t.bfloat16().double() for t in (fc1.weight, fc1.bias, fc2.weight))
    z = q64 @ w1d.t() + b1d
    sg = torch.sigmoid(z)
    dz = (g64 @ w2d) * sg * (1 + z * (1 - sg))
    exact = [dz.t() @ q64, dz.sum(0), g64.t() @ (z * sg), g64.sum(0)]
    for got, ref, ex in zip(gw_op, gw_ref, exact):
        e_got, e_ref = (got.double() - ex).abs(), (ref.double() - ex).abs()
        floor = 1e-6 * float(ex.abs().max())
        assert float(e_got.max()) <= 1.5 * float(e_ref.max()) + floor
        assert float(e_got.mean()) <= 1.5 * float(e_ref.mean()) + floor


def test_coeff_mlp_bwd_intermediates():
    """x1, dz1 and the padded output gradient of the fused backward against
    the torch steps on the same rows: x1 = SiLU(bf16(q·W1 + b1)) and
    dz1 = SiLU'(z1)·bf16(gy·W2) agree but for rare one-ulp flips at bf16
    rounding boundaries; the padding is gy itself and zeros."""
    g = torch.Generator(device=DEV).manual_seed(5)
    rows, O = 4096, 41
    q = torch.randn((rows, 128), generator=g, device=DEV).to(torch.bfloat16)
    w1 = torch.randn((256, 128), generator=g, device=DEV) * 0.05
    b1 = torch.randn(256, generator=g, device=DEV) * 0.05
    w2 = torch.randn((O, 256), generator=g, device=DEV) * 0.05
    b2 = torch.randn(O, generator=g, device=DEV) * 0.05
    gy = torch.randn((rows, O), generator=g, device=DEV).to(torch.bfloat16)
    dq, dz1, x1, gyp = ops.coeff_mlp_bwd(q, gy, w1, b1, w2, b2)
    torch.cuda.synchronize()
    z_ref = torch.nn.functional.linear(q, w1.bfloat16(), b1.bfloat16())
    x_ref = torch.nn.functional.silu(z_ref)
    dz_ref = torch.ops.aten.silu_backward(gy.matmul(w2.bfloat16()), z_ref)
    assert torch.equal(gyp[:, :O], gy) and not bool(gyp[:, O:].any())
    for got, ref in ((x1, x_ref), (dz1, dz_ref)):
        diff = (got.float() - ref.float()).abs()
        ulp = ref.float().abs().clamp_min(1e-30) * 2.0 ** -7
        assert bool((diff <= 2 * ulp + 1e-6).all())
        assert float((diff > 0).float().mean()) < 0.02


@pytest.mark.parametrize("rows", [256, 640, 4096, 131072])
def test_coeff_mlp_wgrad_matches_split_row_kernel(rows):
    """The fused weight and bias gradients (z1, x1, dz1 recomputed per tile)
    against the split-row kernel on the stored x1 / dz1 of the same rows, and
    both against fp64 sums of those bf16 intermediates: the two add in
    different orders and both round to bf16 at the end, so they agree to one
    bf16 step, on all but a few elements exactly.  256 rows make four row
    groups (fewer than the 8 XCDs: the plain workgroup order), 640 rows eight
    groups of which three hold no tile."""
    g = torch.Generator(device=DEV).manual_seed(rows)
    O = 41
    q = torch.randn((rows, 128), generator=g, device=DEV).to(torch.bfloat16)
    w1 = torch.randn((256, 128), generator=g, device=DEV) * 0.05
    b1 = torch.randn(256, generator=g, device=DEV) * 0.05
    w2 = torch.randn((O, 256), generator=g, device=DEV) * 0.05
    b2 = torch.randn(O, generator=g, device=DEV) * 0.05
    gy = torch.randn((rows, O), generator=g, device=DEV).to(torch.bfloat16)
    dq, dz1, x1, gyp = ops.coeff_mlp_bwd(q, gy, w1, b1, w2, b2)
    dq2, none1, none2, gyp2 = ops.coeff_mlp_bwd(q, gy, w1, b1, w2, b2, intermediates=False)
    assert none1 is None and none2 is None
    assert torch.equal(dq, dq2) and torch.equal(gyp, gyp2)
    fused = ops.coeff_mlp_wgrad(q, gyp, w1, b1, w2)
    dw1, db1 = ops.linear_wgrad(dz1, q, round_bf16=True)
    dw2, db2 = ops.linear_wgrad(gyp, x1, round_bf16=True)
    split = (dw1, db1, dw2[:O], db2[:O])
    torch.cuda.synchronize()
    q64, d64, x64, g64 = (t.double() for t in (q, dz1, x1, gyp[:, :O]))
    exact = (d64.t() @ q64, d64.sum(0), g64.t() @ x64, g64.sum(0))
    for name, a, b, ex in zip(("dw1", "db1", "dw2", "db2"), fused, split, exact):
        assert a.shape == b.shape == ex.shape, name
        step = ex.abs() * 2.0 ** -7 + 1e-6 * float(ex.abs().max())
        assert bool(((a.double() - b.double()).abs() <= step).all()), name
        assert float((a != b).float().mean()) < 0.05, name
        # each within bf16 rounding of the fp64 sum (a rounded fp32 sum)
        assert bool(((a.double() - ex).abs() <= step).all()), name


def test_coeff_mlp_wgrad_rejects_bad_layouts():
    q = torch.zeros((4, 96, 128), device=DEV, dtype=torch.bfloat16)  # segments of 96 rows
    w1, b1, w2 = torch.zeros((256, 128), device=DEV), torch.zeros(256, device=DEV), torch.zeros((41, 256), device=DEV)
    gyp = torch.zeros((4, 96, 64), device=DEV, dtype=torch.bfloat16)
    assert not ops.coeff_mlp_wgrad_fused(q[:, :, :])
    with pytest.raises(RuntimeError):
        ops.coeff_mlp_wgrad(q.transpose(0, 1), gyp, w1, b1, w2)
    with pytest.raises(RuntimeError):
        ops.coeff_mlp_wgrad(torch.zeros((128, 128), device=DEV, dtype=torch.bfloat16),
                            torch.zeros((128, 41), device=DEV, dtype=torch.bfloat16), w1, b1, w2)


def test_coeff_mlp_fp32_takes_the_torch_steps():
    """fp32 rows are not the fused kernels' case: the operator runs the
    reference's torch steps, equal to the oracle's forward."""
    H, D, T = 2, 128, 256
    sb = SpectralBias(head_dim=D, num_heads=H, L_train=T, K=6, M=8).to(DEV).train()
    q = torch.randn((1, H, T, D), device=DEV)
    fc1, fc2 = sb.mlp[0], sb.mlp[2]
    assert not ops.coeff_mlp_fused(q, fc1.weight, fc2.weight)
    y = library.coeff_mlp(q, fc1.weight, fc1.bias, fc2.weight, fc2.bias)
    assert torch.equal(y, mlp_forward(sb, q))


def _mlp_run(fn, q0, params, gy):
    q = q0.detach().clone().requires_grad_()
    for p_ in params:
        p_.grad = None
    y = fn(q)
    y.backward(gy)
    if q.is_cuda:
        torch.cuda.synchronize()
    return [y.detach(), q.grad] + [p_.grad.clone() for p_ in params]


@pytest.mark.parametrize("case", ["bf16_L96", "bf16_D64", "bf16_B2", "fp32", "per_head_bf16", "per_head_fp32"])
def test_coeff_mlp_other_shapes_vs_fp64(case):
    """The shapes the fused weight-gradient kernel does not take: segments of
    96 rows (fused forward and row-wise backward, the weight gradients on the
    torch product), head_dim 64 (torch steps; the split-row kernel for the
    second layer's weights), batch 2 (copied to one segment of rows), fp32
    rows, and per-head weights (share_across_heads=False, in bf16 and fp32).
    Output, dq and the four weight and bias gradients against fp64 on the
    CPU from the same operands (weights rounded to q's dtype): at least as
    close as the reference's torch steps run on the CPU in q's dtype (1.5x
    their error, max and mean, plus 1e-6 of the largest value)."""
    import copy

    B, H, L, D, dt, shared = {"bf16_L96": (1, 8, 96, 128, torch.bfloat16, True),
                              "bf16_D64": (1, 8, 256, 64, torch.bfloat16, True),
                              "bf16_B2": (2, 4, 256, 128, torch.bfloat16, True),
                              "fp32": (1, 4, 256, 128, torch.float32, True),
                              "per_head_bf16": (1, 4, 256, 128, torch.bfloat16, False),
                              "per_head_fp32": (1, 4, 256, 128, torch.float32, False)}[case]
    sb = SpectralBias(head_dim=D, num_heads=H, L_train=L, K=6, M=8, share_across_heads=shared).to(DEV).train()
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():
        for p_ in sb.parameters():
            if p_.requires_grad and p_.dim() >= 1 and p_.numel() > 8:
                p_.copy_((torch.randn(p_.shape, generator=g) * 0.05).to(DEV))
    params = list(sb.mlp.parameters()) if shared else [sb.w1, sb.b1, sb.w2, sb.b2]
    q0 = torch.randn((B, H, L, D), generator=g).to(dt)
    O = 5 * 8 + (1 if sb.use_slope else 0)
    gy = torch.randn((B, H, L, O), generator=g).to(dt)
    if shared and dt == torch.bfloat16:
        fc1, fc2 = sb.mlp[0], sb.mlp[2]
        fused = ops.coeff_mlp_fused(q0.to(DEV), fc1.weight, fc2.weight)
        assert fused == (D == 128), case
        assert not (fused and ops.coeff_mlp_wgrad_fused(q0.to(DEV))), case  # the fused weight gradients do not run
    got = _mlp_run(lambda q: sb._mlp_forward(q), q0.to(DEV), params, gy.to(DEV))
    sb_cpu = copy.deepcopy(sb).cpu()
    params_cpu = list(sb_cpu.mlp.parameters()) if shared else [sb_cpu.w1, sb_cpu.b1, sb_cpu.w2, sb_cpu.b2]
    ref = _mlp_run(lambda q: mlp_forward(sb_cpu, q), q0, params_cpu, gy)
    sb64 = copy.deepcopy(sb_cpu).double()
    with torch.no_grad():
        for p_, p32 in zip(sb64.mlp.parameters() if shared else [sb64.w1, sb64.b1, sb64.w2, sb64.b2], params_cpu):
            p_.copy_(p32.to(dt).double())
    params64 = list(sb64.mlp.parameters()) if shared else [sb64.w1, sb64.b1, sb64.w2, sb64.b2]
    exact = _mlp_run(lambda q: mlp_forward(sb64, q), q0.double(), params64, gy.double())
    for name, a, r, ex in zip(("y", "dq", "dw1", "db1", "dw2", "db2"), got, ref, exact):
        assert a.shape == ex.shape and a.dtype == r.dtype, name
        e_got, e_ref = (a.double().cpu() - ex).abs(), (r.double() - ex).abs()
        floor = 1e-6 * float(ex.abs().max())
        print(f"  {case} {name}: max err {float(e_got.max()):.3g} (torch steps {float(e_ref.max()):.3g})", flush=True)
        assert float(e_got.max()) <= 1.5 * float(e_ref.max()) + floor, name
        assert float(e_got.mean()) <= 1.5 * float(e_ref.mean()) + floor, name

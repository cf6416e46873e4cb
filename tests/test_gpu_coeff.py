"""Fused coefficient head (scope_coeff_head_fwd / _bwd) on the GPU against
the reference's golden vectors (eval outputs; training outputs, each
regulariser and the gradients w.r.t. q and the MLP weights), the bf16 input
path against the fp32 one, and the torch steps of the same module at the
training shape (T=65536, H=8).  The head is fp32 arithmetic: the bar is
rtol 1e-4 (atol 1e-5·max|ref|) against the fp32 reference, written in each
comparison."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.golden import load_flat

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ["coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width"]
PARAMS = ("q", "w1", "b1", "w2", "b2")


def _close(got: torch.Tensor, ref: torch.Tensor, rtol=1e-4, atol_frac=1e-5, what=""):
    got = got.detach().float().cpu().reshape(ref.shape)
    ref = ref.float()
    atol = atol_frac * max(ref.abs().max().item(), 1e-30)
    err = (got - ref).abs()
    ok = bool((err <= atol + rtol * ref.abs()).all())
    assert ok, f"{what}: max err {err.max().item():.3e} (atol {atol:.1e}, rtol {rtol})"


def _module(g: dict, **kw):
    from scope_amd import SpectralBias

    sb = SpectralBias(head_dim=int(g["Dh"]), num_heads=int(g["H"]), L_train=int(g["L_train"]), L_max=int(g["L_max"]),
                      M=int(g["M"]), K=int(g["K"]), **kw)
    with torch.no_grad():
        sb.mlp[0].weight.copy_(torch.from_numpy(g["w1"]))
        sb.mlp[0].bias.copy_(torch.from_numpy(g["b1"]))
        sb.mlp[2].weight.copy_(torch.from_numpy(g["w2"]))
        sb.mlp[2].bias.copy_(torch.from_numpy(g["b2"]))
    return sb.to(DEV)


def test_fused_head_eval_matches_reference_vectors():
    g = load_flat("coeff_head_vectors.npz")
    sb = _module(g).eval()
    out = sb(torch.from_numpy(g["q"])[None].to(DEV))
    for i, n in enumerate(NAMES):
        _close(out[i][0], torch.from_numpy(g[n]), what=n)
    assert float(out[11]) == 0.0


def _train_run(g, lams, G=None):
    sb = _module(g, pi_entropy_floor_frac=float(g["pi_entropy_floor_frac"]),
                 delta_edge_eps=float(g["delta_edge_eps"]), **lams).train()
    q = torch.from_numpy(g["q"])[None].to(DEV).requires_grad_()
    out = sb(q)
    params = [q, sb.mlp[0].weight, sb.mlp[0].bias, sb.mlp[2].weight, sb.mlp[2].bias]
    go = None
    if G is not None:
        lo = sum((out[i] * G[i].to(DEV)).sum() for i in range(len(G)))
        go = torch.autograd.grad(lo, params, retain_graph=True)
    gr = torch.autograd.grad(out[11], params, allow_unused=True)
    gr = [torch.zeros_like(p_) if x is None else x for x, p_ in zip(gr, params)]
    return out, go, gr


def test_fused_head_training_matches_reference_vectors():
    g = load_flat("coeff_head_train_vectors.npz")
    lam = {k: float(g[k]) for k in ("lambda_omega", "lambda_zero_mean", "lambda_entropy", "lambda_delta_edge")}
    G = [torch.from_numpy(g[f"G_{n}"])[None] for n in NAMES]
    out, go, gr = _train_run(g, lam, G)
    for i, n in enumerate(NAMES):
        _close(out[i][0], torch.from_numpy(g[n]), what=n)
    _close(out[11], torch.tensor(g["reg_all"]), what="reg_all")
    for n, x in zip(PARAMS, go):
        _close(x, torch.from_numpy(g[f"gout_{n}"]), rtol=2e-4, what=f"d<out,G>/d{n}")
    for n, x in zip(PARAMS, gr):
        _close(x, torch.from_numpy(g[f"greg_all_{n}"]), rtol=2e-4, what=f"dreg/d{n}")
    for k in lam:
        tag = k.replace("lambda_", "")
        out1, _, gr1 = _train_run(g, {**{k2: 0.0 for k2 in lam}, k: lam[k]})
        _close(out1[11], torch.tensor(g[f"reg_{tag}"]), what=f"reg_{tag}")
        for n, x in zip(PARAMS, gr1):
            _close(x, torch.from_numpy(g[f"greg_{tag}_{n}"]), rtol=2e-4, what=f"dreg_{tag}/d{n}")


def _prm(M, K, L, training):
    return dict(M=M, K=K, L=L, use_slope=True, subtract_b0=True, training=training, delta_cap=float(L - 1),
                logw_min=-11.0, logw_max=-3.0, c_scale=0.01, width_min=32.0, width_max=256.0, eps=1e-9,
                lambda_omega=1e-5, lambda_entropy=1e-4, lambda_zero_mean=1e-4, lambda_delta_edge=1e-4,
                entropy_floor=0.25 * float(np.log(M)), delta_edge_eps=0.05)


@pytest.mark.parametrize("M,K", [(2, 6), (8, 8), (4, 12)])
def test_bf16_input_equals_fp32_input(M, K):
    from scope_amd import ops

    g = torch.Generator().manual_seed(M * 100 + K)
    L, H = 512, 2
    y = (torch.randn((1, H, L, 5 * M + 1), generator=g) * 2).to(torch.bfloat16).to(DEV)
    om = torch.logspace(-4.5, -1.0, K).to(DEV)
    lo = om.log()
    cm, sm = torch.rand(K, generator=g).to(DEV) * 0.1, torch.rand(K, generator=g).to(DEV) * 0.1
    prm = _prm(M, K, L, True)
    a = ops.coeff_head_fwd(y, prm, om, lo, cm, sm)
    b = ops.coeff_head_fwd(y.float(), prm, om, lo, cm, sm)
    for n in NAMES + ["reg"]:
        assert torch.equal(a[n], b[n]), n
    grads = {n: torch.randn(a[n].shape, generator=g).to(DEV) for n in NAMES}
    gr = torch.tensor(0.7, device=DEV)
    da = ops.coeff_head_bwd(y, prm, om, lo, cm, sm, grads, gr, a["reg"])
    db = ops.coeff_head_bwd(y.float(), prm, om, lo, cm, sm, grads, gr, b["reg"])
    assert da.dtype == torch.bfloat16
    assert torch.equal(da, db.to(torch.bfloat16))


def test_fused_head_matches_torch_steps_at_training_shape():
    """T=65536, H=8, M=8, K=8 in bf16 (the module's MLP dtype follows q): the
    fused kernels against the oracle's torch steps with the same module's
    parameters on the same GPU.  The head's arithmetic is checked tightly on
    the fused MLP's own output y; the whole path against the torch MLP within
    what one bf16 ulp of y moves the outputs (the two MLPs round their bf16
    intermediates at different boundaries)."""
    from oracle.coeff_head import coeff_head_forward
    from scope_amd import SpectralBias, library

    torch.manual_seed(0)
    sb = SpectralBias(head_dim=128, num_heads=8, L_train=65536, M=8, K=8).to(DEV).train()
    with torch.no_grad():
        for p_ in sb.mlp.parameters():
            p_.normal_(0, 0.05)
    q = torch.randn((1, 8, 65536, 128), device=DEV).to(torch.bfloat16).requires_grad_()
    out_f = sb(q)
    q2 = q.detach().clone().requires_grad_()
    fc1, fc2 = sb.mlp[0], sb.mlp[2]
    with torch.no_grad():
        y_f = library.coeff_mlp(q2, fc1.weight, fc1.bias, fc2.weight, fc2.bias)
        out_h = coeff_head_forward(sb, q2, y=y_f)  # the oracle's head on the same y
    for i, n in enumerate(NAMES):
        a, b = out_f[i].float(), out_h[i].float()
        tol = 1e-4 * b.abs().max().item() + 1e-4 * b.abs()
        assert ((a - b).abs() <= tol).all(), f"{n}: max err {(a - b).abs().max().item():.3e}"
    out_t = coeff_head_forward(sb, q2)  # the oracle, on the same GPU
    for i, n in enumerate(NAMES):
        a, b = out_f[i].float(), out_t[i].float()
        tol = 2.0 ** -6 * b.abs().max().item() + 2.0 ** -6 * b.abs()
        assert ((a - b).abs() <= tol).all(), f"{n}: max err {(a - b).abs().max().item():.3e}"
    assert torch.allclose(out_f[11], out_t[11], rtol=1e-3), (float(out_f[11]), float(out_t[11]))
    g = torch.Generator(device=DEV).manual_seed(1)
    G = [torch.randn(out_f[i].shape, generator=g, device=DEV) for i in range(9)]
    lf = sum((out_f[i] * G[i]).sum() for i in range(9)) + 100.0 * out_f[11]
    lt = sum((out_t[i] * G[i]).sum() for i in range(9)) + 100.0 * out_t[11]
    gf, = torch.autograd.grad(lf, [q])
    gt, = torch.autograd.grad(lt, [q2])
    gf, gt = gf.float(), gt.float()
    # both run the MLP backward in bf16; the head's dy is rounded to bf16 in both
    err = (gf - gt).abs().max().item()
    assert err <= 2e-2 * gt.abs().max().item(), f"dq max err {err:.3e} vs max {gt.abs().max().item():.3e}"


def test_fused_head_ragged_rows():
    """600 rows (H=3, L=200: not a multiple of a forward workgroup's 128 rows,
    so its last passes hold no rows) with M=5 peaks (three of a row's eight
    lanes idle), training mode with the regularisers: the fused head against
    the oracle's torch steps on the same y (outputs, reg_loss, and dy of
    Σ⟨out, G⟩ + reg_loss)."""
    from oracle.coeff_head import coeff_head_forward
    from scope_amd import SpectralBias

    torch.manual_seed(3)
    H, L, M, K = 3, 200, 5, 6
    sb = SpectralBias(head_dim=128, num_heads=H, L_train=L, M=M, K=K).to(DEV).train()
    q = torch.randn((1, H, L, 128), device=DEV)
    y0 = torch.randn((1, H, L, 5 * M + 1), device=DEV) * 2
    y1, y2 = y0.clone().requires_grad_(), y0.clone().requires_grad_()
    sb._mlp_forward = lambda _q: y1  # the head alone, on the given y
    out_f = sb(q)
    out_t = coeff_head_forward(sb, q, y=y2)
    for i, n in enumerate(NAMES):
        a, b = out_f[i].float(), out_t[i].float()
        tol = 1e-4 * b.abs().max().item() + 1e-4 * b.abs()
        assert ((a - b).abs() <= tol).all(), f"{n}: max err {(a - b).abs().max().item():.3e}"
    assert torch.allclose(out_f[11], out_t[11], rtol=2e-4), (float(out_f[11]), float(out_t[11]))
    g = torch.Generator(device=DEV).manual_seed(4)
    G = [torch.randn(out_f[i].shape, generator=g, device=DEV) for i in range(9)]
    lf = sum((out_f[i] * G[i]).sum() for i in range(9)) + out_f[11]
    lt = sum((out_t[i] * G[i]).sum() for i in range(9)) + out_t[11]
    gf, = torch.autograd.grad(lf, [y1])
    gt, = torch.autograd.grad(lt, [y2])
    tol = 2e-4 * gt.abs().max().item() + 2e-4 * gt.abs()
    assert ((gf - gt).abs() <= tol).all(), f"dy max err {(gf - gt).abs().max().item():.3e}"


def test_disabled_forward_on_gpu():
    """enabled=False returns zeros and uniform π like the reference
    (model/attn_bias.py:411-417), on the GPU."""
    from scope_amd import SpectralBias

    sb = SpectralBias(head_dim=16, num_heads=2, L_train=64, M=3, enabled=False).to(DEV)
    out = sb(torch.randn(1, 2, 64, 16, device=DEV))
    assert len(out) == 12 and out[0].is_cuda
    assert all(torch.all(out[i] == 0) for i in (0, 1, 2, 3, 4, 6, 7, 8, 11))
    assert torch.allclose(out[5], torch.full_like(out[5], 1 / 3))

"""CPU: the host-side mirror of the reference interface — configuration
errors, schedule setters, the oracle's coefficient head against the
reference's golden vectors (the fused kernels are checked against the same
vectors on the GPU), the GPU-only forward, shape assertions, and the
BlockMask export logic."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pointer as P
from oracle.coeff_head import coeff_head_forward
from scope_amd import ScopeBlockMask, SpectralBias
from tests.golden import load_cases, load_flat


def test_config_errors_match_reference():
    kw = dict(head_dim=32, num_heads=2, L_train=128)
    with pytest.raises(ValueError, match="K must be positive"):
        SpectralBias(K=0, **kw)
    with pytest.raises(ValueError, match="M must be positive"):
        SpectralBias(M=0, **kw)
    with pytest.raises(ValueError, match="gate_kind"):
        SpectralBias(gate_kind="tanh", **kw)
    with pytest.raises(ValueError, match="pointer_radius_mode"):
        SpectralBias(pointer_radius_mode="budget", **kw)
    with pytest.raises(ValueError, match="pointer_qblock_rep"):
        SpectralBias(pointer_qblock_rep="first", **kw)
    with pytest.raises(ValueError, match="invalid"):
        SpectralBias(w_min=1.0, w_max=0.5, **kw)


def test_setters_clamp_and_validate():
    sb = SpectralBias(head_dim=32, num_heads=2, L_train=128, use_pointer_mask=True, pointer_half_blocks=3,
                      pointer_global_blocks=2)
    sb.set_pointer_mask_state(enabled=True, half_blocks=10, global_blocks=9)
    assert sb._pointer_half_blocks_active.item() == 3 and sb._st["half"] == 3
    assert sb._pointer_global_blocks_active.item() == 2 and sb._st["glob"] == 2
    with pytest.raises(ValueError):
        sb.set_pointer_mask_state(enabled=True, half_blocks=-1)
    with pytest.raises(ValueError):
        sb.set_pointer_reset_state(enabled=True, reset_len=-3)
    sb.set_pointer_reset_state(enabled=False, reset_len=50)
    assert sb._pointer_reset_len_active.item() == 0
    sb.set_delta_star_max_active(max_tokens=10 ** 9)
    assert sb._delta_star_max_active.item() == 127
    with pytest.raises(ValueError):
        sb.set_delta_edge_eps_active(eps=-1.0)
    sb.set_gumbel_seed(seed=77)
    assert sb._gumbel_seed.item() == 77 and sb._st["seed"] == 77


def test_coefficient_head_matches_reference_vectors():
    g = load_flat("coeff_head_vectors.npz")
    sb = SpectralBias(head_dim=int(g["Dh"]), num_heads=int(g["H"]), L_train=int(g["L_train"]), L_max=int(g["L_max"]),
                      M=int(g["M"]), K=int(g["K"]))
    with torch.no_grad():
        sb.mlp[0].weight.copy_(torch.from_numpy(g["w1"]))
        sb.mlp[0].bias.copy_(torch.from_numpy(g["b1"]))
        sb.mlp[2].weight.copy_(torch.from_numpy(g["w2"]))
        sb.mlp[2].bias.copy_(torch.from_numpy(g["b2"]))
    sb.eval()
    assert np.allclose(sb.omegas.numpy(), g["omegas"])
    out = coeff_head_forward(sb, torch.from_numpy(g["q"])[None])
    names = ["coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width"]
    for i, n in enumerate(names):
        ref = torch.from_numpy(g[n])
        assert torch.allclose(out[i][0], ref, rtol=1e-5, atol=1e-6), n


def test_oracle_disabled_head_returns_zeros_and_uniform_pi():
    sb = SpectralBias(head_dim=16, num_heads=2, L_train=64, M=3, enabled=False)
    out = coeff_head_forward(sb, torch.randn(1, 2, 64, 16))
    assert torch.all(out[0] == 0) and torch.allclose(out[5], torch.full_like(out[5], 1 / 3))


@pytest.mark.parametrize("enabled", [True, False])
def test_forward_has_no_cpu_path(enabled):
    sb = SpectralBias(head_dim=16, num_heads=2, L_train=64, M=3, enabled=enabled)
    with pytest.raises(RuntimeError, match="no CPU path"):
        sb(torch.randn(1, 2, 64, 16))


def test_build_pointer_blockmask_shape_assertions():
    sb = SpectralBias(head_dim=16, num_heads=2, L_train=256, M=2, use_pointer_mask=True)
    docs = torch.zeros(256, dtype=torch.long)
    x = torch.zeros(1, 2, 256, 2)
    with pytest.raises(AssertionError):
        sb.build_pointer_blockmask(docs=docs, input_seq=docs, delta_star=x, pi=x, budget_logits=x)
    with pytest.raises(AssertionError):
        sb.build_pointer_blockmask(docs=torch.zeros(200, dtype=torch.long), delta_star=x, pi=x, budget_logits=x)
    with pytest.raises(AssertionError):
        sb.build_pointer_blockmask(docs=docs, delta_star=torch.zeros(1, 3, 256, 2), pi=x, budget_logits=x)
    with pytest.raises(AssertionError):
        sb.build_pointer_blockmask(docs=docs, delta_star=torch.zeros(2, 2, 256, 2), pi=x, budget_logits=x)


def test_blockmask_export_matches_reference():
    """ScopeBlockMask.kv_indices_export / to_torch_blockmask (pure torch, CPU)
    reproduce the reference's NB-wide export and q lists."""
    cases = load_cases("pointer_ref_vectors.npz")
    from tests.golden import pointer_case_args, pointer_case_reps

    for name in ("c1_pi_single_doc", "export_truncation", "gumbel_multi_doc"):
        c = cases[name]
        a = pointer_case_args(c)
        dr, br = pointer_case_reps(c)
        out = P.pointer_mask_reference(dr, br, c["docs"], gumbel_u=c["gumbel_u"], **a)
        bs = int(c["bs"])
        docs = torch.from_numpy(c["docs"])
        bm = ScopeBlockMask(kv_num_blocks=torch.from_numpy(out["kv_num"])[None],
                            kv_indices=torch.from_numpy(out["packed"])[None], BLOCK_SIZE=bs, docs=docs,
                            ds_tok_end=torch.from_numpy(P.doc_start_blocks(c["docs"], bs)[2]))
        assert np.array_equal(bm.kv_indices_export().numpy(), c["kv_indices"])
        tbm = bm.to_torch_blockmask()
        assert np.array_equal(tbm.q_indices.numpy(), c["q_indices"])
        assert tbm.BLOCK_SIZE == (bs, bs)


def _coeff_train_run(g: dict, lams: dict, G=None):
    """The oracle's coefficient head in training mode on the recorded inputs:
    (outputs, reg_loss, grads of Σ<out_i, G_i> (if G), grads of reg_loss)."""
    sb = SpectralBias(head_dim=int(g["Dh"]), num_heads=int(g["H"]), L_train=int(g["L_train"]),
                      L_max=int(g["L_max"]), M=int(g["M"]), K=int(g["K"]),
                      pi_entropy_floor_frac=float(g["pi_entropy_floor_frac"]),
                      delta_edge_eps=float(g["delta_edge_eps"]), **lams)
    with torch.no_grad():
        sb.mlp[0].weight.copy_(torch.from_numpy(g["w1"]))
        sb.mlp[0].bias.copy_(torch.from_numpy(g["b1"]))
        sb.mlp[2].weight.copy_(torch.from_numpy(g["w2"]))
        sb.mlp[2].bias.copy_(torch.from_numpy(g["b2"]))
    sb.train()
    q = torch.from_numpy(g["q"])[None].clone().requires_grad_()
    out = coeff_head_forward(sb, q)
    params = [q, sb.mlp[0].weight, sb.mlp[0].bias, sb.mlp[2].weight, sb.mlp[2].bias]
    go = None
    if G is not None:
        lo = sum((out[i] * G[i]).sum() for i in range(len(G)))
        go = torch.autograd.grad(lo, params, retain_graph=True)
    gr = torch.autograd.grad(out[11], params, allow_unused=True)
    gr = [torch.zeros_like(p_) if x is None else x for x, p_ in zip(gr, params)]
    return out, out[11], go, gr


COEFF_NAMES = ["coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width"]
PARAM_NAMES = ("q", "w1", "b1", "w2", "b2")


def test_coefficient_head_training_regularisers_and_grads_match_reference():
    g = load_flat("coeff_head_train_vectors.npz")
    lam = {k: float(g[k]) for k in ("lambda_omega", "lambda_zero_mean", "lambda_entropy", "lambda_delta_edge")}
    G = [torch.from_numpy(g[f"G_{n}"])[None] for n in COEFF_NAMES]
    out, reg, go, gr = _coeff_train_run(g, lam, G)
    for i, n in enumerate(COEFF_NAMES):
        assert torch.allclose(out[i][0], torch.from_numpy(g[n]), rtol=1e-5, atol=1e-6), n
    assert np.isclose(reg.item(), g["reg_all"], rtol=1e-5, atol=1e-9)
    for n, x in zip(PARAM_NAMES, go):
        ref = torch.from_numpy(g[f"gout_{n}"])
        assert torch.allclose(x.reshape(ref.shape), ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item()), n
    for n, x in zip(PARAM_NAMES, gr):
        ref = torch.from_numpy(g[f"greg_all_{n}"])
        assert torch.allclose(x.reshape(ref.shape), ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item()), n
    # each regulariser alone
    for k in lam:
        tag = k.replace("lambda_", "")
        _, reg1, _, gr1 = _coeff_train_run(g, {**{k2: 0.0 for k2 in lam}, k: lam[k]})
        assert np.isclose(reg1.item(), g[f"reg_{tag}"], rtol=1e-5, atol=1e-9), tag
        assert abs(float(g[f"reg_{tag}"])) > 0, tag
        for n, x in zip(PARAM_NAMES, gr1):
            ref = torch.from_numpy(g[f"greg_{tag}_{n}"])
            assert torch.allclose(x.reshape(ref.shape), ref, rtol=1e-4, atol=1e-5 * max(ref.abs().max().item(), 1e-30)), (tag, n)


def test_pointer_arguments_outlive_their_temporaries_until_the_call_returns():
    """A copy made inside a call's argument list (``_p(_i32(x))``) stays
    referenced until ``call`` returns, also when the call fails; otherwise the
    caching allocator could give its memory to the next copy in the same
    list.  The call here fails its argument check in the library before any
    GPU work (a null pointer)."""
    import weakref

    from scope_amd import ScopeLibraryError, ops

    refs = []

    def copy(x):
        y = ops._i32(x)  # int64 -> a new int32 tensor
        refs.append(weakref.ref(y))
        return y

    x = torch.arange(8, dtype=torch.int64)
    with pytest.raises(ScopeLibraryError, match="null pointer"):
        ops.call("scope_transpose_blocks", ops._p(copy(x)), ops._p(copy(x)), 1, 2, 2, 4, None, None, None, None)
    assert all(r() is None for r in refs)  # released once the call returned
    p1, p2 = ops._p(copy(x)), ops._p(copy(x))
    assert all(r() is not None for r in refs[2:]) and p1.value != p2.value  # held, so not reused
    ops._held.ts.clear()

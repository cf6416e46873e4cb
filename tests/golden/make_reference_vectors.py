"""Write golden input/output vectors for the SCOPE pointer mask and its debug
statistics by running the reference's own Python module on the CPU.

This script is the only place that imports the reference, and it runs only in
the build container (the reference tree is not present where the GPU tests
run). It writes small compressed ``.npz`` fixtures next to itself; the tests
load those fixtures and never import the reference.

What is pinned here, and why an import is needed for it:

* ``SpectralBias.build_pointer_blockmask`` end to end
  (reference ``model/attn_bias.py:623-873``): the stick-breaking radius
  allocation with largest-remainder rounding, the Gumbel top-k over peaks,
  the three pieces, sort/dedupe/pack and the NB-wide export.  Invariants
  and brute force pin parts of it; only the reference pins the composition.
* its debug statistics (``:839-849``) and the forward debug statistics
  (``:510-606``).
* the coefficient head of ``SpectralBias.forward`` (``:379-478``), used to pin
  the host-side restatement of the coefficient head and the fused kernel; in
  training mode also its regularisers (``:480-506``) and the gradients of the
  head (through autograd) w.r.t. q and the MLP weights.

Usage (build container only)::

    python tests/golden/make_reference_vectors.py [/path/to/reference]
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load_reference(ref_root: str):
    sys.path.insert(0, ref_root)
    from model.attn_bias import SpectralBias  # noqa: E402  (reference module)

    return SpectralBias


def _docs_multi(T: int, n_docs: int, gen: torch.Generator) -> torch.Tensor:
    """Document ids (non-decreasing) with boundaries at random tokens,
    including boundaries that fall inside a block."""
    cuts = torch.randperm(T - 1, generator=gen)[: n_docs - 1] + 1
    flag = torch.zeros(T, dtype=torch.int64)
    flag[cuts] = 1
    return flag.cumsum(0)


def _rep_values(H: int, NB: int, M: int, bs: int, T: int, gen: torch.Generator) -> torch.Tensor:
    """Representative Δ* values that exercise every branch of the centre
    computation: far pointers, pointers before token 0, near pointers,
    exact block multiples and exact representative offsets."""
    qb = torch.arange(NB, dtype=torch.float32).view(1, NB, 1)
    t_rep = (qb + 1) * bs - 1
    u = torch.rand((H, NB, M), generator=gen)
    far = u * (t_rep + 2 * bs)  # can exceed t_rep -> clamped to 0
    near = torch.rand((H, NB, M), generator=gen) * (3 * bs)
    exact_blk = torch.randint(0, 6, (H, NB, M), generator=gen).float() * bs
    exact_rep = t_rep.expand(H, NB, M).clone()
    sel = torch.randint(0, 8, (H, NB, M), generator=gen)
    out = torch.where(sel < 4, far, torch.where(sel < 6, near, torch.where(sel < 7, exact_blk, exact_rep)))
    return out.float()


def _full_from_rep(rep: torch.Tensor, T: int, bs: int, fill: torch.Tensor | None = None) -> torch.Tensor:
    H, NB, M = rep.shape
    full = torch.zeros((1, H, T, M), dtype=torch.float32) if fill is None else fill.clone()
    t_rep = (torch.arange(NB) + 1) * bs - 1
    full[0, :, t_rep, :] = rep
    return full


def pointer_case(SpectralBias, name: str, *, H: int, T: int, bs: int, M: int, seed: int,
                 n_docs: int = 1, rep_mode: str = "last", training: bool = False,
                 setters: dict | None = None, build_kwargs: dict | None = None, **cfg) -> dict:
    gen = torch.Generator().manual_seed(seed)
    NB = T // bs
    docs = torch.zeros(T, dtype=torch.int64) if n_docs <= 1 else _docs_multi(T, n_docs, gen)
    if rep_mode == "last":
        delta_rep = _rep_values(H, NB, M, bs, T, gen)
        budget_rep = (torch.randn((H, NB, M), generator=gen) * 1.5).float()
        pi_rep = torch.softmax(torch.randn((H, NB, M), generator=gen), dim=-1)
        delta_star = _full_from_rep(delta_rep, T, bs)
        budget_logits = _full_from_rep(budget_rep, T, bs)
        pi = _full_from_rep(pi_rep, T, bs, fill=torch.full((1, H, T, M), 1.0 / M))
    else:
        delta_star = (torch.rand((1, H, T, M), generator=gen) * T).float()
        budget_logits = (torch.randn((1, H, T, M), generator=gen) * 1.5).float()
        pi = torch.softmax(torch.randn((1, H, T, M), generator=gen), dim=-1)

    sb = SpectralBias(head_dim=32, num_heads=H, L_train=T, M=M, K=6, use_pointer_mask=True,
                      pointer_qblock_rep=rep_mode, debug_stats=True, **cfg)
    sb.train(training)
    setters = setters or {}
    if "mask" in setters:
        sb.set_pointer_mask_state(**setters["mask"])
    if "reset" in setters:
        sb.set_pointer_reset_state(**setters["reset"])
    if "seed" in setters:
        sb.set_gumbel_seed(seed=setters["seed"])
    build_kwargs = build_kwargs or {}
    bm = sb.build_pointer_blockmask(docs=docs, delta_star=delta_star, pi=pi, budget_logits=budget_logits,
                                    block_size=bs, **build_kwargs)
    gseed = int(sb._gumbel_seed.item())
    ggen = torch.Generator().manual_seed(gseed)
    gumbel_u = torch.rand((H, NB, M), generator=ggen, dtype=torch.float32)

    rec = dict(
        H=H, T=T, bs=bs, M=M, rep_mode=rep_mode, training=int(training),
        docs=docs.numpy().astype(np.int32),
        gumbel_u=gumbel_u.numpy(),
        kv_num_blocks=bm.kv_num_blocks.numpy(), kv_indices=bm.kv_indices.numpy(),
        q_num_blocks=bm.q_num_blocks.numpy(), q_indices=bm.q_indices.numpy(),
        dbg_kv_unique_hist=sb._dbg_kv_unique_hist.numpy(),
        dbg_ptr_radius_hist=sb._dbg_ptr_radius_hist.numpy(),
        dbg_ptr_extra_sum_hist=sb._dbg_ptr_extra_sum_hist.numpy(),
        dbg_ptr_radius0_frac=sb._dbg_ptr_radius0_frac.numpy(),
    )
    if rep_mode == "last":
        rec.update(delta_rep=delta_rep.numpy(), budget_rep=budget_rep.numpy())
    else:
        rec.update(delta_star=delta_star[0].numpy(), budget_logits=budget_logits[0].numpy())
    # configuration, as the reference saw it after its own normalisation
    conf = dict(
        pointer_local_blocks=sb.pointer_local_blocks, pointer_half_blocks=sb.pointer_half_blocks,
        pointer_global_blocks=sb.pointer_global_blocks, pointer_budget_blocks=sb.pointer_budget_blocks,
        pointer_budget_is_total=int(sb.pointer_budget_is_total), pointer_budget_temp=sb.pointer_budget_temp,
        pointer_radius_mode=sb.pointer_radius_mode, pointer_doc_clamp=int(sb.pointer_doc_clamp),
        gumbel_topk=int(sb.gumbel_topk), gumbel_topk_k=sb.gumbel_topk_k, gumbel_topk_tau=sb.gumbel_topk_tau,
        eps=sb.eps,
        mask_active=int(sb._pointer_mask_active.item()),
        half_active=int(sb._pointer_half_blocks_active.item()),
        global_active=int(sb._pointer_global_blocks_active.item()),
        reset_active=int(sb._pointer_reset_active.item()),
        reset_len_active=int(sb._pointer_reset_len_active.item()),
        gumbel_seed=gseed,
        build_local_blocks=build_kwargs.get("local_blocks", -1) if build_kwargs.get("local_blocks") is not None else -1,
        build_ptr_half_blocks=build_kwargs.get("ptr_half_blocks", -1) if build_kwargs.get("ptr_half_blocks") is not None else -1,
        build_budget_blocks=build_kwargs.get("pointer_budget_blocks", -1) if build_kwargs.get("pointer_budget_blocks") is not None else -1,
        build_global_blocks=build_kwargs.get("global_blocks", -1) if build_kwargs.get("global_blocks") is not None else -1,
    )
    for k_, v_ in conf.items():
        rec["cfg_" + k_] = np.asarray(v_)
    rec["name"] = np.asarray(name)
    return rec


def forward_case(SpectralBias, name: str, *, H: int, T: int, M: int, K: int, seed: int, n_docs: int,
                 rep_mode: str = "last", with_docs: bool = True, reset: dict | None = None,
                 training: bool = True, **cfg) -> dict:
    gen = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    Dh = 32
    sb = SpectralBias(head_dim=Dh, num_heads=H, L_train=T // 2, L_max=4 * T, M=M, K=K, debug_stats=True,
                      pointer_qblock_rep=rep_mode, **cfg)
    # non-trivial output head so Δ*, π, budget carry signal (reference init zeroes it)
    with torch.no_grad():
        for p in sb.mlp.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.3)
    sb.train(training)
    if reset:
        sb.set_pointer_reset_state(**reset)
    docs = torch.zeros(T, dtype=torch.int64) if n_docs <= 1 else _docs_multi(T, n_docs, gen)
    q = torch.randn((1, H, T, Dh), generator=gen, dtype=torch.float32)
    out = sb(q, docs=docs if with_docs else None)
    (coeff_cos, coeff_sin, slope, b0, delta_star, pi, budget_logits, delta_main, width, cos_wD, sin_wD, reg) = out
    def _np(t):
        return t.detach().numpy()

    rec = dict(
        H=H, T=T, M=M, K=K, rep_mode=rep_mode, with_docs=int(with_docs), training=int(training),
        docs=docs.numpy().astype(np.int32),
        delta_star=delta_star[0].detach().numpy(), pi=pi[0].detach().numpy(),
        dbg_delta_tokens_hist=_np(sb._dbg_delta_tokens_hist),
        dbg_delta_blocks_hist=_np(sb._dbg_delta_blocks_hist),
        dbg_ptr_center_hist=_np(sb._dbg_ptr_center_hist),
        dbg_ptr_outside_local_frac=_np(sb._dbg_ptr_outside_local_frac),
        dbg_ptr_block0_frac=_np(sb._dbg_ptr_block0_frac),
        dbg_ptr_block0_frac_excl=_np(sb._dbg_ptr_block0_frac_excl),
        dbg_ptr_docstart_frac=_np(sb._dbg_ptr_docstart_frac),
        dbg_pi_entropy_mean=_np(sb._dbg_pi_entropy_mean),
        cfg_pointer_local_blocks=np.asarray(sb.pointer_local_blocks),
        cfg_pointer_doc_clamp=np.asarray(int(sb.pointer_doc_clamp)),
        cfg_reset_active=np.asarray(int(sb._pointer_reset_active.item())),
        cfg_reset_len_active=np.asarray(int(sb._pointer_reset_len_active.item())),
        cfg_eps=np.asarray(sb.eps),
        name=np.asarray(name),
    )
    return rec


def coeff_case(SpectralBias, *, seed: int = 5) -> dict:
    """Coefficient head outputs for a random-weight MLP (fp32 q, so the
    reference MLP runs in fp32)."""
    gen = torch.Generator().manual_seed(seed)
    H, T, Dh, M, K = 2, 256, 32, 3, 6
    sb = SpectralBias(head_dim=Dh, num_heads=H, L_train=128, L_max=4096, M=M, K=K)
    with torch.no_grad():
        for p in sb.mlp.parameters():
            p.copy_(torch.randn(p.shape, generator=gen) * 0.3)
    sb.eval()
    q = torch.randn((1, H, T, Dh), generator=gen, dtype=torch.float32)
    out = sb(q)
    names = ["coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width"]
    rec = {n: out[i][0].detach().numpy() for i, n in enumerate(names)}
    rec.update(q=q[0].numpy(), H=H, T=T, Dh=Dh, M=M, K=K, L_train=128, L_max=4096,
               w1=sb.mlp[0].weight.detach().numpy(), b1=sb.mlp[0].bias.detach().numpy(),
               w2=sb.mlp[2].weight.detach().numpy(), b2=sb.mlp[2].bias.detach().numpy(),
               omegas=sb.omegas.numpy())
    return rec


def coeff_train_case(SpectralBias, *, seed: int = 6) -> dict:
    """Training-mode coefficient head: outputs, reg_loss with every
    regulariser on and with each one alone, and the gradients w.r.t. q and
    the MLP weights of (a) Σ_i <out_i, G_i> for random G_i and (b) reg_loss.
    The lambdas are raised above their defaults so that each term carries
    weight in the gradient."""
    gen = torch.Generator().manual_seed(seed)
    H, T, Dh, M, K = 2, 256, 32, 3, 6
    lam = dict(lambda_omega=1e-2, lambda_zero_mean=1e-1, lambda_entropy=1e-1, lambda_delta_edge=1e-1)
    base = dict(head_dim=Dh, num_heads=H, L_train=128, L_max=4096, M=M, K=K, pi_entropy_floor_frac=0.9,
                delta_edge_eps=0.2)
    sb = SpectralBias(**base, **lam)
    with torch.no_grad():
        for p_ in sb.mlp.parameters():
            p_.copy_(torch.randn(p_.shape, generator=gen) * 0.3)
    weights = {n: p_.detach().clone() for n, p_ in sb.mlp.named_parameters()}
    q0 = torch.randn((1, H, T, Dh), generator=gen, dtype=torch.float32)
    names = ["coeff_cos", "coeff_sin", "slope", "b0", "delta_star", "pi", "budget_logits", "delta_main", "width"]
    rec = dict(q=q0[0].numpy(), H=H, T=T, Dh=Dh, M=M, K=K, L_train=128, L_max=4096, pi_entropy_floor_frac=0.9,
               delta_edge_eps=0.2, omegas=sb.omegas.numpy(), **{k: np.asarray(v) for k, v in lam.items()},
               w1=weights["0.weight"].numpy(), b1=weights["0.bias"].numpy(), w2=weights["2.weight"].numpy(),
               b2=weights["2.bias"].numpy())

    def run(lams: dict, tag: str, with_outputs: bool):
        m = SpectralBias(**base, **lams)
        with torch.no_grad():
            for n, p_ in m.mlp.named_parameters():
                p_.copy_(weights[n])
        m.train()
        q = q0.clone().requires_grad_()
        out = m(q)
        params = [q] + [p_ for _, p_ in m.mlp.named_parameters()]
        if with_outputs:
            for i, n in enumerate(names):
                rec[n] = out[i][0].detach().numpy()
            G = [torch.randn(out[i].shape, generator=gen) for i in range(len(names))]
            rec.update({f"G_{n}": G[i][0].numpy() for i, n in enumerate(names)})
            lo = sum((out[i] * G[i]).sum() for i in range(len(names)))
            go = torch.autograd.grad(lo, params, retain_graph=True)
            rec.update({f"gout_{n}": g_.numpy() for n, g_ in zip(("q", "w1", "b1", "w2", "b2"), go)})
        reg = out[11]
        rec[f"reg_{tag}"] = reg.detach().numpy()
        gr = torch.autograd.grad(reg, params, allow_unused=True)
        rec.update({f"greg_{tag}_{n}": (np.zeros(p_.shape, np.float32) if g_ is None else g_.numpy())
                    for n, g_, p_ in zip(("q", "w1", "b1", "w2", "b2"), gr, params)})

    run(lam, "all", True)
    zero = {k: 0.0 for k in lam}
    for k in lam:
        run({**zero, k: lam[k]}, k.replace("lambda_", ""), False)
    return rec


def main() -> None:
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    SpectralBias = _load_reference(ref_root)
    torch.set_num_threads(1)

    cases = [
        # C1-shaped: H=6, T=4096, bs=128, one document, radius from π and the budget
        pointer_case(SpectralBias, "c1_pi_single_doc", H=6, T=4096, bs=128, M=4, seed=1,
                     pointer_local_blocks=3, pointer_half_blocks=2, pointer_global_blocks=1,
                     pointer_budget_blocks=12, pointer_budget_temp=1.0),
        pointer_case(SpectralBias, "gumbel_multi_doc", H=4, T=4096, bs=128, M=8, seed=2, n_docs=9,
                     training=True, setters={"seed": 1234},
                     pointer_local_blocks=4, pointer_half_blocks=4, pointer_global_blocks=2,
                     pointer_budget_blocks=40, pointer_budget_temp=0.5,
                     gumbel_topk=True, gumbel_topk_k=3, gumbel_topk_tau=1.0),
        pointer_case(SpectralBias, "fixed_radius_schedule", H=3, T=2048, bs=128, M=3, seed=3, n_docs=4,
                     setters={"mask": dict(enabled=True, half_blocks=1, global_blocks=1)},
                     pointer_radius_mode="fixed", pointer_local_blocks=2, pointer_half_blocks=3,
                     pointer_global_blocks=2),
        pointer_case(SpectralBias, "reset_segments", H=2, T=4096, bs=256, M=4, seed=4, n_docs=3,
                     setters={"reset": dict(enabled=True, reset_len=700)},
                     pointer_local_blocks=2, pointer_half_blocks=2, pointer_global_blocks=2,
                     pointer_budget_blocks=14, pointer_budget_temp=1.0),
        pointer_case(SpectralBias, "rep_mean", H=2, T=1024, bs=128, M=4, seed=5, rep_mode="mean", n_docs=2,
                     pointer_local_blocks=2, pointer_half_blocks=2, pointer_global_blocks=1,
                     pointer_budget_blocks=10),
        pointer_case(SpectralBias, "no_extra_budget_p0", H=2, T=2048, bs=128, M=4, seed=6, n_docs=3,
                     pointer_local_blocks=3, pointer_half_blocks=0, pointer_global_blocks=1,
                     pointer_budget_blocks=3),
        pointer_case(SpectralBias, "pointer_disabled", H=2, T=2048, bs=128, M=2, seed=7, n_docs=2,
                     setters={"mask": dict(enabled=False, half_blocks=0)},
                     pointer_local_blocks=3, pointer_half_blocks=2, pointer_global_blocks=1,
                     pointer_budget_blocks=9),
        pointer_case(SpectralBias, "extra_budget_no_doc_clamp", H=2, T=2048, bs=128, M=3, seed=8, n_docs=5,
                     pointer_local_blocks=2, pointer_half_blocks=2, pointer_global_blocks=1,
                     pointer_budget_blocks=5, pointer_budget_is_total=False, pointer_doc_clamp=False),
        pointer_case(SpectralBias, "export_truncation", H=2, T=1024, bs=128, M=2, seed=9, n_docs=2,
                     pointer_local_blocks=4, pointer_half_blocks=2, pointer_global_blocks=1,
                     pointer_budget_blocks=20),
        pointer_case(SpectralBias, "build_overrides", H=2, T=2048, bs=128, M=3, seed=10, n_docs=2,
                     build_kwargs=dict(local_blocks=2, ptr_half_blocks=1, pointer_budget_blocks=8, global_blocks=1),
                     pointer_local_blocks=4, pointer_half_blocks=3, pointer_global_blocks=2,
                     pointer_budget_blocks=30),
    ]
    np.savez_compressed(os.path.join(HERE, "pointer_ref_vectors.npz"),
                        **{f"{c['name']}__{k}": v for c in cases for k, v in c.items()})

    fcases = [
        forward_case(SpectralBias, "fwd_docs_last", H=2, T=1024, M=4, K=6, seed=11, n_docs=3,
                     pointer_local_blocks=3),
        forward_case(SpectralBias, "fwd_nodocs_mean", H=2, T=1024, M=4, K=6, seed=12, n_docs=1,
                     rep_mode="mean", with_docs=False, pointer_local_blocks=2),
        forward_case(SpectralBias, "fwd_reset_noclamp", H=2, T=1024, M=3, K=6, seed=13, n_docs=4,
                     reset=dict(enabled=True, reset_len=300), pointer_doc_clamp=False, pointer_local_blocks=2),
    ]
    np.savez_compressed(os.path.join(HERE, "forward_stats_vectors.npz"),
                        **{f"{c['name']}__{k}": v for c in fcases for k, v in c.items()})

    np.savez_compressed(os.path.join(HERE, "coeff_head_vectors.npz"), **coeff_case(SpectralBias))
    np.savez_compressed(os.path.join(HERE, "coeff_head_train_vectors.npz"), **coeff_train_case(SpectralBias))
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()

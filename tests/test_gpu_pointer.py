"""GPU parity of kernel 1 (pointer selection), the q-list transpose and
kernel 3 (statistics) against the reference's golden vectors and the oracle.
Bar: bit-exact for every index list and integer statistic."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pointer as OP
from oracle import stats as OS
from tests.golden import load_cases
from tests.helpers import docs_with_boundaries, qkv

pytestmark = pytest.mark.gpu

POINTER_CASES = load_cases("pointer_ref_vectors.npz")
FORWARD_CASES = load_cases("forward_stats_vectors.npz")
DEV = "cuda"


def _full(rep: np.ndarray, T: int, bs: int) -> torch.Tensor:
    H, NB, M = rep.shape
    full = torch.zeros((1, H, T, M), dtype=torch.float32)
    t_rep = (torch.arange(NB) + 1) * bs - 1
    full[0, :, t_rep, :] = torch.from_numpy(rep)
    return full


def _spectral_bias_for(c: dict):
    from scope_amd import SpectralBias

    sb = SpectralBias(head_dim=32, num_heads=int(c["H"]), L_train=int(c["T"]), M=int(c["M"]), K=6,
                      use_pointer_mask=True, pointer_qblock_rep=str(c["rep_mode"]), debug_stats=True,
                      pointer_local_blocks=int(c["cfg_pointer_local_blocks"]),
                      pointer_half_blocks=int(c["cfg_pointer_half_blocks"]),
                      pointer_global_blocks=int(c["cfg_pointer_global_blocks"]),
                      pointer_budget_blocks=int(c["cfg_pointer_budget_blocks"]),
                      pointer_budget_is_total=bool(c["cfg_pointer_budget_is_total"]),
                      pointer_budget_temp=float(c["cfg_pointer_budget_temp"]),
                      pointer_radius_mode=str(c["cfg_pointer_radius_mode"]),
                      pointer_doc_clamp=bool(c["cfg_pointer_doc_clamp"]), gumbel_topk=bool(c["cfg_gumbel_topk"]),
                      gumbel_topk_k=int(c["cfg_gumbel_topk_k"]), gumbel_topk_tau=float(c["cfg_gumbel_topk_tau"]))
    sb.set_pointer_mask_state(enabled=bool(c["cfg_mask_active"]), half_blocks=int(c["cfg_half_active"]),
                              global_blocks=int(c["cfg_global_active"]))
    sb.set_pointer_reset_state(enabled=bool(c["cfg_reset_active"]), reset_len=int(c["cfg_reset_len_active"]))
    sb.set_gumbel_seed(seed=int(c["cfg_gumbel_seed"]))
    sb.train(bool(c["training"]))
    return sb.to(DEV)


@pytest.mark.parametrize("name", sorted(POINTER_CASES))
def test_build_pointer_blockmask_matches_reference_vectors(name):
    """SpectralBias.build_pointer_blockmask on the GPU vs the reference's own
    outputs (kv lists, NB-wide export, q lists, debug statistics)."""
    c = POINTER_CASES[name]
    T, bs, M, H = int(c["T"]), int(c["bs"]), int(c["M"]), int(c["H"])
    print(f"case {name}: H={H} T={T} bs={bs} M={M}", flush=True)
    sb = _spectral_bias_for(c)
    if c["rep_mode"] == "last":
        delta_star = _full(c["delta_rep"], T, bs)
        budget = _full(c["budget_rep"], T, bs)
    else:
        delta_star = torch.from_numpy(c["delta_star"])[None]
        budget = torch.from_numpy(c["budget_logits"])[None]
    pi = torch.full_like(delta_star, 1.0 / M)
    kw = {}
    for key, arg in (("cfg_build_local_blocks", "local_blocks"), ("cfg_build_ptr_half_blocks", "ptr_half_blocks"),
                     ("cfg_build_budget_blocks", "pointer_budget_blocks"),
                     ("cfg_build_global_blocks", "global_blocks")):
        if int(c[key]) >= 0:
            kw[arg] = int(c[key])
    bm = sb.build_pointer_blockmask(docs=torch.from_numpy(c["docs"]).long().to(DEV), delta_star=delta_star.to(DEV),
                                    pi=pi.to(DEV), budget_logits=budget.to(DEV), block_size=bs,
                                    gumbel_u=torch.from_numpy(c["gumbel_u"]).to(DEV), **kw)
    torch.cuda.synchronize()
    assert np.array_equal(bm.kv_num_blocks.cpu().numpy(), c["kv_num_blocks"])
    assert np.array_equal(bm.kv_indices_export().cpu().numpy(), c["kv_indices"])
    tbm = bm.to_torch_blockmask()
    assert np.array_equal(tbm.q_num_blocks.cpu().numpy(), c["q_num_blocks"])
    assert np.array_equal(tbm.q_indices.cpu().numpy(), c["q_indices"])
    for key in ("kv_unique_hist", "ptr_radius_hist", "ptr_extra_sum_hist"):
        assert np.array_equal(getattr(sb, "_dbg_" + key).cpu().numpy(), c["dbg_" + key]), key
    assert sb._dbg_ptr_radius0_frac.item() == float(c["dbg_ptr_radius0_frac"])


@pytest.mark.parametrize("seed,H,T,bs,M,n_docs", [(0, 8, 65536, 128, 8, 1), (1, 8, 131072, 256, 8, 16),
                                                  (2, 6, 4096, 128, 4, 5)])
def test_pointer_mask_ref_vs_oracle_large(seed, H, T, bs, M, n_docs):
    """Reference mode at training shapes (T up to 128k) vs the oracle."""
    from scope_amd import ops

    print(f"ref-mode seed={seed} H={H} T={T} bs={bs} M={M}", flush=True)
    rng = np.random.default_rng(seed)
    NB = T // bs
    docs = docs_with_boundaries(T, n_docs, seed)
    t_rep = (np.arange(NB) + 1) * bs - 1
    delta_rep = (rng.random((H, NB, M)) * (t_rep[None, :, None] + bs)).astype(np.float32)
    budget_rep = (rng.standard_normal((H, NB, M)) * 1.5).astype(np.float32)
    u = rng.random((H, NB, M)).astype(np.float32)
    budget_blocks = 4 + M + 18
    rem = OP.budget_rem_blocks(M=M, local_blocks=4, ptr_half_blocks=3, budget_blocks=budget_blocks,
                               budget_is_total=True)
    ref = OP.pointer_mask_reference(delta_rep, budget_rep, docs.numpy(), bs=bs, M=M, local_blocks=4,
                                    ptr_half_blocks=3, global_blocks_cfg=2, global_active=2,
                                    budget_blocks=budget_blocks, budget_is_total=True, budget_temp=0.5,
                                    radius_mode="pi", doc_clamp=True, mask_active=True, half_active=3,
                                    gumbel_active=True, gumbel_k=M // 2, gumbel_tau=1.0, gumbel_u=u)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    kv_num, kv_idx, radius, centre = ops.pointer_mask_ref(
        _full(delta_rep, T, bs).to(DEV), _full(budget_rep, T, bs).to(DEV), ds_ptr, ds_local, bs=bs,
        local_blocks=4, ptr_half_blocks=3, global_blocks_cfg=2, global_active=2, radius_mode="pi",
        budget_rem=rem, budget_temp=0.5, mask_active=True, half_active=3, gumbel_k=M // 2, gumbel_tau=1.0,
        gumbel_u=torch.from_numpy(u).to(DEV))
    assert np.array_equal(radius.cpu().numpy(), ref["radius"])
    assert np.array_equal(centre.cpu().numpy(), ref["centre"])
    assert np.array_equal(kv_num.cpu().numpy(), ref["kv_num"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])


def test_doc_starts_vs_oracle():
    from scope_amd import ops

    for T, bs, n_docs, clamp, reset in ((4096, 128, 7, True, 0), (131072, 256, 16, True, 0),
                                        (8192, 128, 40, False, 0), (8192, 256, 9, True, 1000)):
        docs = docs_with_boundaries(T, n_docs, T + n_docs)
        got = [x.cpu().numpy() for x in ops.doc_starts(docs.to(DEV), bs, doc_clamp=clamp, reset_len=reset)]
        ref = OP.doc_start_blocks(docs.numpy(), bs, doc_clamp=clamp, reset_active=reset > 0, reset_len=reset)
        for g, r in zip(got, ref):
            assert np.array_equal(g, r), (T, bs, n_docs, clamp, reset)


# ---------------------------------------------------------------------------
# block-scoring mode
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("H,T,bs,W,G,B,n_docs,ninf", [
    (6, 4096, 128, 3, 1, 2, 1, 0), (8, 65536, 128, 4, 1, 4, 1, 0), (8, 131072, 256, 2, 2, 8, 16, 0),
    (2, 8192, 256, 2, 2, 16, 5, 0),
    # edges: a window as wide as the sequence, no pointer budget, one block, a
    # document per block, and half of the logits -inf (rows with fewer finite
    # candidates than the budget pick -inf ones in block order)
    (2, 1024, 128, 8, 2, 3, 2, 0), (2, 2048, 128, 2, 1, 0, 3, 0), (1, 128, 128, 2, 1, 2, 1, 0),
    (2, 4096, 128, 2, 2, 4, 32, 0), (4, 8192, 128, 2, 1, 6, 3, 1)])
def test_pointer_select_given_logits_exact(H, T, bs, W, G, B, n_docs, ninf):
    """Selection given the same fp32 logits (with ties) is bit-exact."""
    from scope_amd import ops

    print(f"select H={H} T={T} bs={bs} W={W} G={G} B={B} docs={n_docs} -inf={ninf}", flush=True)
    NB = T // bs
    rng = np.random.default_rng(T + B)
    logits = (np.round(rng.standard_normal((H, NB, NB)) * 4) / 4).astype(np.float32)  # many ties
    if ninf:
        logits[rng.random((H, NB, NB)) < 0.5] = -np.inf
    docs = docs_with_boundaries(T, n_docs, 3)
    ref = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=W, n_global=G, budget=B, temp=0.5)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    kv_num, kv_idx, picks = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=W, n_global=G, budget=B,
                                               logits_in=torch.from_numpy(logits).to(DEV), temp=0.5)
    assert np.array_equal(picks.cpu().numpy(), ref["picks"])
    assert np.array_equal(kv_num.cpu().numpy(), ref["kv_num"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])


@pytest.mark.parametrize("noise", ["uniform", "counter"])
def test_pointer_select_gumbel_exact(noise):
    from scope_amd import ops

    H, T, bs, W, G, B = 4, 16384, 128, 4, 1, 4
    NB = T // bs
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    docs = docs_with_boundaries(T, 3, 11)
    seed = 0x1234_5678_9ABC
    if noise == "uniform":
        u = rng.random((H, NB, NB)).astype(np.float32)
    else:
        hh, qq, kk = np.meshgrid(np.arange(H), np.arange(NB), np.arange(NB), indexing="ij")
        u = OP.counter_uniform(seed, hh, qq, kk)
    g = OP.gumbel_from_u(u)
    ref = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=W, n_global=G, budget=B, gumbel=g)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    kv_num, kv_idx, picks = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=W, n_global=G, budget=B,
                                               logits_in=torch.from_numpy(logits).to(DEV), noise=noise,
                                               gumbel_u=torch.from_numpy(u).to(DEV) if noise == "uniform" else None,
                                               seed=seed)
    assert np.array_equal(picks.cpu().numpy(), ref["picks"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])


@pytest.mark.parametrize("H,T,bs", [(6, 4096, 128), (8, 131072, 256), (4, 131072, 128), (2, 140800, 128)])
def test_block_means_and_logits(H, T, bs):
    """Fused block means + q̄·k̄ logits vs fp64; selection exact given the kernel's logits.
    From 1024 blocks on (the last two cases; 1100 blocks is no multiple of the
    64-block tiles) the logits come from the bf16 MFMA product of the split means."""
    from scope_amd import ops

    q, k, _ = qkv(H, T, seed=5)
    NB = T // bs
    docs = docs_with_boundaries(T, 4, 2)
    qbar, kbar = ops.block_means(q.to(DEV), k.to(DEV), bs)
    rq = OP.block_means(q[0].double().numpy(), bs)
    rk = OP.block_means(k[0].double().numpy(), bs)
    assert np.abs(qbar.cpu().numpy() - rq).max() < 1e-6
    assert np.abs(kbar.cpu().numpy() - rk).max() < 1e-6
    prior = (-0.05 * np.log1p(np.arange(NB))).astype(np.float32)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    scale = bs / np.sqrt(128.0)
    kv_num, kv_idx, picks, lg = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=2, n_global=1,
                                                   budget=4, qbar=qbar, kbar=kbar, prior=torch.from_numpy(prior).to(DEV),
                                                   logit_scale=scale, return_logits=True)
    lg = lg.cpu().numpy()
    ref_lg = OP.pointer_logits(rq, rk, logit_scale=scale, prior=prior)
    ds = ds_ptr.cpu().numpy()
    causal = (np.arange(NB)[None, :] <= np.arange(NB)[:, None]) & (np.arange(NB)[None, :] >= ds[:, None])
    diff = np.abs(lg - ref_lg)[:, causal]
    rel = (diff / (1 + np.abs(ref_lg[:, causal]))).max()
    print(f"  NB={NB}: logits within {rel:.3g}·(1 + |ref|) of fp64", flush=True)
    assert rel < 1e-4
    assert np.all(np.isneginf(lg[:, ~causal]))
    ref = OP.pointer_select_blockscore(lg, docs.numpy(), bs=bs, window=2, n_global=1, budget=4)
    assert np.array_equal(picks.cpu().numpy(), ref["picks"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])


@pytest.mark.parametrize("H,T,bs,budget,noise,n_docs", [(4, 131072, 128, 4, "counter", 3), (2, 140800, 128, 8, "counter", 1),
                                                         (2, 140800, 128, 2, "none", 5), (2, 262144, 256, 8, "uniform", 2),
                                                         (2, 140800, 128, 12, "counter", 2)])
def test_scratch_logits_selection_equals_logits_path(H, T, bs, budget, noise, n_docs):
    """From 1024 blocks on, a selection whose logits the caller does not read
    (SCOPE_PTR_LOGITS_SCRATCH: the buffer's non-candidate entries are left
    unset) must give the picks and lists of the call that returns the
    logits, and those must equal the oracle's selection on the returned
    logits, for every noise mode and budgets up to 12."""
    from scope_amd import ops

    q, k, _ = qkv(H, T, seed=11)
    NB = T // bs
    docs = docs_with_boundaries(T, n_docs, 3).to(DEV)
    qbar, kbar = ops.block_means(q.to(DEV), k.to(DEV), bs)
    ds_ptr, ds_local, _ = ops.doc_starts(docs, bs)
    prior = torch.from_numpy((-0.05 * np.log1p(np.arange(NB))).astype(np.float32)).to(DEV)
    gu = (torch.rand((H, NB, NB), generator=torch.Generator(device=DEV).manual_seed(4), device=DEV)
          if noise == "uniform" else None)
    kw = dict(bs=bs, NB=NB, H=H, window=2, n_global=1, budget=budget, qbar=qbar, kbar=kbar, prior=prior,
              logit_scale=bs / np.sqrt(128.0), noise=noise, gumbel_u=gu, seed=99)
    kn1, ki1, pk1 = ops.pointer_select(ds_ptr, ds_local, **kw)
    kn2, ki2, pk2, lg = ops.pointer_select(ds_ptr, ds_local, return_logits=True, **kw)
    torch.cuda.synchronize()
    print(f"  NB={NB} budget={budget} noise={noise}: {int(kn1.sum())} listed blocks", flush=True)
    assert torch.equal(pk1, pk2)
    assert torch.equal(kn1, kn2)
    assert torch.equal(ki1, ki2)
    # and the logits path against the oracle's selection on those logits (head 0)
    lg0 = lg[:1].cpu().numpy()
    g0 = None
    if noise == "counter":
        qq, kk = np.meshgrid(np.arange(NB), np.arange(NB), indexing="ij")
        g0 = OP.gumbel_from_u(OP.counter_uniform(99, np.zeros_like(qq), qq, kk))[None]
    elif noise == "uniform":
        g0 = OP.gumbel_from_u(gu[:1].cpu().numpy())
    ref = OP.pointer_select_blockscore(lg0, docs.cpu().numpy(), bs=bs, window=2, n_global=1, budget=budget, gumbel=g0)
    assert np.array_equal(pk2[:1].cpu().numpy(), ref["picks"])
    assert np.array_equal(ki2[:1].cpu().numpy(), ref["packed"])


def test_planted_needle_is_selected():
    """C3-style needle: a key block = 3 × a query block's mean query, ≥64
    blocks back; the noise-free selection must pick it for that q-block."""
    from scope_amd import ops

    H, T, bs = 2, 65536, 256
    NB = T // bs
    q, k, _ = qkv(H, T, seed=9)
    qb, kb = 200, 100
    mq = q[0, :, qb * bs:(qb + 1) * bs].float().mean(dim=1)  # [H,D]
    k[0, :, kb * bs:(kb + 1) * bs] = (3.0 * mq[:, None, :]).to(k.dtype)
    docs = torch.zeros(T, dtype=torch.int32)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    qbar, kbar = ops.block_means(q.to(DEV), k.to(DEV), bs)
    _, _, picks = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=2, n_global=2, budget=2,
                                     qbar=qbar, kbar=kbar, logit_scale=bs / np.sqrt(128.0))
    assert all(kb in picks[h, qb].tolist() for h in range(H))


# ---------------------------------------------------------------------------
# transpose and statistics
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("H,T,bs,W,G,B", [(2, 8192, 128, 3, 1, 2), (8, 131072, 256, 2, 2, 8)])
def test_transpose_blocks_vs_oracle(H, T, bs, W, G, B):
    from scope_amd import ops

    NB = T // bs
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    docs = docs_with_boundaries(T, 6, 1)
    sel = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=W, n_global=G, budget=B)
    q_num, q_off, q_list = OP.transpose_blocks(sel["kv_num"], sel["packed"], NB)
    got_off, got_list = ops.transpose_blocks(torch.from_numpy(sel["kv_num"]).to(DEV),
                                             torch.from_numpy(sel["packed"]).to(DEV), NB)
    got_off, got_list = got_off.cpu().numpy(), got_list.cpu().numpy()
    assert np.array_equal(got_off, q_off)
    for h in range(H):
        n = q_off[h, -1]
        assert np.array_equal(got_list[h, :n], q_list[h, :n])


@pytest.mark.parametrize("H,QB,maxkv,hot", [(2, 300, 7, 0), (3, 2000, 12, 2), (1, 4096, 5, 1)])
def test_transpose_blocks_long_buckets_and_repeats(H, QB, maxkv, hot):
    """The transpose straight through the C ABI (no list check) against a
    sort of each key block's q-blocks: buckets from 1 to QB entries (``hot``
    key blocks listed by every row, as a long document's global blocks are;
    the long ones are sorted by counting), entries outside the key blocks
    skipped, and rows that list a key block more than once keeping every
    repeat (the count, fill and sort treat list slots independently)."""
    from scope_amd import ops

    print(f"transpose H={H} QB={QB} maxkv={maxkv} hot={hot}", flush=True)
    NB = QB
    rng = np.random.default_rng(QB)
    kn = rng.integers(0, maxkv + 1, size=(H, QB)).astype(np.int32)
    ki = rng.integers(-3, NB + 3, size=(H, QB, maxkv)).astype(np.int32)  # a few outside [0, NB)
    ki[:, :, :hot] = np.arange(hot, dtype=np.int32)  # key blocks 0 .. hot-1 in every row
    kn[:, :] = np.maximum(kn, hot)
    dup = rng.random((H, QB)) < 0.1
    ki[:, :, -1][dup] = ki[:, :, 0][dup]  # a repeat of the row's first entry
    want = {}
    for h in range(H):
        for qb in range(QB):
            for e in range(kn[h, qb]):
                kb = int(ki[h, qb, e])
                if 0 <= kb < NB:
                    want.setdefault((h, kb), []).append(qb)
    tn, ti = torch.from_numpy(kn).to(DEV), torch.from_numpy(ki).to(DEV)
    q_off = torch.empty((H, NB + 1), dtype=torch.int32, device=DEV)
    q_list = torch.empty((H, QB * maxkv), dtype=torch.int32, device=DEV)
    ws = torch.empty(max(1, ops.query("scope_transpose_workspace_bytes", H, NB)), dtype=torch.uint8, device=DEV)
    ops.call("scope_transpose_blocks", ops._p(tn), ops._p(ti), H, QB, NB, maxkv, ops._p(q_off), ops._p(q_list),
             ops._p(ws), ops._stream(torch.device(DEV)))
    off, lst = q_off.cpu().numpy(), q_list.cpu().numpy()
    longest = 0
    for h in range(H):
        for kb in range(NB):
            got = lst[h, off[h, kb]:off[h, kb + 1]].tolist()
            exp = sorted(want.get((h, kb), []))
            longest = max(longest, len(exp))
            assert got == exp, (h, kb)
        assert np.all(lst[h, off[h, NB]:] == -1)
    assert hot == 0 or longest >= QB  # the hot buckets hold every row (and its repeats)


@pytest.mark.parametrize("name", sorted(FORWARD_CASES))
def test_forward_stats_match_reference_vectors(name):
    from scope_amd import ops

    c = FORWARD_CASES[name]
    H, T, M = int(c["H"]), int(c["T"]), int(c["M"])
    has_docs = bool(c["with_docs"])
    clamp, reset_on = bool(c["cfg_pointer_doc_clamp"]), bool(c["cfg_reset_active"])
    rl = int(c["cfg_reset_len_active"]) if reset_on else 0
    ds_ptr = ds_local = None
    if has_docs:
        ds_ptr, ds_local, _ = ops.doc_starts(torch.from_numpy(c["docs"]).to(DEV), 128, doc_clamp=clamp, reset_len=rl)
    counts, values = ops.mask_stats(H=H, QB=T // 128, bs=128, delta_star=torch.from_numpy(c["delta_star"]).to(DEV),
                                    pi=torch.from_numpy(c["pi"]).to(DEV), rep_mode=str(c["rep_mode"]),
                                    has_docs=has_docs, docstart_enabled=has_docs and (clamp or reset_on),
                                    local_blocks_cfg=int(c["cfg_pointer_local_blocks"]), eps=float(c["cfg_eps"]),
                                    ds_ptr_fwd=ds_ptr, ds_local_fwd=ds_local)
    u = ops.unpack_counts(counts.cpu(), 1, 1)
    for key in ("delta_tokens_hist", "delta_blocks_hist", "ptr_center_hist"):
        assert np.array_equal(u[key].numpy(), c["dbg_" + key]), key
    v = values.cpu().numpy()
    for i, key in enumerate(["pi_entropy_mean", "ptr_docstart_frac", "ptr_outside_local_frac", "ptr_block0_frac",
                             "ptr_block0_frac_excl"]):
        if key == "pi_entropy_mean":
            assert abs(v[i] - float(c["dbg_" + key])) <= 1e-5 * max(1.0, abs(float(c["dbg_" + key]))), key
        else:
            assert v[i] == float(c["dbg_" + key]), key


def test_blockscore_stats_vs_oracle():
    from scope_amd import ops

    H, T, bs, W, G, B = 8, 131072, 256, 2, 2, 8
    NB = T // bs
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    docs = docs_with_boundaries(T, 16, 4)
    sel = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=W, n_global=G, budget=B)
    ref = OS.blockscore_stats(sel["kv_num"], sel["picks"], sel["ds_ptr"], sel["ds_local"], maxkv=sel["maxkv"],
                              local_blocks=W)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    counts, values = ops.mask_stats(H=H, QB=NB, bs=bs, kv_num=torch.from_numpy(sel["kv_num"]).to(DEV),
                                    picks=torch.from_numpy(sel["picks"]).to(DEV), ds_ptr=ds_ptr, ds_local=ds_local,
                                    maxkv_bins=sel["maxkv"] + 1, bs_local_blocks=W)
    u = ops.unpack_counts(counts.cpu(), sel["maxkv"] + 1, 0)
    assert np.array_equal(u["kv_unique_hist"].numpy(), ref["kv_unique_hist"])
    assert np.array_equal(u["ptr_dist_hist"].numpy(), ref["ptr_dist_hist"])
    assert int(u["bs_n"]) == int(ref["n_picks"])
    v = values.cpu().numpy()
    assert v[6] == ref["ptr_outside_local_frac"]
    assert v[7] == ref["ptr_block0_frac"]
    assert v[8] == ref["ptr_block0_frac_excl"]
    assert v[9] == ref["ptr_docstart_frac"]


@pytest.mark.parametrize("budget,noise", [(8, "counter"), (12, "none"), (3, "uniform")])
def test_pointer_select_given_logits_past_4096_candidates(budget, noise):
    """Rows with up to 4200 candidates (more than one 4096-candidate pass of
    a wavefront's 64 lanes over 64 chunks) equal the oracle's selection on the
    same logits, ties and -inf logits included, in a second document that
    starts at block 300 (the oracle computes only the checked rows)."""
    from scope_amd import ops

    H, NB, bs = 1, 4500, 128
    T = NB * bs
    print(f"select past 4096 candidates NB={NB} budget={budget} noise={noise}", flush=True)
    rng = np.random.default_rng(budget)
    logits = (np.round(rng.standard_normal((H, NB, NB)) * 4) / 4).astype(np.float32)  # many ties
    logits[rng.random((H, NB, NB)) < 0.2] = -np.inf
    docs = torch.zeros(T, dtype=torch.int32)
    docs[300 * bs:] = 1  # the second document starts at block 300
    rows = [0, 5, 299, 300, 301, 363, 364, 2000, 4095, 4395, 4396, 4397, 4459, 4460, 4499]
    seed = 0xBEEF_1234
    g = u = None
    if noise == "uniform":
        u = rng.random((H, NB, NB)).astype(np.float32)
        g = OP.gumbel_from_u(u)
    elif noise == "counter":
        g = np.zeros((H, NB, NB), dtype=np.float32)
        for qb in rows:
            g[0, qb] = OP.gumbel_from_u(OP.counter_uniform(seed, np.zeros(NB, np.int64), np.full(NB, qb), np.arange(NB)))
    ref = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=2, n_global=1, budget=budget, gumbel=g,
                                       temp=0.5, rows=rows)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), bs)
    kv_num, kv_idx, picks = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=2, n_global=1,
                                               budget=budget, logits_in=torch.from_numpy(logits).to(DEV), temp=0.5,
                                               noise=noise, seed=seed,
                                               gumbel_u=torch.from_numpy(u).to(DEV) if u is not None else None)
    picks, kv_num, kv_idx = picks.cpu().numpy(), kv_num.cpu().numpy(), kv_idx.cpu().numpy()
    for qb in rows:
        assert np.array_equal(picks[0, qb], ref["picks"][0, qb]), qb
        assert kv_num[0, qb] == ref["kv_num"][0, qb], qb
        assert np.array_equal(kv_idx[0, qb], ref["packed"][0, qb]), qb

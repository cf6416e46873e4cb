"""CPU: pin the pointer oracle (reference mode + block-scoring mode + pack +
transpose) against the reference's golden vectors, torch's BlockMask, brute
force and closed forms."""
from __future__ import annotations

import itertools
from collections import Counter

import numpy as np
import pytest
import torch

from oracle import pointer as P
from tests.golden import load_cases, pointer_case_args, pointer_case_reps

CASES = load_cases("pointer_ref_vectors.npz")


@pytest.mark.parametrize("name", sorted(CASES))
def test_reference_mode_matches_golden(name):
    c = CASES[name]
    a = pointer_case_args(c)
    dr, br = pointer_case_reps(c)
    out = P.pointer_mask_reference(dr, br, c["docs"], gumbel_u=c["gumbel_u"], **a)
    NB = int(c["T"]) // int(c["bs"])
    assert np.array_equal(out["kv_num"], c["kv_num_blocks"][0])
    assert np.array_equal(P.export_nb_wide(out["packed"], NB), c["kv_indices"][0])
    qn, qi = P.transpose_dense_export(out["kv_num"], out["packed"], NB)
    assert np.array_equal(qn, c["q_num_blocks"][0])
    assert np.array_equal(qi, c["q_indices"][0])


def test_golden_cases_cover_every_branch():
    names = set(CASES)
    assert {"gumbel_multi_doc", "fixed_radius_schedule", "reset_segments", "rep_mean", "no_extra_budget_p0",
            "pointer_disabled", "extra_budget_no_doc_clamp", "export_truncation", "build_overrides"} <= names
    assert any(int(c["training"]) and int(c["cfg_gumbel_topk"]) for c in CASES.values())


def test_doc_starts_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(20):
        T, bs = 512, 32
        docs = np.cumsum(rng.random(T) < 0.02).astype(np.int32)
        if rng.random() < 0.3:  # non-monotone ids (doc start = last change point)
            docs = rng.integers(0, 3, T).repeat(1)[:T]
        dst = np.array([max(s for s in range(t + 1) if s == 0 or docs[s] != docs[s - 1]) for t in range(T)])
        ptr, loc, tok = P.doc_start_blocks(docs, bs)
        for b in range(T // bs):
            assert ptr[b] == dst[(b + 1) * bs - 1] // bs
            assert loc[b] == dst[b * bs] // bs
            assert tok[b] == dst[(b + 1) * bs - 1]


def test_radius_alloc_invariants():
    """Largest remainder: Σ r = budget_rem when no clamp binds; each r within
    1 of the stick-breaking allocation; M = 1 takes everything."""
    rng = np.random.default_rng(1)
    for M in (1, 2, 3, 8):
        br = (rng.standard_normal((3, 50, M)) * 2).astype(np.float32)
        for rem in (1, 3, 7):
            r = P.radius_alloc_pi(br, budget_rem=rem, temp=1.0, p=100)
            assert np.all(r.sum(-1) == rem)
            if M == 1:
                assert np.all(r[..., 0] == rem)
    assert np.all(P.radius_alloc_pi(br, budget_rem=0, temp=1.0, p=4) == 0)


def test_radius_alloc_matches_hand_computed_case():
    # M=3, rem=5, logits 0 -> sigmoid = 0.5: alloc = 2.5, 1.25, 1.25; floors 2,1,1 (sum 4),
    # one extra to the largest fraction (0.5, peak 0) -> r = 3,1,1
    r = P.radius_alloc_pi(np.zeros((1, 1, 3), np.float32), budget_rem=5, temp=1.0, p=8)
    assert r.tolist() == [[[3, 1, 1]]]


def test_gumbel_closed_form():
    u = np.array([0.5, 0.1, 0.9], np.float32)
    g = P.gumbel_from_u(u)
    ref = -np.log(-np.log(u.astype(np.float64) + 1e-9) + 1e-9)
    assert np.allclose(g, ref, rtol=1e-6)


def test_counter_uniform_known_answers():
    """Fixed values of the in-kernel uniform generator (integer hash)."""
    u = P.counter_uniform(0x123456789ABC, np.array([0, 1, 7]), np.array([0, 5, 511]), np.array([0, 3, 100]))
    assert u.dtype == np.float32 and np.all((u >= 0) & (u < 1))
    # recompute with plain Python integers (independent of numpy's uint32 arithmetic)
    def mix(x):
        x &= 0xFFFFFFFF
        x ^= x >> 16
        x = (x * 0x7FEB352D) & 0xFFFFFFFF
        x ^= x >> 15
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        x ^= x >> 16
        return x

    def cu(seed, h, qb, kb):
        x = mix((seed & 0xFFFFFFFF) ^ mix(seed >> 32))
        x = mix(x ^ ((h + 0x9E3779B9) & 0xFFFFFFFF))
        x = mix(x ^ ((qb + 0x3C6EF372) & 0xFFFFFFFF))
        x = mix(x ^ ((kb + 0xDAA66D2B) & 0xFFFFFFFF))
        return (x >> 8) / 16777216.0

    for i, (h, qb, kb) in enumerate([(0, 0, 0), (1, 5, 3), (7, 511, 100)]):
        assert u[i] == np.float32(cu(0x123456789ABC, h, qb, kb))


def test_pack_matches_brute_force_set_union():
    rng = np.random.default_rng(2)
    x = rng.integers(0, 12, (40, 9)).astype(np.int32)
    n, packed = P.pack_sorted_unique(x)
    for row, k, pk in zip(x, n, packed):
        uniq = sorted(set(row.tolist()))
        assert k == len(uniq)
        assert pk[:k].tolist() == uniq
        cnt = Counter(row.tolist())
        dups = sorted(v for v, c in cnt.items() for _ in range(c - 1))
        assert pk[k:].tolist() == dups


def test_reference_mode_invariants_random():
    rng = np.random.default_rng(3)
    for trial in range(10):
        H, bs, M = 2, 64, 3
        T = 64 * 24
        NB = T // bs
        docs = np.cumsum(rng.random(T) < 0.004).astype(np.int32)
        t_rep = (np.arange(NB) + 1) * bs - 1
        dr = (rng.random((H, NB, M)) * (t_rep[None, :, None] + 100)).astype(np.float32)
        br = rng.standard_normal((H, NB, M)).astype(np.float32)
        out = P.pointer_mask_reference(dr, br, docs, bs=bs, M=M, local_blocks=3, ptr_half_blocks=2,
                                       global_blocks_cfg=1, global_active=1, budget_blocks=14, budget_is_total=True,
                                       budget_temp=1.0, radius_mode="pi", doc_clamp=True, mask_active=True,
                                       half_active=2)
        ds_ptr, ds_local, _ = P.doc_start_blocks(docs, bs)
        for h in range(H):
            for qb in range(NB):
                n = out["kv_num"][h, qb]
                lst = out["packed"][h, qb, :n]
                assert np.all(np.diff(lst) > 0)
                assert qb in lst
                assert lst.max() <= qb and lst.min() >= min(ds_local[qb], ds_ptr[qb])


def test_transpose_matches_torch_blockmask():
    """q lists == torch's own _transpose_ordered (library code)."""
    from torch.nn.attention.flex_attention import BlockMask

    rng = np.random.default_rng(4)
    H, NB = 3, 16
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    docs = np.zeros(NB * 32, np.int32)
    sel = P.pointer_select_blockscore(logits, docs, bs=32, window=2, n_global=1, budget=3)
    exp = P.export_nb_wide(sel["packed"], NB)
    kv_num = torch.from_numpy(sel["kv_num"])[None]
    bm = BlockMask.from_kv_blocks(kv_num, torch.from_numpy(exp)[None], BLOCK_SIZE=32)
    qn, qi = P.transpose_dense_export(sel["kv_num"], sel["packed"], NB)
    assert np.array_equal(bm.q_num_blocks[0].numpy(), qn)
    assert np.array_equal(bm.q_indices[0].numpy(), qi)
    q_num, q_off, q_list = P.transpose_blocks(sel["kv_num"], sel["packed"], NB)
    for h in range(H):
        for kb in range(NB):
            assert q_list[h, q_off[h, kb]:q_off[h, kb + 1]].tolist() == qi[h, kb, :qn[h, kb]].tolist()


def test_blockscore_selection_brute_force():
    """Top-budget over all candidate subsets, tiny NB."""
    rng = np.random.default_rng(5)
    H, NB, bs = 2, 9, 16
    T = NB * bs
    for trial in range(6):
        docs = np.cumsum(rng.random(T) < 0.01).astype(np.int32)
        logits = (np.round(rng.standard_normal((H, NB, NB)) * 2) / 2).astype(np.float32)
        W, G, B = 2, 1, 2
        sel = P.pointer_select_blockscore(logits, docs, bs=bs, window=W, n_global=G, budget=B)
        ds_ptr, ds_local, _ = P.doc_start_blocks(docs, bs)
        for h in range(H):
            for qb in range(NB):
                win = {max(max(qb - o, 0), ds_local[qb]) for o in range(W)}
                glb = {min(ds_ptr[qb] + g, qb) for g in range(G)}
                cand = [kb for kb in range(ds_ptr[qb], qb + 1) if kb not in win | glb]
                best = None
                for sub in itertools.combinations(cand, min(B, len(cand))):
                    key = sorted(((-logits[h, qb, kb], kb) for kb in sub))
                    score = [k[0] for k in key]
                    if best is None or (score, sorted(sub)) < best[0]:
                        best = ((score, sorted(sub)), sub)
                want = set(best[1]) if best else set()
                got = {int(x) for x in sel["picks"][h, qb] if x >= 0}
                assert got == want
                lst = sel["packed"][h, qb, :sel["kv_num"][h, qb]].tolist()
                assert lst == sorted(win | glb | want)

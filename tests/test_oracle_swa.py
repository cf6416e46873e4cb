"""Pins of the sliding-window block-mask oracle (oracle/swa.py) against what
the mathematics and torch fix: token-level brute force of the block rules,
torch's argsort for the row order, closed forms, a hand-computed boundary
row, and torch's eager flex_attention over the exported BlockMask."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import swa as S


def _docs(T: int, cuts) -> np.ndarray:
    flag = np.zeros(T, dtype=np.int64)
    flag[list(cuts)] = 1
    return flag.cumsum()


def _random_docs(T: int, n_cuts: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return _docs(T, rng.choice(np.arange(1, T), size=n_cuts, replace=False))


@pytest.mark.parametrize("seed", range(6))
def test_block_rules_match_token_pairs(seed):
    bs, T = 8, 128
    docs = _random_docs(T, 1 + seed * 2, seed)
    any_, all_ = S.block_rules(docs, bs)
    NB = T // bs
    i = np.arange(T)
    vis = (i[:, None] >= i[None, :]) & (docs[:, None] == docs[None, :])
    blk = vis.reshape(NB, bs, NB, bs)
    assert np.array_equal(any_, blk.any(axis=(1, 3)))
    assert np.array_equal(all_, blk.all(axis=(1, 3)))


def test_dense_to_ordered_matches_torch():
    rng = np.random.default_rng(3)
    dense = rng.random((17, 23)) < 0.3
    num, idx = S.dense_to_ordered(dense)
    t = torch.from_numpy(dense)
    t_idx = t.argsort(dim=-1, descending=False, stable=True).flip(-1)
    assert np.array_equal(num, t.sum(dim=-1, dtype=torch.int32).numpy())
    assert np.array_equal(idx, t_idx.numpy())


@pytest.mark.parametrize("W", [1, 2, 3, 7, 14, 40])
def test_single_document_is_the_last_w_blocks(W):
    bs, T = 16, 512
    NB = T // bs
    m = S.create_blockmasks(np.zeros(T, dtype=np.int64), bs, W)
    for name, w in (("long", W), ("short", W // 2)):
        r = m[name]
        for qb in range(NB):
            want = set(range(max(0, qb - max(w, 1) + 1), qb + 1))
            got = set(r["kv_idx"][qb, :r["kv_num"][qb]].tolist())
            assert got == want, (name, qb)
            assert r["kv_num"][qb] == len(want)
            assert r["kv_num_blocks"][qb] == 1  # only the diagonal block is partial
            assert r["full_kv_num_blocks"][qb] == min(qb, w - 1)


def test_boundary_inside_a_block_hand_row():
    # bs 4, 6 blocks; document 1 starts at token 9 (inside block 2)
    bs, T = 4, 24
    docs = _docs(T, [9])
    m = S.create_blockmasks(docs, bs, 4)
    # block 5 (tokens 20-23, doc 1): full = blocks 4, 3 (all doc 1); partial = 5 (diag), 2 (holds the boundary)
    assert m["full_num"][5] == 2 and list(m["full_idx"][5, :2]) == [4, 3]
    assert m["partial_num"][5] == 2 and list(m["partial_idx"][5, :2]) == [5, 2]
    # the rest of each row: the other blocks descending
    assert list(m["full_idx"][5, 2:]) == [5, 2, 1, 0]
    assert list(m["partial_idx"][5, 2:]) == [4, 3, 1, 0]
    # long window 4: full min(2, 3) = 2, partial min(2, max(4 - 2, 1)) = 2 -> {4, 3, 5, 2}
    assert m["long"]["full_kv_num_blocks"][5] == 2 and m["long"]["kv_num_blocks"][5] == 2
    assert list(m["long"]["kv_idx"][5]) == [4, 3, 5, 2]
    # short window 2: full min(2, 1) = 1, partial min(2, max(2 - 2, 1)) = 1 -> {4, 5}
    assert m["short"]["full_kv_num_blocks"][5] == 1 and m["short"]["kv_num_blocks"][5] == 1
    assert list(m["short"]["kv_idx"][5]) == [4, 5]
    # block 2 (tokens 8-11) spans both documents: no full entries, partial = 2, 1, 0
    assert m["full_num"][2] == 0 and m["partial_num"][2] == 3
    assert list(m["long"]["kv_idx"][2, :3]) == [2, 1, 0]


def test_window_zero_and_one():
    bs, T = 8, 64
    docs = _random_docs(T, 2, 1)
    m0 = S.create_blockmasks(docs, bs, 0)
    for name in ("long", "short"):
        r = m0[name]
        # clamp_max(n_full, -1) = -1 (FlexAttention then reads no full block); one partial entry: the diagonal
        assert (r["full_kv_num_blocks"] == -1).all()
        assert (r["kv_num"] == 1).all()
        assert np.array_equal(r["kv_idx"][:, 0], np.arange(T // bs))
    m1 = S.create_blockmasks(docs, bs, 1)
    assert (m1["long"]["full_kv_num_blocks"] == 0).all()
    assert np.array_equal(m1["long"]["kv_idx"][:, 0], np.arange(T // bs))


def _flex_swa(q, k, v, m, name, docs, bs):
    """torch's eager flex_attention with the semantics of its fused kernels
    over the reference-format BlockMask: mask_mod on the listed partial
    blocks, none on the listed full blocks, nothing elsewhere.  The eager
    path applies only a mask_mod, so the block lists are expanded with
    torch's own ``_ordered_to_dense`` and folded into it."""
    from torch.nn.attention.flex_attention import BlockMask, _ordered_to_dense, flex_attention

    r = m[name]
    docs_l = torch.from_numpy(docs).long()

    def document_causal(b, h, qi, ki):  # scoped_medium.py:539-544
        return (qi >= ki) & (docs_l[qi] == docs_l[ki])

    as4 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.int32)[None, None]
    bm = BlockMask.from_kv_blocks(as4(r["kv_num_blocks"]), as4(m["partial_idx"]),
                                  as4(np.maximum(r["full_kv_num_blocks"], 0)), as4(m["full_idx"]),
                                  BLOCK_SIZE=bs, mask_mod=document_causal)
    part = _ordered_to_dense(bm.kv_num_blocks, bm.kv_indices)[0, 0].bool()
    full = _ordered_to_dense(bm.full_kv_num_blocks, bm.full_kv_indices)[0, 0].bool()
    assert not (part & full).any()

    def visited(b, h, qi, ki):
        qb, kb = qi // bs, ki // bs
        return full[qb, kb] | (part[qb, kb] & document_causal(b, h, qi, ki))

    bm_eager = BlockMask.from_kv_blocks(bm.kv_num_blocks, bm.kv_indices, BLOCK_SIZE=bs, mask_mod=visited)
    o, lse = flex_attention(q[None], k[None], v[None], block_mask=bm_eager, scale=0.1, return_lse=True)
    return o[0], lse[0]


@pytest.mark.parametrize("W", [3, 6])
def test_flex_attention_over_exported_mask_matches_compact_lists(W):
    bs, T, H, D = 16, 256, 2, 16
    docs = _docs(T, [37, 90, 91, 200])
    m = S.create_blockmasks(docs, bs, W)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn((H, T, D), generator=g, dtype=torch.float64) for _ in range(3))
    for name in ("long", "short"):
        o_ref, l_ref = _flex_swa(q, k, v, m, name, docs, bs)
        kv_num = torch.from_numpy(m[name]["kv_num"])[None].expand(H, -1)
        kv_idx = torch.from_numpy(m[name]["kv_idx"])[None].expand(H, -1, -1)
        o, lse = OA.scope_attention_reference(q, k, v, kv_num, kv_idx, torch.from_numpy(docs), bs=bs, scale=0.1)
        assert torch.allclose(o, o_ref, atol=1e-10), name
        fin = torch.isfinite(l_ref)
        assert torch.equal(fin, torch.isfinite(lse))
        assert torch.allclose(lse[fin], l_ref[fin], atol=1e-10), name

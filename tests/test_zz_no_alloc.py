"""The entry point that allocates nothing, scope_transpose_blocks_noalloc,
against scope_transpose_blocks (the same kernels with a caller workspace)
through the C ABI: two calls in a row, the second with a smaller input (the
static cursor array keeps the first call's contents and must be cleared by
the second), bit-exact on the q-list offsets and on every filled q-list
entry; and the size limit rejected with an error before any launch."""
from __future__ import annotations

import pytest
import torch

from tests.helpers import docs_with_boundaries

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _lists(H, T, bs, W, G, B, n_docs, seed):
    """Block-scoring lists over random logits (the selection kernel)."""
    from scope_amd import ops

    NB = T // bs
    docs = docs_with_boundaries(T, n_docs, seed).to(DEV)
    logits = torch.randn((H, NB, NB), generator=torch.Generator(device=DEV).manual_seed(seed), device=DEV)
    ds_ptr, ds_local, _ = ops.doc_starts(docs, bs)
    kv_num, kv_idx, _ = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=W, n_global=G, budget=B,
                                           logits_in=logits)
    return kv_num, kv_idx


def test_transpose_noalloc_equals_workspace_entry_point():
    from scope_amd import ops

    # the million-token shape (H·NB = 32768 cursors), then a smaller one
    for H, T, bs, W, G, B, n_docs in ((8, 1 << 20, 256, 2, 1, 8, 1), (3, 16384, 128, 2, 2, 3, 4)):
        NB = T // bs
        print(f"noalloc transpose H={H} T={T} bs={bs}", flush=True)
        kv_num, kv_idx = _lists(H, T, bs, W, G, B, n_docs, seed=T + H)
        want_off, want_list = ops.transpose_blocks(kv_num, kv_idx, NB)
        q_off = torch.full((H, NB + 1), -7, dtype=torch.int32, device=DEV)
        q_list = torch.full((H, NB * kv_idx.shape[-1]), -7, dtype=torch.int32, device=DEV)
        ops.transpose_blocks_noalloc(kv_num, kv_idx, q_off, q_list)
        torch.cuda.synchronize()
        assert torch.equal(q_off, want_off)
        for h in range(H):
            n = int(want_off[h, NB])
            assert n == int(kv_num[h].sum())
            assert torch.equal(q_list[h, :n], want_list[h, :n]), f"head {h}"
            assert bool((q_list[h, n:] == -1).all())  # the entries past the filled ones are set to -1


def test_transpose_noalloc_rejects_sizes_beyond_the_static_scratch():
    from scope_amd import ops
    from scope_amd._lib import ScopeLibraryError

    H, QB = 65, ops.NOALLOC_MAX_HNB // 64  # H·NB one head beyond the limit
    kv_num = torch.ones((H, QB), dtype=torch.int32, device=DEV)
    kv_idx = torch.zeros((H, QB, 1), dtype=torch.int32, device=DEV)
    q_off = torch.zeros((H, QB + 1), dtype=torch.int32, device=DEV)
    q_list = torch.zeros((H, QB), dtype=torch.int32, device=DEV)
    with pytest.raises(ScopeLibraryError, match="exceeds the static scratch"):
        ops.transpose_blocks_noalloc(kv_num, kv_idx, q_off, q_list)
    torch.cuda.synchronize()
    assert bool((q_off == 0).all())


def test_transpose_noalloc_replayed_from_a_captured_graph():
    """Captured once in a HIP graph (torch.cuda.CUDAGraph) after one eager
    call, then replayed three times with new lists copied into the captured
    inputs and the outputs overwritten by eager work between the replays:
    every replay equals scope_transpose_blocks on those lists, bit for bit."""
    from scope_amd import ops

    H, T, bs, W, G, B = 4, 65536, 128, 2, 1, 4
    NB = T // bs
    kv_num, kv_idx = _lists(H, T, bs, W, G, B, 3, seed=100)
    q_off = torch.zeros((H, NB + 1), dtype=torch.int32, device=DEV)
    q_list = torch.zeros((H, NB * kv_idx.shape[-1]), dtype=torch.int32, device=DEV)
    ops.transpose_blocks_noalloc(kv_num, kv_idx, q_off, q_list)  # eager: the scratch address is looked up here
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.transpose_blocks_noalloc(kv_num, kv_idx, q_off, q_list)
    torch.cuda.synchronize()
    for seed in (101, 102, 103):
        print(f"graph replay with lists of seed {seed}", flush=True)
        kn, ki = _lists(H, T, bs, W, G, B, 1 + seed % 5, seed=seed)
        kv_num.copy_(kn)
        kv_idx.copy_(ki)
        q_off.fill_(-7)
        q_list.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want_off, want_list = ops.transpose_blocks(kn, ki, NB)
        assert torch.equal(q_off, want_off)
        assert torch.equal(q_list, want_list)

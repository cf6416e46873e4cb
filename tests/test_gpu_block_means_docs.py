"""scope_block_means_docs against its two halves: the block means and the
document starts of one fused call equal, bit for bit, those of
scope_block_means and scope_doc_starts (both pinned against the oracle in
test_gpu_pointer.py), for document layouts with boundaries inside blocks, on
block edges and at token 0 only, with and without the clamp and the reset
segments."""
from __future__ import annotations

import pytest
import torch

from tests.helpers import docs_with_boundaries

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _docs(T, bs, kind, seed):
    if kind == "random":
        return docs_with_boundaries(T, 7, seed=seed)
    if kind == "one":
        return torch.zeros(T, dtype=torch.int32)
    d = torch.zeros(T, dtype=torch.int32)  # boundaries on block edges
    for i, b in enumerate(range(3 * bs, T, 5 * bs)):
        d[b:] = i + 1
    return d


@pytest.mark.parametrize("H,T,D,bs", [(2, 4096, 128, 128), (3, 8192, 128, 256), (1, 2048, 64, 128),
                                      (8, 131072, 128, 256)])
@pytest.mark.parametrize("kind", ["random", "one", "edges"])
@pytest.mark.parametrize("clamp,reset", [(True, 0), (False, 0), (True, 1024)])
def test_block_means_docs_equals_the_two_calls(H, T, D, bs, kind, clamp, reset):
    from scope_amd import ops

    print(f"block means + docs H={H} T={T} D={D} bs={bs} {kind} clamp={clamp} reset={reset}", flush=True)
    g = torch.Generator().manual_seed(T + H)
    q = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn((1, H, T, D), generator=g).to(torch.bfloat16).to(DEV)
    docs = _docs(T, bs, kind, seed=H).to(DEV)
    got = ops.block_means_docs(q, k, docs, bs, doc_clamp=clamp, reset_len=reset)
    qbar, kbar = ops.block_means(q, k, bs)
    ds = ops.doc_starts(docs, bs, doc_clamp=clamp, reset_len=reset)
    for name, a, b in zip(("qbar", "kbar", "ds_ptr", "ds_local", "ds_tok_end"), got, (qbar, kbar) + tuple(ds)):
        assert torch.equal(a, b), name

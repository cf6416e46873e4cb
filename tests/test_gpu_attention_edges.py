"""Edge cases of kernel 2 against the fp64 oracle, forward and backward:
rows with an empty list (kv_num = 0), rows whose only listed block lies in
an earlier document (every key masked), and a sequence of a single block.
Such a row sees no key: the oracle (FlexAttention's convention) gives
lse = -inf, an output of 0 and no gradient; the kernels must give exactly
that, and the other rows stay within |got - ref| <= 2e-2 + 1e-2·|ref|."""
from __future__ import annotations

import pytest
import torch

from tests.helpers import docs_with_boundaries, qkv, random_blockscore_mask, tol_check
from tests.test_gpu_attention import _oracle, _run_fwd, _token_terms
from tests.test_gpu_attention_bwd import NAMES, _gpu_grads, _ref_grads, _terms

pytestmark = pytest.mark.gpu
ATOL, RTOL = 2e-2, 1e-2


def _edge_lists(H, T, bs, docs, seed):
    """Random block-scoring lists with one empty row (head 0, q-block 1) and,
    in the last head, the last q-block listing only block 0 of an earlier
    document."""
    QB = T // bs
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=2, n_global=1, budget=2, seed=seed)
    if QB > 1:
        kv_num[0, 1] = 0
    assert int(docs[0]) != int(docs[(QB - 1) * bs]), "the last q-block must start in a later document"
    kv_num[H - 1, QB - 1] = 1
    kv_idx[H - 1, QB - 1, 0] = 0
    return kv_num, kv_idx


def _fwd_check(q, k, v, kv_num, kv_idx, docs, bs, mode, terms):
    out, lse = _run_fwd(q, k, v, kv_num, kv_idx, docs, bs, mode, terms)
    ref_out, ref_lse = _oracle(q, k, v, kv_num, kv_idx, docs, bs, mode, terms)
    out, lse = out[0].float().cpu(), lse[0].float().cpu()
    blind = torch.isinf(ref_lse)
    assert bool(torch.isneginf(lse[blind]).all()), "rows without a visible key must have lse = -inf"
    assert bool((out[blind] == 0).all()), "rows without a visible key must output 0"
    assert bool(torch.isfinite(lse[~blind]).all())
    ok, worst = tol_check(lse[~blind], ref_lse.float()[~blind], ATOL, RTOL)
    assert ok, f"lse: worst ratio {worst:.3f}"
    ok, worst = tol_check(out, ref_out.float(), ATOL, RTOL)
    assert ok, f"out: worst ratio {worst:.3f}"
    return blind


@pytest.mark.parametrize("bs,mode", [(128, "none"), (128, "block"), (128, "token"), (256, "none"), (256, "block"),
                                     (256, "token")])
def test_empty_and_blind_rows(bs, mode):
    H, T = 2, 4 * bs
    print(f"edge rows bs={bs} mode={mode}", flush=True)
    q, k, v = qkv(H, T, seed=31 + bs)
    docs = torch.zeros(T, dtype=torch.int32)
    docs[T // 2:] = 1  # two documents of two blocks each
    kv_num, kv_idx = _edge_lists(H, T, bs, docs, seed=5)
    fterms = _token_terms(H, T, 6, seed=3) if mode == "token" else _terms(mode, q, H, T, seed=3)
    blind = _fwd_check(q, k, v, kv_num, kv_idx, docs, bs, mode, fterms)
    assert int(blind.sum()) == 2 * bs, "one empty and one masked q-block"
    # backward (the token mode with the softplus gate, as the backward tests)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    terms = _terms(mode, q, H, T, seed=3)
    got = _gpu_grads(q, k, v, dout, kv_num, kv_idx, docs, bs, mode, terms)
    ref = _ref_grads(q, k, v, dout, kv_num, kv_idx, docs, bs, mode, terms)
    assert bool((got[0][0][blind] == 0).all()), "dq of rows without a visible key must be 0"
    for name, gg, rr in zip(NAMES, got, ref):
        assert bool(torch.isfinite(gg).all()), f"{name} not finite"
        ok, worst = tol_check(gg, rr, ATOL, RTOL)
        print(f"  {name}: worst ratio {worst:.3f}", flush=True)
        assert ok, f"{name}: worst ratio {worst:.3f}"


@pytest.mark.parametrize("bs,mode", [(128, "block"), (256, "none"), (256, "token")])
def test_single_block_sequence(bs, mode):
    H, T = 1, bs
    print(f"single block bs={bs} mode={mode}", flush=True)
    q, k, v = qkv(H, T, seed=41 + bs)
    docs = docs_with_boundaries(T, 1, seed=0)
    kv_num = torch.ones((H, 1), dtype=torch.int32)
    kv_idx = torch.zeros((H, 1, 3), dtype=torch.int32)
    fterms = _token_terms(H, T, 6, seed=4) if mode == "token" else _terms(mode, q, H, T, seed=4)
    _fwd_check(q, k, v, kv_num, kv_idx, docs, bs, mode, fterms)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    terms = _terms(mode, q, H, T, seed=4)
    got = _gpu_grads(q, k, v, dout, kv_num, kv_idx, docs, bs, mode, terms)
    ref = _ref_grads(q, k, v, dout, kv_num, kv_idx, docs, bs, mode, terms)
    for name, gg, rr in zip(NAMES, got, ref):
        ok, worst = tol_check(gg, rr, ATOL, RTOL)
        assert ok, f"{name}: worst ratio {worst:.3f}"

"""Sliding-window block masks (scoped_medium.py:535-576) on the GPU: the
builder's lists exactly equal to the oracle's, and the attention forward /
backward through the long and short masks against fp64 autograd.  Bar for
attention (written in every comparison): |got - ref| <= 2e-2 + 1e-2·|ref|."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import swa as S
from tests.helpers import docs_with_boundaries, qkv, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_lists(docs: torch.Tensor, bs: int, W: int, export: bool = True):
    from scope_amd import ops

    print(f"swa lists T={docs.numel()} bs={bs} W={W}", flush=True)
    ref = S.create_blockmasks(docs.numpy(), bs, W)
    r = ops.swa_blockmask(docs.to(DEV), bs, W, export=export)
    c = r["counts"].cpu().numpy()
    assert np.array_equal(c[0], ref["partial_num"])
    assert np.array_equal(c[1], ref["full_num"])
    for i, name in enumerate(("long", "short")):
        assert np.array_equal(c[2 + 2 * i], ref[name]["kv_num_blocks"]), name
        assert np.array_equal(c[3 + 2 * i], ref[name]["full_kv_num_blocks"]), name
        kv_num, kv_idx = (x.cpu().numpy() for x in r[name])
        assert np.array_equal(kv_num, ref[name]["kv_num"]), name
        assert np.array_equal(kv_idx, ref[name]["kv_idx"]), name
    if export:
        assert np.array_equal(r["partial_idx"].cpu().numpy(), ref["partial_idx"])
        assert np.array_equal(r["full_idx"].cpu().numpy(), ref["full_idx"])


@pytest.mark.parametrize("T,bs,n_docs,W", [(4096, 128, 1, 14), (4096, 128, 9, 14), (8192, 128, 40, 5),
                                           (8192, 64, 3, 0), (8192, 128, 3, 1), (8192, 128, 5, 2),
                                           (16384, 256, 7, 3), (4096, 128, 4, 100)])
def test_swa_lists_exact(T, bs, n_docs, W):
    _check_lists(docs_with_boundaries(T, n_docs, seed=T + n_docs + W), bs, W)


def test_swa_lists_boundaries_on_block_edges_and_short_documents():
    bs, T = 128, 8192
    flag = np.zeros(T, dtype=np.int64)
    flag[[128, 256, 300, 301, 302, 1024, 4096, 4097, 8191]] = 1  # edges, one-token documents, the last token
    _check_lists(torch.from_numpy(flag.cumsum()).to(torch.int32), bs, 6)


def test_swa_lists_long_sequence_compact_only():
    """65536 tokens, the reference's final window (1792 tokens = 14 blocks)."""
    _check_lists(docs_with_boundaries(65536, 9, seed=5), 128, 14, export=False)


def test_create_blockmasks_defaults_docs_from_tokens():
    import scope_amd

    T = 2048
    g = torch.Generator().manual_seed(3)
    toks = torch.randint(0, 50000, (T,), generator=g)
    toks[[100, 700, 701, 1500]] = 50256
    docs = (toks == 50256).cumsum(0).to(torch.int32)
    long_bm, short_bm = scope_amd.create_blockmasks(toks.to(DEV), torch.tensor(6), num_heads=2)
    ref = S.create_blockmasks(docs.numpy(), 128, 6)
    for bm, name in ((long_bm, "long"), (short_bm, "short")):
        assert bm.kv_num_blocks.shape == (1, 2, T // 128)
        assert torch.equal(bm.docs.cpu(), docs)
        for h in range(2):
            assert np.array_equal(bm.kv_num_blocks[0, h].cpu().numpy(), ref[name]["kv_num"])
            assert np.array_equal(bm.kv_indices[0, h].cpu().numpy(), ref[name]["kv_idx"])


def _grads_gpu(q, k, v, dout, bm):
    import scope_amd

    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    out, lse = scope_amd.scope_attention(qd, kd, vd, block_mask=bm, scale=0.12, return_lse=True)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    return [x.float().cpu() for x in (out, lse, qd.grad, kd.grad, vd.grad)]


@pytest.mark.parametrize("T,n_docs,W", [(2048, 1, 4), (4096, 6, 6), (4096, 3, 3)])
def test_swa_attention_fwd_bwd_vs_fp64(T, n_docs, W):
    import scope_amd

    H, bs = 2, 128
    docs = docs_with_boundaries(T, n_docs, seed=T + W)
    q, k, v = qkv(H, T, seed=11)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    long_bm, short_bm = scope_amd.create_blockmasks(None, W, docs=docs.to(DEV), num_heads=H)
    for bm, name in ((long_bm, "long"), (short_bm, "short")):
        print(f"swa attention T={T} docs={n_docs} W={W} {name}", flush=True)
        got = _grads_gpu(q, k, v, dout, bm)
        kv_num, kv_idx = bm.kv_num_blocks[0].cpu(), bm.kv_indices[0].cpu()
        qq, kk, vv = (x[0].double().requires_grad_() for x in (q, k, v))
        out, lse = OA.scope_attention_blocksparse(qq, kk, vv, kv_num, kv_idx, docs, bs=bs, scale=0.12)
        out.backward(dout[0].double())
        want = [out.detach()[None], lse.detach()[None], qq.grad[None], kk.grad[None], vv.grad[None]]
        for nm, g_, w_ in zip(("out", "lse", "dq", "dk", "dv"), got, want):
            ok, worst = tol_check(g_, w_)
            assert ok, f"{name} {nm}: worst tolerance ratio {worst:.3f}"

"""List validation on the GPU: ``scope_check_lists`` (through
``ops.check_lists``) gives the host path's counters on malformed lists, and the
ops entry points and ``ScopeBlockMask`` reject a malformed list with a
``RuntimeError`` before any kernel reads it.  No malformed list reaches an
attention or transpose kernel here: the check runs first and raises."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from scope_amd import ops
from tests.test_lists_check import malformed_lists

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("H,QB,maxkv,seed", [(3, 40, 9, 0), (8, 512, 12, 1), (2, 4096, 11, 2), (1, 300, 64, 3)])
def test_device_counters_equal_host(H, QB, maxkv, seed):
    kn, ki = malformed_lists(H, QB, maxkv, seed)
    tn, ti = torch.from_numpy(kn), torch.from_numpy(ki)
    for causal in (True, False):
        want = ops._check_lists_host(tn, ti, QB, causal)
        res = torch.empty(5, dtype=torch.int32, device=DEV)
        # two device copies made in the argument list: each stays referenced
        # until the call returns, so the second cannot take the first's memory
        ops.call("scope_check_lists", ops._p(tn.to(DEV)), ops._p(ti.to(DEV)), H, QB, QB, maxkv, int(causal),
                 ops._p(res), ops._stream(torch.device(DEV)))
        got = res.tolist()
        print(f"  H={H} QB={QB} causal={causal}: {got}", flush=True)
        assert got == want


def _valid_lists(H, QB, W):
    kn = torch.full((H, QB), W, dtype=torch.int32)
    ki = torch.zeros((H, QB, W), dtype=torch.int32)
    for qb in range(QB):
        n = min(W, qb + 1)
        kn[:, qb] = n
        ki[:, qb, :n] = torch.arange(qb - n + 1, qb + 1)
    return kn.to(DEV), ki.to(DEV)


def test_entry_points_reject_malformed_lists():
    from scope_amd.blockmask import ScopeBlockMask

    H, T, D, bs, W = 2, 1024, 128, 128, 3
    QB = T // bs
    g = torch.Generator(device=DEV).manual_seed(0)
    q, k, v = (torch.randn((1, H, T, D), generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    docs = torch.zeros(T, dtype=torch.int32, device=DEV)
    _, _, ds_tok_end = ops.doc_starts(docs, bs)
    kn, ki = _valid_lists(H, QB, W)
    out, lse = ops.attn_fwd(q, k, v, kn, ki, docs, ds_tok_end, bs=bs, scale=0.1)  # valid lists pass
    q_off, q_list = ops.transpose_blocks(kn, ki, QB)
    bad = ki.clone()
    bad[1, 5, 0] = QB + 7  # outside the key blocks
    late = ki.clone()
    late[0, 2, 0] = 6      # after its q-block
    rep = ki.clone()
    rep[1, 7, 2] = rep[1, 7, 1]
    for lists, msg in ((bad, "entries outside"), (late, "after their q-block"), (rep, "repeated entries")):
        with pytest.raises(RuntimeError, match=msg):
            ops.attn_fwd(q, k, v, kn, lists, docs, ds_tok_end, bs=bs, scale=0.1)
        with pytest.raises(RuntimeError, match=msg):
            ops.transpose_blocks(kn, lists, QB)
        with pytest.raises(RuntimeError, match=msg):
            ops.attn_bwd(q, k, v, out, out, lse, kn, lists, q_off, q_list, docs, ds_tok_end, bs=bs, scale=0.1)
        with pytest.raises(RuntimeError, match=msg):
            ScopeBlockMask(kv_num_blocks=kn[None], kv_indices=lists[None], BLOCK_SIZE=bs, docs=docs,
                           ds_tok_end=ds_tok_end)
    with pytest.raises(RuntimeError, match="kv_num outside"):
        ops.attn_fwd(q, k, v, kn.clone().fill_(W + 1), ki, docs, ds_tok_end, bs=bs, scale=0.1)
    # the decode list of one token: distinct blocks of the cache (no causal rule)
    kc = k[0].contiguous()
    vc = v[0].contiguous()
    lst = torch.tensor([[0, 3, 7], [1, 2, 8]], dtype=torch.int32, device=DEV)  # 8 is past the 8 cache blocks
    with pytest.raises(RuntimeError, match="entries outside"):
        ops.decode_attn(q[0, :, 5], kc, vc, torch.tensor([3, 3], dtype=torch.int32, device=DEV), lst, docs, 900,
                        bs=bs, scale=0.1)
    torch.cuda.synchronize()
    assert np.isfinite(out.float().cpu().numpy()).all()


def test_int64_lists_and_documents_equal_int32():
    """Lists and document ids in int64 (the reference's dtypes) are copied to
    int32 inside the call's argument list: outputs equal the int32 call's bit
    for bit, forward and backward."""
    H, T, D, bs, W = 2, 2048, 128, 128, 3
    QB = T // bs
    g = torch.Generator(device=DEV).manual_seed(5)
    q, k, v, do = (torch.randn((1, H, T, D), generator=g, device=DEV).to(torch.bfloat16) for _ in range(4))
    docs = torch.zeros(T, dtype=torch.int32, device=DEV)
    docs[700:] = 1
    docs[1500:] = 2
    _, _, ds_tok_end = ops.doc_starts(docs, bs)
    kn, ki = _valid_lists(H, QB, W)
    q_off, q_list = ops.transpose_blocks(kn, ki, QB)
    out, lse = ops.attn_fwd(q, k, v, kn, ki, docs, ds_tok_end, bs=bs, scale=0.1)
    out64, lse64 = ops.attn_fwd(q, k, v, kn.long(), ki.long(), docs.long(), ds_tok_end.long(), bs=bs, scale=0.1)
    assert torch.equal(out, out64) and torch.equal(lse, lse64)
    g32 = ops.attn_bwd(q, k, v, out, do, lse, kn, ki, q_off, q_list, docs, ds_tok_end, bs=bs, scale=0.1)
    g64 = ops.attn_bwd(q, k, v, out, do, lse, kn.long(), ki.long(), q_off.long(), q_list.long(), docs.long(),
                       ds_tok_end.long(), bs=bs, scale=0.1)
    assert g32.keys() == g64.keys()
    for key, a in g32.items():
        assert (a is None and g64[key] is None) or torch.equal(a, g64[key]), key

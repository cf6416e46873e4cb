"""Teacher block mass (scoped_medium.py:1799-1819) on the GPU
(scope_attn_block_mass) against the fp64 oracle: the teacher's dense
document-causal attention with the token-offset band term and slope, a
pointer list with the block-offset bias, and the row-sum invariant at the
training shape.  Bar (written in each comparison): |got - ref| <= 2e-2 +
1e-2·|ref| per (head, q-block, key block) entry."""
from __future__ import annotations

import pytest
import torch

from oracle import attention as OA
from oracle.pointer import doc_start_blocks
from tests.helpers import band_coefficients, docs_with_boundaries, omegas_block, qkv, random_blockscore_mask, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE, BETA = 0.12, 0.5


def test_teacher_mass_dense_with_token_bias():
    import scope_amd

    H, T, bs, K = 4, 4096, 128, 6
    print(f"teacher mass T={T} H={H}", flush=True)
    docs = docs_with_boundaries(T, 5, seed=21)
    q, k, _ = qkv(H, T, seed=22)
    g = torch.Generator().manual_seed(23)
    cc = torch.randn((1, H, T, K), generator=g) * 0.3
    cs = torch.randn((1, H, T, K), generator=g) * 0.3
    sl = torch.randn((1, H, T), generator=g) * 0.002
    om = OA.omegas_logspaced(K, 1024, 1 << 20)
    sp = scope_amd.SpectralTerms(coeff_cos=cc.to(DEV), coeff_sin=cs.to(DEV), omegas=om.to(DEV), offset="token",
                                 beta=BETA, slope=sl.to(DEV), use_slope=True)
    got = scope_amd.attention.teacher_block_mass(q.to(DEV), k.to(DEV), docs.to(DEV), scale=SCALE, spectral=sp,
                                                 block_size=bs)
    ref = OA.block_mass(q[0].double(), k[0].double(), docs, bs=bs, scale=SCALE, beta=BETA, bias_mode="token",
                        coeff_cos=cc[0].double(), coeff_sin=cs[0].double(), omegas=om.double(),
                        token_kwargs=dict(slope=sl[0].double()))
    ok, worst = tol_check(got.cpu(), ref)
    assert ok, f"teacher mass: worst tolerance ratio {worst:.3f}"


def test_block_mass_pointer_lists_block_bias():
    from scope_amd import ops
    from scope_amd.attention import spectral_table

    H, T, bs = 2, 8192, 256
    print(f"block mass pointer lists T={T} bs={bs}", flush=True)
    docs = docs_with_boundaries(T, 3, seed=31)
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=2, n_global=1, budget=4, seed=32)
    q, k, _ = qkv(H, T, seed=33)
    A, B = band_coefficients(q)
    om = omegas_block(8)
    ds_end = torch.from_numpy(doc_start_blocks(docs.numpy(), bs)[2])
    mass, _ = ops.attn_block_mass(q.to(DEV), k.to(DEV), kv_num.to(DEV), kv_idx.to(DEV), docs.to(DEV),
                                  ds_end.to(DEV), bs=bs, scale=SCALE, beta=BETA, bias_mode="block",
                                  table=spectral_table(om.to(DEV), T, bs, "block"), coeff_cos=A.to(DEV),
                                  coeff_sin=B.to(DEV))
    ref = OA.block_mass(q[0].double(), k[0].double(), docs, bs=bs, scale=SCALE, beta=BETA, bias_mode="block",
                        coeff_cos=A[0].double(), coeff_sin=B[0].double(), omegas=om.double(), kv_num=kv_num,
                        kv_idx=kv_idx)
    ok, worst = tol_check(mass.cpu(), ref)
    assert ok, f"pointer-list mass: worst tolerance ratio {worst:.3f}"


def test_teacher_mass_row_sums_at_training_shape():
    """T=65536, H=8, bs=128 (512 blocks): every q-block's mass sums to bs, and
    three sampled q-blocks equal the oracle (no bias)."""
    import scope_amd

    H, T, bs = 8, 65536, 128
    NB = T // bs
    print(f"teacher mass T={T} H={H}", flush=True)
    docs = docs_with_boundaries(T, 8, seed=41)
    q, k, _ = qkv(H, T, seed=42)
    got = scope_amd.attention.teacher_block_mass(q.to(DEV), k.to(DEV), docs.to(DEV), scale=SCALE, block_size=bs)
    torch.cuda.synchronize()
    rs = got.sum(-1).cpu()
    assert (rs - bs).abs().max().item() <= 2e-2 * bs, f"row sums off by {(rs - bs).abs().max().item():.3e}"
    qbs = [0, NB // 3, NB - 1]
    kv_num = torch.zeros((1, NB), dtype=torch.int32)
    kv_idx = torch.zeros((1, NB, NB), dtype=torch.int32)
    for qb in range(NB):
        kv_num[0, qb] = qb + 1
        kv_idx[0, qb, :qb + 1] = torch.arange(qb + 1)
    for h in (0, H - 1):
        for qb in qbs:
            rows = slice(qb * bs, (qb + 1) * bs)
            qq = q[0, h:h + 1].double()
            kk = k[0, h:h + 1].double()
            res = OA.attention_blocksparse(qq, kk, torch.nn.functional.one_hot(torch.arange(T) // bs, NB).double()[None],
                                           kv_num, kv_idx, docs, bs=bs, scale=SCALE, heads=[0], qblocks=[qb])
            want = res[(0, qb)][0].sum(0)
            ok, worst = tol_check(got[h, qb].cpu(), want)
            assert ok, f"head {h} q-block {qb}: worst tolerance ratio {worst:.3f}"

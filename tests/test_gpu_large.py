"""Parity at the million-token shape (T=1048576, bs=256, NB=4096; the C5
layer): pointer selection over 4096 candidates with in-kernel counter Gumbel
noise (bit-exact), the block means feeding it, the mask statistics, and the
block-sparse attention forward and backward on sampled blocks (also at the
64k-token training shape, bs=128, with all eight heads: heads 0 and 7 are
compared).

The attention oracle is evaluated only where it is cheap and still complete:
out / lse / dq of a few q-blocks (each depends only on its own list), and dk /
dv of one key block, which receive contributions exactly from the q-blocks in
its transposed list; all of those are run through the oracle.  Bar:
2e-2 abs + 1e-2·|ref| against the fp32 oracle (fp64 accumulation is not
needed at these row lengths)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import pointer as OP
from oracle import stats as OS
from tests.helpers import band_coefficients, omegas_block, qkv, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
T, BS = 1 << 20, 256
NB = T // BS


def _select(H, W, G, B, seed):
    """Tie-heavy logits + counter Gumbel noise: kernel vs oracle."""
    from scope_amd import ops

    rng = np.random.default_rng(seed)
    logits = (np.round(rng.standard_normal((H, NB, NB)) * 4) / 4).astype(np.float32)
    docs = torch.zeros(T, dtype=torch.int32)  # one document, as in the C5 layer
    nseed = 0x5EED_0000 + seed
    hh, qq, kk = np.meshgrid(np.arange(H), np.arange(NB), np.arange(NB), indexing="ij")
    g = OP.gumbel_from_u(OP.counter_uniform(nseed, hh, qq, kk))
    del hh, qq, kk
    ref = OP.pointer_select_blockscore(logits, docs.numpy(), bs=BS, window=W, n_global=G, budget=B, gumbel=g)
    ds_ptr, ds_local, _ = ops.doc_starts(docs.to(DEV), BS)
    kv_num, kv_idx, picks = ops.pointer_select(ds_ptr, ds_local, bs=BS, NB=NB, H=H, window=W, n_global=G, budget=B,
                                               logits_in=torch.from_numpy(logits).to(DEV), noise="counter", seed=nseed)
    return ref, kv_num, kv_idx, picks, ds_ptr, ds_local


def test_c5_pointer_select_counter_noise_exact():
    H, W, G, B = 2, 2, 1, 8
    print(f"select T={T} NB={NB} H={H} budget={B}", flush=True)
    ref, kv_num, kv_idx, picks, ds_ptr, ds_local = _select(H, W, G, B, seed=1)
    assert np.array_equal(picks.cpu().numpy(), ref["picks"])
    assert np.array_equal(kv_num.cpu().numpy(), ref["kv_num"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])
    # mask statistics of the same selection
    from scope_amd import ops

    st = OS.blockscore_stats(ref["kv_num"], ref["picks"], ref["ds_ptr"], ref["ds_local"], maxkv=ref["maxkv"],
                             local_blocks=W)
    counts, values = ops.mask_stats(H=H, QB=NB, bs=BS, kv_num=kv_num, picks=picks, ds_ptr=ds_ptr, ds_local=ds_local,
                                    maxkv_bins=ref["maxkv"] + 1, bs_local_blocks=W)
    u = ops.unpack_counts(counts.cpu(), ref["maxkv"] + 1, 0)
    assert np.array_equal(u["kv_unique_hist"].numpy(), st["kv_unique_hist"])
    assert np.array_equal(u["ptr_dist_hist"].numpy(), st["ptr_dist_hist"])
    assert int(u["bs_n"]) == int(st["n_picks"])
    v = values.cpu().numpy()
    assert v[6] == st["ptr_outside_local_frac"]
    assert v[7] == st["ptr_block0_frac"]
    assert v[8] == st["ptr_block0_frac_excl"]
    assert v[9] == st["ptr_docstart_frac"]


def test_c5_block_means():
    from scope_amd import ops

    print(f"block means T={T}", flush=True)
    q, k, _ = qkv(1, T, seed=3)
    qbar, kbar = ops.block_means(q.to(DEV), k.to(DEV), BS)
    rq = OP.block_means(q[0].double().numpy(), BS)
    rk = OP.block_means(k[0].double().numpy(), BS)
    assert np.abs(qbar.cpu().numpy() - rq).max() < 1e-6
    assert np.abs(kbar.cpu().numpy() - rk).max() < 1e-6


@pytest.mark.parametrize("T,BS,W,G,B,H", [(1 << 20, 256, 2, 1, 8, 1), (65536, 128, 4, 1, 4, 8)])
def test_attention_sampled_blocks(T, BS, W, G, B, H):
    """The million-token layer (bs 256, one head) and the 64k training shape
    (bs 128, all eight heads run, heads 0 and 7 compared)."""
    import scope_amd
    from scope_amd import ops
    from scope_amd.blockmask import ScopeBlockMask

    NB = T // BS
    scale, beta = 0.12, 0.5
    print(f"attention fwd+bwd T={T} H={H} bs={BS} W{W} G{G} B{B}", flush=True)
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    docs = torch.zeros(T, dtype=torch.int32)
    sel = OP.pointer_select_blockscore(logits, docs.numpy(), bs=BS, window=W, n_global=G, budget=B)
    kv_num, kv_idx = torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])
    q, k, v = qkv(H, T, seed=4)
    dout = torch.randn((1, H, T, 128), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    A, Bc = band_coefficients(q)
    om = omegas_block(8)

    bm = ScopeBlockMask(kv_num_blocks=kv_num[None].to(DEV), kv_indices=kv_idx[None].to(DEV), BLOCK_SIZE=BS,
                        docs=docs.to(DEV), ds_tok_end=torch.from_numpy(OP.doc_start_blocks(docs.numpy(), BS)[2]).to(DEV))
    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    cd, sd = A.to(DEV).requires_grad_(), Bc.to(DEV).requires_grad_()
    sp = scope_amd.SpectralTerms(coeff_cos=cd, coeff_sin=sd, omegas=om.to(DEV), offset="block", beta=beta)
    out, lse = scope_amd.scope_attention(qd, kd, vd, block_mask=bm, scale=scale, spectral=sp, return_lse=True)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    print("  gpu done", flush=True)
    q_off, q_list = ops.transpose_blocks(kv_num.to(DEV).int(), kv_idx.to(DEV).int(), NB)

    def check(name, got, want):
        ok, worst = tol_check(got, want)
        print(f"    {name}: worst ratio {worst:.3f}", flush=True)
        assert ok, f"{name}: worst tolerance ratio {worst:.3f}"

    # sampled q-blocks: first, a middle one, last
    qbs = [0, NB // 2 + 3, NB - 1]
    for h in sorted({0, H - 1}):
        # one key block (not the global block 0) and every q-block that lists it
        kb = NB // 3
        o0, o1 = int(q_off[h, kb]), int(q_off[h, kb + 1])
        users = sorted(set(q_list[h, o0:o1].cpu().tolist()))
        assert users and all(int(u_) >= kb for u_ in users)
        rows = sorted(set(qbs) | set(users))
        print(f"  head {h}: oracle over {len(rows)} q-blocks (key block {kb} has {len(users)})", flush=True)

        qq, kk, vv = (x[0, h:h + 1].float().requires_grad_() for x in (q, k, v))
        cc, cs = A[0, h:h + 1].float().requires_grad_(), Bc[0, h:h + 1].float().requires_grad_()
        res = OA.attention_blocksparse(qq, kk, vv, kv_num[h:h + 1], kv_idx[h:h + 1], docs, bs=BS, scale=scale,
                                       beta=beta, bias_mode="block", coeff_cos=cc, coeff_sin=cs, omegas=om,
                                       heads=[0], qblocks=rows)
        loss = 0.0
        for qb in rows:
            o, _ = res[(0, qb)]
            loss = loss + (o * dout[0, h, qb * BS:(qb + 1) * BS].float()).sum()
        loss.backward()

        for qb in qbs:
            sl = slice(qb * BS, (qb + 1) * BS)
            ro, rl = res[(0, qb)]
            check(f"q-block {qb} out", out[0, h, sl].float().cpu(), ro.detach())
            check(f"q-block {qb} lse", lse[0, h, sl].float().cpu(), rl.detach())
            check(f"q-block {qb} dq", qd.grad[0, h, sl].float().cpu(), qq.grad[0, sl])
            # coefficient gradients of the sampled rows
            check(f"q-block {qb} dcoeff_cos", cd.grad[0, h, sl].cpu(), cc.grad[0, sl])
            check(f"q-block {qb} dcoeff_sin", sd.grad[0, h, sl].cpu(), cs.grad[0, sl])
        sl = slice(kb * BS, (kb + 1) * BS)
        check(f"key block {kb} dk", kd.grad[0, h, sl].float().cpu(), kk.grad[0, sl])
        check(f"key block {kb} dv", vd.grad[0, h, sl].float().cpu(), vv.grad[0, sl])

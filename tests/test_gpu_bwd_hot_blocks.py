"""GPU parity of the backward on hot key blocks.

A key block listed by more than 32 q-blocks (the global block of a long
document, a document's start block; model/attn_bias.py:809-823 makes them)
has its dK/dV summed over several kv-major work items of up to 32 q-blocks:
each item writes fp32 partials, and a reduce kernel adds them in chunk order
and writes bf16 (the FlexAttention backward reduces the same sums over its
q_indices, torch:_inductor/kernel/flex/templates/flex_backwards.py.jinja).

Every case here has key blocks with 2 to 4 chunks, a ragged last chunk, and
heads without any multi-chunk block (the reduce walks the heads' multi-chunk
lists and must skip an empty one), in every dK/dV kernel family: the 16-key
kernel (no bias, block bias, token offsets, each with a pair bias too) and
the 32-key kernel of the gated token mode (softplus gate).  The whole dq / dk / dv (and coefficient and
pair-bias gradients) are compared with fp64 autograd through the oracle's
block-sparse attention.  Bar written in every comparison:
|got - ref| <= 2e-2 + 1e-2·|ref| elementwise (dpair_bias: 2e-2·max|ref|)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle.pointer import doc_start_blocks
from tests.helpers import band_coefficients, omegas_block, qkv, random_blockscore_mask, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2
SCALE, BETA = 0.12, 0.5
CHUNK = 32  # q-blocks per kv-major work item below 2048 key blocks per head (attn_bwd.hip bwd_chunk)


def _docs(T: int, cuts: list[int]) -> torch.Tensor:
    flag = torch.zeros(T, dtype=torch.int64)
    flag[cuts] = 1
    return flag.cumsum(0).to(torch.int32)


def _lists(T: int, bs: int, docs: torch.Tensor, per_head, seed: int):
    """Block-scoring lists per head (W, G, budget), padded to a common width
    with each row's first entry (the reference's export padding rule)."""
    rows = [random_blockscore_mask(1, T, bs, docs, window=W, n_global=G, budget=B, seed=seed + 17 * h)
            for h, (W, G, B) in enumerate(per_head)]
    L = max(ki.shape[-1] for _, ki in rows)
    kv_num = torch.cat([kn for kn, _ in rows], 0)
    kv_idx = torch.cat([torch.cat([ki, ki[..., :1].expand(*ki.shape[:-1], L - ki.shape[-1])], -1) for _, ki in rows], 0)
    return kv_num, kv_idx.contiguous()


def _users(kv_num: torch.Tensor, kv_idx: torch.Tensor, NB: int) -> np.ndarray:
    """users[h, kb] = number of q-blocks whose list holds kb."""
    H, QB, _ = kv_idx.shape
    u = np.zeros((H, NB), dtype=np.int64)
    for h in range(H):
        for qb in range(QB):
            for kb in kv_idx[h, qb, :int(kv_num[h, qb])].tolist():
                u[h, kb] += 1
    return u


CASES = [
    # id, H, T, bs, document cuts, per-head (W, G, budget), bias mode, pair bias
    # one document: the global block 0 has 128 users, 4 full chunks
    ("bs128-none", 4, 16384, 128, [], [(2, 0, 2), (2, 1, 2), (2, 0, 3), (2, 1, 3)], "none", False),
    # a document of 100 blocks first: its start block has 100 users, chunks of 32, 32, 32 and 4
    ("bs128-block", 4, 16384, 128, [100 * 128 + 5], [(2, 0, 2), (2, 1, 2), (2, 0, 3), (2, 1, 3)], "block", False),
    ("bs128-block-pair", 4, 16384, 128, [100 * 128 + 5], [(2, 1, 2), (2, 0, 2), (2, 0, 3), (2, 1, 3)], "block",
     True),
    ("bs128-token", 2, 16384, 128, [9000], [(2, 0, 2), (2, 1, 3)], "token", False),
    ("bs128-token-pair", 2, 16384, 128, [9000], [(2, 1, 2), (2, 0, 3)], "token", True),
    ("bs128-token-gate", 2, 16384, 128, [9000], [(2, 0, 2), (2, 1, 3)], "token-gate", False),
    ("bs256-token", 2, 32768, 256, [100 * 256 + 77], [(2, 2, 3), (2, 0, 2)], "token", False),
    ("bs256-none", 2, 32768, 256, [100 * 256 + 77], [(2, 2, 3), (2, 0, 2)], "none", False),
    ("bs256-block", 3, 32768, 256, [100 * 256 + 77], [(2, 0, 3), (2, 2, 3), (2, 0, 2)], "block", False),
]


@pytest.mark.parametrize("cid,H,T,bs,cuts,per_head,mode,pair", CASES, ids=[c[0] for c in CASES])
def test_multichunk_dkv_vs_fp64(cid, H, T, bs, cuts, per_head, mode, pair):
    import scope_amd
    from scope_amd.blockmask import ScopeBlockMask

    print(f"multi-chunk dK/dV {cid}: H={H} T={T} bs={bs} cuts={cuts} heads={per_head}", flush=True)
    NB = T // bs
    docs = _docs(T, cuts)
    kv_num, kv_idx = _lists(T, bs, docs, per_head, seed=T + bs)
    users = _users(kv_num, kv_idx, NB)
    nch = (users + CHUNK - 1) // CHUNK
    for h, (_, G, _) in enumerate(per_head):
        # global heads hold blocks of 2+ chunks (one with a ragged last chunk); the others none at all
        if G:
            assert nch[h].max() >= 2, (h, users[h].max())
            if cuts:  # the first document's start block ends in a ragged chunk
                assert ((users[h] > CHUNK) & (users[h] % CHUNK != 0)).any(), (h, users[h].max())
        else:
            assert nch[h].max() == 1, (h, users[h].max())
    print(f"  users of the hottest block per head: {users.max(axis=1).tolist()} "
          f"(chunks {nch.max(axis=1).tolist()})", flush=True)

    gate = mode == "token-gate"
    mode = "token" if gate else mode
    q, k, v = qkv(H, T, seed=T + 3 * bs + H)
    g = torch.Generator().manual_seed(41)
    dout = torch.randn((1, H, T, 128), generator=g).to(torch.bfloat16)
    terms, tok_kw = {}, None
    if mode == "block":
        A, B = band_coefficients(q)
        terms = dict(coeff_cos=A, coeff_sin=B, omegas=omegas_block(8))
    elif mode == "token":
        K = 6
        terms = dict(coeff_cos=torch.randn((1, H, T, K), generator=g) * 0.3,
                     coeff_sin=torch.randn((1, H, T, K), generator=g) * 0.3,
                     omegas=OA.omegas_logspaced(K, 1024, 1 << 20))
        tok_kw = dict(b0=terms["coeff_cos"].sum(-1), slope=torch.randn((1, H, T), generator=g) * 0.002,
                      delta_main=torch.rand((1, H, T), generator=g) * 300,
                      width=32 + torch.rand((1, H, T), generator=g) * 200)
    pb = None
    if pair:
        pb = -3.0 * torch.rand(kv_idx.shape, generator=g, dtype=torch.float64)
        pb = torch.where(torch.arange(kv_idx.shape[-1])[None, None] < kv_num[..., None], pb, torch.zeros_like(pb))

    # GPU, through the C ABI
    extras = {}
    pbd = None
    if pair:
        pbd = pb.float().to(DEV).requires_grad_()
        extras["pair_bias"] = pbd
    bm = ScopeBlockMask(kv_num_blocks=kv_num[None].to(DEV), kv_indices=kv_idx[None].to(DEV), BLOCK_SIZE=bs,
                        docs=docs.to(DEV), ds_tok_end=torch.from_numpy(doc_start_blocks(docs.numpy(), bs)[2]).to(DEV),
                        extras=extras)
    qd, kd, vd = (x.to(DEV).requires_grad_() for x in (q, k, v))
    sp, leaves = None, []
    if mode != "none":
        cd, sd = terms["coeff_cos"].to(DEV).requires_grad_(), terms["coeff_sin"].to(DEV).requires_grad_()
        sp = scope_amd.SpectralTerms(coeff_cos=cd, coeff_sin=sd, omegas=terms["omegas"].to(DEV), offset=mode, beta=BETA)
        leaves = [cd, sd]
        if mode == "token":
            # without a gate delta_main and width do not enter the scores
            tok_names = ("b0", "slope", "delta_main", "width") if gate else ("b0", "slope")
            extra = {n: tok_kw[n].to(DEV).requires_grad_() for n in tok_names}
            sp.b0, sp.slope = extra["b0"], extra["slope"]
            sp.use_slope = sp.subtract_b0 = True
            if gate:
                sp.delta_main, sp.width = extra["delta_main"], extra["width"]
                sp.gate_kind, sp.ramp_lambda, sp.tau = "softplus", 0.2, 64.0
            leaves += [extra[n] for n in tok_names]
    out = scope_amd.scope_attention(qd, kd, vd, block_mask=bm, scale=SCALE, spectral=sp)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    print("  gpu done", flush=True)

    # fp64 oracle
    qq, kk, vv = (x[0].double().requires_grad_() for x in (q, k, v))
    kw = dict(bias_mode=mode)
    rleaves = []
    if mode != "none":
        rc, rs = terms["coeff_cos"][0].double().requires_grad_(), terms["coeff_sin"][0].double().requires_grad_()
        kw.update(coeff_cos=rc, coeff_sin=rs, omegas=terms["omegas"].double())
        rleaves = [rc, rs]
    if mode == "token":
        rt = {n: x[0].double().requires_grad_() for n, x in tok_kw.items()}
        gk = dict(gate="softplus", ramp_lambda=0.2, tau=64.0) if gate else dict(gate="none")
        kw["token_kwargs"] = dict(**gk, **rt)
        rleaves += [rt[n] for n in tok_names]
    pr = pb.clone().requires_grad_() if pair else None
    ro, _ = OA.scope_attention_blocksparse(qq, kk, vv, kv_num, kv_idx, docs, bs=bs, scale=SCALE, beta=BETA,
                                           pair_bias=pr, **kw)
    ro.backward(dout[0].double())

    names = ["dq", "dk", "dv", "dcoeff_cos", "dcoeff_sin", "db0", "dslope", "ddelta_main", "dwidth"]
    got = [qd.grad[0], kd.grad[0], vd.grad[0]] + [x.grad[0] for x in leaves]
    ref = [qq.grad, kk.grad, vv.grad] + [x.grad for x in rleaves]
    for name, gg, rr in zip(names, got, ref):
        ok, worst = tol_check(gg.float().cpu(), rr, ATOL, RTOL)
        print(f"  {name}: worst ratio {worst:.3f} (max |ref| {rr.abs().max().item():.3g})", flush=True)
        assert ok, f"{name} violates 2e-2 abs / 1e-2 rel: worst ratio {worst:.3f}"
    # the hot blocks themselves, named in the failure message
    for h in range(H):
        for kb in np.flatnonzero(nch[h] >= 2):
            sl = slice(int(kb) * bs, (int(kb) + 1) * bs)
            for name, gg, rr in (("dk", kd.grad[0, h, sl], kk.grad[h, sl]), ("dv", vd.grad[0, h, sl], vv.grad[h, sl])):
                ok, worst = tol_check(gg.float().cpu(), rr, ATOL, RTOL)
                assert ok, f"{name} of head {h} key block {kb} ({users[h, kb]} users): worst ratio {worst:.3f}"
    if pair:
        dref = pr.grad
        bar = 2e-2 * float(dref.abs().max())
        err = float((pbd.grad.double().cpu() - dref).abs().max())
        print(f"  dpair_bias: max err {err:.4g} (bar {bar:.4g})", flush=True)
        assert err <= bar

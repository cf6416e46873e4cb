"""GPU parity of the timed layer at its own shapes.

* The long-context prefill layer (T=131072, H=8, D=128, bs=256, window 2,
  2 doc-local global blocks, 16 documents at seeded positions, planted needle,
  radius prior, counter Gumbel noise) at pointer budgets 2, 4 and 8, built
  from the benchmark's own inputs and run by the benchmark's own step.
* The million-token layer (T=1048576, H=8, one document, window 2, one global
  block, budget 8): 2 GiB per bf16 tensor, so the last head's rows sit just
  under the 2^31-byte mark and the dK/dV partials span several GiB.

What is compared:

* lists: exactly the oracle's block-scoring selection on the kernel's own
  fp32 logits (block means + prior) with the oracle's counter noise;
* block means (million-token layer, every head): within 1e-6 of fp64;
* heads 0 and H-1, sampled q-blocks (the first, document-boundary blocks, the
  needle's q-block, a middle and the last block): out, lse, dq and the
  spectral coefficient gradients against the fp32 oracle;
* dK/dV of one ordinary key block against the fp32 oracle over every q-block
  that lists it;
* out and lse of every row of heads 0 and H-1 against a row reference: fp32
  torch on the device over each q-block's listed key blocks (the block term,
  the document-causal mask and the list applied as in the oracle), computed
  from q, k, v and the coefficients alone;
* dK/dV of every hot key block (more users than one kv-major work item
  takes: 32 q-blocks, 64 from 2048 key blocks per head; the global blocks
  whose sums run through the multi-chunk partials and the reduce; up to 4096
  users, 64 chunks, at a million tokens) against a column reference: the key
  block's column of P and dS in fp32 torch on the device from the row
  reference's lse and out (not the kernel's), and the same column reference
  is checked against the oracle on the ordinary key block.

Bar written in every comparison: |got - ref| <= 2e-2 + 1e-2·|ref|."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import pointer as OP
from tests.helpers import tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
SCALE, BETA = 0.12, 0.5


def _chunk(NB: int) -> int:
    """q-blocks per kv-major work item: 32, or 64 from 2048 key blocks per head."""
    return 64 if NB >= 2048 else 32


def _rows_ref(h, bs, q, k, v, kv_num, kv_idx, docs, cc, cs, om, batch=32):
    """out [T, D] and lse [T] (fp32, natural log) of every row of head h: each
    q-block attends over its first kv_num listed key blocks with
    s = scale·q·k + β·Σ_k (A_k cos ω_k r + B_k sin ω_k r), r = qb - kb, and the
    document-causal mask; fp32 torch on the device, q-blocks in batches."""
    T, D = q.shape[2], q.shape[3]
    NB, L = T // bs, kv_idx.shape[-1]
    Qh, Kh, Vh = q[0, h], k[0, h], v[0, h]
    ar = torch.arange(bs, device=DEV)
    out = torch.empty((T, D), dtype=torch.float32, device=DEV)
    lse = torch.empty(T, dtype=torch.float32, device=DEV)
    for i0 in range(0, NB, batch):
        qb = torch.arange(i0, min(NB, i0 + batch), device=DEV)
        G = qb.numel()
        idx = kv_idx[h, qb].long()  # [G, L]
        valid = torch.arange(L, device=DEV)[None] < kv_num[h, qb][:, None]
        keys = (idx[..., None] * bs + ar).reshape(G, L * bs)
        rows = (qb[:, None] * bs + ar).reshape(G, bs)
        s = SCALE * torch.matmul(Qh[rows].float(), Kh[keys].float().transpose(1, 2).contiguous())  # [G, bs, L·bs]
        ph = (qb[:, None] - idx).float()[..., None] * om  # [G, L, K]
        bt = torch.matmul(cc[0, h][rows], torch.cos(ph).transpose(1, 2).contiguous())
        bt = BETA * (bt + torch.matmul(cs[0, h][rows], torch.sin(ph).transpose(1, 2).contiguous()))  # [G, bs, L]
        s = s.view(G, bs, L, bs) + bt[..., None]
        ok = (valid[:, None, :, None] & (keys.view(G, 1, L, bs) <= rows.view(G, bs, 1, 1))
              & (docs[keys].view(G, 1, L, bs) == docs[rows].view(G, bs, 1, 1)))
        s = torch.where(ok, s, torch.full_like(s, -math.inf)).view(G, bs, L * bs)
        lg = torch.logsumexp(s, dim=-1)  # [G, bs]; -inf for a row without visible keys
        p = torch.where(torch.isinf(lg)[..., None], torch.zeros_like(s), torch.exp(s - lg[..., None]))
        out[rows.reshape(-1)] = torch.matmul(p, Vh[keys].float()).reshape(G * bs, D)
        lse[rows.reshape(-1)] = lg.reshape(-1)
    return out, lse


def _check_dev(name, got, want):
    """The bar on the device (float64), for whole heads."""
    got, want = got.double(), want.double()
    both_inf = torch.isinf(got) & torch.isinf(want) & (torch.sign(got) == torch.sign(want))
    err = torch.where(both_inf, torch.zeros_like(got), (got - want).abs())
    ratio = (err / (2e-2 + 1e-2 * want.abs().nan_to_num(posinf=0.0, neginf=0.0))).nan_to_num(nan=math.inf)
    worst = float(ratio.max())
    print(f"    {name}: worst ratio {worst:.3f}", flush=True)
    assert worst <= 1.0, f"{name}: worst tolerance ratio {worst:.3f}"


def _column_ref(h, kb, bs, q, k, v, dout, out, lse, kv_num, kv_idx, docs, cc, cs, om):
    """dK, dV [bs, D] of key block kb in head h: fp32 torch on the device,
    P_ij = exp(s_ij - lse_i) over the rows whose q-block lists kb,
    dS = P∘(dO·V^T - rowsum(dO∘O)), dV = P^T·dO, dK = scale·dS^T·Q.
    out [T, D] and lse [T] are head h's rows (the row reference's)."""
    T = q.shape[2]
    cols = slice(kb * bs, (kb + 1) * bs)
    Qh, dO = q[0, h].float(), dout[0, h].float()
    Kb, Vb = k[0, h, cols].float(), v[0, h, cols].float()
    L = kv_idx.shape[-1]
    listed = ((kv_idx[h] == kb) & (torch.arange(L, device=DEV)[None] < kv_num[h][:, None])).any(-1)  # [QB]
    rowq = torch.arange(T, device=DEV) // bs
    s = SCALE * (Qh @ Kb.T)
    ph = om[None, :] * (rowq - kb).float()[:, None]  # [T, K]
    s = s + BETA * (cc[0, h] * torch.cos(ph) + cs[0, h] * torch.sin(ph)).sum(-1)[:, None]
    i = torch.arange(T, device=DEV)[:, None]
    j = torch.arange(kb * bs, (kb + 1) * bs, device=DEV)[None, :]
    ok = (i >= j) & (docs[:, None] == docs[cols][None, :]) & listed[rowq][:, None]
    P = torch.where(ok, torch.exp(s - lse[:, None]), torch.zeros_like(s))
    del s
    dV = P.T @ dO
    dS = P * (dO @ Vb.T - (dO * out).sum(-1)[:, None])
    dK = SCALE * (dS.T @ Qh)
    return dK.cpu(), dV.cpu()


def _oracle_rows(h, rows, kb_users, bs, q, k, v, dout, docs, kv_num, kv_idx, cc, cs, om):
    """fp32 oracle over head h's q-blocks `rows`: per-block (out, lse) and
    the gradients of Σ_rows ⟨out, dout⟩ w.r.t. q, k, v, coeff_cos, coeff_sin."""
    qq, kk, vv = (x[0, h:h + 1].float().cpu().requires_grad_() for x in (q, k, v))
    rc, rs = (x[0, h:h + 1].float().cpu().requires_grad_() for x in (cc, cs))
    res = OA.attention_blocksparse(qq, kk, vv, kv_num[h:h + 1].cpu(), kv_idx[h:h + 1].cpu(), docs.cpu(), bs=bs,
                                   scale=SCALE, beta=BETA, bias_mode="block", coeff_cos=rc, coeff_sin=rs,
                                   omegas=om.cpu(), heads=[0], qblocks=sorted(set(rows) | set(kb_users)))
    loss = 0.0
    do = dout[0, h].float().cpu()
    for qb, (o, _) in res.items():
        loss = loss + (o * do[qb[1] * bs:(qb[1] + 1) * bs]).sum()
    loss.backward()
    return res, qq.grad[0], kk.grad[0], vv.grad[0], rc.grad[0], rs.grad[0]


def _users(q_off, q_list, h, kb):
    o0, o1 = int(q_off[h, kb]), int(q_off[h, kb + 1])
    return sorted(set(q_list[h, o0:o1].tolist()))


def _check(name, got, want):
    ok, worst = tol_check(got, want)
    print(f"    {name}: worst ratio {worst:.3f}", flush=True)
    assert ok, f"{name}: worst tolerance ratio {worst:.3f}"


def _layer_checks(step, inp, heads, sample_qbs, bs, n_hot_max=None):
    """The comparisons of the module docstring on one run of the bench step."""
    t, last = step.t, step.last
    kv_num, kv_idx = last["kv_num"], last["kv_idx"]
    q_off, q_list = last["q_off"].cpu(), last["q_list"].cpu()
    out, lse, gr = last["out"], last["lse"], last["grads"]
    NB = kv_num.shape[-1]
    docs = t["docs"]
    om = t["omegas"].float()
    for h in heads:
        print(f"  head {h}", flush=True)
        # an ordinary key block (fp32 oracle over all of its users) and every hot one (column reference)
        kb_o = next(kb for kb in range(NB // 3, NB) if 1 <= len(_users(q_off, q_list, h, kb)) <= _chunk(NB))
        users_o = _users(q_off, q_list, h, kb_o)
        res, gq, gk, gv, gc, gs = _oracle_rows(h, sample_qbs, users_o, bs, t["q"], t["k"], t["v"], t["dout"], docs,
                                               kv_num, kv_idx, t["coeff_cos"], t["coeff_sin"], om)
        for qb in sample_qbs:
            sl = slice(qb * bs, (qb + 1) * bs)
            ro, rl = res[(0, qb)]
            print(f"   q-block {qb} ({int(kv_num[h, qb])} listed)", flush=True)
            _check("out", out[0, h, sl].float().cpu(), ro.detach())
            _check("lse", lse[0, h, sl].cpu(), rl.detach())
            _check("dq", gr["dq"][0, h, sl].float().cpu(), gq[sl])
            _check("dcoeff_cos", gr["dcoeff_cos"][0, h, sl].cpu(), gc[sl])
            _check("dcoeff_sin", gr["dcoeff_sin"][0, h, sl].cpu(), gs[sl])
        sl = slice(kb_o * bs, (kb_o + 1) * bs)
        print(f"   key block {kb_o} ({len(users_o)} users)", flush=True)
        _check("dk", gr["dk"][0, h, sl].float().cpu(), gk[sl])
        _check("dv", gr["dv"][0, h, sl].float().cpu(), gv[sl])
        # every row of the head: the row reference against the oracle's
        # sampled blocks, then the kernel against the row reference
        ro_all, rl_all = _rows_ref(h, bs, t["q"], t["k"], t["v"], kv_num, kv_idx, docs, t["coeff_cos"],
                                   t["coeff_sin"], om)
        for qb in sample_qbs:
            sl_q = slice(qb * bs, (qb + 1) * bs)
            ro, rl = res[(0, qb)]
            _check(f"row reference out of q-block {qb} vs oracle", ro_all[sl_q].cpu(), ro.detach())
            _check(f"row reference lse of q-block {qb} vs oracle", rl_all[sl_q].cpu(), rl.detach())
        print(f"   every row of head {h}", flush=True)
        _check_dev("out", out[0, h].float(), ro_all)
        _check_dev("lse", lse[0, h], rl_all)
        ck, cv = _column_ref(h, kb_o, bs, t["q"], t["k"], t["v"], t["dout"], ro_all, rl_all, kv_num, kv_idx, docs,
                             t["coeff_cos"], t["coeff_sin"], om)
        _check("column reference dk vs oracle", ck, gk[sl])
        _check("column reference dv vs oracle", cv, gv[sl])
        n_users = np.diff(q_off[h].numpy())
        hot = np.flatnonzero(n_users > _chunk(NB))
        assert hot.size, f"no key block with more than {_chunk(NB)} users"
        if n_hot_max is not None:
            hot = hot[np.argsort(-n_users[hot], kind="stable")][:n_hot_max]
        for kb in hot.tolist():
            ck, cv = _column_ref(h, kb, bs, t["q"], t["k"], t["v"], t["dout"], ro_all, rl_all, kv_num, kv_idx,
                                 docs, t["coeff_cos"], t["coeff_sin"], om)
            sl = slice(kb * bs, (kb + 1) * bs)
            print(f"   hot key block {kb} ({int(n_users[kb])} users, {-(-int(n_users[kb]) // _chunk(NB))} chunks)",
                  flush=True)
            _check("dk", gr["dk"][0, h, sl].float().cpu(), ck)
            _check("dv", gr["dv"][0, h, sl].float().cpu(), cv)
        del ro_all, rl_all


def _lists_vs_oracle(step, window, n_global, budget):
    """The step's lists = the oracle's selection on the kernel's own logits."""
    from scope_amd import ops

    t = step.t
    bs, NB, H = step.bs, step.NB, step.H
    ds_ptr, ds_local, _ = ops.doc_starts(t["docs"], bs)
    qbar, kbar = ops.block_means(t["q"], t["k"], bs)
    ls = bs / math.sqrt(t["q"].shape[-1])
    kv_num, kv_idx, picks, lg = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=window,
                                                   n_global=n_global, budget=budget, qbar=qbar, kbar=kbar,
                                                   prior=step.prior, temp=1.0, logit_scale=ls, noise="counter",
                                                   seed=step.seed, return_logits=True)
    assert torch.equal(kv_num, step.last["kv_num"]) and torch.equal(kv_idx, step.last["kv_idx"])
    hh, qq, kk = np.meshgrid(np.arange(H), np.arange(NB), np.arange(NB), indexing="ij")
    g = OP.gumbel_from_u(OP.counter_uniform(step.seed, hh, qq, kk))
    ref = OP.pointer_select_blockscore(lg.cpu().numpy(), t["docs"].cpu().numpy(), bs=bs, window=window,
                                       n_global=n_global, budget=budget, gumbel=g)
    assert np.array_equal(picks.cpu().numpy(), ref["picks"])
    assert np.array_equal(kv_idx.cpu().numpy(), ref["packed"])
    return ref


@pytest.fixture(scope="module")
def c3_inputs():
    import bench

    print("C3 inputs (T=131072, H=8)", flush=True)
    return bench.make_inputs(8, 131072, 128, 256)


@pytest.mark.parametrize("budget", [2, 4, 8])
def test_c3_layer_vs_oracle(c3_inputs, budget):
    import bench

    inp = c3_inputs
    bs, W, G = 256, 2, 2
    print(f"C3 layer budget {budget}", flush=True)
    step = bench.Step(inp, bs=bs, window=W, n_global=G, budget=budget)
    step()
    torch.cuda.synchronize()
    NB = step.NB
    ref = _lists_vs_oracle(step, W, G, budget)
    print(f"  lists exact (N_act {int(ref['kv_num'].sum())})", flush=True)
    qb_n, kb_n = inp["needle"]
    if budget == 8:  # the planted needle wins in every head
        assert bool((step.last["picks"][:, qb_n] == kb_n).any(dim=-1).all())
    docs = inp["docs"]
    cuts = torch.nonzero(docs[1:] != docs[:-1]).flatten() + 1
    boundary = sorted({int(c) // bs for c in cuts})[:5]
    sample = sorted({0, qb_n, NB // 2 + 1, NB - 1, *boundary})
    _layer_checks(step, inp, [0, 7], sample, bs)


def test_c5_h8_layer():
    """The million-token layer at H=8 (the bench's --T 1048576 --n-global 1 --docs 1 --no-needle)."""
    import bench
    from scope_amd import ops

    H, T, D, bs = 8, 1 << 20, 128, 256
    NB = T // bs
    print(f"C5 inputs T={T} H={H} (device generator)", flush=True)
    g = torch.Generator(device=DEV).manual_seed(21)
    inp = {n: torch.randn((1, H, T, D), generator=g, device=DEV).to(torch.bfloat16) for n in ("q", "k", "v", "dout")}
    W_b = torch.randn((D, 16), generator=torch.Generator().manual_seed(22)) * 0.02
    c = inp["q"].float() @ W_b.to(DEV)
    inp["coeff_cos"], inp["coeff_sin"] = c[..., :8].contiguous(), c[..., 8:].contiguous()
    del c
    inp["docs"] = torch.zeros(T, dtype=torch.int32, device=DEV)
    inp["omegas"] = torch.tensor([math.pi * 2.0 ** (-i) for i in range(8)], dtype=torch.float32, device=DEV)
    # block means of every head within 1e-6 of fp64
    qbar, kbar = ops.block_means(inp["q"], inp["k"], bs)
    for h in range(H):
        for name, got, x in (("q", qbar, inp["q"]), ("k", kbar, inp["k"])):
            want = x[0, h].double().reshape(NB, bs, D).mean(dim=1)
            err = float((got[h].double() - want).abs().max())
            assert err < 1e-6, f"block mean of {name}, head {h}: {err:.3g}"
    print("  block means within 1e-6 of fp64 in every head", flush=True)
    step = bench.Step(inp, bs=bs, window=2, n_global=1, budget=8)
    step()
    torch.cuda.synchronize()
    print(f"  layer done (N_act {int(step.last['kv_num'].sum())})", flush=True)
    # the selection over 4096 candidates (logits on bf16 MFMA from the split means at this length):
    # the step's lists again with the logits returned, each sampled row's
    # logits within 1e-4·(1 + |ref|) of fp64 from the block means, and heads
    # 0 and H-1 equal to the oracle's selection on those logits
    ds_ptr, ds_local, _ = ops.doc_starts(inp["docs"], bs)
    ls = bs / math.sqrt(D)
    kv_num, kv_idx, picks, lg = ops.pointer_select(ds_ptr, ds_local, bs=bs, NB=NB, H=H, window=2, n_global=1,
                                                   budget=8, qbar=qbar, kbar=kbar, prior=step.prior, temp=1.0,
                                                   logit_scale=ls, noise="counter", seed=step.seed,
                                                   return_logits=True)
    assert torch.equal(kv_num, step.last["kv_num"]) and torch.equal(kv_idx, step.last["kv_idx"])
    prior64 = step.prior.double().cpu()
    for h in (0, H - 1):
        rows = [0, 1, 777, NB // 2, NB - 2, NB - 1]
        q64, k64 = qbar[h, rows].double().cpu(), kbar[h].double().cpu()
        want = ls * (q64 @ k64.T)
        for i, qb in enumerate(rows):
            want[i, :qb + 1] += prior64[qb - torch.arange(qb + 1)]
            got = lg[h, qb, :qb + 1].double().cpu()
            err = float(((got - want[i, :qb + 1]).abs() / (1 + want[i, :qb + 1].abs())).max())
            assert err <= 1e-4, f"head {h}, q-block {qb}: logits off by {err:.3g}"
        lgh = lg[h:h + 1].cpu().numpy()
        qq, kk = np.meshgrid(np.arange(NB), np.arange(NB), indexing="ij")
        gh = OP.gumbel_from_u(OP.counter_uniform(step.seed, np.full_like(qq, h), qq, kk))[None]
        ref = OP.pointer_select_blockscore(lgh, inp["docs"].cpu().numpy(), bs=bs, window=2, n_global=1, budget=8,
                                           gumbel=gh)
        assert np.array_equal(picks[h:h + 1].cpu().numpy(), ref["picks"]), f"picks of head {h}"
        assert np.array_equal(kv_idx[h:h + 1].cpu().numpy(), ref["packed"]), f"lists of head {h}"
        print(f"  head {h}: logits within 1e-4 of fp64, lists equal to the oracle's selection", flush=True)
    del lg
    sample = [0, NB // 2 + 3, NB - 1]
    _layer_checks(step, inp, [0, H - 1], sample, bs, n_hot_max=2)

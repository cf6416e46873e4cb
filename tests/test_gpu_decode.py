"""Decode path on the GPU: scope_decode_attn against the fp64 oracle; the
decoder's token loop against its own prefill (KV cache, rotary positions,
value embeddings, skips and the per-block lists) on a window that lists every
causal block, so that both paths attend over the same keys; and the
decode-time pointer reselection against the oracle's block-scoring choice.
Bars (written in each comparison): attention |got - ref| <= 2e-2 +
1e-2·|ref|; logits of the bf16 model |step - prefill| <= 5e-2 (the logits are
30·σ(x/7.5), in [0, 30]) with equal argmax."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import pointer as OP
from tests.helpers import docs_with_boundaries, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("bs,t", [(128, 0), (128, 1000), (128, 1023), (256, 2047), (64, 777)])
def test_decode_attn_vs_oracle(bs, t):
    from scope_amd import ops

    H, T_cap, D = 4, 2048, 128
    print(f"decode attn bs={bs} t={t}", flush=True)
    g = torch.Generator().manual_seed(t + bs)
    kc = torch.randn((H, T_cap, D), generator=g).to(torch.bfloat16)
    vc = torch.randn((H, T_cap, D), generator=g).to(torch.bfloat16)
    q = torch.randn((H, D), generator=g).to(torch.bfloat16)
    docs = docs_with_boundaries(T_cap, 4, seed=t)
    qb = t // bs
    maxkv = 6
    kv_idx = torch.zeros((H, maxkv), dtype=torch.int32)
    kv_num = torch.zeros(H, dtype=torch.int32)
    for h in range(H):
        cand = sorted(set([qb, max(qb - 1, 0), 0] + torch.randint(0, qb + 1, (3,), generator=g).tolist()))
        kv_num[h] = len(cand)
        kv_idx[h, :len(cand)] = torch.tensor(cand)
    out, lse = ops.decode_attn(q.to(DEV), kc.to(DEV), vc.to(DEV), kv_num.to(DEV), kv_idx.to(DEV), docs.to(DEV), t,
                               bs=bs, scale=0.12)
    ro, rl = OA.decode_attention(q.double(), kc.double(), vc.double(), kv_num, kv_idx, docs, t, bs=bs, scale=0.12)
    for name, a, b in (("out", out, ro), ("lse", lse, rl)):
        ok, worst = tol_check(a.float().cpu(), b)
        assert ok, f"{name}: worst tolerance ratio {worst:.3f}"
    # the position read from device memory (scope_decode_attn_at) gives the same result
    args = (q.to(DEV), kc.to(DEV), vc.to(DEV), kv_num.to(DEV), kv_idx.to(DEV), docs.to(DEV))
    out2, lse2 = ops.decode_attn(*args, torch.tensor([t], dtype=torch.int64, device=DEV), bs=bs, scale=0.12)
    assert torch.equal(out2, out) and torch.equal(lse2, lse)
    # a device position outside the cache: no mass, zero output (checked in the kernel)
    out3, lse3 = ops.decode_attn(*args, torch.tensor([T_cap], dtype=torch.int64, device=DEV), bs=bs, scale=0.12)
    assert torch.all(out3.float() == 0) and torch.all(lse3 == -float("inf"))


def test_qkv_glue_matches_torch_ops():
    """The fused glue against the torch ops it replaces (scoped_medium.py:
    339-345: rms_norm of q and k, the half-truncated Rotary, v = a·v + b·ve):
    v bit-exact, q and k equal up to the norm's sum order (under 1% of the
    elements, by at most 2^-6 on rows of RMS 1); with caches, k and v land in rows pos and nowhere else; a
    position outside the tables writes a zero q and no cache row."""
    from scope_amd import ops
    from scope_amd.decode import _Rotary, _norm

    H, D, T, rows = 4, 128, 300, 512
    print(f"qkv glue T={T} H={H}", flush=True)
    g = torch.Generator().manual_seed(11)
    qkv = (torch.randn((T, 3 * H * D), generator=g) * 2).to(torch.bfloat16).to(DEV)
    ve = torch.randn((T, H * D), generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.randperm(rows, generator=g)[:T].to(DEV)
    rot = _Rotary(D, rows, DEV)
    q, k, v = qkv.view(T, 3 * H, D).chunk(3, dim=-2)
    q, k = rot(_norm(q), pos), rot(_norm(k), pos)
    v = 0.5 * v + 0.5 * ve.view_as(v)
    q2, k2, v2 = ops.decoder_qkv_glue(qkv, ve, pos, rot.cos, rot.sin, heads=H, va=0.5, vb=0.5)
    assert torch.equal(v2, v)
    for name, a, b in (("q", q2, q), ("k", k2, k)):
        # rows have RMS 1 after the norm: a one-step difference of a normed
        # value moves a rotated one by at most ~2^-7 (more than one step of a
        # small rotated value when its two terms cancel)
        d = (a.float() - b.float()).abs()
        assert d.max().item() <= 2.0 ** -6, f"{name}: max difference {d.max().item():.3e}"
        assert (d > 0).float().mean().item() < 0.01, f"{name}: too many differing elements"
    kc = torch.zeros((H, rows, D), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    q3, _, _ = ops.decoder_qkv_glue(qkv, ve, pos, rot.cos, rot.sin, heads=H, va=0.5, vb=0.5, k_out=kc, v_out=vc)
    assert torch.equal(q3, q2)
    assert torch.equal(kc[:, pos], k2.transpose(0, 1)) and torch.equal(vc[:, pos], v2.transpose(0, 1))
    untouched = torch.ones(rows, dtype=torch.bool, device=DEV)
    untouched[pos] = False
    assert torch.all(kc[:, untouched] == 0) and torch.all(vc[:, untouched] == 0)
    bad = torch.full((T,), rows, dtype=torch.int64, device=DEV)
    kc2 = torch.zeros_like(kc)
    vc2 = torch.zeros_like(kc)
    q4, _, _ = ops.decoder_qkv_glue(qkv, ve, bad, rot.cos, rot.sin, heads=H, va=0.5, vb=0.5, k_out=kc2, v_out=vc2)
    assert torch.all(q4.float() == 0) and torch.all(kc2 == 0) and torch.all(vc2 == 0)


def _small_model(window: int, max_len: int, use_graph: bool = True):
    from scope_amd.decode import DecoderConfig, ScopeDecoder

    cfg = DecoderConfig(vocab_size=50257, num_layers=6, num_heads=2, model_dim=256, head_dim=128, block_size=128,
                        window=window, budget=2, n_global=1, no_attn_layer=2)
    return ScopeDecoder(cfg, max_len=max_len, device=DEV, seed=3, use_graph=use_graph)


@pytest.mark.parametrize("N,K,norm,epi,skip", [(3072, 1024, True, "plain", True), (3072, 1024, True, "plain", False),
                                                (4096, 1024, True, "relu2", False), (1024, 4096, False, "resid", False),
                                                (1024, 1024, False, "resid", False), (50304, 1024, True, "logit", False),
                                                (13, 256, True, "relu2", True), (9, 2048, False, "logit", False),
                                                (768, 512, True, "resid", False)])
def test_decoder_gemv_matches_torch_ops(N, K, norm, epi, skip):
    """The fused row-vector products of the token step (decoder's sizes and
    ragged ones) against the torch chains they replace on the same bf16
    inputs: bf16(x + skip), F.rms_norm, F.linear, then relu(z)² / res + z /
    30·σ(z / 7.5).  The linear's fp32 sums run in another order than the
    library GEMM's, so z may round to a neighbouring bf16 value: the bar is
    two bf16 steps of |z| (plus one of the epilogue's own rounding), and at
    least 97% of the bf16 outputs equal."""
    import torch.nn.functional as F

    from scope_amd import ops

    print(f"decoder gemv N={N} K={K} norm={norm} epi={epi} skip={skip}", flush=True)
    g = torch.Generator().manual_seed(N * 7 + K)
    x = torch.randn(K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn((N, K), generator=g) * K ** -0.5).to(torch.bfloat16).to(DEV)
    s_ = torch.randn(K, generator=g).to(torch.bfloat16).to(DEV) if skip else None
    res = torch.randn(N, generator=g).to(torch.bfloat16).to(DEV) if epi == "resid" else None
    got = ops.decoder_gemv(x, w, norm=norm, epi=epi, res=res, addx=s_)
    xi = x
    if skip:
        got, xpost = got
        xi = x + s_
        assert torch.equal(xpost, xi)
    xn = F.rms_norm(xi, (K,)) if norm else xi
    z = F.linear(xn[None], w)[0]
    ref = {"plain": z, "relu2": F.relu(z).square(), "resid": (res + z) if res is not None else None,
           "logit": 30 * torch.sigmoid(z.float() / 7.5)}[epi]
    assert got.shape == ref.shape and got.dtype == ref.dtype
    zf, gf, rf = z.float(), got.float(), ref.float()
    step = 2.0 ** -8  # one bf16 step, relative
    grow = {"plain": 1.0, "relu2": 2.0 * zf.abs(), "resid": 1.0, "logit": 1.0}[epi]  # d(epi)/dz bound
    bar = 2 * step * zf.abs() * grow + step * rf.abs() + 1e-6
    err = (gf - rf).abs()
    assert bool((err <= bar).all()), f"max err {err.max().item():.3e} (worst ratio {(err / bar).max().item():.2f})"
    if epi != "logit":
        eq = (got == ref).float().mean().item()
        print(f"  equal bf16 outputs {eq:.4f}, max err {err.max().item():.3e}", flush=True)
        assert eq >= 0.97


def test_decoder_gemv_rejects_bad_arguments():
    from scope_amd import ops

    x = torch.zeros(1024, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((64, 1024), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="K in"):
        ops.decoder_gemv(torch.zeros(1000, dtype=torch.bfloat16, device=DEV), torch.zeros((64, 1000),
                         dtype=torch.bfloat16, device=DEV))
    with pytest.raises(ValueError, match="res is given"):
        ops.decoder_gemv(x, w, epi="resid")
    with pytest.raises(RuntimeError, match="aligned"):
        ops.decoder_gemv(torch.zeros(1028, dtype=torch.bfloat16, device=DEV)[4:], w)  # 8-byte offset
    with pytest.raises(RuntimeError, match="bfloat16"):
        ops.decoder_gemv(x.float(), w)


def test_decoder_step_prologue_matches_torch_ops():
    """The fused start of a token step against the torch ops it replaces:
    tokens[t] and docs[t] (t = 0, an end-of-text token opening a document,
    a plain token) exactly, the value-embedding rows exactly, x0 =
    F.rms_norm(embedding) within one bf16 step (the sum of squares runs in
    another order) and equal on at least 99% of its features; a token
    outside the vocabulary changes neither and gives zero rows."""
    import torch.nn.functional as F

    from scope_amd import ops

    V, dm, T_cap, eot = 50257, 1024, 256, 50256
    g = torch.Generator().manual_seed(17)
    embed = torch.randn((V, dm), generator=g).to(torch.bfloat16).to(DEV)
    ves = [torch.randn((V, dm), generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    tokens = torch.zeros(T_cap, dtype=torch.int64, device=DEV)
    docs = torch.zeros(T_cap, dtype=torch.int32, device=DEV)
    docs[:10] = 3
    for t, tk in ((0, 123), (10, eot), (11, 4567), (12, V + 5)):
        print(f"step prologue t={t} tok={tk}", flush=True)
        tok = torch.tensor([tk], dtype=torch.int64, device=DEV)
        td = torch.tensor([t], dtype=torch.int64, device=DEV)
        tok_before, doc_before = tokens.clone(), docs.clone()
        if tk >= V:
            x0, ve = ops.decoder_step_prologue(tok, td, tokens, docs, embed, ves[:2], eot=eot)
            torch.cuda.synchronize()
            assert torch.equal(tokens, tok_before) and torch.equal(docs, doc_before)
            assert torch.all(x0 == 0) and ve.shape == (2, dm) and torch.all(ve == 0)
            continue
        x0, ve = ops.decoder_step_prologue(tok, td, tokens, docs, embed, ves, eot=eot)
        exp_doc = (int(doc_before[t - 1]) if t > 0 else 0) + (1 if tk == eot else 0)
        assert int(tokens[t]) == tk and int(docs[t]) == exp_doc
        others = torch.ones(T_cap, dtype=torch.bool, device=DEV)
        others[t] = False
        assert torch.equal(tokens[others], tok_before[others]) and torch.equal(docs[others], doc_before[others])
        for i in range(3):
            assert torch.equal(ve[i], ves[i][tk])
        ref = F.rms_norm(embed[tk][None], (dm,))[0]
        err = (x0.float() - ref.float()).abs()
        assert bool((err <= 2.0 ** -8 * ref.float().abs() + 1e-6).all()), f"max err {err.max().item():.3e}"
        assert (x0 == ref).float().mean().item() >= 0.99


@pytest.mark.parametrize("bs,t,with_ve", [(128, 1000, True), (128, 1023, False), (64, 0, True), (256, 777, False)])
def test_decode_attn_glue_equals_glue_then_attention(bs, t, with_ve):
    """The glue fused into the decode attention against the glue kernel
    followed by the plain attention on copies of the same caches: the same
    output, LSE, q and cache rows, bit for bit (the same arithmetic; the
    fused kernel takes the token's own k, v row from LDS)."""
    from scope_amd import ops

    H, T_cap, D, maxkv = 4, 2048, 128, 6
    print(f"decode attn glue bs={bs} t={t} ve={with_ve}", flush=True)
    g = torch.Generator().manual_seed(bs + t)
    kc = torch.randn((H, T_cap, D), generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn((H, T_cap, D), generator=g).to(torch.bfloat16).to(DEV)
    qkv = torch.randn(3 * H * D, generator=g).to(torch.bfloat16).to(DEV)
    ve = torch.randn(H * D, generator=g).to(torch.bfloat16).to(DEV) if with_ve else None
    docs = docs_with_boundaries(T_cap, 4, seed=t).to(DEV)
    qb = t // bs
    kv_idx = torch.zeros((H, maxkv), dtype=torch.int32)
    kv_num = torch.zeros(H, dtype=torch.int32)
    for h in range(H):
        cand = sorted(set([qb, max(qb - 1, 0), 0] + torch.randint(0, qb + 1, (2,), generator=g).tolist()))
        kv_num[h] = len(cand)
        kv_idx[h, :len(cand)] = torch.tensor(cand)
    kv_num, kv_idx = kv_num.to(DEV), kv_idx.to(DEV)
    theta = torch.arange(T_cap, dtype=torch.float32)[:, None] * torch.rand(D // 2, generator=g)[None]
    cos, sin = theta.cos().to(DEV), theta.sin().to(DEV)
    td = torch.tensor([t], dtype=torch.int64, device=DEV)
    k2, v2 = kc.clone(), vc.clone()
    q_ref, _, _ = ops.decoder_qkv_glue(qkv[None], ve, td, cos, sin, heads=H, va=0.5, vb=0.5, k_out=k2, v_out=v2)
    o_ref, l_ref = ops.decode_attn(q_ref[0], k2, v2, kv_num, kv_idx, docs, td, bs=bs, scale=0.12)
    out, lse, q = ops.decode_attn_glue(qkv, ve, td, cos, sin, kc, vc, kv_num, kv_idx, docs, heads=H, va=0.5, vb=0.5,
                                       bs=bs, scale=0.12, want_q=True)
    assert torch.equal(q, q_ref[0])
    assert torch.equal(kc, k2) and torch.equal(vc, v2)
    assert torch.equal(out, o_ref) and torch.equal(lse, l_ref)


def test_argmax_matches_torch():
    """The greedy choice against torch.argmax: random logits, ties (the first
    index wins), the maximum in the last element, one element, -inf runs."""
    from scope_amd import ops

    g = torch.Generator().manual_seed(23)
    cases = [torch.rand(50257, generator=g) * 30, torch.zeros(5000), torch.arange(4096, dtype=torch.float32),
             torch.tensor([3.0]), torch.full((777,), -float("inf"))]
    cases[0][[100, 40000]] = 31.0  # a tie at the maximum
    cases[1][[17, 4000]] = 2.0
    for x in cases:
        xd = x.to(DEV)
        assert int(ops.argmax(xd)) == int(xd.argmax()), (x.numel(), int(ops.argmax(xd)), int(xd.argmax()))


def test_graph_steps_equal_eager_steps():
    """The steps inside a block run as one captured graph, replayed per
    token; every replay gives the logits of the eager step (same operations),
    across block opens and closes (positions 384 .. 533, blocks of 128) and
    with end-of-text tokens before and during the loop; each replay is
    followed by eager work (the comparison) and a synchronization."""
    T0, n = 384, 150
    g = torch.Generator().manual_seed(9)
    toks = torch.randint(0, 50257, (T0 + n,), generator=g)
    toks[[100, 450, 520]] = 50256
    print("graph steps vs eager steps", flush=True)
    eager = _small_model(window=8, max_len=1024, use_graph=False)
    graph = _small_model(window=8, max_len=1024, use_graph=True)
    eager.prefill(toks[:T0])
    graph.prefill(toks[:T0])
    worst = 0.0
    for s_ in range(n):
        a = eager.step(toks[T0 + s_])
        b = graph.step(toks[T0 + s_])
        torch.cuda.synchronize()
        d = (a - b).abs().max().item()
        worst = max(worst, d)
        assert d <= 1e-6, f"position {T0 + s_}: |graph - eager| = {d:.3e}"
        assert int(a.argmax()) == int(b.argmax())
    assert graph._graph is not None, "no step ran as a graph"
    assert torch.equal(eager.k_cache[0], graph.k_cache[0]) and torch.equal(eager.docs, graph.docs)
    assert int(graph._t_dev.item()) == graph.t == T0 + n
    print(f"  max |graph - eager| {worst:.3e}", flush=True)


def test_token_loop_matches_prefill():
    """Prefill 384 tokens, then 140 steps (crossing the block starts at 384
    and 512, with end-of-text tokens opening documents before and during the
    loop) equal the prefill of the whole sequence at those positions."""
    T0, n = 384, 140
    g = torch.Generator().manual_seed(5)
    toks = torch.randint(0, 50257, (768,), generator=g)
    toks[[50, 300, 450]] = 50256
    print("token loop vs prefill", flush=True)
    m = _small_model(window=8, max_len=1024)
    m.prefill(toks[:T0])
    got = torch.stack([m.step(toks[T0 + s]) for s in range(n)])
    full = _small_model(window=8, max_len=1024)
    ref = full.prefill(toks[:640], all_logits=True)[T0:T0 + n]
    err = (got - ref).abs().max().item()
    print(f"  max |step - prefill| logit diff {err:.3e}", flush=True)
    assert err <= 5e-2, f"max logit difference {err:.3e}"
    agree = (got.argmax(-1) == ref.argmax(-1)).float().mean().item()
    assert agree == 1.0, f"argmax agreement {agree:.3f}"


def test_block_start_reselection_matches_oracle_choice():
    """At a q-block's first position each layer reselects its list from the
    new token's query (the block's only known query) and the cached key-block
    means: for the first attention layer the list equals the oracle's
    block-scoring selection on the same logits."""
    import torch.nn.functional as F

    from scope_amd.decode import _norm

    m = _small_model(window=2, max_len=2048)
    cfg = m.cfg
    T0 = 1024
    g = torch.Generator().manual_seed(6)
    toks = torch.randint(0, 50257, (T0 + 1,), generator=g)
    toks[[200, 700]] = 50256
    print("block-start reselection", flush=True)
    m.prefill(toks[:T0])
    m.step(toks[T0])
    qb = T0 // cfg.block_size
    nb = qb + 1
    D = cfg.head_dim
    i0 = next(i for i, lay in enumerate(m.layers) if "qkv" in lay)
    assert i0 == 0  # its input is x0 alone, so its query can be recomputed here
    lay = m.layers[i0]
    with torch.no_grad():
        tok = toks[T0:T0 + 1].to(DEV)
        x0 = _norm(F.embedding(tok, m.embed))
        a, b = lay["lambdas"]
        q, _, _ = m._qkv(lay, _norm(a * x0 + b * x0), m._ve(tok)[i0], torch.tensor([T0], device=DEV))
    qbar = np.zeros((cfg.num_heads, nb, D), dtype=np.float64)
    qbar[:, qb] = q[0].double().cpu().numpy()
    kbar = m.kbar[i0][:, :nb].double().cpu().numpy()
    logits = (cfg.block_size / math.sqrt(D)) * np.einsum("hqd,hkd->hqk", qbar, kbar)
    docs = m.docs[:nb * cfg.block_size].cpu().numpy()
    ref = OP.pointer_select_blockscore(logits.astype(np.float32), docs, bs=cfg.block_size, window=cfg.window,
                                       n_global=cfg.n_global, budget=cfg.budget)
    kv_num, kv_idx = m.list_num[i0].cpu(), m.list_idx[i0].cpu()
    for h in range(cfg.num_heads):
        want = ref["packed"][h, qb, :ref["kv_num"][h, qb]]
        assert list(kv_idx[h, :int(kv_num[h])].numpy()) == list(want), h


def test_block_start_reselection_every_layer_full_config():
    """The full decoder configuration (16 layers, d_model 1024, window 4,
    budget 4, one global block) after a 20-block prompt with three documents:
    at the next block start, every attention layer's reselection (the new
    token's query against the cached key-block means of blocks 0..20) gives
    logits within 1e-4·(1 + |ref|) of fp64 from the recorded query and means
    (on the candidates: the kernel marks the window, the global block and
    later blocks -inf), and lists equal to the oracle's block-scoring
    selection on those logits."""
    from scope_amd.decode import DecoderConfig, ScopeDecoder

    cfg = DecoderConfig()
    bs, D = cfg.block_size, cfg.head_dim
    T0 = 20 * bs
    g = torch.Generator().manual_seed(8)
    toks = torch.randint(0, 50257, (T0 + 1,), generator=g)
    toks[[100, 200]] = 50256  # the current document starts in block 1: 15 candidates beyond window and global
    print("full-config block-start reselection, every layer", flush=True)
    m = ScopeDecoder(cfg, max_len=T0 + bs, device=DEV, seed=0, use_graph=False)
    m.prefill(toks[:T0])
    m.record = {}
    m.step(toks[T0])
    torch.cuda.synchronize()
    qb = T0 // bs
    nb = qb + 1
    docs = m.docs[:nb * bs].cpu().numpy()
    layers = sorted(m.record)
    assert layers == [i for i, lay in enumerate(m.layers) if "qkv" in lay] and len(layers) == cfg.num_layers - 1
    n_far = 0
    for i in layers:
        rec = m.record[i]
        lg = rec["logits"].cpu()
        want = (bs / math.sqrt(D)) * torch.einsum("hd,hkd->hk", rec["q"].double().cpu(), m.kbar[i][:, :nb].double().cpu())
        fin = torch.isfinite(lg[:, qb])  # the window, the global block and later blocks are no candidates
        assert bool((fin.sum(-1) > cfg.budget).all()), f"layer {i}: the selection has no choice to make"
        err = ((lg[:, qb].double() - want).abs() / (1 + want.abs()))[fin].max().item()
        assert err <= 1e-4, f"layer {i}: logits off by {err:.3g}"
        ref = OP.pointer_select_blockscore(lg.numpy(), docs, bs=bs, window=cfg.window, n_global=cfg.n_global,
                                           budget=cfg.budget)
        kv_num, kv_idx = rec["kv_num"].cpu(), rec["kv_idx"].cpu()
        got_num, got_idx = m.list_num[i].cpu(), m.list_idx[i].cpu()
        for h in range(cfg.num_heads):
            want_list = list(ref["packed"][h, qb, :ref["kv_num"][h, qb]])
            assert list(kv_idx[h, qb, :int(kv_num[h, qb])].numpy()) == want_list, (i, h)
            assert list(got_idx[h, :int(got_num[h])].numpy()) == want_list, (i, h)
            n_far += sum(1 for kb in want_list if kb < qb - cfg.window + 1 and kb != 0)
    print(f"  {len(layers)} layers x {cfg.num_heads} heads equal the oracle; {n_far} picks outside the window "
          f"and the global block", flush=True)
    assert n_far > 0

"""GPU parity of kernel 2 (block-sparse attention with the spectral bias)
against the fp64 dense-masked oracle.  Bar (written in every comparison):
|got - ref| <= 2e-2 + 1e-2·|ref| elementwise, for outputs, LSE and gradients."""
from __future__ import annotations

import pytest
import torch

from oracle import attention as OA
from tests.helpers import band_coefficients, docs_with_boundaries, omegas_block, qkv, random_blockscore_mask, tol_check

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-2, 1e-2
SCALE, BETA = 0.12, 0.5


def _token_terms(H, T, K, seed, gate="softplus"):
    g = torch.Generator().manual_seed(seed)
    cc = torch.randn((1, H, T, K), generator=g) * 0.3
    cs = torch.randn((1, H, T, K), generator=g) * 0.3
    b0 = cc.sum(-1)
    slope = torch.randn((1, H, T), generator=g) * 0.002
    dm = torch.rand((1, H, T), generator=g) * 300
    wd = 32 + torch.rand((1, H, T), generator=g) * 200
    om = OA.omegas_logspaced(K, 1024, 1 << 20)
    return dict(coeff_cos=cc, coeff_sin=cs, omegas=om, b0=b0, slope=slope, delta_main=dm, width=wd, gate=gate)


def _run_fwd(q, k, v, kv_num, kv_idx, docs, bs, mode, terms):
    from scope_amd import ops
    from scope_amd.attention import spectral_table

    kw = dict(bias_mode=mode)
    if mode != "none":
        kw.update(table=spectral_table(terms["omegas"].to(DEV), q.shape[2], bs, mode),
                  coeff_cos=terms["coeff_cos"].to(DEV), coeff_sin=terms["coeff_sin"].to(DEV))
    if mode == "token":
        gate = terms["gate"]
        kw.update(b0=terms["b0"].to(DEV), slope=terms["slope"].to(DEV), delta_main=terms["delta_main"].to(DEV),
                  width=terms["width"].to(DEV), use_slope=True, subtract_b0=True, gate_kind=gate, ramp_lambda=0.2,
                  tau=64.0)
    return ops.attn_fwd(q.to(DEV), k.to(DEV), v.to(DEV), kv_num.to(DEV), kv_idx.to(DEV), docs.to(DEV),
                        ds_tok_end_of(docs, bs).to(DEV), bs=bs, scale=SCALE, beta=BETA, **kw)


def ds_tok_end_of(docs, bs):
    from oracle.pointer import doc_start_blocks

    return torch.from_numpy(doc_start_blocks(docs.numpy(), bs)[2])


def _oracle(q, k, v, kv_num, kv_idx, docs, bs, mode, terms):
    H = q.shape[1]
    kw = dict(bias_mode=mode)
    if mode != "none":
        kw.update(coeff_cos=terms["coeff_cos"][0].double(), coeff_sin=terms["coeff_sin"][0].double(),
                  omegas=terms["omegas"].double())
    if mode == "token":
        kw["token_kwargs"] = dict(b0=terms["b0"][0].double(), slope=terms["slope"][0].double(),
                                  delta_main=terms["delta_main"][0].double(), width=terms["width"][0].double(),
                                  gate=terms["gate"], ramp_lambda=0.2, tau=64.0)
    return OA.scope_attention_reference(q[0].double(), k[0].double(), v[0].double(), kv_num, kv_idx, docs, bs=bs,
                                        scale=SCALE, beta=BETA, **kw)


CASES = [
    # (H, T, bs, mode, n_docs, W, G, B)
    (2, 1024, 128, "none", 1, 2, 1, 2),
    (2, 1024, 128, "block", 3, 2, 1, 2),
    (2, 2048, 256, "block", 4, 2, 2, 3),
    (2, 1024, 128, "token", 3, 2, 1, 2),
    (1, 2048, 256, "token", 2, 2, 1, 2),
    (2, 2048, 256, "none", 6, 1, 0, 4),
]


@pytest.mark.parametrize("H,T,bs,mode,n_docs,W,G,B", CASES)
def test_attn_fwd_vs_dense_oracle(H, T, bs, mode, n_docs, W, G, B):
    print(f"fwd H={H} T={T} bs={bs} mode={mode} docs={n_docs}", flush=True)
    q, k, v = qkv(H, T, seed=T + bs)
    docs = docs_with_boundaries(T, n_docs, seed=bs)
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=W, n_global=G, budget=B, seed=H + T)
    if mode == "block":
        A, Bc = band_coefficients(q)
        terms = dict(coeff_cos=A, coeff_sin=Bc, omegas=omegas_block(8))
    elif mode == "token":
        terms = _token_terms(H, T, 6, seed=T)
    else:
        terms = {}
    out, lse = _run_fwd(q, k, v, kv_num, kv_idx, docs, bs, mode, terms)
    ref_out, ref_lse = _oracle(q, k, v, kv_num, kv_idx, docs, bs, mode, terms)
    ok, worst = tol_check(out[0].float(), ref_out, ATOL, RTOL)
    assert ok, f"out violates 2e-2 abs / 1e-2 rel: worst ratio {worst:.3f}"
    ok, worst = tol_check(lse[0], ref_lse, ATOL, RTOL)
    assert ok, f"lse violates 2e-2 abs / 1e-2 rel: worst ratio {worst:.3f}"


def test_attn_fwd_strided_inputs_match_contiguous():
    """q/k/v as transposed [1,T,H,D] views (the reference's layout) give the
    same bits as contiguous [1,H,T,D]."""
    H, T, bs = 4, 2048, 256
    q, k, v = qkv(H, T, seed=3)
    docs = docs_with_boundaries(T, 3, seed=1)
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=2, n_global=1, budget=2, seed=5)
    A, Bc = band_coefficients(q)
    terms = dict(coeff_cos=A, coeff_sin=Bc, omegas=omegas_block(8))
    out_c, lse_c = _run_fwd(q, k, v, kv_num, kv_idx, docs, bs, "block", terms)
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    out_s, lse_s = _run_fwd(qt, kt, vt, kv_num, kv_idx, docs, bs, "block", terms)
    assert out_s.stride() == qt.stride()
    assert torch.equal(out_c.cpu(), out_s.cpu())
    assert torch.equal(lse_c.cpu(), lse_s.cpu())


def test_attn_fwd_c1_full_size_blocksparse_oracle():
    """Config 1 (H=6, T=4096, bs=128, window 3, global 1, budget 2, 8 block
    bands) over every q-block, against the block-sparse fp64 oracle."""
    H, T, bs = 6, 4096, 128
    q, k, v = qkv(H, T, seed=11)
    docs = torch.zeros(T, dtype=torch.int32)
    kv_num, kv_idx = random_blockscore_mask(H, T, bs, docs, window=3, n_global=1, budget=2, seed=2)
    A, Bc = band_coefficients(q)
    terms = dict(coeff_cos=A, coeff_sin=Bc, omegas=omegas_block(8))
    out, lse = _run_fwd(q, k, v, kv_num, kv_idx, docs, bs, "block", terms)
    out, lse = out[0].float().cpu(), lse[0].cpu()
    res = OA.attention_blocksparse(q[0].double(), k[0].double(), v[0].double(), kv_num, kv_idx, docs, bs=bs,
                                   scale=SCALE, beta=BETA, bias_mode="block", coeff_cos=A[0].double(),
                                   coeff_sin=Bc[0].double(), omegas=omegas_block(8).double())
    worst = 0.0
    for (h, qb), (o, l) in res.items():
        ok, w1 = tol_check(out[h, qb * bs:(qb + 1) * bs], o, ATOL, RTOL)
        ok2, w2 = tol_check(lse[h, qb * bs:(qb + 1) * bs], l, ATOL, RTOL)
        worst = max(worst, w1, w2)
        assert ok and ok2, f"(h={h}, qb={qb}) worst ratio {max(w1, w2):.3f}"
    print(f"C1 worst tolerance ratio {worst:.3f}")


@pytest.mark.parametrize("mode", ["block", "token"])
def test_spectral_table_cache_follows_the_tensor(mode):
    """The cached cos/sin table belongs to the ω tensor it was built from: a
    new ω of other values (here allocated where a freed one lay, as per-call
    .to(device) copies are) gets its own table, and an in-place change of ω
    rebuilds it."""
    from scope_amd import library
    from scope_amd.attention import spectral_table

    T, bs = 4096, 128
    m = {"block": 1, "token": 2}[mode]
    om1 = omegas_block(8).to(DEV)
    spectral_table(om1, T, bs, mode)
    del om1
    om2 = (omegas_block(8) * 1.5).to(DEV)
    assert torch.equal(spectral_table(om2, T, bs, mode), library.spectral_table(om2, T, bs, m))
    om2.mul_(0.5)
    assert torch.equal(spectral_table(om2, T, bs, mode), library.spectral_table(om2, T, bs, m))

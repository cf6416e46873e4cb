"""GPU: the ``torch.ops.scope`` operators under torch's operator checks and
under torch.compile.

* ``torch.library.opcheck`` (schema / mutation and aliasing, autograd
  registration, fake-tensor agreement with the real outputs, AOT dispatch
  with dynamic shapes) on every operator with small real inputs, including
  the differentiable ones with inputs that require grad.
* A block-scoring SCOPE layer and the reference's default layer path
  (SpectralBias.forward -> build_pointer_blockmask -> attention with the
  token-offset terms, scoped_medium.py:361-466) compiled with
  ``fullgraph=True`` (a graph break is an error) on the aot_eager backend
  (AOT autograd traces the registered backward formulas; no code
  generation): forward outputs and every gradient equal eager execution bit
  for bit."""
from __future__ import annotations

import math

import pytest
import torch

from scope_amd import SpectralBias, SpectralTerms, library, scope_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"
S = torch.ops.scope


def _inputs(H=2, T=1024, D=128, bs=128, seed=0, grad=False):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q, k, v = (torch.randn((1, H, T, D), generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
    docs = torch.zeros(T, dtype=torch.int32, device=DEV)
    docs[T // 2 + 77:] = 1
    cc, cs = (0.05 * torch.randn((1, H, T, 8), generator=g, device=DEV) for _ in range(2))
    om = torch.tensor([math.pi * 2.0 ** (-i) for i in range(8)], device=DEV)
    if grad:
        for t in (q, k, v, cc, cs):
            t.requires_grad_()
    return q, k, v, docs, cc, cs, om


def _lists(q, k, docs, bs, W=2, G=1, B=2):
    NB = q.shape[2] // bs
    ds_ptr, ds_local, dse = S.doc_starts(docs, bs, True, 0)
    qbar, kbar = S.block_means(q, k, bs)
    kn, ki, pk, _ = S.pointer_select(ds_ptr, ds_local, qbar, kbar, None, None, None, bs, NB, q.shape[1], W, G, B, 1.0,
                                     bs / math.sqrt(q.shape[-1]), 0, 0, 1e-9, False)
    return ds_ptr, ds_local, dse, qbar, kbar, kn, ki, pk


def test_opcheck_selection_and_list_operators():
    bs = 128
    q, k, v, docs, cc, cs, om = _inputs()
    NB = q.shape[2] // bs
    torch.library.opcheck(S.doc_starts.default, (docs, bs, True, 0))
    torch.library.opcheck(S.block_means.default, (q, k, bs))
    torch.library.opcheck(S.block_means_docs.default, (q, k, docs, bs, True, 0))
    ds_ptr, ds_local, dse, qbar, kbar, kn, ki, pk = _lists(q, k, docs, bs)
    for noise, seed in ((0, 0), (2, library.seed_to_signed(2 ** 64 - 3))):
        torch.library.opcheck(S.pointer_select.default, (ds_ptr, ds_local, qbar, kbar, None, None, None, bs, NB, 2, 2,
                                                          1, 3, 1.0, 11.3, noise, seed, 1e-9, True))
    torch.library.opcheck(S.transpose_blocks.default, (kn, ki, NB))
    torch.library.opcheck(S.mask_stats.default, (None, None, None, None, kn, None, pk, ds_ptr, ds_local, 2, NB, bs, 0,
                                                  False, False, False, 1, 1e-9, ki.shape[-1] + 1, 1, 1, 2))
    torch.library.opcheck(S.spectral_table.default, (om, q.shape[2], bs, 1))
    torch.library.opcheck(S.spectral_table.default, (om, q.shape[2], bs, 2))
    lg = torch.randn((2, NB, NB), device=DEV)
    torch.library.opcheck(S.pair_bias_from_logits.default, (kn, ki, pk, lg, bs, 2, 1, 2.0))
    # reference mode
    M = 4
    g = torch.Generator(device=DEV).manual_seed(3)
    dstar = torch.rand((1, 2, q.shape[2], M), generator=g, device=DEV) * 600
    bl = torch.randn((1, 2, q.shape[2], M), generator=g, device=DEV)
    torch.library.opcheck(S.pointer_mask_ref.default, (dstar, bl, ds_ptr, ds_local, None, bs, 2, 1, 1, 1, True, 2, 1.0,
                                                       True, 1, False, 0, 1.0, 1e-9))


@pytest.mark.parametrize("mode", ["block", "token"])
def test_opcheck_attention_with_gradients(mode):
    bs = 128
    q, k, v, docs, cc, cs, om = _inputs(seed=1)
    _, _, dse, _, _, kn, ki, _ = _lists(q, k, docs, bs)
    q_off, q_list = S.transpose_blocks(kn, ki, q.shape[2] // bs)
    for t in (q, k, v, cc, cs):
        t.requires_grad_()
    m = 1 if mode == "block" else 2
    tab = S.spectral_table(om, q.shape[2], bs, m)
    extra = (None, None, None, None)
    if mode == "token":
        g = torch.Generator(device=DEV).manual_seed(4)
        extra = (cc.detach().sum(-1).requires_grad_(), (torch.randn((1, 2, q.shape[2]), generator=g, device=DEV)
                                                        * 1e-3).requires_grad_(),
                 (torch.rand((1, 2, q.shape[2]), generator=g, device=DEV) * 300).requires_grad_(),
                 (32 + torch.rand((1, 2, q.shape[2]), generator=g, device=DEV) * 200).requires_grad_())
    tok = mode == "token"
    args = (q, k, v, kn, ki, docs, dse, q_off, q_list, tab, cc, cs, *extra, None, bs, 0.12, 0.5, m, tok, tok,
            1 if tok else 0, 0.2 if tok else 0.0, 64.0)
    torch.library.opcheck(S.attn_fwd.default, args)


def test_opcheck_soft_pointer_and_coefficient_head():
    bs = 128
    q, k, v, docs, cc, cs, om = _inputs(seed=2)
    _, _, _, _, _, kn, ki, pk = _lists(q, k, docs, bs)
    qg, kg = q.clone().requires_grad_(), k.clone().requires_grad_()
    torch.library.opcheck(S.soft_pointer_bias.default, (qg, kg, kn, ki, pk, None, bs, 2, 1, 11.3, 2.0))
    sb = SpectralBias(head_dim=128, num_heads=2, L_train=1024, M=8, K=6).to(DEV).train()
    iprm, fprm = library.pack_head_params(sb._head_params(1024))
    _, _, cm, sm = sb._get_trig_tables(1024, q.device)
    y = (torch.randn((1, 2, 1024, 41), device=DEV) * 2).requires_grad_()
    torch.library.opcheck(S.coeff_head_fwd.default, (y, sb.omegas, sb.log_omegas, cm, sm, iprm, fprm))


class _Layer(torch.nn.Module):
    def __init__(self, H, T, bs):
        super().__init__()
        self.sb, self.bs = SpectralBias(head_dim=128, num_heads=H, L_train=T), bs

    def forward(self, q, k, v, docs, cc, cs, om):
        bm = self.sb.build_blockscore_mask(q, k, docs=docs, block_size=self.bs, window_blocks=2, global_blocks=1,
                                           budget_blocks=2, noise="none", soft_temp=2.0)
        sp = SpectralTerms(coeff_cos=cc, coeff_sin=cs, omegas=om, offset="block")
        return scope_attention(q, k, v, block_mask=bm, scale=0.12, spectral=sp)


class _RefLayer(torch.nn.Module):
    def __init__(self, H, T):
        super().__init__()
        self.sb = SpectralBias(head_dim=128, num_heads=H, L_train=T, use_pointer_mask=True, pointer_half_blocks=2)

    def forward(self, q, k, v, docs):
        out = self.sb(q, docs=docs)
        bm = self.sb.build_pointer_blockmask(docs=docs, delta_star=out[4], pi=out[5], budget_logits=out[6],
                                             block_size=128)
        y = scope_attention(q, k, v, block_mask=bm, scale=0.12, spectral=self.sb.score_terms(out, offset="token"))
        return y, out[11]


def _run(fn, args, leaves, seed):
    outs = fn(*args)
    outs = outs if isinstance(outs, tuple) else (outs,)
    g = torch.Generator(device=DEV).manual_seed(seed)
    loss = sum((o.float() * torch.randn(o.shape, generator=g, device=DEV)).sum() for o in outs)
    grads = torch.autograd.grad(loss, leaves)
    torch.cuda.synchronize()
    return [o.detach().clone() for o in outs], [x.clone() for x in grads]


def test_compiled_block_scoring_layer_equals_eager():
    torch._dynamo.reset()
    q, k, v, docs, cc, cs, om = _inputs(H=2, T=2048, seed=5, grad=True)
    layer = _Layer(2, 2048, 128).to(DEV)
    comp = torch.compile(layer, backend="aot_eager", fullgraph=True)
    leaves = (q, k, v, cc, cs)
    eo, eg = _run(layer, (q, k, v, docs, cc, cs, om), leaves, 9)
    co, cg = _run(comp, (q, k, v, docs, cc, cs, om), leaves, 9)
    for a, b in zip(eo + eg, co + cg):
        assert torch.equal(a, b)


def test_compiled_reference_mode_layer_equals_eager():
    torch._dynamo.reset()
    H, T = 2, 2048
    q, k, v, docs, _, _, _ = _inputs(H=H, T=T, seed=6, grad=True)
    layer = _RefLayer(H, T).to(DEV).train()
    with torch.no_grad():
        for p_ in layer.sb.mlp.parameters():
            p_.normal_(0, 0.05)
    comp = torch.compile(layer, backend="aot_eager", fullgraph=True)
    leaves = (q, k, v) + tuple(layer.sb.mlp.parameters())
    eo, eg = _run(layer, (q, k, v, docs.long()), leaves, 10)
    co, cg = _run(comp, (q, k, v, docs.long()), leaves, 10)
    for a, b in zip(eo + eg, co + cg):
        assert torch.equal(a, b)

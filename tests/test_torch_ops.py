"""CPU: the ``torch.ops.scope`` operators without a GPU.

* Every operator's fake (shape) implementation gives the shapes, dtypes and
  strides of the C layouts; where the library has a host-side size function
  (list width of the reference mode, statistics length, table bytes) the
  fake agrees with it for many parameter sets.
* A SCOPE layer (block-scoring mask build + attention with the spectral
  bias) exports with ``torch.export`` (always a full graph, no breaks) over
  fake CUDA tensors, and its forward + backward traces into one graph whose
  backward runs through the registered autograd formulas.
* The operators' real implementations refuse CPU tensors (no CPU path).

The GPU side (tests/test_gpu_torch_ops.py) runs ``torch.library.opcheck`` on
each operator and compares a ``torch.compile(fullgraph=True)`` layer with
eager execution."""
from __future__ import annotations

import ctypes as C
import os

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

import scope_amd  # noqa: F401  (registers the operators)
from scope_amd import SpectralBias, SpectralTerms, library, ops, scope_attention

S = torch.ops.scope
LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "scope_amd", "libscope_amd.so")
needs_lib = pytest.mark.skipif(not os.path.exists(LIB), reason="libscope_amd.so not built")
OPS = ["doc_starts", "pointer_mask_ref", "block_means", "pointer_select", "soft_pointer_bias", "pair_bias_from_logits",
       "soft_pointer_bwd", "transpose_blocks", "mask_stats", "spectral_table", "attn_fwd", "attn_bwd",
       "coeff_head_fwd", "coeff_head_bwd"]


def test_every_operator_is_registered():
    for n in OPS:
        assert hasattr(S, n), n
        assert str(getattr(S, n).default._schema).startswith(f"scope::{n}(")


def _fake_cuda():
    return FakeTensorMode(allow_non_fake_inputs=True)


def test_attention_fakes_keep_q_layout_and_gradient_presence():
    H, T, D, bs, L = 3, 2048, 128, 256, 6
    QB = T // bs
    with _fake_cuda():
        # [1,T,H,D] memory viewed as [1,H,T,D], as the reference passes it (scoped_medium.py:460-462)
        q, k, v = (torch.empty(1, T, H, D, device="cuda", dtype=torch.bfloat16).transpose(1, 2) for _ in range(3))
        kv_num = torch.empty(H, QB, device="cuda", dtype=torch.int32)
        kv_idx = torch.empty(H, QB, L, device="cuda", dtype=torch.int32)
        docs = torch.empty(T, device="cuda", dtype=torch.int32)
        dse = torch.empty(QB, device="cuda", dtype=torch.int32)
        e = kv_num.new_empty(0)
        cc = torch.empty(1, H, T, 8, device="cuda")
        out, lse = S.attn_fwd(q, k, v, kv_num, kv_idx, docs, dse, e, e, None, cc, cc, None, None, None, None, None, bs,
                              0.12, 0.5, 1, False, False, 0, 0.0, 64.0)
        assert out.shape == q.shape and out.stride() == q.stride() and out.dtype == torch.bfloat16
        assert lse.shape == (1, H, T) and lse.dtype == torch.float32
        for mode, K, need_c, use_slope, sub_b0, gate, need_p in ((0, 0, True, False, False, 0, False),
                                                                (1, 8, True, False, False, 0, True),
                                                                (2, 8, True, True, True, 1, False),
                                                                (2, 8, False, True, True, 1, False)):
            ccm = cc if mode else None
            g = S.attn_bwd(q, k, v, out, out, lse, kv_num, kv_idx, kv_num, kv_idx, docs, dse, None, ccm, ccm, None,
                           None, None, None, None, bs, 0.12, 0.5, mode, use_slope, sub_b0, gate, 0.2, 64.0, need_c,
                           need_p)
            assert all(x.stride() == q.stride() for x in g[:3])
            pres = library.bwd_outputs_present(mode, K, need_c, use_slope, sub_b0, gate, need_p)
            for name, x in zip(library._BWD_NAMES, g[3:]):
                assert (x.numel() > 0) == pres[name], (mode, name)
            if pres["dpair_bias"]:
                assert g[-1].shape == (H, QB, L)


@needs_lib
def test_fake_sizes_agree_with_the_library_size_functions():
    from scope_amd._lib import PtrRefParams, StatsParams, load

    lib = load()
    for T, bs, M, local, p, G in ((4096, 128, 8, 8, 4, 1), (8192, 256, 3, 1, 0, 2), (1024, 128, 32, 20, 2, 40),
                                  (131072, 256, 8, 8, 4, 1)):
        prm = PtrRefParams(H=2, M=M, bs=bs, T=T, local_blocks=local, ptr_half_blocks=p, global_blocks_cfg=G)
        assert library.ref_maxkv(T, bs, M, local, p, G) == lib.scope_ptr_ref_maxkv(C.byref(prm))
        with _fake_cuda():
            ds = torch.empty(1, 2, T, M, device="cuda")
            blk = torch.empty(T // bs, device="cuda", dtype=torch.int32)
            kn, ki, rad, cen = S.pointer_mask_ref(ds, ds, blk, blk, None, bs, local, p, G, G, True, 3, 1.0, True, p,
                                                  False, 0, 1.0, 1e-9)
            assert ki.shape == (2, T // bs, lib.scope_ptr_ref_maxkv(C.byref(prm))) and kn.dtype == torch.int32
            assert rad.shape == cen.shape == (2, T // bs, M)
    for mk, rb, eb in ((1, 1, 1), (13, 5, 9), (81, 2, 33)):
        sp = StatsParams(maxkv_bins=mk, radius_bins=rb, extra_bins=eb)
        with _fake_cuda():
            kn = torch.empty(2, 16, device="cuda", dtype=torch.int32)
            counts, values = S.mask_stats(None, None, None, None, kn, kn, None, None, None, 2, 16, 128, 2, False, False,
                                          False, 1, 1e-9, mk, rb, eb, 1)
        assert counts.shape == (lib.scope_stats_counts_len(C.byref(sp)),) and counts.dtype == torch.int32
        assert values.shape == (len(ops.SV_NAMES),)
    for mode in (1, 2):
        for T, bs in ((4096, 128), (131072, 256)):
            with _fake_cuda():
                tab = S.spectral_table(torch.empty(8, device="cuda"), T, bs, mode)
            assert tab.numel() == lib.scope_spectral_table_bytes(mode, T, bs) and tab.dtype == torch.uint8


def test_selection_and_list_fakes():
    H, T, D, bs, W, G, B = 4, 8192, 128, 128, 2, 1, 3
    NB = T // bs
    with _fake_cuda():
        docs = torch.empty(T, device="cuda", dtype=torch.int32)
        ds_ptr, ds_local, dse = S.doc_starts(docs, bs, True, 0)
        assert ds_ptr.shape == ds_local.shape == dse.shape == (NB,)
        q = torch.empty(1, H, T, D, device="cuda", dtype=torch.bfloat16)
        qbar, kbar = S.block_means(q, q, bs)
        assert qbar.shape == (H, NB, D) and qbar.dtype == torch.float32
        for ret in (False, True):
            kn, ki, pk, lg = S.pointer_select(ds_ptr, ds_local, qbar, kbar, None, None, None, bs, NB, H, W, G, B, 1.0,
                                              11.3, 2, library.seed_to_signed(2 ** 64 - 5), 1e-9, ret)
            assert kn.shape == (H, NB) and ki.shape == (H, NB, W + B + G) and pk.shape == (H, NB, B)
            assert lg.shape == ((H, NB, NB) if ret else (0,))
        q_off, q_list = S.transpose_blocks(kn, ki, NB)
        assert q_off.shape == (H, NB + 1) and q_list.shape == (H, NB * (W + B + G))
        pb, qb_, kb_ = S.soft_pointer_bias(q, q, kn, ki, pk, None, bs, W, G, 11.3, 2.0)
        assert pb.shape == ki.shape and pb.dtype == torch.float32 and qb_.shape == (H, NB, D)
        assert S.pair_bias_from_logits(kn, ki, pk, lg, bs, W, G, 2.0).shape == ki.shape
        dq, dk = S.soft_pointer_bwd(qb_, kb_, kn, ki, q_off, q_list, pb, pb, q, q, bs, 11.3, 2.0)
        assert dq.shape == q.shape and dq.dtype == torch.bfloat16


def test_coefficient_head_fakes():
    M, K = 8, 6
    sb = SpectralBias(head_dim=64, num_heads=2, L_train=1024, M=M, K=K)
    iprm, fprm = library.pack_head_params(sb._head_params(1024))
    with _fake_cuda():
        y = torch.empty(1, 2, 1024, 5 * M + 1, device="cuda", dtype=torch.bfloat16)
        om = torch.empty(K, device="cuda")
        outs = S.coeff_head_fwd(y, om, om, om, om, iprm, fprm)
        shapes = [(1, 2, 1024, K)] * 2 + [(1, 2, 1024)] * 2 + [(1, 2, 1024, M)] * 3 + [(1, 2, 1024)] * 2 + [(6,)]
        assert [tuple(o.shape) for o in outs] == shapes
        dy = S.coeff_head_bwd(y, om, om, om, om, [outs[0], None, None, None, None, None, None, None, None], outs[9][:1],
                              outs[9], iprm, fprm)
        assert dy.shape == y.shape and dy.dtype == y.dtype


class _Layer(torch.nn.Module):
    """One SCOPE layer: block-scoring mask from q, k, then the attention with
    the block-offset spectral bias."""

    def __init__(self, H, T, D, bs):
        super().__init__()
        self.sb, self.bs = SpectralBias(head_dim=D, num_heads=H, L_train=T), bs

    def forward(self, q, k, v, docs, cc, cs, om):
        bm = self.sb.build_blockscore_mask(q, k, docs=docs, block_size=self.bs, window_blocks=2, global_blocks=1,
                                           budget_blocks=2, noise="none")
        sp = SpectralTerms(coeff_cos=cc, coeff_sin=cs, omegas=om, offset="block")
        return scope_attention(q, k, v, block_mask=bm, scale=0.12, spectral=sp)


def _layer_inputs(H, T, D, device):
    q, k, v = (torch.randn(1, H, T, D, device=device, dtype=torch.bfloat16) for _ in range(3))
    docs = torch.zeros(T, dtype=torch.int32, device=device)
    cc, cs = torch.randn(1, H, T, 8, device=device), torch.randn(1, H, T, 8, device=device)
    return q, k, v, docs, cc, cs, torch.randn(8, device=device)


def test_layer_exports_as_one_graph():
    H, T, D, bs = 2, 1024, 128, 128
    layer = _Layer(H, T, D, bs)
    with _fake_cuda():
        ep = torch.export.export(layer, _layer_inputs(H, T, D, "cuda"))
    targets = [str(n.target) for n in ep.graph_module.graph.nodes if n.op == "call_function"]
    assert "scope.attn_fwd.default" in targets and "scope.spectral_table.default" in targets
    # the mask build runs under no_grad: its operators sit in the wrapped submodule
    sub = "".join(str(m.code) for _, m in ep.graph_module.named_modules())
    for n in ("block_means_docs", "pointer_select"):
        assert f"torch.ops.scope.{n}.default" in sub, n


class _RefLayer(torch.nn.Module):
    """The reference's default layer path (scoped_medium.py:361-466):
    SpectralBias.forward (MLP + coefficient head), build_pointer_blockmask
    (reference mode), attention with the token-offset score_mod terms."""

    def __init__(self, H, T, D):
        super().__init__()
        self.sb = SpectralBias(head_dim=D, num_heads=H, L_train=T, use_pointer_mask=True)

    def forward(self, q, k, v, docs):
        out = self.sb(q, docs=docs)
        bm = self.sb.build_pointer_blockmask(docs=docs, delta_star=out[4], pi=out[5], budget_logits=out[6],
                                             block_size=128)
        y = scope_attention(q, k, v, block_mask=bm, scale=0.12, spectral=self.sb.score_terms(out, offset="token"))
        return y, out[11]


def test_reference_mode_layer_exports_as_one_graph():
    H, T, D = 2, 1024, 128
    with _fake_cuda(), torch.device("cuda"):
        layer = _RefLayer(H, T, D)
        q, k, v = (torch.randn(1, H, T, D, dtype=torch.bfloat16) for _ in range(3))
        ep = torch.export.export(layer, (q, k, v, torch.zeros(T, dtype=torch.int64)))
    code = "".join(str(m.code) for _, m in ep.graph_module.named_modules())
    for n in ("coeff_head_fwd", "doc_starts", "pointer_mask_ref", "spectral_table", "transpose_blocks", "attn_fwd"):
        assert f"torch.ops.scope.{n}.default" in code, n


def test_forward_backward_traces_through_the_autograd_formulas():
    H, T, D, bs = 2, 1024, 128, 128
    layer = _Layer(H, T, D, bs)
    with FakeTensorMode(allow_non_fake_inputs=True):
        # CPU fakes: the fakes do not look at the device, and the autograd engine
        # needs a real GPU context for CUDA ones
        q, k, v, docs, cc, cs, om = _layer_inputs(H, T, D, "cpu")
        for t in (q, k, v, cc, cs):
            t.requires_grad_()

        def f(q, k, v, cc, cs):
            out = layer(q, k, v, docs, cc, cs, om)
            return torch.autograd.grad(out.float().sum(), (q, k, v, cc, cs))

        gm = make_fx(f)(q, k, v, cc, cs)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    order = [t.split(".")[1] for t in targets if t.startswith("scope.")]
    assert order == ["block_means_docs", "pointer_select", "spectral_table", "transpose_blocks", "attn_fwd",
                     "attn_bwd"], order


def test_real_implementations_refuse_cpu_tensors():
    x = torch.zeros(1, 2, 256, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        S.block_means(x, x, 128)
    with pytest.raises(RuntimeError, match="no CPU path"):
        S.doc_starts(torch.zeros(256, dtype=torch.int32), 128, True, 0)

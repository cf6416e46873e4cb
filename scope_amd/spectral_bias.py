"""``SpectralBias``: the call surface of ``model/attn_bias.py:68-874`` with the
pointer mask, its statistics and the attention running on the gfx950 kernels.

* constructor, configuration checks and schedule setters mirror
  ``model/attn_bias.py:75-377`` (same keyword names, same ValueErrors);
* ``forward`` is the coefficient head (``:379-478``) plus the regularisers
  (``:480-508``): the MLP GEMMs run in torch (BLAS) and everything after them
  in the fused coefficient-head kernels, forward and backward
  (``scope::coeff_head_fwd`` / ``_bwd``).  GPU tensors only: there is no CPU
  path.  The debug statistics (``:510-606``) run in the fused statistics
  kernel without host syncs;
* ``build_pointer_blockmask`` (``:623-873``) runs the doc-start and
  reference-mode pointer kernels and returns a ``ScopeBlockMask``;
* ``build_blockscore_mask`` is the block-mean q·k selection (this project's
  block-scoring mode).

The scheduled state lives both in the reference's int buffers and in Python
integers, so that no kernel argument needs a ``.item()`` sync.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import library, ops
from .attention import SpectralTerms
from .blockmask import ScopeBlockMask

TOKEN_EDGES = [0, 127, 255, 511, 1023, 2047, 4095, 8191, 16383, 32767, 65535, 131071, 262143, 524287, 1048575]
BLOCK_EDGES = [0, 1, 3, 7, 15, 31, 63, 127, 255, 511, 1023, 2047, 4095, 8191]


class _PerHeadMLP(torch.autograd.Function):
    """The per-head MLP of ``share_across_heads=False`` (model/attn_bias.py:387-398):
    y[b,h,l] = W2[h]·SiLU(W1[h]·q[b,h,l] + b1[h]) + b2[h] in q's dtype, the
    weights cast to it, as the reference's two einsums.  Every batched
    product here takes contiguous operands (weights transposed once and
    copied, rows of every head gathered), forward and backward, so no batched
    bf16 product sees a transposed view.  The weights' gradients are those
    of their cast copies, in the weights' dtype, as autograd through the
    reference's ``.to(dt)`` gives them."""

    @staticmethod
    def _hidden(q, w1, b1):
        dt = q.dtype
        w1t = w1.to(dt).transpose(1, 2).contiguous()  # [H, D, K]
        z = torch.matmul(q.contiguous(), w1t[None]) + b1.to(dt)[None, :, None, :]
        return z, F.silu(z)

    @staticmethod
    def forward(ctx, q, w1, b1, w2, b2):
        dt = q.dtype
        _, x = _PerHeadMLP._hidden(q, w1, b1)
        w2t = w2.to(dt).transpose(1, 2).contiguous()  # [H, K, O]
        ctx.save_for_backward(q, w1, b1, w2, b2)
        return torch.matmul(x, w2t[None]) + b2.to(dt)[None, :, None, :]

    @staticmethod
    def backward(ctx, gy):
        q, w1, b1, w2, b2 = ctx.saved_tensors
        dt = q.dtype
        B, H, L, D = q.shape
        gy = gy.to(dt).contiguous()
        z, x = _PerHeadMLP._hidden(q, w1, b1)
        dz = torch.ops.aten.silu_backward(torch.matmul(gy, w2.to(dt).contiguous()[None]), z)
        dq = torch.matmul(dz, w1.to(dt).contiguous()[None]) if ctx.needs_input_grad[0] else None

        def rows_t(t):  # [B, H, L, C] -> [H, C, B·L]
            return t.permute(1, 3, 0, 2).reshape(H, t.shape[-1], B * L).contiguous()

        def rows(t):  # [B, H, L, C] -> [H, B·L, C]
            return t.permute(1, 0, 2, 3).reshape(H, B * L, t.shape[-1]).contiguous()

        dw1 = torch.bmm(rows_t(dz), rows(q))
        dw2 = torch.bmm(rows_t(gy), rows(x))
        db1, db2 = dz.sum(dim=(0, 2)), gy.sum(dim=(0, 2))
        return dq, dw1.to(w1.dtype), db1.to(b1.dtype), dw2.to(w2.dtype), db2.to(b2.dtype)


class SpectralBias(nn.Module):
    """Query-conditioned Fourier bias over Δ = q_idx - kv_idx plus the
    pointer-driven block mask (model/attn_bias.py:68-73)."""

    def __init__(self, *, head_dim: int, num_heads: int, L_train: int, L_max: int = 1_000_000, K: int = 6,
                 M: int = 2, beta: float = 0.5, ramp_lambda: float = 0.2, tau: float = 64.0,
                 w_min: float | None = None, w_max: float | None = None, share_across_heads: bool = True,
                 use_slope: bool = True, gate_kind: str = "softplus", c_scale: float = 0.01,
                 width_min: float = 32.0, width_max: float = 256.0, delta_star_max: int | None = None,
                 detach_q: bool = False, subtract_b0: bool = True, eps: float = 1e-9,
                 use_pointer_mask: bool = False, pointer_local_blocks: int = 16, pointer_half_blocks: int = 4,
                 pointer_global_blocks: int = 0, pointer_budget_blocks: int = 0,
                 pointer_budget_is_total: bool = True, pointer_budget_temp: float = 1.0,
                 pointer_radius_mode: str = "pi", pointer_qblock_rep: str = "last", pointer_doc_clamp: bool = True,
                 gumbel_topk: bool = False, gumbel_topk_k: int = 0, gumbel_topk_tau: float = 1.0,
                 gumbel_topk_seed: int = 0, pointer_reset_len: int = 0, lambda_omega: float = 1e-5,
                 lambda_zero_mean: float = 1e-4, lambda_entropy: float = 1e-4, pi_entropy_floor_frac: float = 0.25,
                 lambda_delta_edge: float = 0.0, delta_edge_eps: float = 0.0, debug_stats: bool = False,
                 enabled: bool = True):
        super().__init__()
        # configuration checks: model/attn_bias.py:124-131, 159-163, 222-223
        if K <= 0:
            raise ValueError("K must be positive")
        if M <= 0:
            raise ValueError("M must be positive")
        if gate_kind not in {"none", "softplus", "relu"}:
            raise ValueError("gate_kind must be one of: none|softplus|relu")
        if not share_across_heads and num_heads <= 0:
            raise ValueError("num_heads must be set when share_across_heads=False")
        self.enabled = enabled
        self.head_dim, self.num_heads, self.K, self.M = head_dim, num_heads, K, M
        self.beta, self.ramp_lambda, self.tau = float(beta), float(ramp_lambda), float(tau)
        self.gate_kind = gate_kind
        self.share_across_heads = share_across_heads
        self.use_slope = use_slope
        self.c_scale = float(c_scale)
        self.width_min, self.width_max = float(width_min), float(width_max)
        self.delta_star_max = int(delta_star_max) if delta_star_max is not None else int(L_train - 1)
        self.detach_q, self.subtract_b0, self.eps = detach_q, subtract_b0, float(eps)
        self.use_pointer_mask = bool(use_pointer_mask)
        self.pointer_local_blocks = int(pointer_local_blocks)
        self.pointer_half_blocks = int(pointer_half_blocks)
        self.pointer_global_blocks = int(pointer_global_blocks)
        self.pointer_budget_blocks = int(pointer_budget_blocks)
        self.pointer_budget_is_total = bool(pointer_budget_is_total)
        self.pointer_budget_temp = float(pointer_budget_temp)
        self.pointer_radius_mode = str(pointer_radius_mode).strip().lower()
        if self.pointer_radius_mode not in {"fixed", "pi"}:
            raise ValueError("pointer_radius_mode must be one of: fixed|pi")
        self.pointer_qblock_rep = str(pointer_qblock_rep)
        if self.pointer_qblock_rep not in {"last", "mean"}:
            raise ValueError("pointer_qblock_rep must be one of: last|mean")
        self.pointer_doc_clamp = bool(pointer_doc_clamp)
        self.gumbel_topk = bool(gumbel_topk)
        self.gumbel_topk_k = int(gumbel_topk_k)
        self.gumbel_topk_tau = float(gumbel_topk_tau)
        self.gumbel_topk_seed = int(gumbel_topk_seed)
        self.pointer_reset_len = int(pointer_reset_len)
        self.debug_stats = bool(debug_stats)
        # scheduled state: buffers (model/attn_bias.py:171-206) + host mirror
        self._st = dict(mask=1 if self.use_pointer_mask else 0,
                        half=self.pointer_half_blocks if self.use_pointer_mask else 0,
                        glob=self.pointer_global_blocks if self.use_pointer_mask else 0,
                        reset=0, reset_len=max(0, self.pointer_reset_len), seed=self.gumbel_topk_seed,
                        dmax=self.delta_star_max, edge_eps=float(delta_edge_eps))
        i32 = dict(dtype=torch.int32)
        self.register_buffer("_pointer_mask_active", torch.tensor(self._st["mask"], **i32), persistent=False)
        self.register_buffer("_pointer_half_blocks_active", torch.tensor(self._st["half"], **i32), persistent=False)
        self.register_buffer("_pointer_global_blocks_active", torch.tensor(self._st["glob"], **i32), persistent=False)
        self.register_buffer("_pointer_reset_active", torch.tensor(0, **i32), persistent=False)
        self.register_buffer("_pointer_reset_len_active", torch.tensor(self._st["reset_len"], **i32),
                             persistent=False)
        self.register_buffer("_gumbel_seed", torch.tensor(self.gumbel_topk_seed, dtype=torch.int64), persistent=False)
        self.register_buffer("_delta_star_max_active", torch.tensor(self.delta_star_max, **i32), persistent=False)
        self.lambda_omega, self.lambda_zero_mean = float(lambda_omega), float(lambda_zero_mean)
        self.lambda_entropy, self.pi_entropy_floor_frac = float(lambda_entropy), float(pi_entropy_floor_frac)
        self.lambda_delta_edge, self.delta_edge_eps = float(lambda_delta_edge), float(delta_edge_eps)
        self.register_buffer("_delta_edge_eps_active", torch.tensor(self.delta_edge_eps, dtype=torch.float32),
                             persistent=False)

        w_min = float(w_min) if w_min is not None else (2 * math.pi / L_max)
        w_max = float(w_max) if w_max is not None else (2 * math.pi / L_train)
        if not (w_min > 0 and w_max > 0 and w_min < w_max):
            raise ValueError(f"invalid (w_min, w_max)=({w_min}, {w_max})")
        omegas = torch.logspace(math.log10(w_min), math.log10(w_max), K, dtype=torch.float32)  # :225
        self.register_buffer("omegas", omegas, persistent=False)
        self.register_buffer("log_omegas", omegas.log(), persistent=False)
        self.register_buffer("omega_sq", omegas.square(), persistent=False)
        self.register_buffer("logw_min", torch.tensor(math.log(w_min), dtype=torch.float32), persistent=False)
        self.register_buffer("logw_max", torch.tensor(math.log(w_max), dtype=torch.float32), persistent=False)
        # the same fp32 values on the host (kernel arguments without a device read)
        self._logw = (float(np.float32(math.log(w_min))), float(np.float32(math.log(w_max))))
        self._trig_cache: dict = {}

        # debug statistics buffers (model/attn_bias.py:239-265)
        self.register_buffer("_dbg_token_edges", torch.tensor(TOKEN_EDGES, dtype=torch.int64), persistent=False)
        self.register_buffer("_dbg_block_edges", torch.tensor(BLOCK_EDGES, dtype=torch.int64), persistent=False)
        z32 = lambda n: torch.zeros(n, dtype=torch.int32)  # noqa: E731
        self.register_buffer("_dbg_delta_tokens_hist", z32(len(TOKEN_EDGES) + 1), persistent=False)
        self.register_buffer("_dbg_delta_blocks_hist", z32(len(BLOCK_EDGES) + 1), persistent=False)
        self.register_buffer("_dbg_ptr_center_hist", z32(len(BLOCK_EDGES) + 1), persistent=False)
        max_kv = int(self.pointer_local_blocks + (2 * self.pointer_half_blocks + 1) * self.M + self.pointer_global_blocks)
        self.register_buffer("_dbg_kv_unique_hist", z32(max_kv + 1), persistent=False)
        for name in ("ptr_outside_local_frac", "ptr_block0_frac", "ptr_block0_frac_excl", "ptr_docstart_frac"):
            self.register_buffer("_dbg_" + name, torch.zeros((), dtype=torch.float32), persistent=False)
        self.register_buffer("_dbg_ptr_radius_hist", z32(self.pointer_half_blocks + 1), persistent=False)
        max_extra = max(1, int(self.pointer_half_blocks * self.M))
        self.register_buffer("_dbg_ptr_extra_sum_hist", z32(max_extra + 1), persistent=False)
        for name in ("ptr_radius0_frac", "pi_entropy_mean", "reg_omega", "reg_entropy", "reg_delta_edge",
                     "reg_zero_mean", "reg_total"):
            self.register_buffer("_dbg_" + name, torch.zeros((), dtype=torch.float32), persistent=False)

        hidden = max(128, 2 * head_dim)
        out = 5 * M + (1 if use_slope else 0)
        if share_across_heads:
            self.mlp = nn.Sequential(nn.Linear(head_dim, hidden), nn.SiLU(), nn.Linear(hidden, out))
        else:
            self.w1 = nn.Parameter(torch.empty(num_heads, hidden, head_dim))
            self.b1 = nn.Parameter(torch.zeros(num_heads, hidden))
            self.w2 = nn.Parameter(torch.empty(num_heads, out, hidden))
            self.b2 = nn.Parameter(torch.zeros(num_heads, out))
            self._init_per_head_weights()
        self._init_outputs()

    # ---- initialisation (model/attn_bias.py:280-304)
    def _init_per_head_weights(self):
        std1 = 0.5 * (self.head_dim ** -0.5)
        std2 = 0.5 * (self.w1.size(1) ** -0.5)
        with torch.no_grad():
            self.w1.uniform_(-(3 ** 0.5) * std1, (3 ** 0.5) * std1)
            self.w2.uniform_(-(3 ** 0.5) * std2, (3 ** 0.5) * std2)

    def _init_outputs(self):
        delta_biases = torch.linspace(-6.0, -4.0, steps=self.M)
        with torch.no_grad():
            if self.share_across_heads:
                last: nn.Linear = self.mlp[-1]
                last.weight.zero_()
                last.bias.zero_()
                last.bias[: self.M].copy_(delta_biases)
            else:
                self.w2.zero_()
                self.b2.zero_()
                self.b2[:, : self.M].copy_(delta_biases.view(1, self.M).expand(self.num_heads, -1))

    # ---- schedule setters (model/attn_bias.py:342-377)
    def set_pointer_mask_state(self, *, enabled: bool, half_blocks: int, global_blocks: int | None = None):
        half_blocks = int(half_blocks)
        if half_blocks < 0:
            raise ValueError("half_blocks must be >= 0")
        half_blocks = min(half_blocks, self.pointer_half_blocks)
        self._st["mask"] = 1 if enabled else 0
        self._st["half"] = half_blocks
        self._pointer_mask_active.fill_(self._st["mask"])
        self._pointer_half_blocks_active.fill_(half_blocks)
        if global_blocks is not None:
            gb = int(global_blocks)
            if gb < 0:
                raise ValueError("global_blocks must be >= 0")
            gb = min(gb, self.pointer_global_blocks)
            self._st["glob"] = gb
            self._pointer_global_blocks_active.fill_(gb)

    def set_pointer_reset_state(self, *, enabled: bool, reset_len: int):
        reset_len = int(reset_len)
        if reset_len < 0:
            raise ValueError("reset_len must be >= 0")
        self._st["reset"] = 1 if enabled else 0
        self._st["reset_len"] = reset_len if enabled else 0
        self._pointer_reset_active.fill_(self._st["reset"])
        self._pointer_reset_len_active.fill_(self._st["reset_len"])

    def set_gumbel_seed(self, *, seed: int):
        self._st["seed"] = int(seed)
        self._gumbel_seed.fill_(int(seed))

    def set_delta_star_max_active(self, *, max_tokens: int):
        max_tokens = int(max_tokens)
        if max_tokens < 0:
            raise ValueError("max_tokens must be >= 0")
        max_tokens = min(max_tokens, int(self.delta_star_max))
        self._st["dmax"] = max_tokens
        self._delta_star_max_active.fill_(max_tokens)

    def set_delta_edge_eps_active(self, *, eps: float):
        eps = float(eps)
        if eps < 0:
            raise ValueError("eps must be >= 0")
        self._st["edge_eps"] = eps
        self._delta_edge_eps_active.fill_(eps)

    # ---- coefficient head (model/attn_bias.py:306-340, 379-478)
    def _mlp_forward(self, q: Tensor) -> Tensor:
        if self.detach_q:
            q = q.detach()
        dt = q.dtype
        if self.share_across_heads:
            # the two F.linear and the SiLU of the reference, as one operator:
            # a fused kernel forward, and backward one for dq and one for the
            # weight and bias gradients (a contraction over all B·H·T rows)
            fc1: nn.Linear = self.mlp[0]
            fc2: nn.Linear = self.mlp[2]
            return library.coeff_mlp(q, fc1.weight, fc1.bias, fc2.weight, fc2.bias)
        return _PerHeadMLP.apply(q, self.w1, self.b1, self.w2, self.b2)

    def _get_trig_tables(self, L: int, device: torch.device):
        key = (L, device)
        if key not in self._trig_cache:
            D = torch.arange(L, device=device, dtype=torch.float32)
            w = self.omegas.to(device=device)
            c32 = torch.cos(w[:, None] * D[None, :])
            s32 = torch.sin(w[:, None] * D[None, :])
            self._trig_cache = {key: (c32.to(torch.bfloat16), s32.to(torch.bfloat16), c32.mean(-1), s32.mean(-1))}
        return self._trig_cache[key]

    def _head_params(self, L: int) -> dict:
        """Scalar arguments of the fused coefficient head (host values only)."""
        return dict(M=self.M, K=self.K, L=L, use_slope=self.use_slope, subtract_b0=self.subtract_b0,
                    training=self.training, delta_cap=min(max(float(self._st["dmax"]), 0.0), float(L - 1)),
                    logw_min=self._logw[0], logw_max=self._logw[1], c_scale=self.c_scale, width_min=self.width_min,
                    width_max=self.width_max, eps=self.eps, lambda_omega=self.lambda_omega,
                    lambda_entropy=self.lambda_entropy, lambda_zero_mean=self.lambda_zero_mean,
                    lambda_delta_edge=self.lambda_delta_edge,
                    entropy_floor=float(self.pi_entropy_floor_frac) * math.log(self.M),
                    delta_edge_eps=self._st["edge_eps"])

    def forward(self, q: Tensor, *, docs: Tensor | None = None) -> tuple[Tensor, ...]:
        """q [B,H,L,D] on the GPU -> the reference's 12-tuple
        (model/attn_bias.py:385-401): the MLP and the rest of the head in fused
        HIP kernels.  Disabled, it returns zeros and uniform π
        like the reference (:411-417).  There is no CPU path."""
        if not q.is_cuda:
            raise RuntimeError(f"SpectralBias.forward: q must live on the GPU (got {q.device}); there is no CPU path")
        if not self.enabled:
            return self._forward_disabled(q)
        return self._forward_fused(q, docs)

    def _forward_disabled(self, q: Tensor) -> tuple[Tensor, ...]:
        """model/attn_bias.py:411-417: zero coefficients, uniform π."""
        B, H, L, _ = q.shape
        cos_wD, sin_wD, _, _ = self._get_trig_tables(L, q.device)
        f = dict(dtype=torch.float32, device=q.device)
        z_k = torch.zeros((B, H, L, self.K), **f)
        z_l = torch.zeros((B, H, L), **f)
        z_m = torch.zeros((B, H, L, self.M), **f)
        z_pi = torch.full((B, H, L, self.M), 1.0 / self.M, **f)
        return z_k, z_k, z_l, z_l, z_m, z_pi, z_m, z_l, z_l, cos_wD, sin_wD, torch.zeros((), **f)

    def _forward_fused(self, q: Tensor, docs: Tensor | None) -> tuple[Tensor, ...]:
        """GPU forward: the fused MLP, then the fused coefficient head."""
        B, H, L, Dh = q.shape
        if H != self.num_heads:
            raise ValueError(f"expected H={self.num_heads}, got {H}")
        if Dh != self.head_dim:
            raise ValueError(f"expected head_dim={self.head_dim}, got {Dh}")
        cos_wD, sin_wD, cos_mean, sin_mean = self._get_trig_tables(L, q.device)
        y = self._mlp_forward(q)
        iprm, fprm = library.pack_head_params(self._head_params(L))
        outs = library.coeff_head_fwd(y, self.omegas, self.log_omegas, cos_mean, sin_mean, iprm, fprm)
        coeff_cos, coeff_sin, slope, b0, delta_star, pi, budget_logits, delta_main, width, reg_all = outs
        reg_loss = reg_all[0] if self.training else q.new_zeros((), dtype=torch.float32)
        if self.debug_stats:
            if B == 1 and L % 128 == 0:
                self._forward_stats(delta_star.detach(), pi.detach(), docs, L)
            r = reg_all.detach()
            for i, name in enumerate(("reg_total", "reg_omega", "reg_entropy", "reg_delta_edge", "reg_zero_mean")):
                getattr(self, "_dbg_" + name).copy_(r[i] if self.training else torch.zeros_like(r[i]))
        return (coeff_cos, coeff_sin, slope, b0, delta_star, pi, budget_logits, delta_main, width, cos_wD, sin_wD,
                reg_loss)

    def _forward_stats(self, delta_star: Tensor, pi: Tensor, docs: Tensor | None, L: int, bs: int = 128):
        """model/attn_bias.py:510-600 in the fused statistics kernel."""
        QB = L // bs
        has_docs = docs is not None
        reset_on = bool(self._st["reset"]) and self._st["reset_len"] > 0
        ds_ptr = ds_local = None
        if has_docs:
            ds_ptr, ds_local, _ = library.doc_starts(docs.to(torch.int32), bs, bool(self.pointer_doc_clamp),
                                                     self._st["reset_len"] if reset_on else 0)
        d3, p3 = (delta_star[0], pi[0]) if delta_star.dim() == 4 else (delta_star, pi)
        counts, values = library.mask_stats(d3, p3, ds_ptr, ds_local, None, None, None, None, None, self.num_heads,
                                            QB, bs, self.M, self.pointer_qblock_rep == "mean", has_docs,
                                            has_docs and (self.pointer_doc_clamp or bool(self._st["reset"])),
                                            self.pointer_local_blocks, float(self.eps), 1, 1, 1, 1)
        c = ops.unpack_counts(counts, 1, 1)
        self._dbg_delta_tokens_hist.copy_(c["delta_tokens_hist"])
        self._dbg_delta_blocks_hist.copy_(c["delta_blocks_hist"])
        self._dbg_ptr_center_hist.copy_(c["ptr_center_hist"])
        for i, name in enumerate(ops.SV_NAMES[:5]):
            getattr(self, "_dbg_" + name).copy_(values[i])

    # ---- pointer mask, reference mode (model/attn_bias.py:623-873)
    @torch.no_grad()
    def build_pointer_blockmask(self, *, input_seq: Tensor | None = None, docs: Tensor | None = None,
                                delta_star: Tensor, pi: Tensor, budget_logits: Tensor, block_size: int = 128,
                                local_blocks: int | None = None, ptr_half_blocks: int | None = None,
                                pointer_budget_blocks: int | None = None, global_blocks: int | None = None,
                                eod_token_id: int = 50256, gumbel_u: Tensor | None = None) -> ScopeBlockMask:
        """Same arguments and assertions as the reference; ``gumbel_u``
        optionally replaces the internal draw of the Gumbel uniforms."""
        assert (input_seq is None) != (docs is None), "pass exactly one of: input_seq|docs"
        if docs is None:
            assert input_seq is not None and input_seq.ndim == 1
            docs = (input_seq == eod_token_id).cumsum(0)
        assert docs is not None and docs.ndim == 1
        device = docs.device
        T = int(docs.numel())
        assert T % block_size == 0
        B, H, TT, M = delta_star.shape
        assert B == 1
        assert TT == T
        assert H == self.num_heads
        assert M == self.M
        assert pi.shape == (B, H, T, M)
        assert budget_logits.shape == (B, H, T, M)
        local = self.pointer_local_blocks if local_blocks is None else int(local_blocks)
        p = self.pointer_half_blocks if ptr_half_blocks is None else int(ptr_half_blocks)
        local, p = max(1, local), max(0, p)
        NB = T // block_size
        local = min(local, NB)
        budget_val = self.pointer_budget_blocks if pointer_budget_blocks is None else int(pointer_budget_blocks)
        budget_val = max(0, int(budget_val))
        if self.pointer_budget_is_total:
            cap = int(local + M + 2 * M * p)
            extra = max(min(budget_val, cap) - local - M, 0)
        else:
            extra = budget_val
        budget_rem = min(extra // 2, M * p)
        k = self.gumbel_topk_k
        if k <= 0 or k > M:
            k = M
        gumbel_k = k if (self.training and self.gumbel_topk and p > 0 and k < M) else 0
        if gumbel_k and gumbel_u is None:
            gen = torch.Generator(device=device)
            gen.manual_seed(int(self._st["seed"]))
            gumbel_u = torch.rand((H, NB, M), device=device, generator=gen, dtype=torch.float32)
        reset_on = bool(self._st["reset"]) and self._st["reset_len"] > 0
        docs32 = docs.to(torch.int32)
        ds_ptr, ds_local, ds_tok_end = library.doc_starts(docs32, block_size, bool(self.pointer_doc_clamp),
                                                          self._st["reset_len"] if reset_on else 0)
        ga = self._st["glob"] if global_blocks is None else int(global_blocks)
        kv_num, kv_idx, radius, centre = library.pointer_mask_ref(
            delta_star, budget_logits, ds_ptr, ds_local, gumbel_u if gumbel_k else None, block_size, local, p,
            self.pointer_global_blocks, ga, self.pointer_radius_mode == "pi", budget_rem,
            float(self.pointer_budget_temp), bool(self._st["mask"]), self._st["half"],
            self.pointer_qblock_rep == "mean", gumbel_k, float(self.gumbel_topk_tau), float(self.eps))
        if self.debug_stats:
            mk = self._dbg_kv_unique_hist.numel()
            if kv_idx.shape[-1] + 1 > mk:
                raise RuntimeError(f"kv_unique histogram has {mk} bins, list width is {kv_idx.shape[-1]}")
            rb, eb = self._dbg_ptr_radius_hist.numel(), self._dbg_ptr_extra_sum_hist.numel()
            counts, values = library.mask_stats(None, None, None, None, kv_num, radius, None, None, None, H, NB,
                                                block_size, M, False, False, False, 1, 1e-9, mk, rb, eb, 1)
            c = ops.unpack_counts(counts, mk, rb)
            self._dbg_kv_unique_hist.copy_(c["kv_unique_hist"])
            self._dbg_ptr_radius_hist.copy_(c["ptr_radius_hist"])
            self._dbg_ptr_extra_sum_hist.copy_(c["ptr_extra_sum_hist"])
            self._dbg_ptr_radius0_frac.copy_(values[5])
        return ScopeBlockMask(kv_num_blocks=kv_num[None], kv_indices=kv_idx[None], BLOCK_SIZE=block_size,
                              docs=docs32, ds_tok_end=ds_tok_end, ds_ptr=ds_ptr, ds_local=ds_local,
                              extras=dict(radius=radius, centre=centre), check=False)

    # ---- pointer mask, block-scoring mode
    @torch.no_grad()
    def build_blockscore_mask(self, q: Tensor, k: Tensor, *, docs: Tensor, block_size: int = 128,
                              window_blocks: int = 4, global_blocks: int = 1, budget_blocks: int = 4,
                              budget_temp: float | None = None, logit_scale: float | None = None,
                              prior: Tensor | None = None, noise: str = "counter", gumbel_u: Tensor | None = None,
                              seed: int | None = None, logits: Tensor | None = None,
                              return_logits: bool = False, soft_temp: float | None = None) -> ScopeBlockMask:
        """window ∪ top-``budget_blocks`` block-mean q·k pointers ∪ global
        anchors.  q, k: [1,H,T,D] bf16.  ``noise``: "none" | "uniform"
        (explicit ``gumbel_u`` [H,QB,NB]) | "counter" (in-kernel draw from the
        Gumbel seed; only while training, like the reference's Gumbel).
        ``soft_temp`` > 0 attaches the soft pointer weights log σ(z/soft_temp)
        of the picks (z the noise-free logit) as ``extras["pair_bias"]``:
        ``scope_attention`` adds them to the picked tiles' scores, and their
        gradient flows back to q and k through the block means (with
        ``logits`` given instead of q̄·k̄, the weights are constants)."""
        T = int(docs.numel())
        H = q.shape[1]
        NB = T // block_size
        docs32 = docs.to(torch.int32)
        qbar = kbar = None
        if logits is None:
            # the block means with the document starts folded in (one launch fewer)
            qbar, kbar, ds_ptr, ds_local, ds_tok_end = library.block_means_docs(
                q, k, docs32, block_size, bool(self.pointer_doc_clamp), 0)
        else:
            ds_ptr, ds_local, ds_tok_end = library.doc_starts(docs32, block_size, bool(self.pointer_doc_clamp), 0)
        if noise == "counter" and not self.training:
            noise = "none"
        scale = float(block_size) / math.sqrt(q.shape[-1]) if logit_scale is None else float(logit_scale)
        noise_mode = {"none": 0, "uniform": 1, "counter": 2}[noise]
        kv_num, kv_idx, picks, lg = library.pointer_select(
            ds_ptr, ds_local, qbar, kbar, logits, prior, gumbel_u if noise_mode == 1 else None, block_size, NB, H,
            window_blocks, global_blocks, budget_blocks,
            float(self.pointer_budget_temp if budget_temp is None else budget_temp), scale, noise_mode,
            library.seed_to_signed(self._st["seed"] if seed is None else seed), float(self.eps), bool(return_logits))
        extras = dict(picks=picks)
        if return_logits:
            extras["logits"] = lg
        bm = ScopeBlockMask(kv_num_blocks=kv_num[None], kv_indices=kv_idx[None], BLOCK_SIZE=block_size,
                            docs=docs32, ds_tok_end=ds_tok_end, ds_ptr=ds_ptr, ds_local=ds_local, extras=extras,
                            check=False)
        if soft_temp is not None and soft_temp > 0 and budget_blocks > 0:
            if logits is None:
                from .attention import soft_pointer_bias

                with torch.enable_grad():
                    extras["pair_bias"] = soft_pointer_bias(q, k, bm, window=window_blocks, n_global=global_blocks,
                                                            logit_scale=scale, soft_temp=float(soft_temp),
                                                            prior=prior)
            else:
                extras["pair_bias"] = library.pair_bias_from_logits(kv_num, kv_idx, picks, logits, block_size,
                                                                    window_blocks, global_blocks, float(soft_temp))
        return bm

    def score_terms(self, outputs: tuple, *, offset: str = "token") -> SpectralTerms:
        """SpectralTerms for ``scope_attention`` from the 12-tuple of forward()."""
        coeff_cos, coeff_sin, slope, b0, _, _, _, delta_main, width = outputs[:9]
        return SpectralTerms(coeff_cos=coeff_cos, coeff_sin=coeff_sin, omegas=self.omegas.to(coeff_cos.device),
                             offset=offset, beta=self.beta, b0=b0, slope=slope, delta_main=delta_main, width=width,
                             use_slope=self.use_slope, subtract_b0=self.subtract_b0, gate_kind=self.gate_kind,
                             ramp_lambda=self.ramp_lambda, tau=self.tau)

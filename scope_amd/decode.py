"""Token-loop decoding of the 16-layer SCOPE decoder on one MI355X.

The model mirrors ``GPT`` of scoped_medium.py:266-639 — token and value
embeddings (the 012 ... 012 pattern, :592), per block ``lambdas`` mixing with
x0, QK-norm, half-truncated rotary, value-embedding mix, ReLU² MLP, the
U-net skip connections with ``skip_weights``, no attention in block 7
(:499), and the soft-capped logits ``30·σ(logits/7.5)`` (:618) over the
vocabulary padded to a multiple of 128 (:529).  Every attention layer is a
SCOPE layer with the block-scoring pointer mask (window W, budget B, G
document-start globals) and no spectral bias.  Weights are random (the
reference zero-initialises its output projections and lm_head, which would
make greedy decoding trivial).

* ``prefill(tokens)``: one forward over the prompt (T a multiple of the
  block size) with the block-sparse attention kernel; fills every layer's KV
  cache and key-block means.
* ``step(token)``: one new position t.  When t opens a q-block, every layer
  reselects that block's list over its cache (the query block mean is the
  new token's query, the only one known), and keeps it for the block's other
  positions; the attention of the token runs ``scope_decode_attn`` over the
  list.  When t closes a block, its key mean joins the candidates.
* The steps inside a block (neither opening nor closing it) run as one
  captured HIP graph (``torch.cuda.CUDAGraph``), replayed per token: the
  position lives on the device (``_t_dev``; cache and document writes index
  with it, ``scope_decode_attn_at`` reads it), the lists sit in fixed
  per-layer buffers that a reselection refills, so every replay sees the
  current state.  The eager steps run the same operations, so both paths
  give the same logits.

The reference has no decode path; this is the row of the scope table that
puts the hot-path kernels under a token loop.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from . import ops

EOT = 50256


@dataclass
class DecoderConfig:
    vocab_size: int = 50257
    num_layers: int = 16
    num_heads: int = 8
    model_dim: int = 1024
    head_dim: int = 128
    block_size: int = 128
    window: int = 4
    budget: int = 4
    n_global: int = 1
    attn_scale: float = 0.12
    no_attn_layer: int = 7

    @property
    def vocab_padded(self) -> int:
        return ((self.vocab_size + 127) // 128) * 128


def _norm(x: torch.Tensor) -> torch.Tensor:
    return F.rms_norm(x, (x.size(-1),))


def _mix(a: float, b: float, x: torch.Tensor, x0: torch.Tensor) -> torch.Tensor:
    """a·x + b·x0 (scoped_medium.py:505); a = 1, b = 0 is x itself, exactly."""
    return x if (a == 1.0 and b == 0.0) else a * x + b * x0


def _skip(x: torch.Tensor, w: float, s: torch.Tensor) -> torch.Tensor:
    """x + w·s (scoped_medium.py:607); w = 1 is a plain sum, exactly."""
    return x + s if w == 1.0 else x + w * s


class _Rotary:
    """Half-truncated RoPE tables (scoped_medium.py:282-299)."""

    def __init__(self, dim: int, max_len: int, device):
        freq = (1 / 1024) ** torch.linspace(0, 1, steps=dim // 4, dtype=torch.float32)
        freq = torch.cat([freq, freq.new_zeros(dim // 4)])
        theta = torch.arange(max_len, dtype=torch.float32)[:, None] * freq[None]
        self.cos, self.sin = theta.cos().to(device), theta.sin().to(device)

    def __call__(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """x [T, H, D] at positions pos [T]."""
        cos, sin = self.cos[pos][:, None, :], self.sin[pos][:, None, :]
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos + x2 * sin, x1 * (-sin) + x2 * cos), -1).type_as(x)


class ScopeDecoder(nn.Module):
    def __init__(self, cfg: DecoderConfig, *, max_len: int, device="cuda", seed: int = 0, use_graph: bool = True):
        super().__init__()
        self.cfg = cfg
        g = torch.Generator(device="cpu").manual_seed(seed)
        d, H, D, L = cfg.model_dim, cfg.num_heads, cfg.head_dim, cfg.num_layers
        hd = H * D

        def uni(*shape, fan_in):
            b = math.sqrt(3.0) * 0.5 * fan_in ** -0.5  # CastedLinear / qkv init bound (:270-274, :305-306)
            return ((torch.rand(shape, generator=g) * 2 - 1) * b).to(torch.bfloat16).to(device)

        self.embed = (torch.randn((cfg.vocab_size, d), generator=g)).to(torch.bfloat16).to(device)
        self.value_embeds = [torch.randn((cfg.vocab_size, d), generator=g).to(torch.bfloat16).to(device)
                             for _ in range(3)]
        self.layers = []
        for i in range(L):
            lay = dict(lambdas=(1.0, 0.0), mlp_fc=uni(4 * d, d, fan_in=d), mlp_proj=uni(d, 4 * d, fan_in=4 * d))
            if i != cfg.no_attn_layer:
                lay.update(qkv=uni(3 * hd, d, fan_in=d), proj=uni(d, hd, fan_in=hd), vlam=(0.5, 0.5))
            self.layers.append(lay)
        self.skip_weights = [1.0] * (L // 2)
        self.lm_head = uni(cfg.vocab_padded, d, fan_in=d)
        self.rotary = _Rotary(D, max_len, device)
        self.device = torch.device(device)
        self.max_len = max_len
        # caches
        nbc = max_len // cfg.block_size
        z = dict(dtype=torch.bfloat16, device=device)
        self.k_cache = [torch.zeros((H, max_len, D), **z) if "qkv" in lay else None for lay in self.layers]
        self.v_cache = [torch.zeros((H, max_len, D), **z) if "qkv" in lay else None for lay in self.layers]
        self.kbar = [torch.zeros((H, nbc, D), dtype=torch.float32, device=device) if "qkv" in lay else None
                     for lay in self.layers]
        # current q-block's list per layer, in fixed buffers of the full width
        # (window + budget + globals) that each reselection refills
        width = cfg.window + cfg.budget + cfg.n_global
        self.list_num = [torch.zeros(H, dtype=torch.int32, device=device) if "qkv" in lay else None
                         for lay in self.layers]
        self.list_idx = [torch.zeros((H, width), dtype=torch.int32, device=device) if "qkv" in lay else None
                         for lay in self.layers]
        self.have_lists = False
        # a dict here makes every reselection record, per attention layer, the
        # query row it chose from, its logits and its lists (eager steps only)
        self.record: dict | None = None
        self.docs = torch.zeros(max_len, dtype=torch.int32, device=device)
        self.tokens = torch.zeros(max_len, dtype=torch.int64, device=device)
        self.t = 0
        self._t_dev = torch.zeros(1, dtype=torch.int64, device=device)  # = t, on the device
        self._ws = torch.empty(H * width * (D + 2) * 4, dtype=torch.uint8, device=device)
        self.use_graph = bool(use_graph) and self.device.type == "cuda"
        self._graph = None
        self._g_tok = None
        self._g_out = None
        self._g_warm = 0

    # ---- pieces shared by prefill and step -------------------------------------
    def _ve(self, tok: torch.Tensor):
        ve = [F.embedding(tok, w) for w in self.value_embeds]
        L = self.cfg.num_layers
        return [ve[0], ve[1], ve[2]] + [None] * (L - 6) + [ve[0], ve[1], ve[2]]

    def _qkv(self, lay, x: torch.Tensor, ve, pos: torch.Tensor, i: int | None = None):
        """x [T, d] (normed) -> q [T, H, D] (normed and rotated) and k, v: with
        a layer index i, k and v go to rows pos of that layer's caches (which
        are returned); otherwise they are new [T, H, D] tensors.  The glue runs
        as one kernel (``ops.decoder_qkv_glue``)."""
        cfg = self.cfg
        qkv = F.linear(x, lay["qkv"])
        a, b = lay["vlam"]
        kc = self.k_cache[i] if i is not None else None
        vc = self.v_cache[i] if i is not None else None
        return ops.decoder_qkv_glue(qkv, ve, pos, self.rotary.cos, self.rotary.sin, heads=cfg.num_heads, va=a,
                                    vb=b if ve is not None else 0.0, k_out=kc, v_out=vc)

    def _mlp(self, lay, x: torch.Tensor) -> torch.Tensor:
        h = F.linear(_norm(x), lay["mlp_fc"])
        return F.linear(F.relu(h).square(), lay["mlp_proj"])

    def _logits(self, x: torch.Tensor) -> torch.Tensor:
        return 30 * torch.sigmoid(F.linear(_norm(x), self.lm_head).float() / 7.5)

    def _select(self, qbar: torch.Tensor, kbar: torch.Tensor, nb: int, return_logits: bool = False):
        """Block-scoring lists of blocks 0..nb-1 from q̄, k̄ [H, nb, D]."""
        cfg = self.cfg
        T = nb * cfg.block_size
        ds_ptr, ds_local, _ = ops.doc_starts(self.docs[:T], cfg.block_size)
        return ops.pointer_select(ds_ptr, ds_local, bs=cfg.block_size, NB=nb, H=cfg.num_heads, window=cfg.window,
                                  n_global=cfg.n_global, budget=cfg.budget, qbar=qbar, kbar=kbar, temp=1.0,
                                  logit_scale=cfg.block_size / math.sqrt(cfg.head_dim), noise="none",
                                  return_logits=return_logits)

    # ---- prefill ---------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, tokens: torch.Tensor, *, all_logits: bool = False) -> torch.Tensor:
        """Forward over the prompt; returns the logits of the last position
        (or of every position with ``all_logits``)."""
        cfg = self.cfg
        T = tokens.numel()
        bs = cfg.block_size
        if T % bs or T > self.max_len:
            raise ValueError(f"prefill: T={T} must be a multiple of {bs} and at most {self.max_len}")
        tok = tokens.to(self.device).long()
        self.tokens[:T] = tok
        self.docs[:T] = (tok == EOT).cumsum(0).to(torch.int32)
        docs = self.docs[:T]
        _, _, ds_tok_end = ops.doc_starts(docs, bs)
        pos = torch.arange(T, device=self.device)
        ve = self._ve(tok)
        x = x0 = _norm(F.embedding(tok, self.embed))
        skips = []
        n = len(self.skip_weights)
        for i, lay in enumerate(self.layers):
            if i >= n:
                x = _skip(x, self.skip_weights[i - n], skips.pop())
            a, b = lay["lambdas"]
            x = _mix(a, b, x, x0)
            if "qkv" in lay:
                q, kc, vc = self._qkv(lay, _norm(x), ve[i], pos, i)  # k, v into cache rows 0 .. T-1
                qh, kh, vh = q.transpose(0, 1), kc[:, :T], vc[:, :T]  # [H, T, D] views
                qbar, kbar = ops.block_means(qh, kh, bs)
                self.kbar[i][:, :T // bs] = kbar
                kv_num, kv_idx, _ = self._select(qbar, kbar, T // bs)
                y, _ = ops.attn_fwd(qh[None], kh[None], vh[None], kv_num, kv_idx, docs, ds_tok_end, bs=bs,
                                    scale=cfg.attn_scale, check=False)
                x = x + F.linear(y[0].transpose(0, 1).reshape(T, -1), lay["proj"])
            x = x + self._mlp(lay, x)
            if i < n:
                skips.append(x)
        self.t = T
        self._t_dev.fill_(T)
        self.have_lists = False
        return self._logits(x) if all_logits else self._logits(x[-1:])[0]

    # ---- one decode step ---------------------------------------------------------
    def _body(self, tok: torch.Tensor, t: int, opens: bool, closes: bool) -> torch.Tensor:
        """The step at the position held in ``_t_dev`` (= t), then _t_dev += 1.
        ``opens`` / ``closes`` (eager steps only) add the block's reselection /
        its key-mean update; with both false the body is graph-capturable."""
        cfg = self.cfg
        bs = cfg.block_size
        td = self._t_dev
        # token and document bookkeeping, the embedding, its norm and the
        # value embeddings in one kernel
        x0, ve3 = ops.decoder_step_prologue(tok, td, self.tokens, self.docs, self.embed, self.value_embeds, eot=EOT)
        qb = t // bs
        if opens:  # positions of the new block not yet written carry the current document
            self.docs[t + 1:(qb + 1) * bs] = self.docs[t]
        v0, v1, v2 = ve3[0:1], ve3[1:2], ve3[2:3]
        ve = [v0, v1, v2] + [None] * (cfg.num_layers - 6) + [v0, v1, v2]
        x = x0
        skips = []
        n = len(self.skip_weights)
        H, D = cfg.num_heads, cfg.head_dim
        gemv = ops.decoder_gemv
        for i, lay in enumerate(self.layers):
            # the row-vector products run fused with their norms, activations
            # and residual adds (ops.decoder_gemv); the U-net skip (weight 1)
            # joins the next normed product
            skip = None
            a, b = lay["lambdas"]
            if i >= n:
                if self.skip_weights[i - n] == 1.0 and "qkv" in lay and (a, b) == (1.0, 0.0):
                    skip = skips.pop()
                else:
                    x = _skip(x, self.skip_weights[i - n], skips.pop())
            x = _mix(a, b, x, x0)
            if "qkv" in lay:
                if skip is not None:
                    qkv, x = gemv(x, lay["qkv"], norm=True, addx=skip)
                else:
                    qkv = gemv(x, lay["qkv"], norm=True)
                va, vb = lay["vlam"]
                vb = vb if ve[i] is not None else 0.0
                if opens:
                    # the block's lists are chosen from this token's q: the glue
                    # (k, v into cache row t), the reselection, then the attention
                    q, _, _ = ops.decoder_qkv_glue(qkv[None], ve[i], td, self.rotary.cos, self.rotary.sin, heads=H,
                                                   va=va, vb=vb, k_out=self.k_cache[i], v_out=self.v_cache[i])
                    nb = qb + 1
                    qbar = torch.zeros((H, nb, D), dtype=torch.float32, device=self.device)
                    qbar[:, qb] = q[0].float()
                    if self.record is None:
                        kv_num, kv_idx, _ = self._select(qbar, self.kbar[i][:, :nb].contiguous(), nb)
                    else:
                        kv_num, kv_idx, _, lg = self._select(qbar, self.kbar[i][:, :nb].contiguous(), nb,
                                                             return_logits=True)
                        self.record[i] = dict(q=qbar[:, qb].clone(), logits=lg.clone(), kv_num=kv_num.clone(),
                                              kv_idx=kv_idx.clone())
                    self.list_num[i].copy_(kv_num[:, qb])
                    self.list_idx[i].zero_()
                    self.list_idx[i][:, :kv_idx.shape[-1]].copy_(kv_idx[:, qb])
                    y, _ = ops.decode_attn(q[0], self.k_cache[i], self.v_cache[i], self.list_num[i], self.list_idx[i],
                                           self.docs, td, bs=bs, scale=cfg.attn_scale, workspace=self._ws, check=False)
                else:
                    # lists fixed within the block: the glue runs inside the attention
                    # (k, v into cache row t there)
                    y, _, _ = ops.decode_attn_glue(qkv, ve[i], td, self.rotary.cos, self.rotary.sin, self.k_cache[i],
                                                   self.v_cache[i], self.list_num[i], self.list_idx[i], self.docs,
                                                   heads=H, va=va, vb=vb, bs=bs, scale=cfg.attn_scale,
                                                   workspace=self._ws, check=False)
                x = gemv(y.reshape(H * D), lay["proj"], epi="resid", res=x)
                if closes:  # the block is complete: its key mean joins the candidates
                    self.kbar[i][:, qb] = self.k_cache[i][:, qb * bs:(qb + 1) * bs].float().mean(dim=1)
            h2 = gemv(x, lay["mlp_fc"], norm=True, epi="relu2")
            x = gemv(h2, lay["mlp_proj"], epi="resid", res=x)
            if i < n:
                skips.append(x)
        logits = gemv(x, self.lm_head, norm=True, epi="logit")
        td.add_(1)
        return logits

    @torch.no_grad()
    def step(self, token: int | torch.Tensor) -> torch.Tensor:
        """Append one token at position t; returns its logits [vocab_padded]."""
        bs = self.cfg.block_size
        t = self.t
        if t >= self.max_len:
            raise ValueError("step: the cache is full")
        if not isinstance(token, torch.Tensor) or not token.is_cuda:  # a host token is checked here
            if not 0 <= int(token) < self.cfg.vocab_size:
                raise ValueError(f"step: token {int(token)} outside the vocabulary [0, {self.cfg.vocab_size})")
        tok = torch.as_tensor(token, device=self.device).reshape(1).long()
        opens = t % bs == 0 or not self.have_lists
        closes = t % bs == bs - 1
        if self.use_graph and not opens and not closes:
            out = self._graph_step(tok, t)
        else:
            out = self._body(tok, t, opens, closes)
            self.have_lists = True
        self.t = t + 1
        return out

    def _graph_step(self, tok: torch.Tensor, t: int) -> torch.Tensor:
        """A step inside a block: one eager run of the body first (library
        warm-up), then a capture; every later such step replays the graph."""
        if self._graph is None and self._g_warm == 0:
            self._g_warm = 1
            side = torch.cuda.Stream(self.device)
            side.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(side):
                out = self._body(tok, t, False, False)
            torch.cuda.current_stream(self.device).wait_stream(side)
            return out
        if self._graph is None:
            self._g_tok = tok.clone()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._g_out = self._body(self._g_tok, -1, False, False)
            self._graph = g  # the capture ran nothing: replay for this token below
        else:
            self._g_tok.copy_(tok)
        self._graph.replay()
        return self._g_out.clone()

    @torch.no_grad()
    def generate(self, n_steps: int, first: int | torch.Tensor) -> torch.Tensor:
        """Greedy decoding: feeds ``first``, then each argmax, for n_steps."""
        out = torch.empty(n_steps, dtype=torch.int64, device=self.device)
        tok = torch.as_tensor(first, device=self.device)
        for s in range(n_steps):
            logits = self.step(tok)
            tok = ops.argmax(logits[:self.cfg.vocab_size], out=out[s:s + 1])  # written in place
        return out

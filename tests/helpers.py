"""Input builders shared by the tests (seeded, generated on the CPU)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import pointer as OP


def tol_check(got: torch.Tensor, ref: torch.Tensor, atol: float = 2e-2, rtol: float = 1e-2) -> tuple[bool, float]:
    """|got - ref| <= atol + rtol·|ref| elementwise (the parity bar of the
    attention outputs and gradients: 2e-2 max-abs / 1e-2 relative); returns
    (ok, max violation ratio)."""
    got = got.double().cpu()
    ref = ref.double().cpu()
    both_inf = torch.isinf(got) & torch.isinf(ref) & (torch.sign(got) == torch.sign(ref))
    err = (got - ref).abs()
    err = torch.where(both_inf, torch.zeros_like(err), err)
    bound = atol + rtol * ref.abs().nan_to_num(posinf=0.0, neginf=0.0)
    ratio = (err / bound).nan_to_num(nan=float("inf"))
    return bool((ratio <= 1.0).all()), float(ratio.max())


def docs_with_boundaries(T: int, n_docs: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    if n_docs <= 1:
        return torch.zeros(T, dtype=torch.int32)
    cuts = torch.randperm(T - 1, generator=g)[: n_docs - 1] + 1
    flag = torch.zeros(T, dtype=torch.int64)
    flag[cuts] = 1
    return flag.cumsum(0).to(torch.int32)


def qkv(H: int, T: int, D: int = 128, seed: int = 0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((1, H, T, D), generator=g).to(dtype)
    k = torch.randn((1, H, T, D), generator=g).to(dtype)
    v = torch.randn((1, H, T, D), generator=g).to(dtype)
    return q, k, v


def band_coefficients(q: torch.Tensor, K: int = 8, seed: int = 1, std: float = 0.02):
    """coeff = q·W_b, W_b ~ N(0, std) of shape [D, 2K]; A = first K, B = last K."""
    g = torch.Generator().manual_seed(seed)
    W = torch.randn((q.shape[-1], 2 * K), generator=g) * std
    c = q.float() @ W
    return c[..., :K].contiguous(), c[..., K:].contiguous()


def omegas_block(K: int = 8) -> torch.Tensor:
    return torch.tensor([math.pi * 2.0 ** (-k) for k in range(K)], dtype=torch.float32)


def random_blockscore_mask(H: int, T: int, bs: int, docs: torch.Tensor, *, window: int, n_global: int,
                           budget: int, seed: int):
    """A pointer mask from the oracle's block-scoring selection over random logits."""
    NB = T // bs
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    sel = OP.pointer_select_blockscore(logits, docs.numpy(), bs=bs, window=window, n_global=n_global,
                                       budget=budget)
    return torch.from_numpy(sel["kv_num"]), torch.from_numpy(sel["packed"])

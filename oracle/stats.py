"""CPU oracle: SCOPE debug statistics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

* ``forward_stats`` restates ``model/attn_bias.py:510-600`` (the debug block of
  ``SpectralBias.forward``) with the block size as a parameter (the reference
  hard-codes 128, ``:512``).
* ``mask_stats`` restates ``model/attn_bias.py:839-849``.
* ``blockscore_stats`` defines the statistics of the block-scoring mode
  (this project's specification): the same histograms over the picked
  pointer blocks.

Parity pins (tests/test_oracle_stats.py): golden vectors recorded from the
reference for ``forward_stats`` (3 configurations) and ``mask_stats``
(10 configurations); ``blockscore_stats`` by brute-force counting loops.
"""
from __future__ import annotations

import numpy as np

from .pointer import doc_start_token

F32 = np.float32

TOKEN_EDGES = np.array([0, 127, 255, 511, 1023, 2047, 4095, 8191, 16383, 32767, 65535, 131071, 262143,
                        524287, 1048575], dtype=np.int64)  # model/attn_bias.py:240-243
BLOCK_EDGES = np.array([0, 1, 3, 7, 15, 31, 63, 127, 255, 511, 1023, 2047, 4095, 8191],
                       dtype=np.int64)  # model/attn_bias.py:244


def bucketize(x: np.ndarray, edges: np.ndarray) -> np.ndarray:
    """torch.bucketize(right=False): i with edges[i-1] < x <= edges[i]."""
    return np.searchsorted(edges, np.asarray(x, dtype=np.int64), side="left")


def bincount(x: np.ndarray, minlength: int) -> np.ndarray:
    return np.bincount(np.asarray(x, dtype=np.int64).ravel(), minlength=minlength).astype(np.int32)


def frac(count: int, n: int) -> np.float32:
    """bool.float().mean() for an exact integer count."""
    return F32(F32(count) / F32(n)) if n > 0 else F32(np.nan)


def forward_stats(delta_star: np.ndarray, pi: np.ndarray, docs: np.ndarray | None, *, bs: int = 128,
                  rep_mode: str = "last", local_blocks_cfg: int, doc_clamp: bool, reset_active: bool,
                  reset_len: int, eps: float = 1e-9) -> dict:
    """delta_star, pi: [H,T,M] fp32.  model/attn_bias.py:510-600."""
    H, T, M = delta_star.shape
    NB = T // bs
    qb = np.arange(NB, dtype=np.int64)
    t_rep = (qb + 1) * bs - 1
    if rep_mode == "last":
        d_rep = delta_star[:, t_rep, :].astype(F32)
        p_rep = pi[:, t_rep, :].astype(F32)
    else:
        d_rep = delta_star.reshape(H, NB, bs, M).astype(np.float64).mean(axis=2).astype(F32)
        p_rep = pi.reshape(H, NB, bs, M).astype(np.float64).mean(axis=2).astype(F32)

    d_tok = d_rep.astype(np.int64)  # trunc toward zero, like Tensor.to(int64)
    out = {}
    out["delta_tokens_hist"] = bincount(bucketize(d_tok, TOKEN_EDGES), TOKEN_EDGES.size + 1)
    out["delta_blocks_hist"] = bincount(bucketize(np.floor_divide(d_tok, bs), BLOCK_EDGES), BLOCK_EDGES.size + 1)

    key = np.maximum((t_rep[None, :, None].astype(F32) - d_rep).astype(F32), F32(0.0))
    centre = np.minimum(np.floor_divide(key.astype(np.int64), bs), qb[None, :, None])
    if docs is not None:
        dst = doc_start_token(docs)
        ds_ptr = dst[t_rep] // bs
        ds_local = dst[qb * bs] // bs
        if not doc_clamp:
            ds_ptr = np.zeros_like(ds_ptr)
            ds_local = np.zeros_like(ds_local)
        if reset_active and reset_len > 0:
            ds_ptr = np.maximum(ds_ptr, ((t_rep // reset_len) * reset_len) // bs)
            ds_local = np.maximum(ds_local, ((qb * bs // reset_len) * reset_len) // bs)
        centre = np.maximum(centre, ds_ptr[None, :, None])
        if doc_clamp or reset_active:
            out["ptr_docstart_frac"] = frac(int((centre == ds_ptr[None, :, None]).sum()), centre.size)
        else:
            out["ptr_docstart_frac"] = F32(0.0)
    else:
        out["ptr_docstart_frac"] = F32(0.0)
    out["ptr_center_hist"] = bincount(bucketize(centre, BLOCK_EDGES), BLOCK_EDGES.size + 1)

    local = min(local_blocks_cfg, NB)
    local_start = np.maximum(qb - (local - 1), 0)
    if docs is not None and (doc_clamp or reset_active):
        local_start = np.maximum(local_start, ds_local)
    out["ptr_outside_local_frac"] = frac(int((centre < local_start[None, :, None]).sum()), centre.size)
    out["ptr_block0_frac"] = frac(int((centre == 0).sum()), centre.size)
    if NB > 4:
        sub = centre[:, 4:, :]
        out["ptr_block0_frac_excl"] = frac(int((sub == 0).sum()), sub.size)
    else:
        out["ptr_block0_frac_excl"] = F32(0.0)
    p64 = p_rep.astype(np.float64)
    ent = -(p64 * np.log(p64 + eps)).sum(axis=-1)
    out["pi_entropy_mean"] = F32(ent.mean())
    out["centre"] = centre.astype(np.int32)
    out["delta_rep"] = d_rep
    out["pi_rep"] = p_rep
    return out


def mask_stats(kv_num: np.ndarray, radius: np.ndarray, *, maxkv_cfg: int, half_cfg: int, M: int) -> dict:
    """model/attn_bias.py:839-849 (minlengths from the constructor, :250-258)."""
    max_extra = max(1, int(half_cfg * M))
    extra_sum = np.minimum(radius.astype(np.int64).sum(axis=-1), max_extra)
    return dict(
        kv_unique_hist=bincount(kv_num, maxkv_cfg + 1),
        ptr_radius_hist=bincount(radius, half_cfg + 1),
        ptr_extra_sum_hist=bincount(extra_sum, max_extra + 1),
        ptr_radius0_frac=frac(int((radius == 0).sum()), radius.size),
    )


def blockscore_stats(kv_num: np.ndarray, picks: np.ndarray, ds_ptr: np.ndarray, ds_local: np.ndarray, *,
                     maxkv: int, local_blocks: int) -> dict:
    """Statistics of the block-scoring mode over valid picks (pick ≥ 0).

    * kv_unique_hist        bincount(kv_num, minlength=maxkv+1)
    * ptr_dist_hist         bucketize(qb - pick, block edges), 15 bins
    * ptr_outside_local_frac  picks < max(qb-(local-1), 0, ds_local)
    * ptr_block0_frac / _excl (q-blocks ≥ 4) / ptr_docstart_frac (pick == ds_ptr)
    """
    H, QB, B = picks.shape
    qb = np.arange(QB, dtype=np.int64)[None, :, None]
    valid = picks >= 0
    n = int(valid.sum())
    dist = np.where(valid, qb - picks, 0)
    hist = np.zeros(BLOCK_EDGES.size + 1, dtype=np.int32)
    for d in dist[valid].ravel():
        hist[int(np.searchsorted(BLOCK_EDGES, d, side="left"))] += 1
    local_start = np.maximum(np.maximum(np.arange(QB) - (local_blocks - 1), 0), ds_local)[None, :, None]
    outside = valid & (picks < local_start)
    b0 = valid & (picks == 0)
    sub_valid = valid[:, 4:, :]
    b0x = b0[:, 4:, :]
    ds = valid & (picks == ds_ptr[None, :, None])
    return dict(
        kv_unique_hist=bincount(kv_num, maxkv + 1),
        ptr_dist_hist=hist,
        ptr_outside_local_frac=frac(int(outside.sum()), n) if n else F32(0.0),
        ptr_block0_frac=frac(int(b0.sum()), n) if n else F32(0.0),
        ptr_block0_frac_excl=frac(int(b0x.sum()), int(sub_valid.sum())) if int(sub_valid.sum()) else F32(0.0),
        ptr_docstart_frac=frac(int(ds.sum()), n) if n else F32(0.0),
        n_picks=np.int32(n),
    )

"""CPU oracle: the sliding-window (long / short) block masks of the layers
without the pointer mask — ``GPT.create_blockmasks``, scoped_medium.py:535-576.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Parity pins (tests/test_oracle_swa.py):

* ``block_rules``       – brute force over token pairs: ``any`` holds iff some
                          (query, key) pair of the two blocks is visible under
                          document_causal, ``all`` iff every pair is (document
                          ids non-decreasing, as the reference derives them by
                          cumsum, scoped_medium.py:537-538).
* ``dense_to_ordered``  – torch's stable argsort + flip on the same rows (the
                          library routine the reference calls, :545-548).
* ``create_blockmasks`` – single-document closed form (a window of W blocks is
                          the last W−1 blocks as full entries plus the diagonal
                          block as the partial entry); a hand-computed row with
                          a document boundary inside a block; windows 0 and 1;
                          and token level: torch's eager ``flex_attention`` over
                          the exported ``BlockMask`` (partial + full lists, the
                          mask applied to partial blocks only) equals the dense
                          document-causal attention restricted to the compact
                          list, for the long and the short mask.
"""
from __future__ import annotations

import numpy as np

I32 = np.int32


def block_rules(docs: np.ndarray, bs: int) -> tuple[np.ndarray, np.ndarray]:
    """(any, all) [NB, NB] bool (scoped_medium.py:552-561): block causality
    and document overlap from each block's first / last document id."""
    docs = np.asarray(docs).reshape(-1)
    NB = docs.shape[0] // bs
    lo = docs.reshape(NB, bs)[:, 0]
    hi = docs.reshape(NB, bs)[:, -1]
    qb = np.arange(NB)[:, None]
    kb = np.arange(NB)[None, :]
    any_ = (qb >= kb) & (lo[:, None] <= hi[None, :]) & (hi[:, None] >= lo[None, :])
    all_ = (qb > kb) & (lo[:, None] == hi[None, :]) & (hi[:, None] == lo[None, :])
    return any_, all_


def dense_to_ordered(dense: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(num [NB], indices [NB, NB]) (scoped_medium.py:545-548): the row's set
    blocks descending, then the other blocks descending."""
    num = dense.sum(axis=-1).astype(I32)
    idx = np.argsort(dense, axis=-1, kind="stable")[..., ::-1]
    return num, np.ascontiguousarray(idx).astype(I32)


def window_width(NB: int, window_blocks: int) -> int:
    """Row width of a compact list: max(1, min(W, NB + 1))."""
    return max(1, min(int(window_blocks), NB + 1))


def create_blockmasks(docs: np.ndarray, bs: int, window_blocks: int) -> dict:
    """Both masks of a window of W blocks (scoped_medium.py:535-576).

    Returns ``partial_num``, ``partial_idx``, ``full_num``, ``full_idx``
    (shared) and, for ``"long"`` (W) and ``"short"`` (W // 2):
    ``kv_num_blocks`` / ``full_kv_num_blocks`` (the BlockMask counts, :566-571)
    and the compact ``kv_num`` / ``kv_idx`` (kept full entries, then kept
    partial entries, each descending; the row tail repeats the first entry).
    """
    any_, all_ = block_rules(docs, bs)
    pnum, pidx = dense_to_ordered(any_ & ~all_)
    fnum, fidx = dense_to_ordered(all_)
    NB = pnum.shape[0]
    out = dict(partial_num=pnum, partial_idx=pidx, full_num=fnum, full_idx=fidx)
    for name, W in (("long", int(window_blocks)), ("short", int(window_blocks) // 2)):
        kvn = np.minimum(pnum, np.maximum(W - fnum, 1)).astype(I32)   # :568
        fkn = np.minimum(fnum, W - 1).astype(I32)                     # :570
        width = window_width(NB, W)
        kv_num = np.zeros(NB, dtype=I32)
        kv_idx = np.zeros((NB, width), dtype=I32)
        for qb in range(NB):
            row = list(fidx[qb, :max(int(fkn[qb]), 0)]) + list(pidx[qb, :int(kvn[qb])])
            kv_num[qb] = len(row)
            kv_idx[qb, :len(row)] = row
            kv_idx[qb, len(row):] = row[0]
        out[name] = dict(kv_num_blocks=kvn, full_kv_num_blocks=fkn, kv_num=kv_num, kv_idx=kv_idx)
    return out

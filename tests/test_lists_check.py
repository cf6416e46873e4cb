"""List validation on the host path (CPU tensors): what ``ops.check_lists``
and ``ScopeBlockMask`` accept and reject.

The rules are the guarantees of the reference's pack
(model/attn_bias.py:825-837) that the kernels rely on: per row (h, qb),
0 <= kv_num <= MAXKV, and the first kv_num entries are distinct key blocks in
[0, NB), each <= qb.  The counters are checked against a brute-force loop over
random malformed lists; a mask from the oracle's selection (every golden
pointer case) passes."""
from __future__ import annotations

import re

import numpy as np
import pytest
import torch

from oracle import pointer as P
from scope_amd import ops
from scope_amd.blockmask import ScopeBlockMask
from tests.golden import load_cases, pointer_case_args, pointer_case_reps


def _brute(kn: np.ndarray, ki: np.ndarray, NB: int, causal: bool) -> list[int]:
    H, QB, maxkv = ki.shape
    bad = [0, 0, 0, 0]
    first = 2 ** 31 - 1
    for h in range(H):
        for qb in range(QB):
            n = int(kn[h, qb])
            row_bad = False
            if n < 0 or n > maxkv:
                bad[0] += 1
                row_bad = True
            else:
                seen = set()
                for e in range(n):
                    kb = int(ki[h, qb, e])
                    if kb < 0 or kb >= NB:
                        bad[1] += 1
                        row_bad = True
                    elif causal and kb > qb:
                        bad[2] += 1
                        row_bad = True
                    elif kb in seen:
                        bad[3] += 1
                        row_bad = True
                    else:
                        seen.add(kb)
            if row_bad:
                first = min(first, h * QB + qb)
    return bad + [first]


def malformed_lists(H: int, QB: int, maxkv: int, seed: int):
    """Valid causal lists with a sprinkling of every kind of fault."""
    rng = np.random.default_rng(seed)
    kn = rng.integers(1, maxkv + 1, size=(H, QB)).astype(np.int32)
    ki = np.zeros((H, QB, maxkv), dtype=np.int32)
    for h in range(H):
        for qb in range(QB):
            n = min(int(kn[h, qb]), qb + 1)
            kn[h, qb] = n
            ki[h, qb, :n] = np.sort(rng.choice(qb + 1, size=n, replace=False))
            ki[h, qb, n:] = ki[h, qb, 0]
    flat = rng.random((H, QB))
    kn[flat < 0.03] = maxkv + 1
    kn[(flat >= 0.03) & (flat < 0.05)] = -1
    faults = rng.random((H, QB, maxkv))
    ki[faults < 0.02] = QB + 3                     # outside [0, NB)
    ki[(faults >= 0.02) & (faults < 0.03)] = -2     # negative
    rows = np.arange(QB)[None, :, None]
    late = (faults >= 0.03) & (faults < 0.05)
    ki[late] = np.broadcast_to(np.minimum(rows + 1, QB - 1), ki.shape)[late]  # after its q-block (where one exists)
    dup = (faults >= 0.05) & (faults < 0.08)
    ki[:, :, 1:][dup[:, :, 1:]] = ki[:, :, :-1][dup[:, :, 1:]]  # repeat the previous entry
    return kn, ki


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_host_counters_match_brute_force(seed):
    H, QB, maxkv = 3, 40, 9
    kn, ki = malformed_lists(H, QB, maxkv, seed)
    for causal in (True, False):
        want = _brute(kn, ki, QB, causal)
        got = ops._check_lists_host(torch.from_numpy(kn), torch.from_numpy(ki), QB, causal)
        assert got == want, (causal, got, want)
        assert sum(want[:4]) > 0


def test_check_lists_raises_with_the_first_bad_row():
    H, QB, maxkv = 2, 8, 4
    kn = torch.tensor([[1, 2, 3, 4, 4, 4, 4, 4]] * H, dtype=torch.int32)
    ki = torch.zeros((H, QB, maxkv), dtype=torch.int32)
    for qb in range(QB):
        ki[:, qb, :int(kn[0, qb])] = torch.arange(max(0, qb - int(kn[0, qb]) + 1), qb + 1)
    ops.check_lists(kn, ki, QB)  # valid
    for name, edit, msg in (
            ("kv_num", lambda n, i: n.__setitem__((1, 5), 5), "1 rows with kv_num outside"),
            ("range", lambda n, i: i.__setitem__((1, 6, 0), 8), "1 entries outside [0, 8)"),
            ("negative", lambda n, i: i.__setitem__((1, 6, 0), -1), "1 entries outside [0, 8)"),
            ("causal", lambda n, i: i.__setitem__((1, 3, 0), 4), "1 entries after their q-block"),
            ("repeat", lambda n, i: i.__setitem__((1, 7, 1), 7), "1 repeated entries")):
        n2, i2 = kn.clone(), ki.clone()
        edit(n2, i2)
        with pytest.raises(RuntimeError, match=re.escape(msg)):
            ops.check_lists(n2, i2, QB, who=name)
    # the first bad row is named
    i2 = ki.clone()
    i2[1, 6, 0] = 9
    i2[0, 7, 0] = 9
    with pytest.raises(RuntimeError, match="head 0, q-block 7"):
        ops.check_lists(kn, i2, QB)
    # entries past kv_num are not looked at; a non-causal check accepts later blocks
    i2 = ki.clone()
    i2[0, 0, 1:] = 99
    ops.check_lists(kn, i2, QB)
    i2[0, 2, 0] = 5
    ops.check_lists(kn, i2, QB, causal=False)


def test_scope_block_mask_validates_on_construction():
    cases = load_cases("pointer_ref_vectors.npz")
    for name in ("c1_pi_single_doc", "export_truncation", "gumbel_multi_doc"):
        c = cases[name]
        out = P.pointer_mask_reference(*pointer_case_reps(c), c["docs"], gumbel_u=c["gumbel_u"],
                                       **pointer_case_args(c))
        bs = int(c["bs"])
        docs = torch.from_numpy(c["docs"])
        kv_num, kv_idx = torch.from_numpy(out["kv_num"])[None], torch.from_numpy(out["packed"])[None]
        ds_tok_end = torch.from_numpy(P.doc_start_blocks(c["docs"], bs)[2])
        ScopeBlockMask(kv_num_blocks=kv_num, kv_indices=kv_idx, BLOCK_SIZE=bs, docs=docs, ds_tok_end=ds_tok_end)
        bad = kv_idx.clone()
        bad[0, 0, -1, 0] = kv_num.shape[-1]  # the last q-block lists a block past the end
        with pytest.raises(RuntimeError, match="ScopeBlockMask: malformed block lists"):
            ScopeBlockMask(kv_num_blocks=kv_num, kv_indices=bad, BLOCK_SIZE=bs, docs=docs, ds_tok_end=ds_tok_end)
        # a mask the library's builders made skips the check
        ScopeBlockMask(kv_num_blocks=kv_num, kv_indices=bad, BLOCK_SIZE=bs, docs=docs, ds_tok_end=ds_tok_end,
                       check=False)
        with pytest.raises(RuntimeError, match="do not cover"):
            ScopeBlockMask(kv_num_blocks=kv_num, kv_indices=kv_idx, BLOCK_SIZE=bs, docs=docs[:-bs],
                           ds_tok_end=ds_tok_end)

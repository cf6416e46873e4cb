"""CPU: pin the statistics oracle against the reference's golden vectors and
brute-force counting."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import pointer as P
from oracle import stats as S
from tests.golden import load_cases, pointer_case_args, pointer_case_reps

PCASES = load_cases("pointer_ref_vectors.npz")
FCASES = load_cases("forward_stats_vectors.npz")


@pytest.mark.parametrize("name", sorted(PCASES))
def test_mask_stats_match_golden(name):
    c = PCASES[name]
    a = pointer_case_args(c)
    dr, br = pointer_case_reps(c)
    out = P.pointer_mask_reference(dr, br, c["docs"], gumbel_u=c["gumbel_u"], **a)
    maxkv_cfg = int(c["cfg_pointer_local_blocks"] + (2 * c["cfg_pointer_half_blocks"] + 1) * c["M"]
                    + c["cfg_pointer_global_blocks"])
    st = S.mask_stats(out["kv_num"], out["radius"], maxkv_cfg=maxkv_cfg, half_cfg=int(c["cfg_pointer_half_blocks"]),
                      M=int(c["M"]))
    for key in ("kv_unique_hist", "ptr_radius_hist", "ptr_extra_sum_hist"):
        assert np.array_equal(st[key], c["dbg_" + key]), key
    assert st["ptr_radius0_frac"] == c["dbg_ptr_radius0_frac"]


@pytest.mark.parametrize("name", sorted(FCASES))
def test_forward_stats_match_golden(name):
    c = FCASES[name]
    st = S.forward_stats(c["delta_star"], c["pi"], c["docs"] if c["with_docs"] else None, bs=128,
                         rep_mode=str(c["rep_mode"]), local_blocks_cfg=int(c["cfg_pointer_local_blocks"]),
                         doc_clamp=bool(c["cfg_pointer_doc_clamp"]), reset_active=bool(c["cfg_reset_active"]),
                         reset_len=int(c["cfg_reset_len_active"]), eps=float(c["cfg_eps"]))
    for key in ("delta_tokens_hist", "delta_blocks_hist", "ptr_center_hist"):
        assert np.array_equal(st[key], c["dbg_" + key]), key
    for key in ("ptr_outside_local_frac", "ptr_block0_frac", "ptr_block0_frac_excl", "ptr_docstart_frac"):
        assert st[key] == c["dbg_" + key], key
    assert abs(float(st["pi_entropy_mean"]) - float(c["dbg_pi_entropy_mean"])) < 1e-6


def test_bucketize_matches_torch():
    import torch

    x = np.array([-5, 0, 1, 2, 3, 126, 127, 128, 1048575, 1048576, 5_000_000])
    for edges in (S.TOKEN_EDGES, S.BLOCK_EDGES):
        ref = torch.bucketize(torch.from_numpy(x), torch.from_numpy(edges), right=False).numpy()
        assert np.array_equal(S.bucketize(x, edges), ref)


def test_blockscore_stats_brute_force():
    rng = np.random.default_rng(0)
    H, NB, bs = 2, 12, 16
    docs = np.cumsum(rng.random(NB * bs) < 0.01).astype(np.int32)
    logits = rng.standard_normal((H, NB, NB)).astype(np.float32)
    sel = P.pointer_select_blockscore(logits, docs, bs=bs, window=2, n_global=1, budget=3)
    st = S.blockscore_stats(sel["kv_num"], sel["picks"], sel["ds_ptr"], sel["ds_local"], maxkv=sel["maxkv"],
                            local_blocks=2)
    n = out = b0 = b0x = nx = ds = 0
    hist = [0] * 15
    for h in range(H):
        for qb in range(NB):
            for pk in sel["picks"][h, qb]:
                if pk < 0:
                    continue
                n += 1
                d = qb - pk
                hist[sum(1 for e in S.BLOCK_EDGES if e < d)] += 1
                out += pk < max(qb - 1, 0, sel["ds_local"][qb])
                b0 += pk == 0
                if qb >= 4:
                    nx += 1
                    b0x += pk == 0
                ds += pk == sel["ds_ptr"][qb]
    assert st["ptr_dist_hist"].tolist() == hist
    assert st["n_picks"] == n
    assert st["ptr_outside_local_frac"] == np.float32(out / n)
    assert st["ptr_block0_frac"] == np.float32(b0) / np.float32(n)
    assert st["ptr_docstart_frac"] == np.float32(ds) / np.float32(n)
    assert st["kv_unique_hist"].sum() == H * NB

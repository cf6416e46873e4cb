"""The measurement probes behind the bench line's measured ceilings.  The
data-driven MFMA probe must really multiply the operands it is given: the
sum of a wavefront's outputs is the sum of every 32x32 product it
accumulated, which is the sum over k of (column sum of A)·(row sum of B)
for each product, computed here in fp64 from the operand layout of
v_mfma_f32_32x32x16_bf16 (lane l holds row/column l % 32, k = 8·(l // 32)
.. +7)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _product_sum(ops: np.ndarray, x: int, y: int) -> float:
    """Sum of all entries of A_x·B_y for one wavefront's operands ops [64, 16, 8]."""
    tot = 0.0
    for half in range(2):
        a = ops[32 * half:32 * (half + 1), x, :].sum(0)      # column sums of A over its rows, k = 8·half + 0..7
        b = ops[32 * half:32 * (half + 1), 8 + y, :].sum(0)  # row sums of B over its columns
        tot += float((a * b).sum())
    return tot


def test_mfma_data_probe_multiplies_its_operands():
    from scope_amd import _lib
    from scope_amd.ops import _p, _stream, call

    blocks, iters = 2, 16
    g = torch.Generator(device=DEV).manual_seed(3)
    ops = ((torch.rand((blocks * 256, 16, 8), generator=g, device=DEV) * 2 - 1) / 4).to(torch.bfloat16)
    out = torch.full((blocks * 256,), float("nan"), dtype=torch.float32, device=DEV)
    call("scope_probe_mfma_data", _p(ops), _p(out), blocks, iters, _stream(torch.device(DEV)))
    torch.cuda.synchronize()
    got = out.double().cpu().numpy().reshape(-1, 64).sum(1)  # per wavefront
    host = ops.double().cpu().numpy()
    for w in range(blocks * 4):
        o = host[64 * w:64 * (w + 1)]
        want = 0.0
        for s in range(iters):
            s8, b = s % 8, (s + 3) % 8
            want += sum(_product_sum(o, x, b) for x in (s8, (s8 + 1) % 8, (s8 + 2) % 8, (s8 + 5) % 8))
        assert abs(got[w] - want) <= 1e-4 * max(1.0, abs(want)), (w, got[w], want)
    assert _lib.load().scope_probe_mfma_flops(blocks, iters) == blocks * 4 * iters * 4 * 32768


def test_measure_peaks_reports_both_mfma_ceilings():
    from scope_amd.ops import measure_peaks

    mp = measure_peaks(DEV, mfma_iters=512, copy_mib=16, repeats=1)
    for k in ("mfma_bf16_tflops", "mfma_bf16_tflops_random", "hbm_copy_gbs"):
        assert np.isfinite(mp[k]) and mp[k] > 0, (k, mp[k])

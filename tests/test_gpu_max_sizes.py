"""Parity past 2^31 elements: the C ABI takes int64 counts where the
reference's launchers took `int` (cuda/include/cudaforge/quantization.cuh:40-55,
rmsnorm.cuh:35-62, softmax.cuh:43-65, reduction.cuh:41-55), so every index in
the kernels is 64-bit. These tests run each op once just past 2^31 elements and
check it by properties that hold at any size (round-trip error within half a
step, every code within +-127, unit-RMS rows, rows summing to one, a sum of
ones) on the whole output, plus bit-exact / oracle parity on windows at the
start, across element 2^31 and at the ragged end.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

N_BIG = (1 << 31) + 4096 + 37   # crosses 2^31, ragged last block
CHUNK = 1 << 27


def windows(n: int, width: int = 4096) -> list[tuple[int, int]]:
    """Block-aligned element windows: start, across 2^31, and the end."""
    mid = (1 << 31) - width // 2
    last = (n // 64) * 64 - width
    return [(0, width), (mid, mid + width), (last, n)]


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def test_quantize_round_trip_past_2_31_elements():
    g.announce(f"quantize/dequantize bf16, {N_BIG} elements")
    x = torch.randn(N_BIG, device="cuda", dtype=torch.bfloat16)
    q = g.empty(N_BIG, torch.int8)
    nscales = (N_BIG + 63) // 64
    s = g.empty(nscales, torch.float32)
    g.call("cf_quantize_int8", x.data_ptr(), g.cf("bf16"), q.data_ptr(), s.data_ptr(), N_BIG, g.stream())
    y = g.poison_like(x)
    g.call("cf_dequantize_int8", q.data_ptr(), s.data_ptr(), y.data_ptr(), g.cf("bf16"), N_BIG, g.stream())
    torch.cuda.synchronize()
    assert int((q == -128).sum()) == 0
    for start in range(0, N_BIG, CHUNK):
        end = min(N_BIG, start + CHUNK)
        xs = x[start:end].float()
        step = s[start // 64:(end + 63) // 64].repeat_interleave(64)[: end - start]
        err = (y[start:end].float() - xs).abs()
        # half a quantisation step, plus the bf16 rounding of the dequantised value
        assert bool((err <= 0.5 * step * (1 + 1e-6) + xs.abs() * 2.0**-8).all()), f"chunk at {start}"
    for lo, hi in windows(N_BIG):
        xh = bf16_bits(x[lo:hi])
        q_ref, s_ref = oracle.quantize_int8(xh, "bf16")
        np.testing.assert_array_equal(q[lo:hi].cpu().numpy(), q_ref, err_msg=f"codes at {lo}")
        np.testing.assert_array_equal(s[lo // 64:(hi + 63) // 64].cpu().numpy().view(np.uint32),
                                      s_ref.view(np.uint32), err_msg=f"scales at {lo}")
        y_ref = oracle.dequantize_int8(q_ref, s_ref, "bf16")
        np.testing.assert_array_equal(bf16_bits(y[lo:hi]), y_ref, err_msg=f"dequantised at {lo}")


@pytest.mark.parametrize("op", ["rmsnorm", "softmax"])
def test_row_ops_past_2_31_elements(op):
    cols = 4096
    rows = (1 << 31) // cols + 3
    g.announce(f"{op} bf16 [{rows}, {cols}] = {rows * cols} elements")
    x = torch.randn(rows, cols, device="cuda", dtype=torch.bfloat16)
    y = g.poison_like(x)
    if op == "rmsnorm":
        w = torch.ones(cols, device="cuda", dtype=torch.bfloat16)
        g.call("cf_rmsnorm", x.data_ptr(), w.data_ptr(), y.data_ptr(), g.cf("bf16"), rows, cols, 1e-6, g.stream())
    else:
        g.call("cf_softmax", x.data_ptr(), g.cf("bf16"), y.data_ptr(), g.cf("bf16"), rows, cols, g.stream())
    torch.cuda.synchronize()
    step = CHUNK // cols
    for r0 in range(0, rows, step):
        yr = y[r0:r0 + step].float()
        if op == "rmsnorm":
            stat = yr.pow(2).mean(dim=1)      # unit weight: unit mean square per row
        else:
            stat = yr.sum(dim=1)              # probabilities sum to one
        assert bool(((stat - 1.0).abs() < 1e-2).all()), f"rows at {r0}"
    boundary = (1 << 31) // cols
    for r in (0, boundary - 1, boundary, rows - 1):
        row = x[r].float().cpu().numpy()
        expected = oracle.rmsnorm(row[None], np.ones(cols), 1e-6)[0] if op == "rmsnorm" else oracle.softmax(row[None])[0]
        got = y[r].float().cpu().numpy()
        assert np.abs(got - expected).max() <= 1e-2 * np.abs(expected).max(), f"row {r}"


def test_sum_past_2_31_elements():
    n = (1 << 31) + 77
    g.announce(f"sum fp32 of {n} ones")
    x = torch.ones(n, device="cuda")
    out = g.empty(1, torch.float32)
    lib = g.lib()
    nbytes = lib.cf_reduce_sum_workspace_bytes(n)
    ws = g.empty(nbytes, torch.uint8)
    g.call("cf_reduce_sum", x.data_ptr(), g.cf("f32"), out.data_ptr(), n, ws.data_ptr(), nbytes, 0, g.stream())
    torch.cuda.synchronize()
    # fp32 partial sums of ones are exact below 2^24 per partial; the final
    # fixed-order tree over <= 4096 partials rounds at most ~12 times.
    assert abs(out.item() - n) <= n * 2.0**-20

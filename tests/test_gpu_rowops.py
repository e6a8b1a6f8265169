"""GPU parity of RMSNorm, residual+RMSNorm, softmax, the sums and the activations.

Tolerances (stated per BASELINE): fp32 outputs within 1e-5 relative of the
float64 oracle (elementwise |got - exact| <= 1e-5 |exact| + 1e-7); bf16/fp16
outputs within 1e-2 relative (|got - exact| <= 1e-2 |exact| + 1e-6) - in
practice one rounding of the fp32 result, <= 2^-9 relative. Sums: the
reference's |got - exact| <= max(|exact|, 1) * 1e-5 * sqrt(N)
(tests/cuda/test_reduction.cu:18-20), exact for integer-valued inputs.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from tests import gpu_util as g
from tests.conftest import load_golden, rng

pytestmark = pytest.mark.gpu

RTOL = {"f32": 1e-5, "bf16": 1e-2, "f16": 1e-2}
ATOL = {"f32": 1e-7, "bf16": 1e-6, "f16": 1e-6}


def assert_close(got_stored: np.ndarray, exact: np.ndarray, dtype: str, what: str) -> None:
    got = g.host_values(got_stored, dtype).astype(np.float64)
    err = np.abs(got - exact)
    bound = RTOL[dtype] * np.abs(exact) + ATOL[dtype]
    bad = np.flatnonzero(~(err <= bound).reshape(-1))  # an unwritten (NaN-poisoned) element fails
    assert bad.size == 0, (
        f"{what}: {bad.size} elements out of tolerance; worst rel "
        f"{np.max(err / (np.abs(exact) + 1e-30)):.3e} at {bad[:5]}"
    )


def assert_rmsnorm_rows(y: np.ndarray, x: np.ndarray, w: np.ndarray, dtype: str, eps: float, what: str,
                        chunk: int = 2048) -> None:
    """Every row of y against the float64 oracle, `chunk` rows at a time (bounded host memory)."""
    wv = g.host_values(w, dtype)
    for r0 in range(0, x.shape[0], chunk):
        exact = oracle.rmsnorm(g.host_values(x[r0:r0 + chunk], dtype), wv, eps)
        assert_close(y[r0:r0 + chunk], exact, dtype, f"{what} rows {r0}..{r0 + exact.shape[0] - 1}")


def run_rmsnorm(x: np.ndarray, w: np.ndarray, dtype: str, eps: float, offset: int = 0) -> np.ndarray:
    rows, cols = x.shape
    flat = np.concatenate([np.zeros(offset, x.dtype), x.reshape(-1)])
    xg = g.to_gpu(flat, dtype)
    wg = g.to_gpu(w, dtype)
    yg = g.poison_like(xg)
    es = xg.element_size()
    g.call("cf_rmsnorm", xg.data_ptr() + offset * es, wg.data_ptr(), yg.data_ptr() + offset * es,
           g.cf(dtype), rows, cols, eps, g.stream())
    torch.cuda.synchronize()
    return g.to_host(yg)[offset:].reshape(rows, cols)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize(
    "shape", [(1, 1), (1, 64), (3, 17), (8, 128), (33, 1023), (16, 4096), (3, 2049), (4, 16384), (2, 40000)]
)
def test_rmsnorm_matches_the_oracle(dtype, shape):
    rows, cols = shape
    r = rng(rows * 131 + cols)
    x = g.storage_bits(r.standard_normal((rows, cols)).astype(np.float32), dtype)
    w = g.storage_bits((1 + 0.1 * r.standard_normal(cols)).astype(np.float32), dtype)
    y = run_rmsnorm(x, w, dtype, 1e-6)
    exact = oracle.rmsnorm(g.host_values(x, dtype), g.host_values(w, dtype), 1e-6)
    assert_close(y, exact, dtype, f"rmsnorm {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 128), (4, 2048), (2, 4096), (3, 8192)], ids=str)
def test_rmsnorm_half_inputs_whose_squares_overflow_fp16(dtype, shape):
    """Every input 300 (300^2 = 90000 > 65504, fp16's largest value), weight 1:
    the fp32 sum of squares keeps every output finite and 1 within the
    reference's 2e-2 relative / 1e-2 absolute (tests/cuda/test_rmsnorm.cu:99-134
    for fp16, tests/cuda/test_reduced_precision.cu:69-103 for bf16), here at
    the reference's 2 x 128 and at the row widths of the tiled kernels."""
    rows, cols = shape
    x = g.storage_bits(np.full(shape, 300.0, np.float32), dtype)
    w = g.storage_bits(np.ones(cols, np.float32), dtype)
    stored = run_rmsnorm(x, w, dtype, 1e-6)
    y = g.host_values(stored, dtype).astype(np.float64)
    assert np.isfinite(y).all()
    assert (np.abs(y - 1.0) <= 1e-2 + 2e-2).all()
    exact = oracle.rmsnorm(g.host_values(x, dtype), g.host_values(w, dtype), 1e-6)
    assert_close(stored, exact, dtype, f"rmsnorm |x| = 300 {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rmsnorm_misaligned_rows_take_the_fallback(dtype):
    r = rng(3)
    x = g.storage_bits(r.standard_normal((5, 256)).astype(np.float32), dtype)
    w = g.storage_bits(r.standard_normal(256).astype(np.float32), dtype)
    y = run_rmsnorm(x, w, dtype, 1e-6, offset=1)
    exact = oracle.rmsnorm(g.host_values(x, dtype), g.host_values(w, dtype), 1e-6)
    assert_close(y, exact, dtype, "rmsnorm misaligned")


def test_rmsnorm_golden_cases():
    for case, d in load_golden("rmsnorm.npz").items():
        dtype = "bf16" if case.startswith("bf16") else "f32"
        y = run_rmsnorm(d["x"], d["w"], dtype, 1e-6)
        exact = oracle.rmsnorm(g.host_values(d["x"], dtype), g.host_values(d["w"], dtype), 1e-6)
        assert_close(y, exact, dtype, case)


def test_rmsnorm_unit_input_returns_the_weight_and_is_scale_invariant():
    x = np.ones((4, 256), np.float32)
    w = np.ones(256, np.float32)
    np.testing.assert_allclose(run_rmsnorm(x, w, "f32", 0.0), 1.0, rtol=1e-6)
    z = rng(4).standard_normal((4, 512)).astype(np.float32)
    a = run_rmsnorm(z, np.ones(512, np.float32), "f32", 1e-12)
    b = run_rmsnorm(z * 10, np.ones(512, np.float32), "f32", 1e-12)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


# The workgroup-tiled RMSNorm (rows of 256, 512 or 1024 16-byte vectors, at
# least 16 workgroups per CU = 4096 on MI355X) only runs at these sizes; each
# has a ragged last workgroup.
TILE_SHAPES = [("bf16", (16385, 2048)), ("bf16", (8193, 4096)), ("bf16", (4097, 8192)),
               ("f16", (8193, 4096)), ("f32", (16387, 1024)), ("f32", (4097, 4096))]


@pytest.mark.parametrize("dtype,shape", TILE_SHAPES, ids=[f"{d}-{s[0]}x{s[1]}" for d, s in TILE_SHAPES])
def test_rmsnorm_tiled_kernel_matches_the_oracle(dtype, shape):
    rows, cols = shape
    g.announce(f"rmsnorm tiled {dtype} {shape}")
    r = rng(rows + 7 * cols)
    x = g.storage_bits(r.standard_normal((rows, cols)).astype(np.float32), dtype)
    w = g.storage_bits((1 + 0.1 * r.standard_normal(cols)).astype(np.float32), dtype)
    y = run_rmsnorm(x, w, dtype, 1e-6)
    assert_rmsnorm_rows(y, x, w, dtype, 1e-6, f"tiled rmsnorm {dtype} {shape}")


def test_rmsnorm_tiled_kernel_non_finite_bits():
    """A NaN in a row and an infinite weight: the tiled kernel's fast bf16
    rounding is skipped for them, so NaN outputs carry the reference's
    canonical bits (0x7FC0) and the rest round exactly as the oracle does."""
    rows, cols = 8192, 4096
    g.announce("rmsnorm tiled bf16 non-finite")
    r = rng(99)
    xf = r.standard_normal((rows, cols)).astype(np.float32)
    xf[5, 100] = np.nan
    xf[9, 7] = 0.0
    wf = (1 + 0.1 * r.standard_normal(cols)).astype(np.float32)
    wf[7] = np.inf
    x = g.storage_bits(xf, "bf16")
    w = g.storage_bits(wf, "bf16")
    y = run_rmsnorm(x, w, "bf16", 1e-6)
    np.testing.assert_array_equal(y[5], np.full(cols, 0x7FC0, np.uint16))
    assert y[9, 7] == 0x7FC0  # 0 * inf
    cols_ok = np.arange(cols) != 7
    wv = g.host_values(w, "bf16")
    for r0 in range(0, rows, 2048):  # every row, 2048 at a time
        with np.errstate(invalid="ignore", over="ignore"):
            exact = oracle.rmsnorm(g.host_values(x[r0:r0 + 2048], "bf16"), wv, 1e-6)
        inf_col = oracle.f32_to_bf16_bits(exact[:, 7].astype(np.float32))
        np.testing.assert_array_equal(y[r0:r0 + 2048, 7], inf_col)
        finite = [i for i in range(exact.shape[0]) if r0 + i != 5]
        assert_close(y[r0:r0 + 2048][finite][:, cols_ok], exact[finite][:, cols_ok], "bf16",
                     f"non-finite neighbours, rows {r0}..")


@pytest.mark.parametrize("dtype,shape", [("bf16", (8193, 4096)), ("f32", (4097, 4096)),
                                         ("bf16", (16385, 2048)), ("f16", (16385, 2048))], ids=str)
def test_fused_residual_rmsnorm_tiled_kernel(dtype, shape):
    g.announce(f"fused residual rmsnorm tiled {dtype} {shape}")
    r = rng(shape[0] + 3)
    x = g.storage_bits(r.standard_normal(shape).astype(np.float32), dtype)
    res = g.storage_bits(r.standard_normal(shape).astype(np.float32), dtype)
    w = g.storage_bits((1 + 0.1 * r.standard_normal(shape[1])).astype(np.float32), dtype)
    xg, rg, wg = g.to_gpu(x, dtype), g.to_gpu(res, dtype), g.to_gpu(w, dtype)
    yg, sg = g.poison_like(xg), g.poison_like(xg)
    g.call("cf_fused_residual_rmsnorm", xg.data_ptr(), rg.data_ptr(), wg.data_ptr(), yg.data_ptr(),
           sg.data_ptr(), g.cf(dtype), shape[0], shape[1], 1e-6, g.stream())
    torch.cuda.synchronize()
    summed = g.storage_bits(g.host_values(x, dtype) + g.host_values(res, dtype), dtype)
    got_sum = g.to_host(sg)
    np.testing.assert_array_equal(got_sum.view(np.uint32) if dtype == "f32" else got_sum,
                                  summed.view(np.uint32) if dtype == "f32" else summed)
    assert_rmsnorm_rows(g.to_host(yg), summed, w, dtype, 1e-6, f"fused residual rmsnorm tiled {dtype} {shape}")


def test_config2_rmsnorm_full_size():
    g.announce("config 2: rmsnorm bf16 [16384, 4096]")
    r = rng(2002)
    x = oracle.f32_to_bf16_bits(r.standard_normal((16384, 4096), dtype=np.float32))
    w = oracle.f32_to_bf16_bits((1 + 0.02 * r.standard_normal(4096)).astype(np.float32))
    y = run_rmsnorm(x, w, "bf16", 1e-6)  # into a NaN-poisoned output
    assert_rmsnorm_rows(y, x, w, "bf16", 1e-6, "config 2 rmsnorm")
    # Every row: the output's RMS is the weight's RMS to bf16 precision.
    yv = g.host_values(y, "bf16").astype(np.float64) / g.host_values(w, "bf16")
    rms = np.sqrt(np.mean(yv * yv, axis=1))
    assert np.all(np.abs(rms - 1.0) < 1e-2)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(4, 17), (8, 512), (33, 4096)])
def test_fused_residual_rmsnorm(dtype, shape):
    r = rng(shape[0] + shape[1])
    x = g.storage_bits(r.standard_normal(shape).astype(np.float32), dtype)
    res = g.storage_bits(r.standard_normal(shape).astype(np.float32), dtype)
    w = g.storage_bits(r.standard_normal(shape[1]).astype(np.float32), dtype)
    xg, rg, wg = g.to_gpu(x, dtype), g.to_gpu(res, dtype), g.to_gpu(w, dtype)
    yg, sg = g.poison_like(xg), g.poison_like(xg)
    g.call("cf_fused_residual_rmsnorm", xg.data_ptr(), rg.data_ptr(), wg.data_ptr(), yg.data_ptr(),
           sg.data_ptr(), g.cf(dtype), shape[0], shape[1], 1e-6, g.stream())
    torch.cuda.synchronize()
    summed = g.storage_bits(g.host_values(x, dtype) + g.host_values(res, dtype), dtype)
    got_sum = g.to_host(sg)
    np.testing.assert_array_equal(got_sum.view(np.uint32) if dtype == "f32" else got_sum,
                                  summed.view(np.uint32) if dtype == "f32" else summed)
    exact = oracle.rmsnorm(g.host_values(summed, dtype), g.host_values(w, dtype), 1e-6)
    assert_close(g.to_host(yg), exact, dtype, "fused residual rmsnorm")


# ---------------------------------------------------------------------------
# Softmax.
# ---------------------------------------------------------------------------


def run_softmax(x: np.ndarray, in_dtype: str, out_dtype: str, offset: int = 0) -> np.ndarray:
    rows, cols = x.shape
    flat = np.concatenate([np.zeros(offset, x.dtype), x.reshape(-1)])
    xg = g.to_gpu(flat, in_dtype)
    yg = g.empty(flat.size, g.torch_dtype(out_dtype))
    g.call("cf_softmax", xg.data_ptr() + offset * xg.element_size(), g.cf(in_dtype),
           yg.data_ptr() + offset * yg.element_size(), g.cf(out_dtype), rows, cols, g.stream())
    torch.cuda.synchronize()
    return g.to_host(yg)[offset:].reshape(rows, cols)


def causal(rows: int, cols: int, seed: int) -> np.ndarray:
    x = (rng(seed).standard_normal((rows, cols)) * 2.0).astype(np.float32)
    col = np.arange(cols)[None, :]
    row = (np.arange(rows) % cols)[:, None]
    x[col > row] = -np.inf
    return x


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", [(1, 1), (1, 32), (4, 17), (8, 256), (3, 1025), (64, 4096), (2, 32768)])
def test_softmax_matches_the_oracle(dtype, shape):
    x = g.storage_bits((rng(shape[0] * 31 + shape[1]).standard_normal(shape) * 2).astype(np.float32), dtype)
    y = run_softmax(x, dtype, dtype)
    assert_close(y, oracle.softmax(g.host_values(x, dtype)), dtype, f"softmax {dtype} {shape}")


def test_softmax_golden_and_extreme_logits():
    for case, d in load_golden("softmax.npz").items():
        dtype = "bf16" if case.startswith("bf16") else "f32"
        y = run_softmax(d["x"], dtype, dtype)
        assert_close(y, oracle.softmax(g.host_values(d["x"], dtype)), dtype, case)
    ext = load_golden("softmax.npz")["extreme"]["x"]
    y = run_softmax(ext, "f32", "f32")
    assert np.isfinite(y).all()
    np.testing.assert_allclose(y[0], 0.25, rtol=1e-6)


@pytest.mark.parametrize("cols", [4, 2048])
def test_softmax_bf16_logits_fp16_cannot_represent(cols):
    """Logits 1e5, 9e4, -1e5, 0 in bf16 (tests/cuda/test_reduced_precision.cu:133-173):
    every output finite, the dominant logit takes the mass (> 0.5; exactly 1
    after rounding), and the result matches the oracle. The 2048-column row
    pads with -inf so the wide-row kernel sees the same four logits."""
    logits = np.full((1, cols), -np.inf, np.float32)
    logits[0, :4] = [100000.0, 90000.0, -100000.0, 0.0]
    x = oracle.f32_to_bf16_bits(logits)
    assert g.host_values(x, "bf16")[0, 0] > g.host_values(x, "bf16")[0, 1]
    y = g.host_values(run_softmax(x, "bf16", "bf16"), "bf16")
    assert np.isfinite(y).all()
    assert y[0, 0] > 0.5
    assert_close(oracle.f32_to_bf16_bits(y), oracle.softmax(g.host_values(x, "bf16")), "bf16", "softmax +-1e5")


@pytest.mark.parametrize("in_dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cols", [8, 512, 2048, 32768])
def test_softmax_bf16_rows_that_turn_nan(in_dtype, cols):
    """bf16 probabilities: a row holding NaN, +inf, or nothing but -inf is
    NaN throughout (its sum is NaN), stored as the canonical 0x7FC0 of
    c10::BFloat16's rounding, bit for bit, in every kernel width (two rows
    per wave, one row per wave, a workgroup per row, fp32 logits through the
    8-byte store); the finite rows around them match the oracle."""
    g.announce(f"softmax bf16 NaN rows, {in_dtype} logits, {cols} columns")
    rows = 4096 if cols <= 512 else 6  # 4096 rows of 512 bf16: two rows per wave, row 1 beside row 0
    xf = (rng(cols + 3).standard_normal((rows, cols)) * 2).astype(np.float32)
    xf[1, cols // 2] = np.nan
    xf[3, cols - 1] = np.inf
    xf[4, :] = -np.inf
    x = g.storage_bits(xf, in_dtype)
    y = run_softmax(x, in_dtype, "bf16")
    for r in (1, 3, 4):
        assert (y[r] == 0x7FC0).all(), f"row {r}: {np.unique(y[r])[:4]}"
    finite = [r for r in range(rows) if r not in (1, 3, 4)]
    assert_close(y[finite], oracle.softmax(g.host_values(x, in_dtype)[finite]), "bf16", "finite rows")
    # The scaled entry point follows the same rule (no mask: period 0).
    ys = run_softmax_scaled(x, in_dtype, "bf16", 0.5, 0)
    for r in (1, 3, 4):
        assert (ys[r] == 0x7FC0).all(), f"scaled row {r}"


def test_softmax_bf16_logits_to_fp32_probabilities_and_misaligned():
    x = oracle.f32_to_bf16_bits(causal(128, 512, 8))
    y = run_softmax(x, "bf16", "f32")
    assert_close(y, oracle.softmax(g.host_values(x, "bf16")), "f32", "bf16 -> f32 softmax")
    z = rng(9).standard_normal((6, 128)).astype(np.float32)
    assert_close(run_softmax(z, "f32", "f32", offset=1), oracle.softmax(z), "f32", "misaligned")


def test_config2_softmax_full_size():
    g.announce("config 2: causal softmax bf16 [1024, 2048]")
    x = oracle.f32_to_bf16_bits(causal(1024, 2048, 2048))
    y = run_softmax(x, "bf16", "bf16")
    exact = oracle.softmax(g.host_values(x, "bf16"))
    assert_close(y, exact, "bf16", "config 2 softmax")
    masked = np.arange(2048)[None, :] > np.arange(1024)[:, None]
    assert (g.host_values(y, "bf16")[masked] == 0).all()
    np.testing.assert_allclose(g.host_values(y, "bf16").astype(np.float64).sum(axis=1), 1.0, atol=2e-2)


def run_softmax_scaled(x: np.ndarray, in_dtype: str, out_dtype: str, scale: float, period: int,
                       offset: int = 0, in_place: bool = False) -> np.ndarray:
    rows, cols = x.shape
    flat = np.concatenate([np.zeros(offset, x.dtype), x.reshape(-1)])
    xg = g.to_gpu(flat, in_dtype)
    yg = xg if in_place else g.empty(flat.size, g.torch_dtype(out_dtype))
    g.call("cf_softmax_scaled", xg.data_ptr() + offset * xg.element_size(), g.cf(in_dtype),
           yg.data_ptr() + offset * yg.element_size(), g.cf(out_dtype), rows, cols, scale, period, g.stream())
    torch.cuda.synchronize()
    return g.to_host(yg)[offset:].reshape(rows, cols)


def masked_logits(values: np.ndarray, scale: float, period: int) -> np.ndarray:
    """scale * x in float64 with the causal -inf mask of cf_softmax_scaled."""
    z = scale * values.astype(np.float64)
    if period > 0:
        col = np.arange(z.shape[1])[None, :]
        z = np.where(col > (np.arange(z.shape[0]) % period)[:, None], -np.inf, z)
    return z


@pytest.mark.parametrize(
    "dtype,shape,period",
    [("bf16", (1024, 2048), 2048), ("bf16", (4099, 512), 512), ("f32", (4097, 256), 256), ("f16", (640, 1024), 512),
     ("bf16", (2048, 512), 0), ("f32", (3, 1025), 7), ("bf16", (5, 40000), 3), ("f32", (96, 4096), 96)],
    ids=str,
)
def test_softmax_scaled_causal_matches_the_oracle(dtype, shape, period):
    """softmax(scale * x) with column c of row r masked when c > r mod period
    (period 0: no mask), against the float64 oracle on the same stored
    logits; masked outputs are exactly 0 and whatever the masked inputs hold
    (NaN here) never reaches a result."""
    rows, cols = shape
    g.announce(f"softmax_scaled {dtype} {shape} period {period}")
    scale = 1 / math.sqrt(128)
    x = g.storage_bits((rng(rows + cols + period).standard_normal(shape) * 8).astype(np.float32), dtype)
    xv = g.host_values(x, dtype)
    z = masked_logits(xv, scale, period)
    poisoned = x.copy()
    nan_bits = {"bf16": 0x7FC0, "f16": 0x7E00}
    if dtype == "f32":
        poisoned[np.isinf(z)] = np.nan
    else:
        poisoned[np.isinf(z)] = nan_bits[dtype]
    y = run_softmax_scaled(poisoned, dtype, dtype, scale, period)
    exact = oracle.softmax(z)
    assert_close(y, exact, dtype, f"softmax_scaled {dtype} {shape} period {period}")
    assert (g.host_values(y, dtype)[np.isinf(z)] == 0).all()
    # fp32 probabilities from 16-bit logits, and the same kernel in place.
    if dtype != "f32":
        assert_close(run_softmax_scaled(x, dtype, "f32", scale, period), exact, "f32", "fp32 out")
    assert_close(run_softmax_scaled(x, dtype, dtype, scale, period, in_place=True), exact, dtype, "in place")


@pytest.mark.parametrize("period", [(1 << 32) + 1, 1 << 32, (1 << 31) + 5, 1 << 40], ids=str)
def test_softmax_scaled_periods_past_32_bits(period):
    """A period of rows or more masks column c of row r when c > r, whatever
    its size: 2^32 + 1 must not act as 1 (a 32-bit truncation). Checked
    against the oracle and bit for bit against period = rows."""
    rows, cols = 512, 512  # the one-wave-per-row kernel
    g.announce(f"softmax_scaled bf16 period {period}")
    x = g.storage_bits((rng(period % 997).standard_normal((rows, cols)) * 4).astype(np.float32), "bf16")
    y = run_softmax_scaled(x, "bf16", "bf16", 0.5, period)
    exact = oracle.softmax(masked_logits(g.host_values(x, "bf16"), 0.5, rows))
    assert_close(y, exact, "bf16", f"period {period}")
    np.testing.assert_array_equal(y, run_softmax_scaled(x, "bf16", "bf16", 0.5, rows))


def test_softmax_scaled_misaligned_and_scale_only():
    x = (rng(21).standard_normal((37, 512)) * 3).astype(np.float32)
    exact = oracle.softmax(masked_logits(x, 0.25, 512))
    assert_close(run_softmax_scaled(x, "f32", "f32", 0.25, 512, offset=1), exact, "f32", "misaligned causal")
    # period 0 and scale 1: exactly cf_softmax's result.
    xb = oracle.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(run_softmax_scaled(xb, "bf16", "bf16", 1.0, 0), run_softmax(xb, "bf16", "bf16"))


@pytest.mark.parametrize("dtype,shape", [("bf16", (4099, 512)), ("f32", (4097, 256)), ("bf16", (2049, 384))],
                         ids=str)
def test_softmax_two_rows_per_wave(dtype, shape):
    """Rows of one 16-byte vector per lane at more than 2 x 1024 rows take two
    rows per wave; an odd row count leaves the last wave one row."""
    rows, cols = shape
    g.announce(f"softmax two rows per wave {dtype} {shape}")
    x = g.storage_bits(causal(rows, cols, rows), dtype)
    y = run_softmax(x, dtype, dtype)
    assert_close(y, oracle.softmax(g.host_values(x, dtype)), dtype, f"softmax {dtype} {shape}")


@pytest.mark.parametrize(
    "in_dtype,out_dtype,shape",
    [
        ("f32", "f32", (128, 8192)),     # the reference's benchmark shape (README.md:420-431): 2 vectors per thread
        ("f32", "f32", (7, 4100)),       # 1025 vectors: just past one wave's registers, ragged
        ("f32", "f32", (3, 12000)),      # 4 vectors per thread, ragged
        ("f32", "f32", (2, 32772)),      # 8193 vectors: past the workgroup kernel, three-pass fallback
        ("bf16", "bf16", (5, 65536)),    # 8 vectors per thread, full
        ("bf16", "f32", (6, 16384)),     # bf16 logits to fp32 probabilities
        ("f16", "f16", (4, 20000)),      # ragged 16-bit row
    ],
    ids=str,
)
def test_softmax_long_rows(in_dtype, out_dtype, shape):
    """Rows longer than one wave's registers take a 1024-thread workgroup per
    row with the row in registers (up to 8 16-byte vectors per thread); past
    that, the three-pass kernel. Both against the float64 oracle, the
    workgroup kernel in place and causally masked too."""
    rows, cols = shape
    g.announce(f"softmax long rows {in_dtype}->{out_dtype} {shape}")
    x = g.storage_bits((rng(rows * 7 + cols).standard_normal(shape) * 4).astype(np.float32), in_dtype)
    xv = g.host_values(x, in_dtype)
    assert_close(run_softmax(x, in_dtype, out_dtype), oracle.softmax(xv), out_dtype, f"softmax {shape}")
    if in_dtype == out_dtype:
        assert_close(run_softmax_scaled(x, in_dtype, in_dtype, 1.0, 0, in_place=True), oracle.softmax(xv), in_dtype,
                     f"in place {shape}")
    period = max(rows // 2, 1) if rows > 4 else cols
    z = masked_logits(xv, 0.125, period)
    assert_close(run_softmax_scaled(x, in_dtype, out_dtype, 0.125, period), oracle.softmax(z), out_dtype,
                 f"causal period {period} {shape}")


@pytest.mark.parametrize(
    "in_dtype,out_dtype,shape",
    [
        ("bf16", "bf16", (256, 4096)),   # 512 vectors: 512 threads, full
        ("bf16", "bf16", (128, 3000)),   # 375 vectors: 512 threads, ragged
        ("f16", "f16", (7, 6000)),       # 750 vectors: 1024 threads, ragged
        ("bf16", "bf16", (64, 8192)),    # 1024 vectors: 1024 threads, full
        ("f32", "f32", (1024, 1028)),    # 257 vectors at 1024 rows: the shortest such row, the most rows
        ("f32", "bf16", (100, 2048)),    # fp32 logits to bf16 probabilities
        ("bf16", "f32", (33, 4104)),     # bf16 logits to fp32 probabilities, 513 vectors
        ("f32", "f32", (1025, 1028)),    # one row more than SIMDs: the one-wave form
    ],
    ids=str,
)
def test_softmax_few_rows_spread_over_a_workgroup(in_dtype, out_dtype, shape):
    """No more rows than SIMDs with 257-1024 16-byte vectors a row: a 512- or
    1024-thread workgroup per row, one vector per thread. Plain, in place, and
    causally masked with NaN in every masked input, against the float64
    oracle; masked outputs are exactly 0."""
    rows, cols = shape
    g.announce(f"softmax few rows {in_dtype}->{out_dtype} {shape}")
    x = g.storage_bits((rng(rows * 5 + cols).standard_normal(shape) * 4).astype(np.float32), in_dtype)
    xv = g.host_values(x, in_dtype)
    assert_close(run_softmax(x, in_dtype, out_dtype), oracle.softmax(xv), out_dtype, f"softmax {shape}")
    if in_dtype == out_dtype:
        assert_close(run_softmax_scaled(x, in_dtype, in_dtype, 1.0, 0, in_place=True), oracle.softmax(xv), in_dtype,
                     f"in place {shape}")
    for period in (max(rows // 2, 1), cols):
        z = masked_logits(xv, 0.125, period)
        poisoned = x.copy()
        poisoned[np.isinf(z)] = {"f32": np.nan, "bf16": 0x7FC0, "f16": 0x7E00}[in_dtype]
        y = run_softmax_scaled(poisoned, in_dtype, out_dtype, 0.125, period)
        assert_close(y, oracle.softmax(z), out_dtype, f"causal period {period} {shape}")
        assert (g.host_values(y, out_dtype)[np.isinf(z)] == 0).all()


def test_softmax_in_place():
    x = rng(10).standard_normal((16, 1024)).astype(np.float32)
    xg = g.to_gpu(x)
    g.call("cf_softmax", xg.data_ptr(), g.cf("f32"), xg.data_ptr(), g.cf("f32"), 16, 1024, g.stream())
    torch.cuda.synchronize()
    assert_close(g.to_host(xg), oracle.softmax(x), "f32", "in place")


# ---------------------------------------------------------------------------
# Sums.
# ---------------------------------------------------------------------------


def run_sum(x: np.ndarray, dtype: str = "f32", accumulate_onto: float | None = None) -> float:
    xg = g.to_gpu(x, dtype)
    n = x.size
    ws = g.empty(max(1, g.lib().cf_reduce_sum_workspace_bytes(n)), torch.uint8)
    out = torch.full((1,), 0.0 if accumulate_onto is None else accumulate_onto, device=g.DEVICE)
    g.call("cf_reduce_sum", xg.data_ptr(), g.cf(dtype), out.data_ptr(), n, ws.data_ptr(), ws.numel(),
           0 if accumulate_onto is None else 1, g.stream())
    torch.cuda.synchronize()
    return float(out.item())


@pytest.mark.parametrize("n", [1, 31, 32, 33, 255, 256, 1000, 1 << 16, 1 << 20, (1 << 24) + 7])
def test_sum_matches_the_exact_sum(n):
    x = rng(n).standard_normal(n).astype(np.float32)
    exact = oracle.sum_exact(x)
    assert abs(run_sum(x) - exact) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(n)


def test_sum_of_ones_is_exact_and_deterministic():
    assert run_sum(np.ones(100_000, np.float32)) == 100_000.0
    x = rng(11).standard_normal(3_000_001).astype(np.float32)
    first = run_sum(x)
    assert all(run_sum(x) == first for _ in range(3))


def test_sum_accumulates_when_asked_and_handles_bf16():
    x = np.ones(1000, np.float32)
    assert run_sum(x, accumulate_onto=5.0) == 1005.0
    xb = oracle.f32_to_bf16_bits(rng(12).standard_normal(50_000).astype(np.float32))
    exact = oracle.sum_exact(g.host_values(xb, "bf16"))
    assert abs(run_sum(xb, "bf16") - exact) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(50_000)


@pytest.mark.parametrize("dtype,n", [("f32", 65536), ("f32", 65537), ("bf16", 131072), ("bf16", 131073),
                                     ("f16", 131071)], ids=str)
def test_sum_around_the_single_launch_boundary(dtype, n):
    """Inputs of at most 256 KiB are summed by one workgroup in one launch,
    larger ones by the two-stage tree: both within the sqrt(n) bound of the
    exact sum, deterministic, accumulating when asked, and misaligned input
    (scalar loads) too."""
    g.announce(f"sum {dtype} n={n}")
    x = g.storage_bits(rng(n).standard_normal(n).astype(np.float32), dtype)
    exact = oracle.sum_exact(g.host_values(x, dtype))
    got = run_sum(x, dtype)
    assert abs(got - exact) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(n)
    assert run_sum(x, dtype) == got
    assert abs(run_sum(x, dtype, accumulate_onto=100.0) - (exact + 100.0)) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(n)
    padded = np.concatenate([x[:1], x])
    xg = g.to_gpu(padded, dtype)
    out = torch.zeros(1, device=g.DEVICE)
    ws = g.empty(max(1, g.lib().cf_reduce_sum_workspace_bytes(n)), torch.uint8)
    g.call("cf_reduce_sum", xg.data_ptr() + xg.element_size(), g.cf(dtype), out.data_ptr(), n, ws.data_ptr(),
           ws.numel(), 0, g.stream())
    torch.cuda.synchronize()
    assert abs(float(out.item()) - exact) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(n)


def test_an_empty_sum_leaves_the_output_untouched():
    """count 0 returns without launching, so *out keeps its value whether the
    call accumulates or overwrites (tests/cuda/test_reduction.cu:73-83, where
    the reference's launcher always accumulates)."""
    for accumulate in (1, 0):
        out = torch.full((1,), 7.5, device=g.DEVICE)
        g.call("cf_reduce_sum", 0, g.cf("f32"), out.data_ptr(), 0, 0, 0, accumulate, g.stream())
        torch.cuda.synchronize()
        assert float(out.item()) == 7.5


@pytest.mark.parametrize("shape", [(1, 1), (4, 17), (33, 1023), (128, 512), (3, 100_000)])
def test_row_sums(shape):
    x = rng(shape[0] * shape[1]).standard_normal(shape).astype(np.float32)
    xg = g.to_gpu(x)
    out = g.empty(shape[0], torch.float32)
    g.call("cf_row_sum", xg.data_ptr(), g.cf("f32"), out.data_ptr(), shape[0], shape[1], g.stream())
    torch.cuda.synchronize()
    exact = x.astype(np.float64).sum(axis=1)
    np.testing.assert_allclose(g.to_host(out), exact, rtol=1e-4, atol=1e-3)


# ---------------------------------------------------------------------------
# Activations.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 64, 1023, 100_003])
def test_activations(dtype, n):
    r = rng(n)
    x = g.storage_bits((r.standard_normal(n) * 4).astype(np.float32), dtype)
    up = g.storage_bits(r.standard_normal(n).astype(np.float32), dtype)
    xg, ug = g.to_gpu(x, dtype), g.to_gpu(up, dtype)
    xv, uv = g.host_values(x, dtype), g.host_values(up, dtype)
    for name, args, exact in (
        ("cf_silu", (xg,), oracle.silu(xv)),
        ("cf_gelu", (xg,), oracle.gelu_tanh(xv)),
        ("cf_swiglu", (xg, ug), oracle.swiglu(xv, uv)),
    ):
        yg = g.poison_like(xg)
        g.call(name, *[a.data_ptr() for a in args], yg.data_ptr(), g.cf(dtype), n, g.stream())
        torch.cuda.synchronize()
        got = g.host_values(g.to_host(yg), dtype).astype(np.float64)
        bound = (1e-5 if dtype == "f32" else 1e-2) * np.abs(exact) + (1e-6 if dtype == "f32" else 1e-3)
        assert (np.abs(got - exact) <= bound).all(), name

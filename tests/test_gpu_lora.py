"""GPU parity of the LoRA linear (forward, adapter backward) and matmul.

Tolerances: fp32 outputs |got - exact| <= 1e-4 |exact| + 1e-4 max|exact|
(the reference's CUDA tests allow 1e-3 against a double host reference,
tests/cuda/test_lora.cu:220-222); bf16 outputs
|got - exact| <= 1e-2 |exact| + 1e-3 max|exact| - 1e-2 relative with an
absolute floor at 0.1% of the output's scale for entries near zero, where a
bf16 GEMM's rounding of the accumulator (2^-9 of |y|) and of the adapter
intermediate dominate. `exact` is the float64 oracle on the same bf16 inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests import gpu_util as g
from tests.conftest import load_golden, rng

pytestmark = pytest.mark.gpu


def assert_gemm_close(got_stored: np.ndarray, exact: np.ndarray, dtype: str, what: str) -> None:
    got = g.host_values(got_stored, dtype).astype(np.float64)
    rel, floor = (1e-4, 1e-4) if dtype == "f32" else (1e-2, 1e-3)
    scale = np.max(np.abs(exact)) if exact.size else 0.0
    err = np.abs(got - exact)
    bad = np.flatnonzero(~(err <= rel * np.abs(exact) + floor * scale).reshape(-1))  # NaN fails
    assert bad.size == 0, f"{what}: {bad.size} out of tolerance, max err {err.max():.3e} (scale {scale:.3e})"


def make_operands(m: int, k: int, n: int, r: int, dtype: str, seed: int):
    gen = rng(seed)
    x = g.storage_bits(gen.standard_normal((m, k)).astype(np.float32), dtype)
    w = g.storage_bits((0.02 * gen.standard_normal((k, n))).astype(np.float32), dtype)
    a = g.storage_bits((gen.standard_normal((k, r)) / 64).astype(np.float32), dtype)
    b = g.storage_bits((0.02 * gen.standard_normal((r, n))).astype(np.float32), dtype)
    return x, w, a, b


def run_lora(x, w, a, b, dtype: str, scale: float, want_xa: bool = True):
    m, k = x.shape
    n = w.shape[1]
    r = a.shape[1]
    xg, wg, ag, bg = (g.to_gpu(t, dtype) for t in (x, w, a, b))
    yg = g.empty((m, n), g.torch_dtype(dtype))
    xa = g.empty((m, max(r, 1)), torch.float32)
    g.call("cf_lora_linear", xg.data_ptr(), wg.data_ptr(), ag.data_ptr(), bg.data_ptr(), yg.data_ptr(),
           xa.data_ptr() if want_xa else 0, g.cf(dtype), m, k, n, r, scale, g.stream())
    torch.cuda.synchronize()
    return g.to_host(yg), g.to_host(xa)


@pytest.mark.parametrize("shape", [(1, 8, 4, 2), (4, 64, 32, 8), (7, 129, 65, 3), (16, 256, 256, 16), (33, 100, 50, 4)])
def test_fp32_reference_shapes(shape):
    m, k, n, r = shape
    gen = rng(sum(shape))
    x, w, a, b = (gen.standard_normal(s).astype(np.float32) for s in ((m, k), (k, n), (k, r), (r, n)))
    y, _ = run_lora(x, w, a, b, "f32", 0.25)
    assert_gemm_close(y, oracle.lora_linear(x, w, a, b, 0.25, False), "f32", f"fp32 {shape}")


def run_lora_ws(x, w, a, b, scale: float):
    """fp32 through cf_lora_linear_ws with the workspace it asks for."""
    m, k = x.shape
    n = w.shape[1]
    r = a.shape[1]
    xg, wg, ag, bg = (g.to_gpu(t, "f32") for t in (x, w, a, b))
    yg = g.empty((m, n), torch.float32)
    xa = g.empty((m, max(r, 1)), torch.float32)
    nbytes = g.lib().cf_lora_linear_ws_bytes(g.cf("f32"), m, k, n, r)
    ws = g.empty(max(nbytes, 16), torch.uint8)
    g.call("cf_lora_linear_ws", xg.data_ptr(), wg.data_ptr(), ag.data_ptr(), bg.data_ptr(), yg.data_ptr(),
           xa.data_ptr(), g.cf("f32"), m, k, n, r, scale, ws.data_ptr() if nbytes else None, nbytes, g.stream())
    torch.cuda.synchronize()
    return g.to_host(yg), g.to_host(xa), nbytes


@pytest.mark.parametrize(
    "shape",
    [
        (32, 1024, 1024, 8),     # the reference's benchmark shapes (README.md:449-451)
        (64, 2048, 2048, 16),
        (128, 4096, 4096, 16),
        (100, 260, 132, 5),      # ragged M, N, K (multiples of 4), odd rank
        (1000, 512, 520, 12),    # many row tiles
        (3, 4, 8, 1),            # one partial K-step
        (70, 36, 68, 16),        # two K-steps, the second partial
        (40, 8192, 64, 16),      # one tile, long reduction: many slices
        (48, 512, 256, 0),       # no adapter
    ],
)
def test_fp32_mfma_path(shape):
    """fp32 problems with rank <= 16 and K, N multiples of 4 take the MFMA
    kernel (bf16 high/low split): one slice through cf_lora_linear, a split
    reduction through cf_lora_linear_ws; both within the fp32 tolerance of the
    float64 oracle, x @ a too, and the split sum bit-identical between runs."""
    m, k, n, r = shape
    g.announce(f"fp32 MFMA LoRA {shape}")
    gen = rng(7 * m + k + n + r)
    x, w, a, b = (gen.standard_normal(s).astype(np.float32) for s in ((m, k), (k, n), (k, r), (r, n)))
    exact = oracle.lora_linear(x, w, a, b, 0.25, False)
    exact_xa = x.astype(np.float64) @ a.astype(np.float64)
    y1, xa1 = run_lora(x, w, a, b, "f32", 0.25)
    assert_gemm_close(y1, exact, "f32", f"one slice {shape}")
    y2, xa2, nbytes = run_lora_ws(x, w, a, b, 0.25)
    assert_gemm_close(y2, exact, "f32", f"split reduction ({nbytes} B workspace) {shape}")
    if r > 0:
        assert_gemm_close(xa1[:, :r], exact_xa, "f32", f"x @ a one slice {shape}")
        assert_gemm_close(xa2[:, :r], exact_xa, "f32", f"x @ a split {shape}")
    y3, xa3, _ = run_lora_ws(x, w, a, b, 0.25)
    assert np.array_equal(y2.view(np.uint32), y3.view(np.uint32)), f"split sum not deterministic {shape}"
    assert np.array_equal(xa2.view(np.uint32), xa3.view(np.uint32)), f"split x @ a not deterministic {shape}"


def test_fp32_golden_cases():
    for case, d in load_golden("lora.npz").items():
        if not case.startswith("f32"):
            continue
        y, _ = run_lora(d["x"], d["w"], d["a"], d["b"], "f32", 0.25)
        assert_gemm_close(y, oracle.lora_linear(d["x"], d["w"], d["a"], d["b"], 0.25, False), "f32", case)


@pytest.mark.parametrize(
    "shape",
    [
        (256, 256, 256, 16),    # one tile
        (512, 1024, 768, 16),   # several tiles, K loop
        (300, 512, 264, 16),    # ragged M and N (N a multiple of 8 only)
        (256, 512, 256, 8),     # rank below 16
        (64, 128, 512, 3),      # odd rank
        (1024, 4096, 1024, 16), # long K
    ],
)
def test_fused_bf16_matches_the_oracle(shape):
    m, k, n, r = shape
    x, w, a, b = make_operands(m, k, n, r, "bf16", seed=m + k + n + r)
    y, xa = run_lora(x, w, a, b, "bf16", 2.0)
    xv, wv, av, bv = (g.host_values(t, "bf16") for t in (x, w, a, b))
    assert_gemm_close(y, oracle.lora_linear(xv, wv, av, bv, 2.0, True), "bf16", f"bf16 {shape}")
    np.testing.assert_allclose(xa[:, :r], xv.astype(np.float64) @ av, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize(
    "shape",
    [
        (256, 2048, 256, 16),   # one tile, 64 K-steps
        (300, 2048, 264, 12),   # ragged M and N, rank 12
        (513, 4096, 520, 2),    # rank 2, a row past a tile, columns past a tile
        (1024, 6144, 768, 16),  # 96 K-tiles
    ],
    ids=str,
)
def test_fused_bf16_long_reductions(shape):
    """Long reductions (64 to 192 K-steps of the fused kernel's pipeline,
    ragged tiles, small ranks): every output and x @ a against the float64
    oracle."""
    m, k, n, r = shape
    g.announce(f"fused bf16 LoRA, long reduction {shape}")
    x, w, a, b = make_operands(m, k, n, r, "bf16", seed=m + k + n + r)
    y, xa = run_lora(x, w, a, b, "bf16", 2.0)
    xv, wv, av, bv = (g.host_values(t, "bf16") for t in (x, w, a, b))
    assert_gemm_close(y, oracle.lora_linear(xv, wv, av, bv, 2.0, True), "bf16", f"bf16 {shape}")
    np.testing.assert_allclose(xa[:, :r], xv.astype(np.float64) @ av, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("shape", [(256, 2048, 256), (300, 4096, 264), (1000, 2048, 1000)], ids=str)
def test_matmul_bf16_long_reductions(shape):
    """cf_matmul bf16 at K >= 2048 (the rank-0 form of the fused kernel):
    every output against the float64 product."""
    m, k, n = shape
    g.announce(f"bf16 matmul, long reduction {shape}")
    gen = rng(m + 3 * k + n)
    a = g.storage_bits(gen.standard_normal((m, k)).astype(np.float32), "bf16")
    b = g.storage_bits((0.05 * gen.standard_normal((k, n))).astype(np.float32), "bf16")
    ag, bg = g.to_gpu(a, "bf16"), g.to_gpu(b, "bf16")
    cg = g.empty((m, n), torch.bfloat16)
    g.call("cf_matmul", ag.data_ptr(), bg.data_ptr(), cg.data_ptr(), g.cf("bf16"), m, n, k, g.stream())
    torch.cuda.synchronize()
    exact = g.host_values(a, "bf16").astype(np.float64) @ g.host_values(b, "bf16")
    assert_gemm_close(g.to_host(cg), exact, "bf16", f"matmul bf16 {shape}")


def test_bf16_golden_case():
    d = load_golden("lora.npz")["bf16_64x256x128r16"]
    y, _ = run_lora(d["x"], d["w"], d["a"], d["b"], "bf16", 2.0)
    vals = [g.host_values(d[k], "bf16") for k in "xwab"]
    assert_gemm_close(y, oracle.lora_linear(*vals, 2.0, True), "bf16", "golden bf16")


def test_bf16_unfused_shapes_take_the_generic_path():
    # K not a multiple of 64 and rank above 16 cannot take the fused kernel.
    for shape in ((33, 100, 48, 4), (64, 256, 128, 32)):
        m, k, n, r = shape
        x, w, a, b = make_operands(m, k, n, r, "bf16", seed=sum(shape))
        y, _ = run_lora(x, w, a, b, "bf16", 2.0)
        vals = [g.host_values(t, "bf16") for t in (x, w, a, b)]
        assert_gemm_close(y, oracle.lora_linear(*vals, 2.0, True), "bf16", f"generic {shape}")


def test_zero_b_reduces_to_the_base_layer_and_scale_is_linear():
    x, w, a, b = make_operands(256, 512, 256, 16, "bf16", seed=5)
    zero_b = np.zeros_like(b)
    y0, _ = run_lora(x, w, a, zero_b, "bf16", 2.0)
    xv, wv = g.host_values(x, "bf16"), g.host_values(w, "bf16")
    assert_gemm_close(y0, xv.astype(np.float64) @ wv, "bf16", "B = 0")
    zero_w = np.zeros_like(w)
    y1, _ = run_lora(x, zero_w, a, b, "bf16", 1.0)
    y2, _ = run_lora(x, zero_w, a, b, "bf16", 2.0)
    # Doubling a power-of-two scale doubles every bf16 output exactly.
    np.testing.assert_array_equal(g.host_values(y2, "bf16"), 2 * g.host_values(y1, "bf16"))


def test_config3_full_size():
    """Config 3 at full size, every output element against the float64 oracle
    (so every 256 x 256 tile, every row residue and both wave halves of each
    tile are checked), plus float64 column sums over each 256-row band of the
    output against the same sums of the oracle's formula (a check that a tile
    written twice or never cannot pass)."""
    g.announce("config 3: fused LoRA bf16 8192x4096x4096 r16")
    gen = rng(3003)
    m, k, n, r = 8192, 4096, 4096, 16
    # PEFT layout, then the operator layout the reference's test maps it to
    # (tests/python/test_lora.py:54-70): op(x, W^T, A^T, B^T, alpha / r).
    x = oracle.f32_to_bf16_bits(gen.standard_normal((m, k), dtype=np.float32))
    W = oracle.f32_to_bf16_bits((0.02 * gen.standard_normal((n, k), dtype=np.float32)))
    A = oracle.f32_to_bf16_bits((gen.standard_normal((r, k), dtype=np.float32) / 64))
    B = oracle.f32_to_bf16_bits((0.02 * gen.standard_normal((n, r), dtype=np.float32)))
    w, a, b = (np.ascontiguousarray(t.T) for t in (W, A, B))
    y, xa = run_lora(x, w, a, b, "bf16", 32 / 16)
    xv, wv, av, bv = (g.host_values(t, "bf16") for t in (x, w, a, b))
    exact = oracle.lora_linear(xv, wv, av, bv, 2.0, True)
    assert_gemm_close(y, exact, "bf16", "config 3 (all 8192 x 4096 outputs)")
    np.testing.assert_allclose(xa, xv.astype(np.float64) @ av, rtol=1e-3, atol=1e-3)
    # Band column sums: each output's bf16 rounding is at most 2^-8 of it, so
    # a band's sum may move by at most 2^-8 * sum |y| (plus the fp32
    # accumulation error, far smaller); a missing or duplicated 256-row tile
    # moves it by about sqrt(256) times a typical |y|.
    got = g.host_values(y, "bf16").astype(np.float64).reshape(m // 256, 256, n)
    want = exact.reshape(m // 256, 256, n)
    bound = 2.0**-8 * np.abs(got).sum(axis=1) * 1.01 + 1e-6 * np.abs(want).max()
    assert (np.abs(got.sum(axis=1) - want.sum(axis=1)) <= bound).all()


@pytest.mark.parametrize("shape,scale", [((512, 1024, 768, 16), 32 / 12), ((300, 512, 264, 12), 16 / 12)], ids=str)
def test_fused_bf16_non_power_of_two_scale(shape, scale):
    """alpha / rank that is not a power of two: the adapter term must carry no
    rounding beyond the reference's bf16 x @ a. With w = 0 the output is
    scale * bf16(x @ a) @ b alone. Taking bf16(x @ a) from the kernel's own
    fp32 x @ a (xa_out; the oracle's float64 x @ a can round to the other bf16
    neighbour), each stored value must be the exact value rounded once to
    bf16: within 2^-8 of it, plus 2^-14 of sum_j |scale xa_j b_j| for the
    arithmetic. Rounding bf16(scale * b) first leaves up to 2^-9 of that sum."""
    m, k, n, r = shape
    x, w, a, b = make_operands(m, k, n, r, "bf16", seed=m + n + r)
    xv, wv, av, bv = (g.host_values(t, "bf16") for t in (x, w, a, b))
    y, _ = run_lora(x, w, a, b, "bf16", scale)
    assert_gemm_close(y, oracle.lora_linear(xv, wv, av, bv, scale, True), "bf16", f"scale {scale:.4f} {shape}")
    y0, xa = run_lora(x, np.zeros_like(w), a, b, "bf16", scale)
    xa_bf16 = oracle.round_bf16(xa[:, :r].astype(np.float64))
    exact = scale * (xa_bf16 @ bv.astype(np.float64))
    arithmetic = abs(scale) * (np.abs(xa_bf16) @ np.abs(bv.astype(np.float64)))
    err = np.abs(g.host_values(y0, "bf16").astype(np.float64) - exact)
    bad = ~(err <= 2.0**-8 * np.abs(exact) + 2.0**-14 * arithmetic)  # NaN fails
    assert not bad.any(), f"{bad.sum()} outputs off by more than one bf16 rounding, max err {err.max():.3e}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_large_rank_forward_and_backward(dtype):
    """Rank 128 (above the fused kernel's 16): the generic path takes any rank,
    forward and adapter backward, against the oracle."""
    m, k, n, r = 200, 256, 136, 128
    x, w, a, b = make_operands(m, k, n, r, dtype, seed=128)
    y, xa = run_lora(x, w, a, b, dtype, 0.125)
    xv, wv, av, bv = (g.host_values(t, dtype) for t in (x, w, a, b))
    assert_gemm_close(y, oracle.lora_linear(xv, wv, av, bv, 0.125, dtype == "bf16"), dtype, f"rank 128 {dtype}")
    gen = rng(129)
    dy = g.storage_bits(gen.standard_normal((m, n)).astype(np.float32), dtype)
    ga, gb = run_backward(x, dy, b, xa, dtype, 0.125)
    exact_a, exact_b = oracle.lora_backward(xv, g.host_values(dy, dtype), bv, xa, 0.125, dtype == "bf16")
    assert_gemm_close(ga, exact_a, dtype, f"grad_a rank 128 {dtype}")
    assert_gemm_close(gb, exact_b, dtype, f"grad_b rank 128 {dtype}")


def run_backward(x, dy, b, xa, dtype: str, scale: float):
    m, k = x.shape
    r, n = b.shape
    xg, dyg, bg = g.to_gpu(x, dtype), g.to_gpu(dy, dtype), g.to_gpu(b, dtype)
    xag = g.to_gpu(np.ascontiguousarray(xa, dtype=np.float32))
    ga = g.empty((k, r), g.torch_dtype(dtype))
    gb = g.empty((r, n), g.torch_dtype(dtype))
    nbytes = g.lib().cf_lora_backward_workspace_bytes(m, k, n, r)
    ws = g.empty(nbytes, torch.uint8)
    g.call("cf_lora_backward", xg.data_ptr(), dyg.data_ptr(), bg.data_ptr(), xag.data_ptr(), ga.data_ptr(),
           gb.data_ptr(), g.cf(dtype), m, k, n, r, scale, ws.data_ptr(), nbytes, g.stream())
    torch.cuda.synchronize()
    return g.to_host(ga), g.to_host(gb)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize(
    "shape",
    [(64, 96, 80, 4), (130, 64, 96, 5), (300, 256, 520, 16), (8192, 512, 384, 16), (1000, 130, 70, 24),
     (8192, 4096, 4096, 16)],
)
def test_adapter_backward(dtype, shape):
    m, k, n, r = shape
    g.announce(f"adapter backward {dtype} {shape}")
    gen = rng(sum(shape) + 1)
    x = g.storage_bits(gen.standard_normal((m, k)).astype(np.float32), dtype)
    dy = g.storage_bits(gen.standard_normal((m, n)).astype(np.float32), dtype)
    b = g.storage_bits((0.02 * gen.standard_normal((r, n))).astype(np.float32), dtype)
    xa = (gen.standard_normal((m, r)) * 0.5).astype(np.float32)
    ga, gb = run_backward(x, dy, b, xa, dtype, 2.0)
    exact_a, exact_b = oracle.lora_backward(
        g.host_values(x, dtype), g.host_values(dy, dtype), g.host_values(b, dtype), xa, 2.0, dtype == "bf16"
    )
    assert_gemm_close(ga, exact_a, dtype, f"grad_a {dtype} {shape}")
    assert_gemm_close(gb, exact_b, dtype, f"grad_b {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shape", [(1, 8, 4, 2), (7, 129, 65, 3), (128, 256, 256, 16)])
def test_matmul(dtype, shape):
    m, k, n, _ = shape
    gen = rng(m * k + n)
    a = g.storage_bits(gen.standard_normal((m, k)).astype(np.float32), dtype)
    b = g.storage_bits(gen.standard_normal((k, n)).astype(np.float32), dtype)
    ag, bg = g.to_gpu(a, dtype), g.to_gpu(b, dtype)
    cg = g.empty((m, n), g.torch_dtype(dtype))
    g.call("cf_matmul", ag.data_ptr(), bg.data_ptr(), cg.data_ptr(), g.cf(dtype), m, n, k, g.stream())
    torch.cuda.synchronize()
    exact = g.host_values(a, dtype).astype(np.float64) @ g.host_values(b, dtype)
    assert_gemm_close(g.to_host(cg), exact, dtype, f"matmul {dtype} {shape}")

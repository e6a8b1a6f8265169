"""GPU parity of the INT8 quantiser through the C ABI: bit-exact codes and scales.

Bar: int8 codes and fp32 scales bit-identical to the oracle (itself pinned to
the reference's own operators by tests/test_oracle.py) and to the golden
vectors; dequantised values bit-identical too (one IEEE multiply, one RNE).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests import gpu_util as g
from tests.conftest import load_golden, rng

pytestmark = pytest.mark.gpu

QUANT_F32 = load_golden("quant_f32.npz")
QUANT_BF16 = load_golden("quant_bf16.npz")


def gpu_quantize(x_host: np.ndarray, dtype: str = "f32", offset: int = 0):
    """Quantise on the GPU; `offset` elements of padding misalign the input."""
    n = x_host.size
    padded = np.concatenate([np.zeros(offset, x_host.dtype), x_host.reshape(-1)])
    xg = g.to_gpu(padded, dtype)
    q = g.empty(n + offset, torch.int8)
    s = g.empty(max(1, (n + 63) // 64), torch.float32)
    g.call("cf_quantize_int8", xg.data_ptr() + offset * xg.element_size(), g.cf(dtype),
           q.data_ptr() + offset, s.data_ptr(), n, g.stream())
    torch.cuda.synchronize()
    return g.to_host(q)[offset:], g.to_host(s)[: (n + 63) // 64]


def assert_bits_equal(a: np.ndarray, b: np.ndarray) -> None:
    a32 = a.view(np.uint32) if a.dtype == np.float32 else a
    b32 = b.view(np.uint32) if b.dtype == np.float32 else b
    mismatch = np.flatnonzero(a32.reshape(-1) != b32.reshape(-1))
    assert mismatch.size == 0, f"{mismatch.size} mismatches, first at {mismatch[:5]}"


@pytest.mark.parametrize("case", sorted(QUANT_F32))
def test_golden_cases_are_bit_exact(case):
    d = QUANT_F32[case]
    q, s = gpu_quantize(d["x"])
    assert_bits_equal(q, d["q"])
    assert_bits_equal(s, d["s"])


@pytest.mark.parametrize("case", sorted(QUANT_BF16))
def test_bf16_golden_cases_are_bit_exact(case):
    d = QUANT_BF16[case]
    q, s = gpu_quantize(d["x"], "bf16")
    assert_bits_equal(q, d["q"])
    assert_bits_equal(s, d["s"])


def c1_input() -> np.ndarray:
    """Config 1: fp32 [4096, 4096] ~N(0,1), 1% of elements x20 at seeded positions."""
    x = rng(20260101).standard_normal((4096, 4096), dtype=np.float32)
    flat = x.reshape(-1)
    idx = rng(20260102).choice(flat.size, size=flat.size // 100, replace=False)
    flat[idx] *= 20.0
    return x


def test_config1_full_size_is_bit_exact():
    g.announce("config 1: quantise fp32 [4096, 4096]")
    x = c1_input()
    q, s = gpu_quantize(x)
    q_ref, s_ref = oracle.quantize_int8(x)
    assert_bits_equal(q, q_ref.reshape(-1))
    assert_bits_equal(s, s_ref)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 3, 63, 64, 65, 127, 1000, 4097, 100_003])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_ragged_and_misaligned_inputs(dtype, n, offset):
    values = (rng(n * 7 + offset).standard_normal(n) * 3).astype(np.float32)
    x = g.storage_bits(values, dtype)
    q, s = gpu_quantize(x, dtype, offset)
    q_ref, s_ref = oracle.quantize_int8(x, dtype)
    assert_bits_equal(q, q_ref)
    assert_bits_equal(s, s_ref)


def test_quotients_near_half_integers_take_the_exact_divide():
    # Blocks whose quotients sit within a few ulps of k + 0.5 for random
    # scales: exactly the cases where x * (1/s) and x / s can round apart.
    blocks = 4096
    r = rng(99)
    absmax = (r.uniform(0.5, 2.0, blocks) * 10.0 ** r.integers(-20, 20, blocks)).astype(np.float32)
    s = (absmax / np.float32(127)).astype(np.float32)
    k = r.integers(-126, 126, (blocks, 64)).astype(np.float32)
    target = ((k + np.float32(0.5)) * s[:, None]).astype(np.float32)
    nudge = r.integers(-3, 4, (blocks, 64))
    x = target.view(np.int32) + nudge.astype(np.int32)
    x = x.view(np.float32)
    x[:, 0] = absmax  # pins the block's scale
    q, sc = gpu_quantize(x)
    q_ref, s_ref = oracle.quantize_int8(x)
    assert_bits_equal(sc, s_ref)
    assert_bits_equal(q, q_ref.reshape(-1))


def test_ties_over_consecutive_block_maxima():
    """Quotients within a few ulps of k + 0.5 for 8192 consecutive fp32 block
    maxima at each of five magnitudes: the scales' significands run through
    every low-bit pattern there (all-ones included), which is where a
    reciprocal-based quotient could round apart from x / s."""
    r = rng(123)
    starts = np.array([127.0, 1.0, 3.0e-30, 7.5e20, 254.0 - 2.0 ** -16], dtype=np.float32)
    absmax = np.concatenate([(s.view(np.int32) + np.arange(8192, dtype=np.int32)).view(np.float32)
                             for s in starts])
    blocks = absmax.size
    scale = (absmax / np.float32(127)).astype(np.float32)
    k = r.integers(-126, 126, (blocks, 64)).astype(np.float32)
    target = ((k + np.float32(0.5)) * scale[:, None]).astype(np.float32)
    x = (target.view(np.int32) + r.integers(-2, 3, (blocks, 64)).astype(np.int32)).view(np.float32)
    x[:, 0] = absmax
    q, sc = gpu_quantize(x)
    q_ref, s_ref = oracle.quantize_int8(x)
    assert_bits_equal(sc, s_ref)
    assert_bits_equal(q, q_ref.reshape(-1))


def test_exact_half_integer_quotients_round_to_even_bf16():
    """bf16 blocks with absmax 127 * 2^j (so s = 2^j exactly) and elements
    (k + 0.5) * 2^j: every quotient is an exact tie, rounded half to even."""
    r = rng(124)
    blocks = 8192
    j = r.integers(-60, 60, blocks).astype(np.float32)
    k = r.integers(-127, 127, (blocks, 64)).astype(np.float32)
    xf = ((k + np.float32(0.5)) * np.exp2(j)[:, None]).astype(np.float32)
    xf[:, 0] = np.float32(127) * np.exp2(j)
    x = oracle.f32_to_bf16_bits(xf)
    assert np.array_equal(oracle.bf16_bits_to_f32(x), xf)  # all exactly representable
    q, sc = gpu_quantize(x, "bf16")
    q_ref, s_ref = oracle.quantize_int8(xf)
    assert_bits_equal(sc, s_ref)
    assert_bits_equal(q, q_ref.reshape(-1))
    assert np.all(np.abs(q.reshape(blocks, 64)[:, 1:].astype(np.int32)) % 2 == 0)  # ties went to even


def test_blocks_around_the_smallest_fast_scale():
    """Block maxima from just below to just above 127 * 2^-100 (the boundary
    between the reciprocal path and the IEEE divide), elements spread over
    the block's range including near-ties."""
    r = rng(125)
    centre = np.float32(127 * 2.0 ** -100)
    absmax = (centre.view(np.int32) + np.arange(-2048, 2048, dtype=np.int32)).view(np.float32)
    blocks = absmax.size
    frac = r.uniform(-1, 1, (blocks, 64)).astype(np.float32)
    x = (frac * absmax[:, None]).astype(np.float32)
    x[:, 0] = absmax
    x[:, 1] = -absmax
    q, sc = gpu_quantize(x)
    q_ref, s_ref = oracle.quantize_int8(x)
    assert_bits_equal(sc, s_ref)
    assert_bits_equal(q, q_ref.reshape(-1))


@pytest.mark.parametrize("out", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("n", [1, 65, 4096, 100_003])
def test_dequantise_is_bit_exact(out, n):
    x = (rng(n + 5).standard_normal(n) * 4).astype(np.float32)
    q_ref, s_ref = oracle.quantize_int8(x)
    qg = g.to_gpu(q_ref)
    sg = g.to_gpu(s_ref)
    y = g.empty(n, g.torch_dtype(out))
    g.call("cf_dequantize_int8", qg.data_ptr(), sg.data_ptr(), y.data_ptr(), g.cf(out), n, g.stream())
    torch.cuda.synchronize()
    assert_bits_equal(g.to_host(y), oracle.dequantize_int8(q_ref, s_ref, out))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_fake_quantisation_is_bit_exact(dtype):
    n = 70_001
    x = g.storage_bits((rng(17).standard_normal(n) * 3).astype(np.float32), dtype)
    xg = g.to_gpu(x, dtype)
    y = g.poison_like(xg)
    g.call("cf_quantize_dequantize", xg.data_ptr(), y.data_ptr(), g.cf(dtype), n, g.stream())
    torch.cuda.synchronize()
    assert_bits_equal(g.to_host(y), oracle.quantize_dequantize(x, dtype))


def test_config5_largest_tensor_bf16_round_trip_is_bit_exact():
    # Config 5's [11008, 4096] projection: bf16 ~N(0, 0.02), 0.1% outliers x50,
    # quantised then dequantised to bf16.
    g.announce("config 5: quantise bf16 [11008, 4096]")
    r = rng(5005)
    values = r.standard_normal(11008 * 4096, dtype=np.float32) * np.float32(0.02)
    idx = r.choice(values.size, size=values.size // 1000, replace=False)
    values[idx] *= 50.0
    x = oracle.f32_to_bf16_bits(values)
    q, s = gpu_quantize(x, "bf16")
    q_ref, s_ref = oracle.quantize_int8(x, "bf16")
    assert_bits_equal(q, q_ref)
    assert_bits_equal(s, s_ref)
    qg, sg = g.to_gpu(q_ref), g.to_gpu(s_ref)
    y = g.empty(x.size, torch.bfloat16)
    g.call("cf_dequantize_int8", qg.data_ptr(), sg.data_ptr(), y.data_ptr(), g.cf("bf16"), x.size, g.stream())
    torch.cuda.synchronize()
    assert_bits_equal(g.to_host(y), oracle.dequantize_int8(q_ref, s_ref, "bf16"))

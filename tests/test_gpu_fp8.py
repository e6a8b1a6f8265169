"""GPU tests of the fp8 (e4m3fn) MFMA matmul (cf_matmul_fp8, and
cf_matmul_fp8_wt, which takes the right operand K-major as w_t[N, K]).

The reference has no fp8 path, so the oracle is oracle.matmul_fp8 (float64 sum
of the exact fp8 products, pinned in tests/test_fp8_oracle.py).

Two kinds of check:
* Bit-exact, where the sum is exactly representable however it is
  accumulated: one-hot x or w (each output is one operand value), the
  identity, and powers of two in [1/4, 4] (every partial sum is a multiple of
  2^-4 below 2^17). These pin the data movement (layouts, swizzles,
  pipeline, ragged edges) bit for bit, up to 8192^3.
* General inputs: each output is rounded once to bf16 (half a step, at most
  2^-8 |y|), and the fp8 MFMA adds its 64 products with less than fp32
  internal precision (measured on MI355X: at most 2^-15.4 of sum |x w| beyond
  the bf16 rounding at k = 128, less at larger k). The bound used is
  2^-8 |y| + 2^-13 scale (|x| |w|), four times the measured excess.
Also: every finite code (subnormals, +-448, negative zero), the scale, and the
refusal of shapes the kernel cannot tile. Both layouts feed the MFMA the same
fragments, so their outputs must agree bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cuda_force_amd import _lib

from .gpu_util import announce

pytestmark = pytest.mark.gpu

MFMA_REL = 2.0**-13  # bound on the fp8 MFMA's accumulation error, relative to sum |x w|


def finite_codes(gen: np.random.Generator, shape) -> np.ndarray:
    codes = gen.integers(0, 256, size=shape, dtype=np.uint8)
    return np.where((codes & 0x7F) == 0x7F, np.uint8(0x38), codes)


def small_codes(gen: np.random.Generator, shape) -> np.ndarray:
    """Codes of magnitude 2^-3 .. 2^3 (exponent fields 4-10), either sign."""
    exponent = gen.integers(4, 11, size=shape)
    mantissa = gen.integers(0, 8, size=shape)
    sign = gen.integers(0, 2, size=shape)
    return ((sign << 7) | (exponent << 3) | mantissa).astype(np.uint8)


LAYOUTS = ("kn", "nk")  # w[K, N] through cf_matmul_fp8, w_t[N, K] through cf_matmul_fp8_wt


def run_fp8(x: torch.Tensor, w: torch.Tensor, scale: float, layout: str = "kn") -> torch.Tensor:
    """y = bf16(scale x w) for w[K, N]; layout "nk" hands the kernel w^T."""
    m, k = x.shape
    n = w.shape[1]
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    if layout == "kn":
        _lib.check(lib.cf_matmul_fp8(x.data_ptr(), w.data_ptr(), y.data_ptr(), m, n, k, scale, stream))
    else:
        w_t = w.t().contiguous()
        _lib.check(lib.cf_matmul_fp8_wt(x.data_ptr(), w_t.data_ptr(), y.data_ptr(), m, n, k, scale, stream))
    torch.cuda.synchronize()
    return y


def powers_of_two(gen: np.random.Generator, shape) -> np.ndarray:
    """Codes of +-2^-2 .. 2^2 (exponent fields 5-9, mantissa 0), 30% zeros."""
    exponent = gen.integers(5, 10, size=shape)
    sign = gen.integers(0, 2, size=shape)
    codes = ((sign << 7) | (exponent << 3)).astype(np.uint8)
    return np.where(gen.random(shape) < 0.3, np.uint8(0), codes)


def check_exact(x_codes: np.ndarray, w_codes: np.ndarray, layout: str) -> None:
    got = run_fp8(torch.from_numpy(x_codes).cuda(), torch.from_numpy(w_codes).cuda(), 1.0, layout)
    expected = oracle.round_bf16(oracle.matmul_fp8(x_codes, w_codes, 1.0))
    got = got.float().cpu().numpy().astype(np.float64)
    bad = np.argwhere(got != expected)
    assert len(bad) == 0, f"{len(bad)} outputs differ, first at {tuple(bad[0])}"


def check_against_oracle(x_codes: np.ndarray, w_codes: np.ndarray, scale: float, layout: str) -> None:
    x = torch.from_numpy(x_codes).cuda()
    w = torch.from_numpy(w_codes).cuda()
    got = run_fp8(x, w, scale, layout).float().cpu().numpy().astype(np.float64)
    expected = oracle.matmul_fp8(x_codes, w_codes, scale)
    magnitude = abs(scale) * (np.abs(oracle.e4m3fn_to_f64(x_codes)) @ np.abs(oracle.e4m3fn_to_f64(w_codes)))
    bound = 2.0**-8 * np.abs(expected) + MFMA_REL * magnitude
    err = np.abs(got - expected)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert np.all(err <= bound), f"at {worst}: got {got[worst]}, expected {expected[worst]}"


@pytest.mark.parametrize(
    "shape",
    [(1, 16, 128), (256, 256, 128), (300, 272, 384), (513, 528, 256), (64, 1024, 1152), (1000, 48, 640),
     (300, 272, 2176)],
    ids=str,
)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_against_the_oracle(shape, layout):
    """Reduction depths above 2048 with K-major w take the one-wave-per-SIMD
    kernel (here 17 K-tiles of 128: an odd count through its peeled tail)."""
    m, n, k = shape
    announce(f"fp8 matmul {shape} {layout}")
    gen = np.random.default_rng(m * 7 + n * 3 + k)
    check_against_oracle(small_codes(gen, (m, k)), small_codes(gen, (k, n)), 1.0, layout)


@pytest.mark.parametrize("shape", [(256, 256, 128), (300, 272, 384), (513, 528, 1152), (513, 528, 2304)], ids=str)
@pytest.mark.parametrize("layout", LAYOUTS)
def test_data_movement_is_exact(shape, layout):
    m, n, k = shape
    announce(f"fp8 matmul exact cases {shape} {layout}")
    gen = np.random.default_rng(m + n + k)
    one_hot_x = np.zeros((m, k), np.uint8)
    one_hot_x[np.arange(m), (np.arange(m) * 7 + 3) % k] = 0x38
    check_exact(one_hot_x, finite_codes(gen, (k, n)), layout)
    one_hot_w = np.zeros((k, n), np.uint8)
    one_hot_w[(np.arange(n) * 5 + 1) % k, np.arange(n)] = 0x38
    check_exact(finite_codes(gen, (m, k)), one_hot_w, layout)
    check_exact(powers_of_two(gen, (m, k)), powers_of_two(gen, (k, n)), layout)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_every_finite_code_and_the_scale(layout):
    announce(f"fp8 matmul every code {layout}")
    gen = np.random.default_rng(11)
    x = finite_codes(gen, (384, 512))
    w = finite_codes(gen, (512, 320))
    x[0, :256] = np.arange(256, dtype=np.uint8)  # every code once, NaN codes replaced
    x[0] = np.where((x[0] & 0x7F) == 0x7F, np.uint8(0x80), x[0])
    check_against_oracle(x, w, 0.375, layout)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_identity_reproduces_the_decoded_operand(layout):
    announce(f"fp8 matmul identity {layout}")
    gen = np.random.default_rng(12)
    x = finite_codes(gen, (260, 256))
    eye = np.where(np.eye(256, dtype=bool), np.uint8(0x38), np.uint8(0))
    got = run_fp8(torch.from_numpy(x).cuda(), torch.from_numpy(eye).cuda(), 1.0, layout).cpu()
    expected = torch.from_numpy(x).view(torch.float8_e4m3fn).to(torch.bfloat16)  # exact in bf16
    assert torch.equal(got, expected)


@pytest.mark.parametrize("shape", [(1, 16, 128), (300, 272, 384), (777, 1040, 2560), (260, 300 - 300 % 16, 4224)],
                         ids=str)
def test_both_layouts_agree_bit_for_bit(shape):
    """The MFMA receives the same fragments from either layout and each
    kernel adds the K-steps in the same order, so general codes give
    identical bits, ragged tiles included (K above 2048 with K-major w: the
    one-wave-per-SIMD kernel)."""
    m, n, k = shape
    announce(f"fp8 matmul layouts agree {shape}")
    gen = np.random.default_rng(m + 3 * n + 5 * k)
    x = torch.from_numpy(finite_codes(gen, (m, k))).cuda()
    w = torch.from_numpy(finite_codes(gen, (k, n))).cuda()
    a = run_fp8(x, w, 0.75, "kn")
    b = run_fp8(x, w, 0.75, "nk")
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_unsupported_shapes_are_refused():
    lib = _lib.load()
    assert lib.cf_matmul_fp8_shape_supported(16, 16, 128) == 1
    assert lib.cf_matmul_fp8_shape_supported(1, 4096, 8192) == 1
    assert lib.cf_matmul_fp8_shape_supported(16, 16, 64) == 0
    assert lib.cf_matmul_fp8_shape_supported(16, 24, 128) == 0
    assert lib.cf_matmul_fp8_shape_supported(0, 16, 128) == 0
    assert lib.cf_matmul_fp8_shape_supported(16, 65536, 32768) == 0  # k n >= 2^31
    x = torch.zeros(16, 64, dtype=torch.uint8, device="cuda")
    y = torch.zeros(16, 16, dtype=torch.bfloat16, device="cuda")
    status = lib.cf_matmul_fp8(x.data_ptr(), x.data_ptr(), y.data_ptr(), 16, 16, 64, 1.0,
                               torch.cuda.current_stream().cuda_stream)
    assert status == _lib.CF_ERR_UNSUPPORTED
    status = lib.cf_matmul_fp8(None, x.data_ptr(), y.data_ptr(), 16, 16, 128, 1.0, None)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT
    # K-major w: only one 256-row panel of w_t needs 32-bit offsets.
    assert lib.cf_matmul_fp8_wt_shape_supported(16, 65536, 32768) == 1
    assert lib.cf_matmul_fp8_wt_shape_supported(16, 16, 1 << 23) == 0  # 256 k = 2^31
    assert lib.cf_matmul_fp8_wt_shape_supported(16, 24, 128) == 0
    assert lib.cf_matmul_fp8_wt_shape_supported(16, 16, 64) == 0
    status = lib.cf_matmul_fp8_wt(x.data_ptr(), x.data_ptr(), y.data_ptr(), 16, 16, 64, 1.0,
                                  torch.cuda.current_stream().cuda_stream)
    assert status == _lib.CF_ERR_UNSUPPORTED
    status = lib.cf_matmul_fp8_wt(x.data_ptr(), None, y.data_ptr(), 16, 16, 128, 1.0, None)
    assert status == _lib.CF_ERR_INVALID_ARGUMENT


def test_full_size_against_torch_fp32():
    """8192^3: powers of two, whose sums torch's fp32 product also computes
    exactly, must match bit for bit after the bf16 rounding; general codes
    within the bound above plus torch's own fp32 accumulation error."""
    size = 8192
    announce(f"fp8 matmul {size}^3 against torch fp32")
    gen = torch.Generator(device="cuda").manual_seed(5)
    codes = torch.randint(0, 256, (2, size, size), generator=gen, device="cuda", dtype=torch.uint8)
    zero = torch.rand(2, size, size, generator=gen, device="cuda") < 0.3
    exponent = 5 + torch.remainder(codes, 5).to(torch.uint8)  # 5..9
    pow2 = torch.where(zero, torch.zeros_like(codes), (codes & 0x80) | (exponent << 3))
    got = run_fp8(pow2[0], pow2[1], 1.0)
    exact = pow2[0].view(torch.float8_e4m3fn).float() @ pow2[1].view(torch.float8_e4m3fn).float()
    assert torch.equal(got, exact.to(torch.bfloat16))
    assert torch.equal(run_fp8(pow2[0], pow2[1], 1.0, "nk"), got)
    del pow2, zero, exponent, exact

    # Moderate magnitudes, no NaN code: exponent field 3 or 7 (bit 6 clear,
    # bits 4 and 3 set, bit 5 random), any sign and mantissa.
    codes = (codes & 0xA7) | 0x18
    x, w = codes[0], codes[1]
    got = run_fp8(x, w, 0.5).float()
    xd = x.view(torch.float8_e4m3fn).float()
    wd = w.view(torch.float8_e4m3fn).float()
    expected = 0.5 * (xd @ wd)
    magnitude = 0.5 * (xd.abs() @ wd.abs())
    bound = 2.0**-8 * expected.abs() + (MFMA_REL + size * 2.0**-24) * magnitude
    assert bool(((got - expected).abs() <= bound).all())
    assert bool(torch.isfinite(got).all())
    assert torch.equal(run_fp8(x, w, 0.5, "nk").float(), got)

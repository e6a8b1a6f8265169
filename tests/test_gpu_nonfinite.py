"""Non-finite and near-FLT_MAX inputs through the fp32 kernels that run on the
bf16 matrix cores (the fp32 LoRA linear, one slice and split-K; the fp32
matmul, staged and pre-split). Each fp32 value v is split into hi = bf16(v)
and lo = bf16(v - hi); these tests check that the products still follow fp32
arithmetic where it is not finite, as the reference's plain fp32 kernels do
(cuda/src/lora_linear.cu:33-90, cuda/src/tensor_core_matmul.cu):

* x = +-inf gives +-inf in every output of its row (sign of x * w), and NaN
  where infinite terms of both signs meet;
* NaN propagates to its row;
* a finite |x| above bf16's largest value (3.39e38 < |x| <= FLT_MAX) gives
  the finite product, within the fp32 tolerance;
* an infinite weight gives +-inf down its column.

The expected values are float64 products by np.einsum (its own loops, so
inf * 0 = NaN as IEEE says; no BLAS kernel that skips zeros). Outputs must
have the same NaN positions, the same infinities with the same signs, and the
finite ones within 1e-4 relative plus 5e-5 of the sum of the absolute
products (|x| @ |w| + |s| (|x| @ |a|) @ |b|): the split's error is at most
about 3 * 2^-16 of each product.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests import gpu_util as g
from tests.conftest import rng

pytestmark = pytest.mark.gpu

BIG = np.float32(3.4e38)  # above bf16's largest finite value, below FLT_MAX


def f64_matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    with np.errstate(invalid="ignore", over="ignore"):
        return np.einsum("mk,kn->mn", a.astype(np.float64), b.astype(np.float64), optimize=False)


def assert_ieee_close(got: np.ndarray, exact: np.ndarray, arith: np.ndarray, what: str) -> None:
    got = got.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(exact)), (
        f"{what}: NaN at {np.argwhere(np.isnan(got) != np.isnan(exact))[:4].tolist()}")
    inf = np.isinf(exact)
    assert np.array_equal(np.isinf(got), inf), f"{what}: inf at {np.argwhere(np.isinf(got) != inf)[:4].tolist()}"
    assert np.array_equal(np.sign(got[inf]), np.sign(exact[inf])), f"{what}: an infinity has the wrong sign"
    finite = np.isfinite(exact)
    err = np.abs(got[finite] - exact[finite])
    bound = 1e-4 * np.abs(exact[finite]) + 5e-5 * arith[finite]
    assert (err <= bound).all(), f"{what}: {(err > bound).sum()} finite outputs out of tolerance"


def special_operands(m: int, k: int, n: int, r: int, seed: int):
    gen = rng(seed)
    x = gen.standard_normal((m, k)).astype(np.float32)
    w = (0.02 * gen.standard_normal((k, n))).astype(np.float32)
    a = (gen.standard_normal((k, r)) / 64).astype(np.float32)
    b = (0.02 * gen.standard_normal((r, n))).astype(np.float32)
    x[1, 5] = np.inf
    x[2, 7] = -np.inf
    x[3, 9] = BIG
    x[4, 11] = -BIG
    x[5, 3] = np.nan
    x[6, :] = BIG / k  # a whole row of large finite values
    w[13, 2] = np.inf
    # -BIG in w: its row of x is kept small, so no fp32 product overflows.
    w[14, 6] = -BIG
    x[:, 14] *= 0.01
    x[6, 14] = 0.5
    return x, w, a, b


def lora_exact(x, w, a, b, scale: float) -> tuple[np.ndarray, np.ndarray]:
    """(the float64 result, the sum of its absolute products)."""
    with np.errstate(invalid="ignore", over="ignore"):
        exact = f64_matmul(x, w) + scale * np.einsum("mr,rn->mn", f64_matmul(x, a), b.astype(np.float64),
                                                     optimize=False)
        arith = f64_matmul(np.abs(x), np.abs(w)) + abs(scale) * np.einsum(
            "mr,rn->mn", f64_matmul(np.abs(x), np.abs(a)), np.abs(b).astype(np.float64), optimize=False)
    return exact, arith


@pytest.mark.parametrize("shape", [(64, 256, 128, 8), (40, 2048, 64, 16)], ids=str)
def test_fp32_lora_follows_fp32_arithmetic_off_the_finite_range(shape):
    m, k, n, r = shape
    g.announce(f"fp32 MFMA LoRA with inf / NaN / 3.4e38 inputs {shape}")
    x, w, a, b = special_operands(m, k, n, r, seed=sum(shape))
    exact, arith = lora_exact(x, w, a, b, 0.25)
    xg, wg, ag, bg = (g.to_gpu(t, "f32") for t in (x, w, a, b))
    lib = g.lib()
    # One slice (cf_lora_linear) and the split reduction (cf_lora_linear_ws).
    y1 = g.empty((m, n), torch.float32)
    xa = g.empty((m, r), torch.float32)
    g.call("cf_lora_linear", xg.data_ptr(), wg.data_ptr(), ag.data_ptr(), bg.data_ptr(), y1.data_ptr(),
           xa.data_ptr(), g.cf("f32"), m, k, n, r, 0.25, g.stream())
    nbytes = lib.cf_lora_linear_ws_bytes(g.cf("f32"), m, k, n, r)
    ws = g.empty(max(nbytes, 16), torch.uint8)
    y2 = g.empty((m, n), torch.float32)
    g.call("cf_lora_linear_ws", xg.data_ptr(), wg.data_ptr(), ag.data_ptr(), bg.data_ptr(), y2.data_ptr(),
           None, g.cf("f32"), m, k, n, r, 0.25, ws.data_ptr() if nbytes else None, nbytes, g.stream())
    torch.cuda.synchronize()
    assert_ieee_close(g.to_host(xa), f64_matmul(x, a), f64_matmul(np.abs(x), np.abs(a)), f"x @ a {shape}")
    assert_ieee_close(g.to_host(y1), exact, arith, f"one slice {shape}")
    assert_ieee_close(g.to_host(y2), exact, arith, f"split reduction ({nbytes} B) {shape}")


def tensor_core(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    m, k = a.shape
    n = b.shape[1]
    c = g.empty((m, n), torch.float32)
    nbytes = g.lib().cf_matmul_tensor_core_workspace_bytes(m, n, k)
    ws = g.empty(nbytes, torch.uint8)
    g.call("cf_matmul_tensor_core", a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, ws.data_ptr(), nbytes,
           g.stream())
    torch.cuda.synchronize()
    return g.to_host(c)


@pytest.mark.parametrize("shape", [(128, 128, 64), (96, 256, 520)], ids=str)
def test_fp32_matmul_follows_fp32_arithmetic_off_the_finite_range(shape):
    """Both routes: 16-byte aligned a (the kernel that splits while staging)
    and a at a 4-byte offset (the separate split pass, then the bf16 GEMM)."""
    m, n, k = shape
    g.announce(f"fp32 tensor-core matmul with inf / NaN / 3.4e38 inputs {shape}")
    x, w, _, _ = special_operands(m, k, n, 1, seed=m + n + k)
    exact, arith = f64_matmul(x, w), f64_matmul(np.abs(x), np.abs(w))
    ag, bg = g.to_gpu(x, "f32"), g.to_gpu(w, "f32")
    assert_ieee_close(tensor_core(ag, bg), exact, arith, f"aligned {shape}")
    storage = g.empty(m * k + 1, torch.float32)
    shifted = storage[1:].view(m, k)
    shifted.copy_(ag)
    assert_ieee_close(tensor_core(shifted, bg), exact, arith, f"offset a {shape}")


def bf16_operands(m: int, k: int, n: int, r: int, seed: int):
    """bf16 bits of x, w, a, b with +-inf and NaN in x and an infinite weight.
    Row 1 of x is +inf at column 5 where a's row 5, w's row 5 and b's first
    eight columns are positive, so y[1, :8] is exactly +inf: every adapter
    term there is +inf * (scale * b), with no term of the other sign."""
    gen = rng(seed)
    x = gen.standard_normal((m, k)).astype(np.float32)
    w = (0.02 * gen.standard_normal((k, n))).astype(np.float32)
    a = (gen.standard_normal((k, r)) / 64).astype(np.float32)
    b = (0.02 * gen.standard_normal((r, n))).astype(np.float32)
    x[1, 5] = np.inf
    a[5, :] = np.abs(a[5, :])
    w[5, :8] = np.abs(w[5, :8])
    b[:, :8] = np.abs(b[:, :8])
    x[2, 7] = -np.inf
    x[5, 3] = np.nan
    w[13, 10] = np.inf
    return tuple(g.storage_bits(t, "bf16") for t in (x, w, a, b))


@pytest.mark.parametrize("shape", [(256, 512, 256, 8), (256, 512, 256, 16), (256, 2048, 256, 8),
                                   (300, 2048, 264, 16)], ids=str)
def test_fused_bf16_lora_follows_the_reference_off_the_finite_range(shape):
    """The reference's bf16 path: x @ w + scale * (bf16(x @ a) @ b). An
    infinite x @ a times scale * b must be +-inf (the kernel splits scale * b
    into two bf16 parts; the low part is 0 for scale 2), and the adapter
    columns past the rank (rank 8) must not turn inf * 0 into NaN; at short
    and long reductions, with ragged tiles."""
    m, k, n, r = shape
    g.announce(f"bf16 fused LoRA with inf / NaN inputs {shape}")
    bits = bf16_operands(m, k, n, r, seed=sum(shape))
    xv, wv, av, bv = (g.host_values(t, "bf16") for t in bits)
    with np.errstate(invalid="ignore", over="ignore"):
        xa = g.host_values(g.storage_bits(f64_matmul(xv, av).astype(np.float32), "bf16"), "bf16")
        exact = f64_matmul(xv, wv) + 2.0 * np.einsum("mr,rn->mn", xa.astype(np.float64), bv.astype(np.float64),
                                                     optimize=False)
        arith = f64_matmul(np.abs(xv), np.abs(wv)) + 2.0 * np.einsum(
            "mr,rn->mn", np.abs(xa).astype(np.float64), np.abs(bv).astype(np.float64), optimize=False)
    assert np.isposinf(exact[1, :8]).all()
    xg, wg, ag, bg = (g.to_gpu(t, "bf16") for t in bits)
    y = g.empty((m, n), torch.bfloat16)
    g.call("cf_lora_linear", xg.data_ptr(), wg.data_ptr(), ag.data_ptr(), bg.data_ptr(), y.data_ptr(), None,
           g.cf("bf16"), m, k, n, r, 2.0, g.stream())
    torch.cuda.synchronize()
    got = g.host_values(g.to_host(y), "bf16").astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(exact)), (
        f"NaN at {np.argwhere(np.isnan(got) != np.isnan(exact))[:4].tolist()}")
    inf = np.isinf(exact)
    assert np.array_equal(np.isinf(got), inf) and np.array_equal(np.sign(got[inf]), np.sign(exact[inf]))
    finite = np.isfinite(exact)
    err = np.abs(got[finite] - exact[finite])
    assert (err <= 1e-2 * np.abs(exact[finite]) + 1e-3 * arith[finite]).all()

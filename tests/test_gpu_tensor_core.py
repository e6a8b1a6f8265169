"""GPU tests of the fp32 matmul on the bf16 MFMA units (cf_matmul_tensor_core).

The reference's cases (tests/cuda/test_tensor_core_matmul.cu:80-151): its four
shapes against a float64 host product with its TF32 tolerance (relative 2e-2
plus an absolute 3e-3 sqrt(k)), refusal of shapes the kernel cannot tile, and
agreement with the CUDA-core fp32 path without being bit-identical to it. The
hi/lo bf16 split is checked to a much tighter bound than TF32 allows (1e-4
sqrt(k) absolute on N(0, 1) inputs, from about 2^-16 relative error per
product), on ragged shapes the reference refused, and at 4096^3.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from cuda_force_amd import _lib

from . import gpu_util as g
from .gpu_util import announce

pytestmark = pytest.mark.gpu


def tensor_core(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    m, k = a.shape
    n = b.shape[1]
    c = torch.full((m, n), float("nan"), device=a.device)
    nbytes = lib.cf_matmul_tensor_core_workspace_bytes(m, n, k)
    ws = g.empty(nbytes, torch.uint8)
    _lib.check(lib.cf_matmul_tensor_core(a.data_ptr(), b.data_ptr(), c.data_ptr(), m, n, k, ws.data_ptr(),
                                         nbytes, torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return c


def reference_product(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    return a.double().cpu().numpy() @ b.double().cpu().numpy()


@pytest.mark.parametrize("shape", [(16, 16, 8), (64, 32, 16), (128, 128, 64), (256, 64, 128)], ids=str)
def test_reference_shapes_within_tf32_tolerance_and_far_tighter(shape):
    m, n, k = shape
    announce(f"tensor-core matmul {shape}")
    gen = torch.Generator(device="cuda").manual_seed(m + k)
    a = torch.randn(m, k, generator=gen, device="cuda")
    b = torch.randn(k, n, generator=gen, device="cuda")
    got = tensor_core(a, b).cpu().numpy()
    expected = reference_product(a, b)
    tf32_bound = 2e-2 * np.abs(expected) + 3e-3 * math.sqrt(k)
    assert np.all(np.abs(got - expected) <= tf32_bound)
    assert np.abs(got - expected).max() <= 1e-4 * math.sqrt(k)


@pytest.mark.parametrize("shape", [(15, 16, 8), (100, 24, 12), (257, 520, 70), (1, 8, 1)], ids=str)
def test_ragged_shapes(shape):
    m, n, k = shape
    announce(f"tensor-core matmul ragged {shape}")
    gen = torch.Generator(device="cuda").manual_seed(n)
    a = torch.randn(m, k, generator=gen, device="cuda")
    b = torch.randn(k, n, generator=gen, device="cuda")
    got = tensor_core(a, b).cpu().numpy()
    assert np.abs(got - reference_product(a, b)).max() <= 1e-4 * math.sqrt(k)


def test_refuses_shapes_it_cannot_tile():
    lib = _lib.load()
    assert lib.cf_tensor_cores_available() == 1
    assert lib.cf_matmul_tensor_core_shape_supported(16, 17, 8) == 0
    assert lib.cf_matmul_tensor_core_shape_supported(0, 16, 8) == 0
    assert lib.cf_matmul_tensor_core_shape_supported(16, 16, 0) == 0
    assert lib.cf_matmul_tensor_core_shape_supported(16, 16, 8) == 1
    assert lib.cf_matmul_tensor_core_shape_supported(256, 512, 128) == 1
    assert lib.cf_matmul_tensor_core_workspace_bytes(16, 17, 8) == 0
    a = torch.randn(16, 8, device="cuda")
    b = torch.randn(8, 17, device="cuda")
    c = torch.zeros(16, 17, device="cuda")
    status = lib.cf_matmul_tensor_core(a.data_ptr(), b.data_ptr(), c.data_ptr(), 16, 17, 8, None, 0,
                                       torch.cuda.current_stream().cuda_stream)
    assert status == _lib.CF_ERR_UNSUPPORTED
    torch.cuda.synchronize()
    assert torch.count_nonzero(c) == 0  # nothing launched


def test_agrees_with_an_fp32_fma_path_without_being_identical():
    """The reference compares its tensor-core result with its CUDA-core fp32
    path: close, not bit-identical. Here cf_matmul's fp32 path also runs on
    the matrix cores (the same three-product split), so the fp32 FMA product
    compared against is torch's."""
    announce("tensor-core matmul vs an fp32 FMA product")
    gen = torch.Generator(device="cuda").manual_seed(11)
    a = torch.randn(128, 64, generator=gen, device="cuda")
    b = torch.randn(64, 128, generator=gen, device="cuda")
    tc = tensor_core(a, b)
    plain = a @ b
    torch.cuda.synchronize()
    diff = (tc - plain).abs()
    assert diff.max().item() <= 2e-2 * plain.abs().max().item() + 3e-3 * 8
    assert diff.max().item() > 1e-7  # a different arithmetic path, not a copy of the fp32 one


@pytest.mark.parametrize("shape", [(300, 136, 260), (1000, 1000, 1000), (77, 4096, 512), (129, 8, 4)], ids=str)
def test_staged_kernel_shapes_and_the_fallback(shape):
    """Small outputs with 16-byte aligned operands and k a multiple of 4 take
    the kernel that splits fp32 into bf16 parts on the way into LDS (128 x 128
    tiles, fixed-order split K); a misaligned `a` takes the split-pass kernel.
    Both within 1e-4 sqrt(k) of the float64 product, and close to each other."""
    m, n, k = shape
    announce(f"tensor-core matmul staged kernel {shape}")
    gen = torch.Generator(device="cuda").manual_seed(m + n + k)
    a = torch.randn(m, k, generator=gen, device="cuda")
    b = torch.randn(k, n, generator=gen, device="cuda")
    expected = reference_product(a, b)
    staged = tensor_core(a, b)
    assert np.abs(staged.cpu().numpy() - expected).max() <= 1e-4 * math.sqrt(k)
    assert torch.equal(staged.view(torch.int32), tensor_core(a, b).view(torch.int32))
    # The same values at a 4-byte offset: a is no longer 16-byte aligned.
    storage = torch.empty(m * k + 1, device="cuda")
    shifted = storage[1:].view(m, k)
    shifted.copy_(a)
    fallback = tensor_core(shifted, b)
    assert np.abs(fallback.cpu().numpy() - expected).max() <= 1e-4 * math.sqrt(k)
    assert (fallback - staged).abs().max().item() <= 2e-4 * math.sqrt(k)


def test_large_square():
    announce("tensor-core matmul 4096^3")
    gen = torch.Generator(device="cuda").manual_seed(5)
    n = 4096
    a = torch.randn(n, n, generator=gen, device="cuda")
    b = torch.randn(n, n, generator=gen, device="cuda")
    got = tensor_core(a, b)
    rows = [0, 1777, 4095]
    expected = a[rows].double() @ b.double()
    assert (got[rows].double() - expected).abs().max().item() <= 1e-4 * math.sqrt(n)


@pytest.mark.parametrize("shape", [(1024, 1024, 1024), (2048, 1024, 2048), (512, 256, 4096)], ids=str)
def test_split_reduction_range_is_accurate_and_deterministic(shape):
    """Small outputs cut the reduction into slices whose fp32 partial products
    are summed in slice order: as accurate as one pass, and bit-identical
    from call to call."""
    m, n, k = shape
    announce(f"tensor-core matmul split K {shape}")
    gen = torch.Generator(device="cuda").manual_seed(k + 3)
    a = torch.randn(m, k, generator=gen, device="cuda")
    b = torch.randn(k, n, generator=gen, device="cuda")
    got = tensor_core(a, b)
    again = tensor_core(a, b)
    assert torch.equal(got.view(torch.int32), again.view(torch.int32))
    rows = [0, m // 3, m - 1]
    expected = a[rows].double() @ b.double()
    assert (got[rows].double() - expected).abs().max().item() <= 1e-4 * math.sqrt(k)

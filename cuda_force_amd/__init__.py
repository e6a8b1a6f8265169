"""MI355X-native implementation of CudaForge's custom-op hot path.

The operator surface of the reference package (python/cudaforge/__init__.py:17-32)
with gfx950 HIP kernels behind it; see ``cuda_force_amd.ops``. The reference's
serving and training runtime is not part of this package.
"""

from __future__ import annotations

from cuda_force_amd.ops import (
    CUDA_KERNELS_AVAILABLE,
    KERNEL_DTYPES,
    QUANT_BLOCK_SIZE,
    BackendReport,
    ExtensionMissingError,
    backend_report,
    dequantize_int8,
    fake_quantize_int8,
    fused_residual_rmsnorm,
    gelu,
    kernel_supports,
    lora_linear,
    quantization_error,
    quantize_int8,
    rmsnorm,
    row_sum,
    silu,
    softmax,
    softmax_as,
    softmax_scaled,
    sum_reduce,
    swiglu,
)

__version__ = "0.1.0"

__all__ = [
    "CUDA_KERNELS_AVAILABLE",
    "KERNEL_DTYPES",
    "QUANT_BLOCK_SIZE",
    "BackendReport",
    "ExtensionMissingError",
    "backend_report",
    "dequantize_int8",
    "fake_quantize_int8",
    "fused_residual_rmsnorm",
    "gelu",
    "kernel_supports",
    "lora_linear",
    "quantization_error",
    "quantize_int8",
    "rmsnorm",
    "row_sum",
    "silu",
    "softmax",
    "softmax_as",
    "softmax_scaled",
    "sum_reduce",
    "swiglu",
]

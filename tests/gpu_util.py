"""Helpers for the GPU parity tests: host<->device copies and C-ABI calls."""

from __future__ import annotations

import numpy as np
import torch

from cuda_force_amd import _lib

DEVICE = torch.device("cuda:0")


def lib():
    return _lib.load()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def call(name: str, *args) -> None:
    """Call a C-ABI entry point and raise on a non-zero status."""
    _lib.check(getattr(lib(), name)(*args))


def to_gpu(array: np.ndarray, dtype: str = "f32") -> torch.Tensor:
    """Host array -> device tensor; "bf16"/"f16" arrays are uint16 bit patterns."""
    if dtype == "bf16":
        return torch.from_numpy(array.astype(np.int16)).view(torch.bfloat16).to(DEVICE)
    if dtype == "f16":
        return torch.from_numpy(array.astype(np.int16)).view(torch.float16).to(DEVICE)
    return torch.from_numpy(np.ascontiguousarray(array)).to(DEVICE)


def to_host(tensor: torch.Tensor) -> np.ndarray:
    """Device tensor -> host array; 16-bit floats come back as uint16 bits."""
    t = tensor.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().astype(np.uint16)
    return t.numpy()


def empty(shape, dtype: torch.dtype) -> torch.Tensor:
    return torch.empty(shape, dtype=dtype, device=DEVICE)


def cf(dtype: str) -> int:
    return {"f32": _lib.CF_F32, "f16": _lib.CF_F16, "bf16": _lib.CF_BF16}[dtype]


def torch_dtype(dtype: str) -> torch.dtype:
    return {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[dtype]


def host_values(array: np.ndarray, dtype: str) -> np.ndarray:
    """The float values a stored array holds (bits widened for 16-bit types)."""
    if dtype == "bf16":
        return (array.astype(np.uint32) << 16).view(np.float32)
    if dtype == "f16":
        return array.view(np.float16).astype(np.float32)
    return array.astype(np.float32)


def storage_bits(values: np.ndarray, dtype: str) -> np.ndarray:
    """Round float values to a storage dtype (bits for 16-bit types)."""
    import oracle

    if dtype == "bf16":
        return oracle.f32_to_bf16_bits(values.astype(np.float32))
    if dtype == "f16":
        return values.astype(np.float32).astype(np.float16).view(np.uint16)
    return values.astype(np.float32)


def announce(message: str) -> None:
    print(f"[gpu] {message}", flush=True)

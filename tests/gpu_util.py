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


def poison_(t: torch.Tensor) -> torch.Tensor:
    """Fill a buffer in place with a bit pattern no kernel stores, so that an
    element a kernel leaves unwritten fails the comparison that follows
    (the reference's kernel tests zero-fill outputs for the same reason,
    tests/cuda/cuda_test_utils.cuh:93-111):

    * floats: every bit set - a negative NaN with a full payload, never the
      canonical NaN (bf16 0x7FC0, fp16 0x7E00/0xFE00, fp32 0x7FC00000) that
      a kernel writes, and NaN fails every tolerance check;
    * int8: -128, outside the quantiser's code range [-127, 127];
    * other integer buffers (workspaces): 0xA5 bytes."""
    if t.numel() == 0:
        return t
    if t.dtype == torch.int8:
        t.fill_(-128)
    elif t.dtype.is_floating_point:
        ints = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
        t.view(ints).fill_(-1 if ints is not torch.uint8 else 0xFF)
    else:
        t.view(torch.uint8).fill_(0xA5)
    return t


def empty(shape, dtype: torch.dtype) -> torch.Tensor:
    """A poisoned device buffer (see poison_)."""
    return poison_(torch.empty(shape, dtype=dtype, device=DEVICE))


def poison_like(t: torch.Tensor) -> torch.Tensor:
    return poison_(torch.empty_like(t))


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

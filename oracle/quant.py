"""Block-wise INT8 quantisation oracle (test infrastructure only).

Two restatements of the reference's CPU semantics
(python/cudaforge/ops.py:215-240, cpp/src/bindings.cpp:298-329):

* the C one in cf_oracle.c (scalar loops), reached through ctypes;
* an independent vectorised numpy one below.

Arrays of 16-bit floats are passed as their uint16 bit patterns with a dtype
tag ("bf16" / "f16"); fp32 arrays as np.float32.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache
from pathlib import Path

import numpy as np

BLOCK = 64
_DTYPES = {"f32": 0, "f16": 1, "bf16": 2}
LIBRARY = Path(__file__).resolve().parent / "libcf_oracle.so"


@lru_cache(maxsize=1)
def _lib() -> ctypes.CDLL:
    if not LIBRARY.exists():
        raise FileNotFoundError(f"{LIBRARY} is not built; run `make -C oracle`")
    lib = ctypes.CDLL(str(LIBRARY))
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.oracle_quantize_int8.argtypes = [p, i32, i64, p, p]
    lib.oracle_quantize_int8.restype = None
    lib.oracle_dequantize_int8.argtypes = [p, p, i64, p, i32]
    lib.oracle_dequantize_int8.restype = None
    lib.oracle_quantize_dequantize.argtypes = [p, i32, i64, p]
    lib.oracle_quantize_dequantize.restype = None
    lib.oracle_to_bf16.argtypes = [p, p, i64]
    lib.oracle_to_bf16.restype = None
    lib.oracle_to_f16.argtypes = [p, p, i64]
    lib.oracle_to_f16.restype = None
    lib.oracle_from_f16.argtypes = [p, p, i64]
    lib.oracle_from_f16.restype = None
    return lib


def _as_input(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "f32":
        return np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if x.dtype != np.uint16:
        raise TypeError(f"{dtype} input must be passed as uint16 bit patterns")
    return np.ascontiguousarray(x).reshape(-1)


def scale_count(n: int) -> int:
    return 0 if n <= 0 else (n + BLOCK - 1) // BLOCK


def quantize_int8(x: np.ndarray, dtype: str = "f32") -> tuple[np.ndarray, np.ndarray]:
    """(int8 codes shaped like x, fp32 scales [ceil(n/64)]) via the C oracle."""
    flat = _as_input(x, dtype)
    n = flat.size
    q = np.empty(n, dtype=np.int8)
    s = np.empty(scale_count(n), dtype=np.float32)
    if n:
        _lib().oracle_quantize_int8(flat.ctypes.data, _DTYPES[dtype], n, q.ctypes.data, s.ctypes.data)
    return q.reshape(np.shape(x)), s


def dequantize_int8(q: np.ndarray, scales: np.ndarray, dtype: str = "f32") -> np.ndarray:
    """float(q) * s in fp32, rounded to `dtype` (returned as uint16 bits for halves)."""
    flat = np.ascontiguousarray(q, dtype=np.int8).reshape(-1)
    s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
    n = flat.size
    if s.size != scale_count(n):
        raise ValueError(f"expected {scale_count(n)} scales, got {s.size}")
    out = np.empty(n, dtype=np.float32 if dtype == "f32" else np.uint16)
    if n:
        _lib().oracle_dequantize_int8(flat.ctypes.data, s.ctypes.data, n, out.ctypes.data, _DTYPES[dtype])
    return out.reshape(np.shape(q))


def quantize_dequantize(x: np.ndarray, dtype: str = "f32") -> np.ndarray:
    """Fake quantisation in x's dtype via the C oracle."""
    flat = _as_input(x, dtype)
    n = flat.size
    out = np.empty(n, dtype=np.float32 if dtype == "f32" else np.uint16)
    if n:
        _lib().oracle_quantize_dequantize(flat.ctypes.data, _DTYPES[dtype], n, out.ctypes.data)
    return out.reshape(np.shape(x))


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    flat = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    out = np.empty(flat.size, dtype=np.uint16)
    if flat.size:
        _lib().oracle_to_f16(flat.ctypes.data, out.ctypes.data, flat.size)
    return out.reshape(np.shape(x))


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    flat = np.ascontiguousarray(h, dtype=np.uint16).reshape(-1)
    out = np.empty(flat.size, dtype=np.float32)
    if flat.size:
        _lib().oracle_from_f16(flat.ctypes.data, out.ctypes.data, flat.size)
    return out.reshape(np.shape(h))


# ---------------------------------------------------------------------------
# Independent numpy restatement (vectorised), cross-checked against the C one.
# ---------------------------------------------------------------------------


def quantize_int8_numpy(x32: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Same semantics from a float32 array, with numpy's IEEE float32 ops."""
    flat = np.asarray(x32, dtype=np.float32).reshape(-1)
    n = flat.size
    pad = (-n) % BLOCK
    blocks = np.concatenate([flat, np.zeros(pad, np.float32)]).reshape(-1, BLOCK)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        absmax = np.abs(blocks).max(axis=1)  # np.max propagates NaN like torch.amax
        scales = absmax / np.float32(127.0)
        scales = np.where(scales > 0, scales, np.float32(1.0)).astype(np.float32)
        quotient = blocks / scales[:, None]
        rounded = np.rint(quotient)  # round half to even
        codes = np.clip(rounded, -127, 127)
        codes = np.where(np.isnan(codes), 0, codes).astype(np.int8)
    return codes.reshape(-1)[:n].reshape(np.shape(x32)), scales


def dequantize_int8_numpy(q: np.ndarray, scales: np.ndarray) -> np.ndarray:
    flat = np.asarray(q, dtype=np.int8).reshape(-1)
    idx = np.arange(flat.size) // BLOCK
    with np.errstate(invalid="ignore", over="ignore"):
        out = flat.astype(np.float32) * np.asarray(scales, dtype=np.float32)[idx]
    return out.reshape(np.shape(q))

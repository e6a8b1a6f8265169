"""ctypes binding of the C ABI in ``include/cudaforge_hip.h``.

This is the binding a non-PyTorch caller writes; the
parity tests and the benchmark use it to reach the kernels without the
dispatcher in between. Pointers are passed as integers (``tensor.data_ptr()``)
and streams as ``torch.cuda.current_stream().cuda_stream``.

torch must be imported first on a GPU host, so that this library binds to the
HIP runtime torch already loaded (both resolve ``libamdhip64.so.7``).
"""

from __future__ import annotations

import ctypes
import re
from functools import lru_cache
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
HEADER = PACKAGE_DIR.parent / "include" / "cudaforge_hip.h"
LIBRARY = PACKAGE_DIR / "libcudaforge_hip.so"

CF_OK = 0
CF_ERR_INVALID_ARGUMENT = 1
CF_ERR_UNSUPPORTED = 2
CF_ERR_HIP = 3
CF_ERR_OUT_OF_MEMORY = 4

CF_F32 = 0
CF_F16 = 1
CF_BF16 = 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_PP = ctypes.POINTER(ctypes.c_void_p)
_PI64 = ctypes.POINTER(ctypes.c_int64)
_PI32 = ctypes.POINTER(ctypes.c_int)


class StreamStatsC(ctypes.Structure):
    """cf_stream_stats."""

    _fields_ = [("batches_dispatched", ctypes.c_uint64), ("bytes_to_device", ctypes.c_uint64),
                ("bytes_to_host", ctypes.c_uint64)]


class PoolStatsC(ctypes.Structure):
    """cf_pool_stats."""

    _fields_ = [(name, ctypes.c_uint64) for name in (
        "bytes_reserved", "bytes_in_use", "peak_bytes_in_use", "allocation_count",
        "backend_allocations", "reuse_count", "free_count", "free_block_count")]


CF_POOL_HOST = 0
CF_POOL_DEVICE = 1
CF_POOL_DEVICE_ASYNC = 2
CF_POOL_PINNED = 3

# name -> (restype, argtypes); must cover every function the header declares.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "cf_last_error": (ctypes.c_char_p, []),
    "cf_last_hip_error": (_I32, []),
    "cf_hip_error_is_sticky": (_I32, [_I32]),
    "cf_abi_version": (_I32, []),
    "cf_quant_scale_count": (_I64, [_I64]),
    "cf_quantize_int8": (_I32, [_P, _I32, _P, _P, _I64, _P]),
    "cf_dequantize_int8": (_I32, [_P, _P, _P, _I32, _I64, _P]),
    "cf_quantize_int8_group": (_I32, [_P, _I32, _P, _P, _P, _I64, _P]),
    "cf_dequantize_int8_group": (_I32, [_P, _P, _P, _I32, _P, _I64, _P]),
    "cf_quantize_dequantize": (_I32, [_P, _P, _I32, _I64, _P]),
    "cf_rmsnorm": (_I32, [_P, _P, _P, _I32, _I64, _I64, _F, _P]),
    "cf_fused_residual_rmsnorm": (_I32, [_P, _P, _P, _P, _P, _I32, _I64, _I64, _F, _P]),
    "cf_softmax": (_I32, [_P, _I32, _P, _I32, _I64, _I64, _P]),
    "cf_softmax_scaled": (_I32, [_P, _I32, _P, _I32, _I64, _I64, _F, _I64, _P]),
    "cf_reduce_sum_workspace_bytes": (_SZ, [_I64]),
    "cf_reduce_sum": (_I32, [_P, _I32, _P, _I64, _P, _SZ, _I32, _P]),
    "cf_reduce_sum_noalloc": (_I32, [_P, _I32, _P, _I64, _I32, _P]),
    "cf_row_sum": (_I32, [_P, _I32, _P, _I64, _I64, _P]),
    "cf_lora_workspace_bytes": (_SZ, [_I64, _I64]),
    "cf_lora_linear": (_I32, [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _F, _P]),
    "cf_lora_linear_ws_bytes": (_SZ, [_I32, _I64, _I64, _I64, _I64]),
    "cf_lora_linear_ws": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _F, _P, _SZ, _P],
    ),
    "cf_matmul": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _P]),
    "cf_lora_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "cf_lora_backward": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _F, _P, _SZ, _P],
    ),
    "cf_silu": (_I32, [_P, _P, _I32, _I64, _P]),
    "cf_gelu": (_I32, [_P, _P, _I32, _I64, _P]),
    "cf_swiglu": (_I32, [_P, _P, _P, _I32, _I64, _P]),
    "cf_copy_bytes": (_I32, [_P, _P, _I64, _P]),
    "cf_stream_bytes": (_I32, [_P, _P, _I64, _I32, _P]),
    "cf_time_next_launch": (_I32, [_P, _P]),
    "cf_time_next_launch_armed": (_I32, []),
    "cf_tensor_cores_available": (_I32, []),
    "cf_matmul_tensor_core_shape_supported": (_I32, [_I64, _I64, _I64]),
    "cf_matmul_tensor_core_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "cf_matmul_tensor_core": (_I32, [_P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "cf_matmul_fp8_shape_supported": (_I32, [_I64, _I64, _I64]),
    "cf_matmul_fp8": (_I32, [_P, _P, _P, _I64, _I64, _I64, _F, _P]),
    "cf_matmul_fp8_wt_shape_supported": (_I32, [_I64, _I64, _I64]),
    "cf_matmul_fp8_wt": (_I32, [_P, _P, _P, _I64, _I64, _I64, _F, _P]),
    "cf_attention_scores_causal": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P]),
    "cf_attention_pv_causal": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _I64, _P]),
    "cf_paged_attention_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "cf_paged_attention": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I64, _I64, _I64, _F, _P, _SZ, _P],
    ),
    "cf_scheduler_create": (_I32, [_I64, _I32, _PP]),
    "cf_scheduler_destroy": (_I32, [_P]),
    "cf_scheduler_acquire": (_I32, [_P, _PI64, _PP]),
    "cf_scheduler_stream": (_I32, [_P, _I64, _PP]),
    "cf_scheduler_stream_count": (_I64, [_P]),
    "cf_scheduler_copy_to_device": (_I32, [_P, _I64, _P, _P, _SZ]),
    "cf_scheduler_copy_to_host": (_I32, [_P, _I64, _P, _P, _SZ]),
    "cf_scheduler_record_completion": (_I32, [_P, _I64]),
    "cf_scheduler_chain": (_I32, [_P, _I64, _I64]),
    "cf_scheduler_note_dispatch": (_I32, [_P, _I64]),
    "cf_scheduler_synchronize": (_I32, [_P, _I64]),
    "cf_scheduler_query": (_I32, [_P, _I64, _PI32]),
    "cf_scheduler_event_query": (_I32, [_P, _I64, _PI32]),
    "cf_scheduler_synchronize_all": (_I32, [_P]),
    "cf_scheduler_stats": (_I32, [_P, ctypes.POINTER(StreamStatsC), _I64, ctypes.POINTER(StreamStatsC)]),
    "cf_stream_ordered_allocation_supported": (_I32, []),
    "cf_pool_create": (_I32, [_I32, _P, _SZ, _PP]),
    "cf_pool_destroy": (_I32, [_P]),
    "cf_pool_allocate": (_I32, [_P, _SZ, _PP]),
    "cf_pool_deallocate": (_I32, [_P, _P]),
    "cf_pool_trim": (_I32, [_P]),
    "cf_pool_get_stats": (_I32, [_P, ctypes.POINTER(PoolStatsC)]),
    "cf_pool_backend_name": (ctypes.c_char_p, [_I32]),
}


def declared_functions(header: Path = HEADER) -> list[str]:
    """Names of the functions the C header declares."""
    text = re.sub(r"/\*.*?\*/", "", header.read_text(encoding="utf-8"), flags=re.S)
    return sorted(set(re.findall(r"\b(cf_[a-z0-9_]+)\s*\(", text)))


class CfError(RuntimeError):
    """A non-zero cf_status, with the library's message."""

    def __init__(self, status: int, message: str) -> None:
        super().__init__(f"cf status {status}: {message}")
        self.status = status


@lru_cache(maxsize=1)
def load() -> ctypes.CDLL:
    """Load the library and attach every signature; raises if it is not built."""
    if not LIBRARY.exists():
        raise FileNotFoundError(
            f"{LIBRARY} is not built; run `python -m cuda_force_amd.build` or __graft_entry__.build()"
        )
    lib = ctypes.CDLL(str(LIBRARY))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def check(status: int) -> None:
    """Raise CfError for a non-zero status."""
    if status != CF_OK:
        message = load().cf_last_error().decode("utf-8", "replace")
        raise CfError(status, message)


def dtype_code(dtype: object) -> int:
    """cf_dtype for a torch dtype."""
    import torch

    mapping = {torch.float32: CF_F32, torch.float16: CF_F16, torch.bfloat16: CF_BF16}
    if dtype not in mapping:
        raise TypeError(f"no cf_dtype for {dtype}")
    return mapping[dtype]


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000


def pointer_array(values) -> ctypes.Array:
    """A host array of device pointers (ints) for the grouped entry points."""
    return (ctypes.c_void_p * max(len(values), 1))(*values)


def int64_array(values) -> ctypes.Array:
    """A host array of int64 counts for the grouped entry points."""
    return (ctypes.c_int64 * max(len(values), 1))(*values)


@lru_cache(maxsize=1)
def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime this library is linked against (already loaded)."""
    load()
    hip = ctypes.CDLL("libamdhip64.so.7", mode=ctypes.RTLD_GLOBAL)
    hip.hipEventCreateWithFlags.argtypes = [_PP, ctypes.c_uint]
    hip.hipEventDestroy.argtypes = [_P]
    hip.hipEventSynchronize.argtypes = [_P]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _P, _P]
    for name in ("hipEventCreateWithFlags", "hipEventDestroy", "hipEventSynchronize",
                 "hipEventElapsedTime"):
        getattr(hip, name).restype = ctypes.c_int
    return hip


def _hip_check(error: int, what: str) -> None:
    if error != 0:
        raise RuntimeError(f"HIP error {error} in {what}")


class DispatchTimer:
    """A start/stop hipEvent pair that one kernel dispatch of this library
    records itself (cf_time_next_launch): `elapsed_ms()` is that kernel's
    execution time, the figure a kernel trace reports, with no event packets
    queued around the launch. Call `arm()` right before the entry point.

    The events skip the system-scope fence by default: with it, each timed
    dispatch ends with a system-scope cache release, which measured 5.7 us
    per step on MI355X (1.9 us without it), and timing needs no host-visible
    ordering."""

    def __init__(self, flags: int = HIP_EVENT_DISABLE_SYSTEM_FENCE) -> None:
        hip = _hip_runtime()
        self.start = ctypes.c_void_p()
        self.stop = ctypes.c_void_p()
        _hip_check(hip.hipEventCreateWithFlags(ctypes.byref(self.start), flags), "hipEventCreate")
        _hip_check(hip.hipEventCreateWithFlags(ctypes.byref(self.stop), flags), "hipEventCreate")

    def arm(self) -> None:
        check(load().cf_time_next_launch(self.start, self.stop))

    def elapsed_ms(self) -> float:
        hip = _hip_runtime()
        _hip_check(hip.hipEventSynchronize(self.stop), "hipEventSynchronize")
        ms = ctypes.c_float()
        _hip_check(hip.hipEventElapsedTime(ctypes.byref(ms), self.start, self.stop),
                   "hipEventElapsedTime")
        return float(ms.value)

    def close(self) -> None:
        hip = _hip_runtime()
        for ev in (self.start, self.stop):
            if ev:
                hip.hipEventDestroy(ev)
        self.start = ctypes.c_void_p()
        self.stop = ctypes.c_void_p()

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

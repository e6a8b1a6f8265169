"""Python handles for the stream scheduler and the caching pools.

The reference has these in C++ only (``GpuScheduler`` / ``StreamLease``,
cuda/include/cudaforge/gpu_scheduler.cuh:36-142; ``MemoryPool`` and its
backends, cpp/include/cudaforge/memory_pool.hpp:76-216 and
gpu_scheduler.cuh:150-258). The same classes are in include/cudaforge_runtime.hpp
for C++ callers; this module drives them through the C ABI so Python code (and
the tests) can use them with the same names and meaning:

* ``GpuScheduler(stream_count, device=0)``: ``acquire()`` hands out streams
  round-robin as ``StreamLease`` objects; ``copy_to_device`` /
  ``copy_to_host`` queue asynchronous copies and count their bytes per
  stream; ``GpuScheduler.chain(waiter, signaller)`` orders two streams by
  event; ``note_dispatch``, ``synchronize_all`` and ``stats()`` as in C++.
* ``MemoryPool(backend, stream=None, min_block_bytes=256)`` with backend
  ``"host"``, ``"device"``, ``"device-async"`` or ``"pinned"``:
  ``allocate(nbytes) -> int`` address (0 for 0 bytes), ``deallocate(addr)``,
  ``trim()``, ``stats()``. Failures raise what the C++ raised: ``MemoryError``
  for ``std::bad_alloc``, ``ValueError`` for ``std::invalid_argument``.

Streams are plain ``hipStream_t`` handles (``lease.stream`` is an int);
``lease.torch_stream()`` wraps one for torch. Every stream is non-blocking and
at the default priority.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

from . import _lib

BACKENDS = {
    "host": _lib.CF_POOL_HOST,
    "device": _lib.CF_POOL_DEVICE,
    "device-async": _lib.CF_POOL_DEVICE_ASYNC,
    "pinned": _lib.CF_POOL_PINNED,
}


def _check(status: int) -> None:
    if status == _lib.CF_OK:
        return
    message = _lib.load().cf_last_error().decode("utf-8", "replace")
    if status == _lib.CF_ERR_OUT_OF_MEMORY:
        raise MemoryError(message)
    if status == _lib.CF_ERR_INVALID_ARGUMENT:
        raise ValueError(message)
    raise _lib.CfError(status, message)


def supports_stream_ordered_allocation() -> bool:
    """True when the current device backs hipMallocAsync with a memory pool."""
    return bool(_lib.load().cf_stream_ordered_allocation_supported())


@dataclass(frozen=True)
class StreamStats:
    batches_dispatched: int = 0
    bytes_to_device: int = 0
    bytes_to_host: int = 0


@dataclass(frozen=True)
class SchedulerStats:
    stream_count: int
    total_dispatches: int
    total_bytes_to_device: int
    total_bytes_to_host: int
    per_stream: list[StreamStats] = field(default_factory=list)


@dataclass(frozen=True)
class PoolStats:
    bytes_reserved: int
    bytes_in_use: int
    peak_bytes_in_use: int
    allocation_count: int
    backend_allocations: int
    reuse_count: int
    free_count: int
    free_block_count: int

    @property
    def reuse_rate(self) -> float:
        return self.reuse_count / self.allocation_count if self.allocation_count else 0.0


class StreamLease:
    """Use of one scheduler stream (index ``index``, handle ``stream``)."""

    def __init__(self, scheduler: "GpuScheduler", index: int, stream: int) -> None:
        self._scheduler = scheduler
        self.index = index
        self.stream = stream

    def record_completion(self) -> None:
        _check(_lib.load().cf_scheduler_record_completion(self._scheduler._handle, self.index))

    def synchronize(self) -> None:
        _check(_lib.load().cf_scheduler_synchronize(self._scheduler._handle, self.index))

    def complete(self) -> bool:
        flag = ctypes.c_int(0)
        _check(_lib.load().cf_scheduler_query(self._scheduler._handle, self.index, ctypes.byref(flag)))
        return bool(flag.value)

    def completion_event_complete(self) -> bool:
        """Whether the last recorded completion event has completed."""
        flag = ctypes.c_int(0)
        _check(_lib.load().cf_scheduler_event_query(self._scheduler._handle, self.index,
                                                    ctypes.byref(flag)))
        return bool(flag.value)

    def torch_stream(self):
        """This stream as a ``torch.cuda.ExternalStream``."""
        import torch

        return torch.cuda.ExternalStream(self.stream)


class GpuScheduler:
    """A fixed pool of HIP streams handed out round-robin."""

    def __init__(self, stream_count: int, device: int = 0) -> None:
        self._handle = None
        handle = ctypes.c_void_p()
        _check(_lib.load().cf_scheduler_create(int(stream_count), int(device), ctypes.byref(handle)))
        self._handle = handle
        self.device = device

    @property
    def stream_count(self) -> int:
        return int(_lib.load().cf_scheduler_stream_count(self._handle))

    def acquire(self) -> StreamLease:
        index = ctypes.c_int64(0)
        stream = ctypes.c_void_p()
        _check(_lib.load().cf_scheduler_acquire(self._handle, ctypes.byref(index), ctypes.byref(stream)))
        return StreamLease(self, index.value, stream.value or 0)

    def copy_to_device(self, lease: StreamLease, device: int, host: int, nbytes: int) -> None:
        _check(_lib.load().cf_scheduler_copy_to_device(self._handle, lease.index, device, host, nbytes))

    def copy_to_host(self, lease: StreamLease, host: int, device: int, nbytes: int) -> None:
        _check(_lib.load().cf_scheduler_copy_to_host(self._handle, lease.index, host, device, nbytes))

    @staticmethod
    def chain(waiter: StreamLease, signaller: StreamLease) -> None:
        if waiter._scheduler is not signaller._scheduler:
            raise ValueError("chain: both leases must come from the same scheduler")
        _check(_lib.load().cf_scheduler_chain(waiter._scheduler._handle, waiter.index, signaller.index))

    def note_dispatch(self, lease: StreamLease) -> None:
        _check(_lib.load().cf_scheduler_note_dispatch(self._handle, lease.index))

    def synchronize_all(self) -> None:
        _check(_lib.load().cf_scheduler_synchronize_all(self._handle))

    def stats(self) -> SchedulerStats:
        count = self.stream_count
        per = (_lib.StreamStatsC * max(count, 1))()
        totals = _lib.StreamStatsC()
        _check(_lib.load().cf_scheduler_stats(self._handle, per, count, ctypes.byref(totals)))
        return SchedulerStats(
            stream_count=count,
            total_dispatches=totals.batches_dispatched,
            total_bytes_to_device=totals.bytes_to_device,
            total_bytes_to_host=totals.bytes_to_host,
            per_stream=[StreamStats(p.batches_dispatched, p.bytes_to_device, p.bytes_to_host)
                        for p in per[:count]],
        )

    def close(self) -> None:
        """Drains every stream and releases them (also on garbage collection)."""
        if self._handle:
            handle, self._handle = self._handle, None
            _check(_lib.load().cf_scheduler_destroy(handle))

    def __enter__(self) -> "GpuScheduler":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class MemoryPool:
    """Caching allocator with power-of-two size classes over one backend."""

    def __init__(self, backend: str = "host", stream: int | None = None, min_block_bytes: int = 256) -> None:
        self._handle = None
        if backend not in BACKENDS:
            raise ValueError(f"unknown pool backend {backend!r}; expected one of {sorted(BACKENDS)}")
        handle = ctypes.c_void_p()
        _check(_lib.load().cf_pool_create(BACKENDS[backend], stream or None, int(min_block_bytes),
                                          ctypes.byref(handle)))
        self._handle = handle
        self.backend = backend

    @staticmethod
    def backend_name(backend: str) -> str:
        """The name the C++ backend reports ("host", "device", ...)."""
        return _lib.load().cf_pool_backend_name(BACKENDS[backend]).decode()

    def allocate(self, nbytes: int) -> int:
        out = ctypes.c_void_p()
        _check(_lib.load().cf_pool_allocate(self._handle, int(nbytes), ctypes.byref(out)))
        return out.value or 0

    def deallocate(self, address: int) -> None:
        _check(_lib.load().cf_pool_deallocate(self._handle, address or None))

    def trim(self) -> None:
        _check(_lib.load().cf_pool_trim(self._handle))

    def stats(self) -> PoolStats:
        raw = _lib.PoolStatsC()
        _check(_lib.load().cf_pool_get_stats(self._handle, ctypes.byref(raw)))
        return PoolStats(*(getattr(raw, name) for name, _ in _lib.PoolStatsC._fields_))

    def close(self) -> None:
        """Returns every block, cached or checked out, to the backend."""
        if self._handle:
            handle, self._handle = self._handle, None
            _check(_lib.load().cf_pool_destroy(handle))

    def __enter__(self) -> "MemoryPool":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

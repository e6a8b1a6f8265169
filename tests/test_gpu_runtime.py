"""GPU tests of the stream scheduler and the device / stream-ordered / pinned
pools, through the C ABI (cuda_force_amd.runtime). They restate the cases of the
reference's tests/cuda/test_scheduler.cu (:14-385): round-robin leases,
distinct streams, completion events, cross-stream chaining, per-stream copy
statistics, device-pool reuse, pooled memory used by a kernel, concurrent
workers, and the stream-ordered pool (reuse; returning a buffer that queued
work still reads). Kernels here are this library's own (cf_reduce_sum,
cf_copy_bytes); host staging buffers come from the pinned pool.
"""

from __future__ import annotations

import ctypes
import threading

import pytest
import torch

from cuda_force_amd import _lib
from cuda_force_amd.runtime import GpuScheduler, MemoryPool, StreamLease, supports_stream_ordered_allocation

from .gpu_util import announce

pytestmark = pytest.mark.gpu

F32 = ctypes.sizeof(ctypes.c_float)


def host_floats(address: int, count: int):
    return (ctypes.c_float * count).from_address(address)


def reduce_into(lib, pool, x: int, out: int, count: int, stream: int) -> int:
    """cf_reduce_sum of `count` fp32 at x into *out on `stream`; returns the
    workspace block (the caller returns it to the pool)."""
    nbytes = lib.cf_reduce_sum_workspace_bytes(count)
    workspace = pool.allocate(nbytes)
    _lib.check(lib.cf_reduce_sum(x, _lib.CF_F32, out, count, workspace, nbytes, 0, stream))
    return workspace


@pytest.fixture(scope="module")
def lib():
    torch.cuda.init()
    return _lib.load()


def test_round_robin_and_distinct_streams(lib):
    announce("scheduler: round-robin leases")
    with GpuScheduler(4) as scheduler:
        assert scheduler.stream_count == 4
        assert [scheduler.acquire().index for _ in range(12)] == [i % 4 for i in range(12)]
    with GpuScheduler(3) as scheduler:
        first, second, third = scheduler.acquire(), scheduler.acquire(), scheduler.acquire()
        assert len({first.stream, second.stream, third.stream}) == 3
        assert 0 not in (first.stream, second.stream, third.stream)
        assert scheduler.acquire().stream == first.stream


def test_completion_event_records_and_completes(lib):
    announce("scheduler: completion event")
    with GpuScheduler(2) as scheduler, MemoryPool("device") as pool:
        lease = scheduler.acquire()
        src, dst = pool.allocate(1 << 22), pool.allocate(1 << 22)
        _lib.check(lib.cf_copy_bytes(src, dst, 1 << 22, lease.stream))
        lease.record_completion()
        lease.synchronize()
        assert lease.complete()
        assert lease.completion_event_complete()
        pool.deallocate(src)
        pool.deallocate(dst)


def test_chain_orders_a_consumer_after_a_producer(lib):
    announce("scheduler: chain")
    count = 1 << 20
    with GpuScheduler(2) as scheduler, MemoryPool("device") as device, MemoryPool("pinned") as pinned:
        producer, consumer = scheduler.acquire(), scheduler.acquire()
        staging = pinned.allocate(count * F32)
        values = host_floats(staging, count)
        ctypes.memmove(staging, (ctypes.c_float * count)(*([1.0] * count)), count * F32)
        data, out = device.allocate(count * F32), device.allocate(F32)
        scheduler.copy_to_device(producer, data, staging, count * F32)
        producer.record_completion()
        GpuScheduler.chain(consumer, producer)
        workspace = reduce_into(lib, device, data, out, count, consumer.stream)
        result = pinned.allocate(F32)
        scheduler.copy_to_host(consumer, result, out, F32)
        consumer.synchronize()
        assert host_floats(result, 1)[0] == float(count)
        assert values[count - 1] == 1.0
        for block in (data, out, workspace):
            device.deallocate(block)
        for block in (staging, result):
            pinned.deallocate(block)


def test_copy_statistics_are_per_stream(lib):
    announce("scheduler: copy statistics")
    with GpuScheduler(2) as scheduler, MemoryPool("device") as device, MemoryPool("pinned") as pinned:
        nbytes = 256 * F32
        host, dev = pinned.allocate(nbytes), device.allocate(nbytes)
        lease = scheduler.acquire()
        scheduler.copy_to_device(lease, dev, host, nbytes)
        scheduler.copy_to_host(lease, host, dev, nbytes)
        scheduler.copy_to_device(lease, dev, host, 0)  # no-op, not counted
        scheduler.note_dispatch(lease)
        lease.synchronize()
        stats = scheduler.stats()
        assert stats.stream_count == 2
        assert stats.total_bytes_to_device == nbytes
        assert stats.total_bytes_to_host == nbytes
        assert stats.total_dispatches == 1
        assert stats.per_stream[lease.index].batches_dispatched == 1
        assert stats.per_stream[1 - lease.index].bytes_to_device == 0
        with pytest.raises(ValueError, match="out of range"):
            scheduler.note_dispatch(StreamLease(scheduler, 7, 0))
        device.deallocate(dev)
        pinned.deallocate(host)


def test_device_pool_reuses_and_serves_kernels(lib):
    announce("pool: device backend reuse + kernel use")
    with MemoryPool("device") as pool, MemoryPool("pinned") as pinned:
        first = pool.allocate(1 << 20)
        pool.deallocate(first)
        second = pool.allocate(1 << 20)
        assert second == first
        assert pool.stats().backend_allocations == 1 and pool.stats().reuse_count == 1
        pool.deallocate(second)

        count = 1 << 16
        x, out = pool.allocate(count * F32), pool.allocate(F32)
        host = pinned.allocate(count * F32)
        ctypes.memmove(host, (ctypes.c_float * count)(*[float(i % 7) for i in range(count)]), count * F32)
        scheduler = GpuScheduler(1)
        lease = scheduler.acquire()
        scheduler.copy_to_device(lease, x, host, count * F32)
        workspace = reduce_into(lib, pool, x, out, count, lease.stream)
        result = pinned.allocate(F32)
        scheduler.copy_to_host(lease, result, out, F32)
        lease.synchronize()
        assert host_floats(result, 1)[0] == float(sum(i % 7 for i in range(count)))
        scheduler.close()
        for block in (x, out, workspace):
            pool.deallocate(block)
        pinned.deallocate(host)
        pinned.deallocate(result)


def test_concurrent_workers_share_a_scheduler_and_a_pool(lib):
    announce("scheduler + pool: 8 threads x 25 batches")
    threads, per_thread, count = 8, 25, 4096
    failures: list[str] = []
    with GpuScheduler(4) as scheduler, MemoryPool("device") as device, MemoryPool("pinned") as pinned:

        def worker(t: int) -> None:
            try:
                staging = pinned.allocate(count * F32)
                result = pinned.allocate(F32)
                ctypes.memmove(staging, (ctypes.c_float * count)(*([float(t + 1)] * count)), count * F32)
                for _ in range(per_thread):
                    lease = scheduler.acquire()
                    x, out = device.allocate(count * F32), device.allocate(F32)
                    scheduler.copy_to_device(lease, x, staging, count * F32)
                    workspace = reduce_into(lib, device, x, out, count, lease.stream)
                    scheduler.copy_to_host(lease, result, out, F32)
                    scheduler.note_dispatch(lease)
                    lease.synchronize()
                    value = host_floats(result, 1)[0]
                    if value != float(count * (t + 1)):
                        failures.append(f"thread {t}: {value}")
                    for block in (x, out, workspace):
                        device.deallocate(block)
                pinned.deallocate(staging)
                pinned.deallocate(result)
            except Exception as error:  # reported below
                failures.append(f"thread {t}: {error!r}")

        workers = [threading.Thread(target=worker, args=(t,)) for t in range(threads)]
        for w in workers:
            w.start()
        for w in workers:
            w.join(timeout=60)
        assert not any(w.is_alive() for w in workers)
        assert failures == []
        assert scheduler.stats().total_dispatches == threads * per_thread
        assert device.stats().bytes_in_use == 0
        assert device.stats().reuse_rate > 0.9


def test_stream_ordered_pool(lib):
    announce("pool: stream-ordered backend")
    if not supports_stream_ordered_allocation():
        pytest.skip("device does not back hipMallocAsync with a memory pool")
    count = 1 << 16
    with GpuScheduler(1) as scheduler, MemoryPool("pinned") as pinned:
        lease = scheduler.acquire()
        with MemoryPool("device-async", stream=lease.stream) as pool:
            first = pool.allocate(1 << 20)
            assert first != 0
            pool.deallocate(first)
            second = pool.allocate(1 << 20)
            assert second == first
            assert pool.stats().backend_allocations == 1 and pool.stats().reuse_count == 1
            pool.deallocate(second)

            # Return the input while the queued reduction still reads it: the
            # free is ordered after the kernel on the same stream.
            x, out = pool.allocate(count * F32), pool.allocate(F32)
            staging = pinned.allocate(count * F32)
            ctypes.memmove(staging, (ctypes.c_float * count)(*([1.0] * count)), count * F32)
            scheduler.copy_to_device(lease, x, staging, count * F32)
            workspace = reduce_into(lib, pool, x, out, count, lease.stream)
            pool.deallocate(x)
            pool.trim()  # hipFreeAsync of the cached block, ordered after the kernel
            result = pinned.allocate(F32)
            scheduler.copy_to_host(lease, result, out, F32)
            lease.synchronize()
            assert host_floats(result, 1)[0] == float(count)
            pool.deallocate(out)
            pool.deallocate(workspace)
            pinned.deallocate(staging)
            pinned.deallocate(result)
        lease.synchronize()

"""Host-side tests of the runtime pieces: the caching pool and the C ABI of
the scheduler / pools where no GPU is involved.

* tests/cpp/test_pool.cpp (the reference's tests/cpp/test_memory_pool.cpp
  cases, :51-336) is built with g++ against include/cudaforge_pool.hpp and run
  plain, under AddressSanitizer + UBSan and under ThreadSanitizer.
* The Python handles in cuda_force_amd.runtime drive the host-backed pool
  through the C ABI and check the same contract end to end.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from cuda_force_amd import _lib
from cuda_force_amd.runtime import BACKENDS, GpuScheduler, MemoryPool

ROOT = Path(__file__).resolve().parents[1]
POOL_TEST = ROOT / "tests" / "cpp" / "test_pool.cpp"


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
@pytest.mark.parametrize("flags", [[], ["-fsanitize=address,undefined"], ["-fsanitize=thread"]],
                         ids=["plain", "asan-ubsan", "tsan"])
def test_pool_cpp_cases(tmp_path, flags):
    binary = tmp_path / "test_pool"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-Wall", "-Wextra", "-Werror", "-pthread",
                    *flags, f"-I{ROOT / 'include'}", str(POOL_TEST), "-o", str(binary)],
                   check=True, capture_output=True, text=True)
    result = subprocess.run([str(binary)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "0 failures" in result.stdout
    assert "ERROR" not in result.stderr and "WARNING" not in result.stderr, result.stderr


def test_host_pool_through_the_c_abi():
    with MemoryPool("host") as pool:
        assert pool.allocate(0) == 0
        pool.deallocate(0)
        first = pool.allocate(1000)
        assert first != 0
        ctypes.memset(first, 0xAB, 1000)
        pool.deallocate(first)
        again = pool.allocate(1024)  # same 1024-byte class
        assert again == first
        bigger = pool.allocate(1025)
        assert bigger != first
        stats = pool.stats()
        assert stats.allocation_count == 3
        assert stats.backend_allocations == 2
        assert stats.reuse_count == 1
        assert stats.bytes_in_use == 1024 + 2048
        assert stats.bytes_reserved == 1024 + 2048
        pool.deallocate(again)
        pool.deallocate(bigger)
        assert pool.stats().free_block_count == 2
        pool.trim()
        stats = pool.stats()
        assert stats.free_block_count == 0 and stats.bytes_reserved == 0
        assert stats.peak_bytes_in_use == 1024 + 2048
        assert stats.reuse_rate == pytest.approx(1 / 3)


def test_pool_errors_map_to_python_exceptions():
    with MemoryPool("host", min_block_bytes=512) as pool:
        local = ctypes.c_int(0)
        with pytest.raises(ValueError, match="did not hand out"):
            pool.deallocate(ctypes.addressof(local))
        block = pool.allocate(8)
        pool.deallocate(block)
        with pytest.raises(ValueError):
            pool.deallocate(block)  # second return of the same block
        assert pool.allocate(500) == block  # both in the 512-byte floor class
        with pytest.raises(MemoryError):
            pool.allocate(1 << 62)  # the host backend cannot supply 4 EiB
        assert pool.stats().bytes_in_use == 512
    with pytest.raises(ValueError):
        MemoryPool("host", min_block_bytes=0)
    with pytest.raises(ValueError, match="unknown pool backend"):
        MemoryPool("mmap")


def test_backend_names():
    assert {name: MemoryPool.backend_name(name) for name in BACKENDS} == {
        "host": "host", "device": "device", "device-async": "device-async", "pinned": "pinned"}
    assert _lib.load().cf_pool_backend_name(99) is None


def test_scheduler_rejects_zero_streams_without_touching_the_device():
    with pytest.raises(ValueError, match="at least one stream"):
        GpuScheduler(0)
    lib = _lib.load()
    assert lib.cf_scheduler_stream_count(None) == 0
    assert lib.cf_scheduler_destroy(None) == _lib.CF_OK
    assert lib.cf_scheduler_synchronize_all(None) == _lib.CF_ERR_INVALID_ARGUMENT
    assert lib.cf_pool_destroy(None) == _lib.CF_OK
    assert lib.cf_pool_allocate(None, 8, ctypes.byref(ctypes.c_void_p())) == _lib.CF_ERR_INVALID_ARGUMENT

"""Dispatch timing (cf_time_next_launch): a timed launch computes the same
result as an untimed one, its elapsed time is the kernel's own (positive, and
no longer than an event pair recorded around the same launch), an entry point
of two kernels is timed from the first one's start to the second one's end,
and only the next operator call on the thread is timed."""

from __future__ import annotations

import pytest
import torch

from cuda_force_amd import _lib
from tests import gpu_util as g
from tests.gpu_util import call, stream

pytestmark = pytest.mark.gpu


def _rmsnorm(x, w, y):
    call("cf_rmsnorm", x.data_ptr(), w.data_ptr(), y.data_ptr(), _lib.CF_BF16, x.shape[0], x.shape[1],
         1e-6, stream())


def test_timed_launch_matches_untimed_and_is_the_kernel_time():
    print("case: dispatch timer on rmsnorm bf16 [4096, 4096]", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(4096, 4096, generator=gen, device="cuda").to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(4096, generator=gen, device="cuda")).to(torch.bfloat16)
    plain = g.poison_like(x)
    timed = g.poison_like(x)
    for _ in range(3):
        _rmsnorm(x, w, plain)
    torch.cuda.synchronize()

    timer = _lib.DispatchTimer()
    pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    pair[0].record()
    timer.arm()
    _rmsnorm(x, w, timed)
    pair[1].record()
    torch.cuda.synchronize()
    kernel_ms = timer.elapsed_ms()
    around_ms = pair[0].elapsed_time(pair[1])
    timer.close()
    assert torch.equal(plain.view(torch.int16), timed.view(torch.int16))
    assert 0.0 < kernel_ms <= around_ms * 1.02 + 1e-3, (kernel_ms, around_ms)


def test_an_entry_point_of_two_kernels_is_timed_whole():
    """The two-stage sum launches two kernels: the armed interval runs from the
    first one's start to the second one's end, inside an event pair around the
    call, and the result is the untimed one's."""
    print("case: dispatch timer on the two-stage sum of 16M fp32", flush=True)
    n = 1 << 24
    x = torch.randn(n, generator=torch.Generator(device="cuda").manual_seed(3), device="cuda")
    nbytes = _lib.load().cf_reduce_sum_workspace_bytes(n)
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    outs = [torch.empty(1, device="cuda") for _ in range(2)]

    def run(out):
        call("cf_reduce_sum", x.data_ptr(), _lib.CF_F32, out.data_ptr(), n, ws.data_ptr(), nbytes, 0, stream())

    for _ in range(3):
        run(outs[0])
    torch.cuda.synchronize()
    timer = _lib.DispatchTimer()
    pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    pair[0].record()
    timer.arm()
    run(outs[1])
    pair[1].record()
    torch.cuda.synchronize()
    kernel_ms = timer.elapsed_ms()
    around_ms = pair[0].elapsed_time(pair[1])
    timer.close()
    assert torch.equal(outs[0], outs[1])
    # 64 MiB at no more than 8 TB/s: at least 8 us of stage 1 alone.
    assert 0.008 <= kernel_ms <= around_ms * 1.02 + 1e-3, (kernel_ms, around_ms)
    assert _lib.load().cf_time_next_launch_armed() == 0


def test_only_the_next_launch_is_timed():
    print("case: dispatch timer armed once, two launches", flush=True)
    x = torch.ones(256, 1024, device="cuda", dtype=torch.bfloat16)
    w = torch.ones(1024, device="cuda", dtype=torch.bfloat16)
    y = g.poison_like(x)
    timer = _lib.DispatchTimer()
    timer.arm()
    _rmsnorm(x, w, y)
    torch.cuda.synchronize()
    first = timer.elapsed_ms()
    _rmsnorm(x, w, y)  # not armed: must leave the events as they were
    torch.cuda.synchronize()
    assert timer.elapsed_ms() == first
    timer.close()
    assert torch.equal(y, torch.ones_like(y))


@pytest.mark.parametrize("divisor", [1, 2, 4])
def test_stream_bytes_writes_what_it_read(divisor):
    """The streaming-ceiling kernel: divisor 1 copies; 2 and 4 write the xor of
    each 16-byte vector's halves / words."""
    print(f"case: cf_stream_bytes divisor {divisor}", flush=True)
    src = torch.randint(0, 1 << 31, (1 << 14,), dtype=torch.int32, device="cuda")  # 64 KiB
    dst = torch.zeros(src.numel() // divisor, dtype=torch.int32, device="cuda")
    call("cf_stream_bytes", src.data_ptr(), dst.data_ptr(), src.numel() * 4, divisor, stream())
    torch.cuda.synchronize()
    v = src.view(-1, 4)
    if divisor == 1:
        want = src
    elif divisor == 2:
        want = torch.stack([v[:, 0] ^ v[:, 1], v[:, 2] ^ v[:, 3]], dim=1).reshape(-1)
    else:
        want = v[:, 0] ^ v[:, 1] ^ v[:, 2] ^ v[:, 3]
    assert torch.equal(dst, want)


def test_stream_bytes_read_only_and_write_only_modes():
    """Divisor 0 reads only (workgroup b stores thread 0's xor of its four
    vectors, the ones at 16-byte index 1024 b + 256 u); divisor -1 writes only
    (vector i = (i, ~i, i ^ 0x5bd1e995, i + 1))."""
    print("case: cf_stream_bytes read-only / write-only", flush=True)
    src = torch.randint(0, 1 << 31, (1 << 14,), dtype=torch.int32, device="cuda")  # 64 KiB = 4 workgroups
    dst = torch.zeros(4, dtype=torch.int32, device="cuda")
    call("cf_stream_bytes", src.data_ptr(), dst.data_ptr(), src.numel() * 4, 0, stream())
    out = torch.zeros(1 << 14, dtype=torch.int32, device="cuda")
    call("cf_stream_bytes", None, out.data_ptr(), out.numel() * 4, -1, stream())
    torch.cuda.synchronize()
    vectors = src.view(-1, 4)
    for b in range(4):
        picked = vectors[[1024 * b + 256 * u for u in range(4)]]
        want = picked[:, 0] ^ picked[:, 1] ^ picked[:, 2] ^ picked[:, 3]
        assert int(dst[b]) == int(want[0] ^ want[1] ^ want[2] ^ want[3])
    i = torch.arange(1 << 12, dtype=torch.int64, device="cuda")
    expect = torch.stack([i, ~i & 0xFFFFFFFF, i ^ 0x5BD1E995, i + 1], dim=1) & 0xFFFFFFFF
    got = out.view(-1, 4).to(torch.int64) & 0xFFFFFFFF
    assert torch.equal(got, expect)


@pytest.mark.parametrize("divisor", [-2, -3, -4, -5])
def test_stream_bytes_write_once_modes(divisor):
    """Divisors -2 .. -5 write only, one 16-byte store per lane (vector i =
    (i, ~i, i ^ 0x5bd1e995, i + 1)), whatever their cache-policy bits."""
    print(f"case: cf_stream_bytes write-once divisor {divisor}", flush=True)
    out = torch.zeros(1 << 14, dtype=torch.int32, device="cuda")  # 64 KiB
    call("cf_stream_bytes", None, out.data_ptr(), out.numel() * 4, divisor, stream())
    torch.cuda.synchronize()
    i = torch.arange(1 << 12, dtype=torch.int64, device="cuda")
    expect = torch.stack([i, ~i & 0xFFFFFFFF, i ^ 0x5BD1E995, i + 1], dim=1) & 0xFFFFFFFF
    got = out.view(-1, 4).to(torch.int64) & 0xFFFFFFFF
    assert torch.equal(got, expect)

"""cf_reduce_sum_noalloc: the sum without a workspace or any allocation.

Its partial sums live in a static device array that every call on the GPU
shares, so the checks run calls back to back - largest input first, then
smaller ones, whose stage 2 must read only their own partials - and compare
each result bit for bit with cf_reduce_sum given a fresh workspace (the same
two kernels and reduction tree), and with the exact sum within the
reference's bound (tests/cuda/test_reduction.cu:18-20).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from tests import gpu_util as g
from tests.conftest import rng

pytestmark = pytest.mark.gpu


def sum_with_workspace(xg: torch.Tensor, dtype: str, n: int, start: float, accumulate: int) -> float:
    ws = g.empty(max(1, g.lib().cf_reduce_sum_workspace_bytes(n)), torch.uint8)
    out = torch.full((1,), start, device=g.DEVICE)
    g.call("cf_reduce_sum", xg.data_ptr(), g.cf(dtype), out.data_ptr(), n, ws.data_ptr(), ws.numel(),
           accumulate, g.stream())
    torch.cuda.synchronize()
    return float(out.item())


def sum_noalloc(xg: torch.Tensor, dtype: str, n: int, start: float, accumulate: int) -> float:
    out = torch.full((1,), start, device=g.DEVICE)
    g.call("cf_reduce_sum_noalloc", xg.data_ptr(), g.cf(dtype), out.data_ptr(), n, accumulate, g.stream())
    torch.cuda.synchronize()
    return float(out.item())


def test_noalloc_sum_matches_the_workspace_sum_on_consecutive_calls():
    # Largest first: 40M elements use all 4096 partials (ceil(n / 4096),
    # at most 4096, for inputs above 256 KiB); the next tree-path calls use
    # 18 (f32 70,000), 733 (f32 3,000,001) and 74 (bf16 300,001) and leave
    # the 4096-partial call's values in the slots past theirs, so a stage 2
    # that read stale partials would be caught. bf16 100,003 and f16 1000 fit
    # 256 KiB and take the one-launch path (no scratch).
    cases = [(40_000_003, "f32"), (70_000, "f32"), (3_000_001, "f32"), (300_001, "bf16"), (100_003, "bf16"),
             (1000, "f16"), (40_000_003, "f32")]
    for n, dtype in cases:
        g.announce(f"noalloc sum {dtype} n={n}")
        values = rng(n).standard_normal(n).astype(np.float32)
        stored = g.storage_bits(values, dtype)
        xg = g.to_gpu(stored, dtype)
        for start, accumulate in ((0.0, 0), (2.5, 1)):
            expected = sum_with_workspace(xg, dtype, n, start, accumulate)
            got = sum_noalloc(xg, dtype, n, start, accumulate)
            assert got == expected, f"{dtype} n={n} accumulate={accumulate}: {got!r} != {expected!r}"
        exact = oracle.sum_exact(g.host_values(stored, dtype))
        assert abs(sum_noalloc(xg, dtype, n, 0.0, 0) - exact) <= max(abs(exact), 1.0) * 1e-5 * math.sqrt(n)


def test_noalloc_sum_of_ones_is_exact_and_an_empty_sum_leaves_the_output():
    ones = g.to_gpu(np.ones(100_000, np.float32))
    assert sum_noalloc(ones, "f32", 100_000, 0.0, 0) == 100_000.0
    assert sum_noalloc(ones, "f32", 100_000, 5.0, 1) == 100_005.0
    out = torch.full((1,), 7.5, device=g.DEVICE)
    g.call("cf_reduce_sum_noalloc", 0, g.cf("f32"), out.data_ptr(), 0, 1, g.stream())
    torch.cuda.synchronize()
    assert float(out.item()) == 7.5

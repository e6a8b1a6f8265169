"""GPU parity of the paged-attention decode kernel (cf_paged_attention)
against the float64 oracle, through the C ABI.

Cases: the reference's five parity shapes with its fp32 margin (2e-5,
tests/cuda/test_paged_attention.cu:210-213), table following and block-order
invariance (:216-289), an empty sequence (:291-307), grouped-query attention
(:309-), plus what this kernel adds: bf16 caches (tolerance 1e-2 relative to
the output scale), head sizes served by the wide kernel (80, 1024), long
contexts split across workgroups (with and without the workspace), and a
benchmark-sized batch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cuda_force_amd import _lib

from . import gpu_util as g
from .gpu_util import announce
from .paged_util import REFERENCE_CASES, make_case

pytestmark = pytest.mark.gpu

FP32_MARGIN = 2e-5


def run_gpu(case, dtype="f32", workspace=True):
    s, h, kvh, d, bs, mb = case.dims
    tdtype = torch.float32 if dtype == "f32" else torch.bfloat16
    dev = torch.device("cuda:0")
    q = torch.from_numpy(case.query).to(dev, tdtype)
    k = torch.from_numpy(case.k_cache).to(dev, tdtype)
    v = torch.from_numpy(case.v_cache).to(dev, tdtype)
    tables = torch.from_numpy(case.tables.view(np.int32)).to(dev)
    ctx = torch.from_numpy(case.context).to(dev)
    out = torch.full_like(q, float("nan"))
    lib = _lib.load()
    nbytes = lib.cf_paged_attention_workspace_bytes(s, h, kvh, d, bs, mb) if workspace else 0
    ws = g.empty(max(nbytes, 1), torch.uint8)
    code = _lib.CF_F32 if dtype == "f32" else _lib.CF_BF16
    _lib.check(lib.cf_paged_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), tables.data_ptr(),
                                      ctx.data_ptr(), out.data_ptr(), code, s, h, kvh, d, bs, mb,
                                      case.scale, ws.data_ptr() if nbytes else None, nbytes,
                                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def expected_for(case, dtype="f32"):
    if dtype == "bf16":
        r = oracle.round_bf16
        return oracle.paged_attention(r(case.query), r(case.k_cache), r(case.v_cache), case.tables,
                                      case.context, case.scale)
    return run_oracle(case)


def run_oracle(case):
    return oracle.paged_attention(case.query, case.k_cache, case.v_cache, case.tables, case.context,
                                  case.scale)


@pytest.mark.parametrize("dims", REFERENCE_CASES, ids=str)
def test_reference_cases_fp32(dims):
    announce(f"paged attention fp32 {dims}")
    case = make_case(*dims, seed=dims[3] * 7 + dims[4])
    np.testing.assert_allclose(run_gpu(case), run_oracle(case), rtol=0, atol=FP32_MARGIN)


def test_follows_the_table_and_ignores_block_order():
    announce("paged attention: table following / block-order invariance")
    case = make_case(1, 1, 1, 32, 4, [8], seed=3)
    base = run_gpu(case)
    swapped = make_case(1, 1, 1, 32, 4, [8], seed=3)
    swapped.tables[0, [0, 1]] = swapped.tables[0, [1, 0]]
    np.testing.assert_allclose(run_gpu(swapped), base, rtol=0, atol=1e-6)
    repointed = make_case(1, 1, 1, 32, 4, [8], seed=3)
    used = set(repointed.tables[0].tolist())
    repointed.tables[0, 0] = next(b for b in range(repointed.k_cache.shape[0]) if b not in used)
    assert np.abs(run_gpu(repointed) - base).max() > 1e-3
    np.testing.assert_allclose(run_gpu(repointed), run_oracle(repointed), rtol=0, atol=FP32_MARGIN)


def test_empty_sequence_and_gqa():
    announce("paged attention: empty sequence, GQA")
    case = make_case(2, 2, 2, 32, 4, [0, 6], seed=11)
    got = run_gpu(case)
    assert np.all(got[0] == 0.0)
    np.testing.assert_allclose(got, run_oracle(case), rtol=0, atol=FP32_MARGIN)
    gqa = make_case(2, 8, 2, 64, 8, [20, 9], seed=5)
    np.testing.assert_allclose(run_gpu(gqa), run_oracle(gqa), rtol=0, atol=FP32_MARGIN)
    big_group = make_case(2, 32, 2, 128, 16, [70, 33], seed=6)  # 16 heads per KV head: 2 workgroups
    np.testing.assert_allclose(run_gpu(big_group), run_oracle(big_group), rtol=0, atol=FP32_MARGIN)


@pytest.mark.parametrize("dims", [(2, 4, 2, 80, 16, [40, 3]), (1, 2, 1, 1024, 8, [19]),
                                  (2, 2, 2, 8, 4, [13, 4]), (1, 4, 4, 256, 16, [50])], ids=str)
def test_other_head_sizes(dims):
    announce(f"paged attention head size {dims[3]}")
    case = make_case(*dims, seed=dims[3])
    np.testing.assert_allclose(run_gpu(case), run_oracle(case), rtol=0, atol=FP32_MARGIN)


@pytest.mark.parametrize("workspace", [True, False], ids=["split", "unsplit"])
def test_long_contexts(workspace):
    announce(f"paged attention long context, workspace={workspace}")
    case = make_case(2, 8, 2, 128, 16, [3000, 1500], seed=21)
    s, h, kvh, d, bs, mb = case.dims
    if workspace:
        assert _lib.load().cf_paged_attention_workspace_bytes(s, h, kvh, d, bs, mb) > 0
    np.testing.assert_allclose(run_gpu(case, workspace=workspace), run_oracle(case), rtol=0,
                               atol=FP32_MARGIN)


@pytest.mark.parametrize(
    "dims",
    [
        (2, 16, 2, 128, 16, [300, 17]),     # group 8
        (1, 16, 1, 48, 8, [77]),            # group 16, head size 48
        (2, 32, 4, 80, 4, [129, 0]),        # group 8, head size 80, an empty sequence
        (1, 8, 2, 112, 16, [600]),          # group 4 (one round), head size 112, split or not
        (3, 24, 3, 16, 2, [5, 40, 16]),     # group 8, head size 16, two-token blocks
    ],
    ids=str,
)
def test_fp32_matrix_core_path(dims):
    """fp32 caches with GQA groups of 8 or more (or 4, when one round of
    workgroups holds every sequence and KV head) run on the fp32 matrix-core
    kernel (v_mfma_f32_16x16x4_f32: fp32 products and sums), within the
    reference's 2e-5 margin of the float64 oracle, with and without the split
    workspace."""
    announce(f"paged attention fp32 matrix cores {dims}")
    case = make_case(*dims, seed=sum(dims[:5]) * 3 + len(dims[5]))
    expected = run_oracle(case)
    for workspace in (True, False):
        np.testing.assert_allclose(run_gpu(case, workspace=workspace), expected, rtol=0, atol=FP32_MARGIN)


def test_bf16_cache():
    announce("paged attention bf16")
    case = make_case(3, 8, 2, 128, 16, [200, 17, 1], seed=8)
    got = run_gpu(case, "bf16")
    expected = expected_for(case, "bf16")
    scale = np.abs(expected).max()
    assert np.abs(got - expected).max() <= 1e-2 * scale


@pytest.mark.parametrize(
    "dims",
    [
        (2, 1, 1, 128, 16, [300, 17]),      # MHA: the matrix-core kernel
        (2, 4, 2, 64, 16, [33, 0]),         # GQA group 2 (streaming), an empty sequence
        (3, 8, 2, 128, 16, [200, 17, 1]),   # group 4
        (2, 8, 2, 64, 16, [0, 40]),         # group 4, an empty sequence
        (2, 16, 2, 128, 16, [300, 16]),     # group 8
        (1, 32, 2, 32, 8, [100]),           # group 16, the widest the matrix-core kernel takes
        (1, 32, 1, 64, 16, [50]),           # group 32: the streaming kernel
        (2, 16, 4, 96, 2, [15, 64]),        # group 4, head size 96, two-token blocks
        (1, 8, 2, 256, 1, [70]),            # group 4, head size 256, one-token blocks (window reloads)
        (2, 16, 4, 160, 64, [129, 300]),    # group 4, head size 160, 64-token blocks
        (1, 8, 2, 80, 16, [100]),           # head size 80 (not a multiple of 32): the streaming kernel
        (1, 16, 2, 128, 16, [1100]),        # a long context: split across workgroups, or not
        (2, 12, 4, 64, 16, [90, 33]),       # group 3 (not a power of two)
        (1, 10, 2, 224, 8, [61]),           # group 5, head size 224
        (2, 24, 2, 192, 32, [250, 5]),      # group 12, head size 192
        (3, 6, 2, 32, 16, [1, 16, 17]),     # group 3, one token, exactly one chunk, one past it
    ],
    ids=str,
)
def test_bf16_paths(dims):
    """bf16 caches: head sizes that are multiples of 32 (up to 256) with GQA
    groups of 1 and 4 to 16 take the matrix-core kernel (scores and P.V on MFMA,
    probabilities rounded to bf16 for P.V), the rest the streaming kernel;
    each within 1e-2 of the output scale of the float64 oracle on the same
    bf16 inputs, with and without the split workspace. An empty sequence
    gives zeros."""
    announce(f"paged attention bf16 {dims}")
    case = make_case(*dims, seed=sum(dims[:5]) + len(dims[5]))
    expected = expected_for(case, "bf16")
    scale = np.abs(expected).max()
    for workspace in (True, False):
        got = run_gpu(case, "bf16", workspace=workspace)
        err = np.abs(got - expected).max()
        assert err <= 1e-2 * scale, f"workspace={workspace}: max err {err:.3e} (scale {scale:.3e})"
    for s, n in enumerate(dims[5]):
        if n == 0:
            assert (got[s] == 0).all()


def test_benchmark_sized_batch():
    announce("paged attention 64 seq x 1024 ctx, 32 heads / 8 kv, d128")
    case = make_case(64, 32, 8, 128, 16, [1024] * 64, seed=9, spare=0)
    got = run_gpu(case)
    sample = [0, 17, 63]
    sub = make_case(64, 32, 8, 128, 16, [1024] * 64, seed=9, spare=0)
    expected = oracle.paged_attention(sub.query[sample], sub.k_cache, sub.v_cache, sub.tables[sample],
                                      sub.context[sample], sub.scale)
    np.testing.assert_allclose(got[sample], expected, rtol=0, atol=FP32_MARGIN)
    assert np.isfinite(got).all()


@pytest.mark.parametrize("block_size", [1, 2, 64], ids=lambda b: f"block{b}")
def test_block_sizes_around_the_table_window(block_size):
    announce(f"paged attention block size {block_size}")
    # 8-value head (fp32: 2 lanes, 32 tokens per step) with 1-token blocks: a
    # chunk spans more blocks than the 64-entry window; 300 tokens also cross
    # window reloads.
    for dims in ((2, 2, 1, 8, block_size, [300, 77]), (1, 4, 2, 128, block_size, [300])):
        case = make_case(*dims, seed=block_size)
        np.testing.assert_allclose(run_gpu(case), run_oracle(case), rtol=0, atol=FP32_MARGIN)
        np.testing.assert_allclose(run_gpu(case, workspace=False), run_oracle(case), rtol=0, atol=FP32_MARGIN)


@pytest.mark.parametrize("block_size", [3, 7, 31, 33, 100], ids=lambda b: f"block{b}")
def test_block_sizes_that_are_not_powers_of_two(block_size):
    """Block sizes that are not powers of two, through each kernel family:
    the matrix-core kernels walk the table with a per-wave block cursor (an
    exact float quotient below 32 tokens per block, a compare from 32 up) and
    the streaming kernel with a 32-bit quotient per token. Contexts cross
    steps, blocks and (for small blocks) reloads of the 64-entry table window.
    fp32 within the reference's 2e-5 margin, bf16 within 1e-2 of the output
    scale, with and without the split workspace."""
    announce(f"paged attention block size {block_size} (not a power of two)")
    cases = [
        ("f32", (2, 16, 2, 128, [700, 45])),   # group 8: fp32 matrix-core kernel
        ("f32", (2, 4, 4, 128, [700, 45])),    # MHA: fp32 streaming kernel
        ("bf16", (2, 8, 2, 128, [700, 45])),   # group 4: bf16 matrix-core kernel
        ("bf16", (2, 4, 2, 64, [700, 45])),    # group 2: bf16 streaming kernel
    ]
    for dtype, (s, h, kvh, d, ctx) in cases:
        case = make_case(s, h, kvh, d, block_size, ctx, seed=block_size * 7 + h)
        expected = expected_for(case, dtype)
        for workspace in (True, False):
            got = run_gpu(case, dtype, workspace=workspace)
            if dtype == "f32":
                np.testing.assert_allclose(got, expected, rtol=0, atol=FP32_MARGIN)
            else:
                err = np.abs(got - expected).max()
                assert err <= 1e-2 * np.abs(expected).max(), f"{dtype} {h}/{kvh} workspace={workspace}: {err:.3e}"

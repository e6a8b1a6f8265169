"""Grouped quantise/dequantise (cf_quantize_int8_group / cf_dequantize_int8_group):
every member bit-identical to the oracle - and so to the single-tensor entry
points - across several groups (more than CF_QUANT_GROUP_MAX members), empty
and ragged members, members whose pointers are misaligned (they take their own
launch) and special values (NaN, +-inf, all-zero blocks)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from cuda_force_amd import _lib
from tests import gpu_util as g
from tests.conftest import rng

pytestmark = pytest.mark.gpu

GROUP_MAX = 48
SIZES = [0, 1, 63, 64, 65, 1000, 4096, 4097, 65543, 1 << 18, 3 * 64 * 1024 + 17, 11008]


def member_inputs(seed: int, dtype: str):
    """(count, host values, misalign) per member: 110 members, a few misaligned."""
    gen = rng(seed)
    members = []
    for i in range(110):
        n = SIZES[i % len(SIZES)] + (i // len(SIZES))
        x = (gen.standard_normal(n) * (0.02 if i % 3 else 3.0)).astype(np.float32)
        if n > 200:
            x[gen.integers(0, n, n // 100 + 1)] *= 50.0
        if i == 7 and n >= 130:
            x[0], x[1], x[64:128] = np.nan, np.inf, 0.0
        if i == 8 and n >= 70:
            x[5] = -np.inf
        if dtype == "bf16":
            x = (x.view(np.uint32) >> 16).astype(np.uint16)  # truncation keeps specials
        elif dtype == "f16":
            x = oracle.quant.f32_to_f16_bits(x)
        members.append((n, x, i % 17 == 5))
    return members


def carve(members, elem_bytes: int, torch_dtype, poison: bool = False):
    """One device buffer holding every member at 256-byte aligned slots (plus
    one element for misaligned members); returns the buffer and offsets.
    Input buffers start zeroed; output buffers (poison=True) start poisoned,
    so an element no kernel writes fails the comparison."""
    offsets, cursor = [], 0
    for n, _, misaligned in members:
        start = cursor + (elem_bytes if misaligned else 0)
        offsets.append(start)
        cursor = (start + max(n, 1) * elem_bytes + 255) // 256 * 256
    if poison:
        return g.empty(cursor // elem_bytes + 64, torch_dtype), offsets
    buf = torch.zeros(cursor // elem_bytes + 64, dtype=torch_dtype, device="cuda")
    return buf, offsets


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_group_members_match_the_oracle_bit_for_bit(dtype):
    print(f"case: grouped quantise/dequantise, 110 members, {dtype}", flush=True)
    members = member_inputs(31 if dtype == "f32" else 32, dtype)
    elem = 4 if dtype == "f32" else 2
    xbuf, xoff = carve(members, elem, g.torch_dtype(dtype))
    xbytes = xbuf.view(torch.uint8)
    for (n, x, _), off in zip(members, xoff):
        if n:
            host = torch.from_numpy(np.ascontiguousarray(x).view(np.uint8).copy())
            xbytes[off:off + host.numel()].copy_(host.to("cuda"))
    qbuf, qoff = carve(members, 1, torch.int8, poison=True)
    sbuf = g.empty(sum((n + 63) // 64 + 64 for n, _, _ in members), torch.float32)
    soff, cursor = [], 0
    for n, _, _ in members:
        soff.append(cursor)
        cursor += (n + 63) // 64 + 64
    counts = [n for n, _, _ in members]
    x_ptrs = [xbuf.data_ptr() + off for off in xoff]
    q_ptrs = [qbuf.data_ptr() + off for off in qoff]
    s_ptrs = [sbuf.data_ptr() + 4 * off for off in soff]
    g.call("cf_quantize_int8_group", _lib.pointer_array(x_ptrs), g.cf(dtype), _lib.pointer_array(q_ptrs),
           _lib.pointer_array(s_ptrs), _lib.int64_array(counts), len(members), g.stream())
    # Dequantise back into each of the three output types.
    outs = {}
    for out_dtype in ("f32", "bf16", "f16"):
        oelem = 4 if out_dtype == "f32" else 2
        ybuf, yoff = carve(members, oelem, g.torch_dtype(out_dtype), poison=True)
        y_ptrs = [ybuf.data_ptr() + off for off in yoff]
        g.call("cf_dequantize_int8_group", _lib.pointer_array(q_ptrs), _lib.pointer_array(s_ptrs),
               _lib.pointer_array(y_ptrs), g.cf(out_dtype), _lib.int64_array(counts), len(members), g.stream())
        outs[out_dtype] = (ybuf, yoff, oelem)
    torch.cuda.synchronize()
    qhost = qbuf.cpu().numpy().view(np.int8)
    shost = sbuf.cpu().numpy()
    for i, ((n, x, _), qo, so) in enumerate(zip(members, qoff, soff)):
        q_ref, s_ref = oracle.quantize_int8(x, dtype)
        assert np.array_equal(qhost[qo:qo + n], q_ref.reshape(-1)), f"member {i} (n={n}) codes differ"
        assert np.array_equal(shost[so:so + (n + 63) // 64].view(np.uint32), s_ref.view(np.uint32)), \
            f"member {i} (n={n}) scales differ"
        for out_dtype, (ybuf, yoff, oelem) in outs.items():
            got = ybuf.view(torch.uint8)[yoff[i]:yoff[i] + n * oelem].cpu().numpy()
            want = np.ascontiguousarray(oracle.dequantize_int8(q_ref, s_ref, out_dtype).reshape(-1))
            view = np.uint32 if oelem == 4 else np.uint16
            bad = np.flatnonzero(got.view(view) != want.view(view))
            assert bad.size == 0, (f"member {i} (n={n}) dequantised to {out_dtype}: {bad.size} differ, "
                                   f"first {bad[:4]}: got {[hex(v) for v in got.view(view)[bad[:4]]]} "
                                   f"want {[hex(v) for v in want.view(view)[bad[:4]]]}")
    # The slots between members were never written: they still hold the poison (-128).
    for i, (n, _, _) in enumerate(members):
        end = qoff[i] + n
        gap_end = qoff[i + 1] if i + 1 < len(members) else qhost.size
        assert (qhost[end:min(gap_end, end + 64)] == -128).all(), f"write past member {i}"


SHAPES_7B = [(4096, 4096), (11008, 4096), (4096, 11008)]


def test_group_at_the_7b_shapes_matches_the_oracle():
    """One member of each 7B layer shape (config 5: bf16 ~N(0, 0.02) with 0.1%
    outliers x50) through the grouped quantiser, then the grouped dequantiser
    to bf16 - the bench's aggregate kernels - every code, scale and output
    bit against the oracle."""
    print("case: grouped bf16 quantise/dequantise at the 7B shapes vs the oracle", flush=True)
    gen = rng(7007)
    hosts = []
    for rows, cols in SHAPES_7B:
        n = rows * cols
        x = (0.02 * gen.standard_normal(n, dtype=np.float32))
        x[gen.choice(n, n // 1000, replace=False)] *= 50.0
        hosts.append(oracle.f32_to_bf16_bits(x))
    xs = [g.to_gpu(h, "bf16") for h in hosts]
    qs = [g.empty(x.numel(), torch.int8) for x in xs]
    ss = [g.empty(x.numel() // 64, torch.float32) for x in xs]
    ys = [g.poison_like(x) for x in xs]
    g.call("cf_quantize_int8_group", _lib.pointer_array([x.data_ptr() for x in xs]), _lib.CF_BF16,
           _lib.pointer_array([q.data_ptr() for q in qs]), _lib.pointer_array([s.data_ptr() for s in ss]),
           _lib.int64_array([x.numel() for x in xs]), len(xs), g.stream())
    g.call("cf_dequantize_int8_group", _lib.pointer_array([q.data_ptr() for q in qs]),
           _lib.pointer_array([s.data_ptr() for s in ss]), _lib.pointer_array([y.data_ptr() for y in ys]),
           _lib.CF_BF16, _lib.int64_array([x.numel() for x in xs]), len(xs), g.stream())
    torch.cuda.synchronize()
    for shape, h, q, s, y in zip(SHAPES_7B, hosts, qs, ss, ys):
        q_ref, s_ref = oracle.quantize_int8(h, "bf16")
        bad = np.flatnonzero(g.to_host(q).view(np.int8) != q_ref.reshape(-1))
        assert bad.size == 0, f"{shape}: {bad.size} codes differ, first at {bad[:4]}"
        assert np.array_equal(g.to_host(s).view(np.uint32), s_ref.view(np.uint32)), f"{shape}: scales differ"
        want = oracle.dequantize_int8(q_ref, s_ref, "bf16").reshape(-1)
        bad = np.flatnonzero(g.to_host(y) != want.view(np.uint16))
        assert bad.size == 0, f"{shape}: {bad.size} dequantised values differ, first at {bad[:4]}"
        del q_ref, s_ref, want


def test_group_equals_single_calls_at_the_7b_shapes():
    print("case: grouped bf16 quantise at the 7B layer shapes vs single calls", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    shapes = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)]
    xs = [(0.02 * torch.randn(*s, generator=gen, device="cuda")).to(torch.bfloat16) for s in shapes * 8]
    qs = [g.empty(x.numel(), torch.int8) for x in xs]
    ss = [g.empty(x.numel() // 64, torch.float32) for x in xs]
    g.call("cf_quantize_int8_group", _lib.pointer_array([x.data_ptr() for x in xs]), _lib.CF_BF16,
           _lib.pointer_array([q.data_ptr() for q in qs]), _lib.pointer_array([s.data_ptr() for s in ss]),
           _lib.int64_array([x.numel() for x in xs]), len(xs), g.stream())
    for x, q, s in zip(xs, qs, ss):
        q1 = g.poison_like(q)
        s1 = g.poison_like(s)
        g.call("cf_quantize_int8", x.data_ptr(), _lib.CF_BF16, q1.data_ptr(), s1.data_ptr(), x.numel(), g.stream())
        assert torch.equal(q, q1) and torch.equal(s.view(torch.int32), s1.view(torch.int32))
    assert len(xs) > GROUP_MAX

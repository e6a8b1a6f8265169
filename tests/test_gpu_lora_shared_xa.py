"""The fused bf16 LoRA kernel with a workspace (cf_lora_linear_ws): column
tile 0 of each 256-row tile publishes its bf16 x @ a fragments and a flag
holding the dispatch's token, and workgroups that start late copy them
instead of forming x @ a in their K-loop. Whichever happens, the output must
be bit-identical to the call without a workspace (cf_lora_linear): the same
MFMA sequence forms x @ a in either tile. Checked on shapes of one and of
several rounds of workgroups, ragged edges, ranks 2-16 and K-loops of 2, 4
and 6 steps (the peeled steps alone, and with one loop pass), with a workspace
that starts as garbage and is then reused by a call on other inputs (stale
flags of the first call must read as unset in the second), and the
published fragments themselves against bf16(x @ a).
"""

from __future__ import annotations

import pytest
import torch

import cuda_force_amd  # noqa: F401  (registers torch.ops.cudaforge)
from cuda_force_amd import _lib
from tests import gpu_util as g

pytestmark = pytest.mark.gpu

SHAPES = [
    (8192, 4096, 4096, 16),   # config 3: 512 tiles, two rounds on 256 CUs
    (4096, 4096, 11008, 16),  # 16 x 43 tiles
    (5000, 1024, 2056, 6),    # ragged rows and columns
    (16384, 1024, 2048, 2),
    (32768, 1024, 4096, 16),  # 2048 tiles, eight rounds
    (2048, 2048, 4096, 8),    # 128 tiles: one round, nothing shared
    (32768, 64, 2048, 16),    # the shortest K-loops: 2, 4 and 6 K-steps
    (32768, 128, 2048, 8),
    (32768, 192, 2048, 4),
]


def _operands(m, k, n, r, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16)
    w = (0.02 * torch.randn(k, n, generator=gen, device="cuda")).to(torch.bfloat16)
    a = (torch.randn(k, r, generator=gen, device="cuda") / 64).to(torch.bfloat16)
    b = (0.02 * torch.randn(r, n, generator=gen, device="cuda")).to(torch.bfloat16)
    return x, w, a, b


def _plain(x, w, a, b, scale):
    m, k = x.shape
    n, r = w.shape[1], a.shape[1]
    y = g.poison_like(torch.empty(m, n, dtype=torch.bfloat16, device="cuda"))
    xa = g.poison_like(torch.empty(m, r, dtype=torch.float32, device="cuda"))
    g.call("cf_lora_linear", x.data_ptr(), w.data_ptr(), a.data_ptr(), b.data_ptr(), y.data_ptr(),
           xa.data_ptr(), _lib.CF_BF16, m, k, n, r, scale, g.stream())
    return y, xa


def _shared(x, w, a, b, scale, ws):
    m, k = x.shape
    n, r = w.shape[1], a.shape[1]
    y = g.poison_like(torch.empty(m, n, dtype=torch.bfloat16, device="cuda"))
    xa = g.poison_like(torch.empty(m, r, dtype=torch.float32, device="cuda"))
    g.call("cf_lora_linear_ws", x.data_ptr(), w.data_ptr(), a.data_ptr(), b.data_ptr(), y.data_ptr(),
           xa.data_ptr(), _lib.CF_BF16, m, k, n, r, scale, ws.data_ptr(), ws.numel(), g.stream())
    return y, xa


def _published(xa: torch.Tensor, tiles_m: int, r: int) -> torch.Tensor:
    """The fragments column tile 0 publishes, as uint16 [tiles_m, 16, 64, 4]:
    block rb, lane l, element e holds bf16(x @ a) at row 256 tm + 16 rb + l % 16,
    column 4 (l / 16) + e; zero past the rank and past the last row."""
    m = xa.shape[0]
    full = torch.zeros(tiles_m * 256, 16, dtype=torch.float32, device="cuda")
    full[:m, :r] = xa
    bits = full.to(torch.bfloat16).view(torch.int16)
    t = bits.view(tiles_m, 16, 16, 4, 4)            # [tm][rb][row l%16][group l/16][e]
    return t.permute(0, 1, 3, 2, 4).reshape(tiles_m, 16, 64, 4)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_shared_xa_is_bit_identical_to_the_plain_call(shape):
    m, k, n, r = shape
    g.announce(f"fused LoRA bf16 with shared x @ a {m}x{k}x{n} r{r}")
    nbytes = g.lib().cf_lora_linear_ws_bytes(_lib.CF_BF16, m, k, n, r)
    tiles_m = (m + 255) // 256
    flag_bytes = (tiles_m * 8 + 255) // 256 * 256
    assert nbytes == flag_bytes + tiles_m * 8192
    ws = torch.full((nbytes,), 0xFF, dtype=torch.uint8, device="cuda")
    scale = 2.0 if r == 16 else 16 / r
    for seed in (11, 12):  # the second call finds the first call's flags and fragments
        x, w, a, b = _operands(m, k, n, r, seed)
        y0, xa0 = _plain(x, w, a, b, scale)
        y1, xa1 = _shared(x, w, a, b, scale, ws)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), f"seed {seed}: y differs"
        assert torch.equal(xa0.view(torch.int32), xa1.view(torch.int32)), f"seed {seed}: x @ a differs"
        flags = ws[:tiles_m * 8].view(torch.int64)
        assert bool((flags != -1).all()), "a row tile's flag was not set"
        pub = ws[flag_bytes:].view(torch.int16).view(tiles_m, 16, 64, 4)
        assert torch.equal(pub, _published(xa1, tiles_m, r)), f"seed {seed}: published fragments"


def test_the_torch_operator_takes_the_workspace_path():
    """The dispatcher's lora_linear runs cf_lora_linear_ws with a workspace
    from torch's caching allocator: same bits as the plain entry point."""
    g.announce("torch operator lora_linear bf16 8192x4096x4096 r16 against cf_lora_linear")
    m, k, n, r = 8192, 4096, 4096, 16
    x, w, a, b = _operands(m, k, n, r, 21)
    y0, _ = _plain(x, w, a, b, 2.0)
    y1 = torch.ops.cudaforge.lora_linear(x, w, a, b, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_two_streams_with_workspaces_of_their_own():
    """The torch operator on two default-priority streams at once, each call
    with the workspace torch's caching allocator gives it on its stream: the
    flags and fragments of one call never reach the other."""
    g.announce("fused LoRA bf16 with shared x @ a on two streams at once, 8192x4096x4096 r16")
    m, k, n, r = 8192, 4096, 4096, 16
    ops = [_operands(m, k, n, r, seed) for seed in (31, 32)]
    want = [_plain(*op, 2.0)[0] for op in ops]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [None, None]
    for rep in range(3):
        for i, (s, op) in enumerate(zip(streams, ops)):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                outs[i] = torch.ops.cudaforge.lora_linear(*op, 2.0)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(outs[i].view(torch.int16), want[i].view(torch.int16)), f"rep {rep} stream {i}"

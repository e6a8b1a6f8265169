"""The custom operators under HIP graph capture.

Every op of the path is capturable (no allocation in the C ABI, no
hipMemsetAsync anywhere, workspaces come from torch's graph-aware allocator).
Each graph is replayed several times with eager work and synchronisations in
between, and every replay is compared with the eager result: bit-exact for the
custom ops (their kernels are deterministic), within the bf16 tolerance for
the composed block (whose attention products are torch's).
"""

from __future__ import annotations

import pytest
import torch

import cuda_force_amd as cf
from cuda_force_amd.transformer_block import BlockConfig, LlamaBlock

from .gpu_util import announce

pytestmark = pytest.mark.gpu

REPLAYS = 4


def capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def test_custom_ops_replay_bit_exactly():
    announce("graph capture: quantise/dequantise, rmsnorm, softmax, fused LoRA, sum, activations")
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(512, 4096, generator=gen, device="cuda").to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(4096, generator=gen, device="cuda")).to(torch.bfloat16)
    lw = (0.02 * torch.randn(4096, 1024, generator=gen, device="cuda")).to(torch.bfloat16)
    la = (0.02 * torch.randn(4096, 16, generator=gen, device="cuda")).to(torch.bfloat16)
    lb = (0.02 * torch.randn(16, 1024, generator=gen, device="cuda")).to(torch.bfloat16)
    logits = torch.randn(256, 2048, generator=gen, device="cuda")

    def ops():
        q, s = cf.quantize_int8(x)
        return (q, s, cf.dequantize_int8(q, s).to(torch.bfloat16), cf.rmsnorm(x, w), cf.softmax(logits),
                cf.lora_linear(x, lw, la, lb, 2.0), cf.sum_reduce(logits), cf.swiglu(x, x), cf.gelu(x))

    eager = ops()
    graph, outs = capture(ops)
    for r in range(REPLAYS):
        torch.cuda.synchronize()
        noise = cf.rmsnorm(torch.randn_like(x), w)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(e, o), f"replay {r}"
        del noise


def test_block_forward_replays_match_eager():
    announce("graph capture: Llama block forward (hidden 1024, 8 heads, 2 x 128 tokens)")
    config = BlockConfig(hidden=1024, heads=8, intermediate=2816, rank=16, alpha=32.0)
    gen = torch.Generator(device="cuda").manual_seed(5)
    block = LlamaBlock(config, "cuda", torch.bfloat16, gen)
    x = torch.randn(2, 128, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    res = torch.randn(2, 128, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    eager_out, eager_res = block.forward(x, res)
    graph, (out, out_res) = capture(lambda: block.forward(x, res))
    scale = eager_out.float().abs().max().item()
    for r in range(REPLAYS):
        torch.cuda.synchronize()
        block.forward(torch.randn_like(x), res)  # eager forward between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_res, eager_res), f"replay {r}: residual"
        assert (out.float() - eager_out.float()).abs().max().item() <= 1e-2 * scale, f"replay {r}"


def test_fused_lora_with_shared_xa_replays_on_new_inputs():
    """Config 3's shape (512 output tiles, two rounds of workgroups) through the
    torch operator, whose workspace lets late column tiles take x @ a from the
    first tile of their rows. Each replay runs on new x (copied into the
    captured input) and must equal the plain entry point on that x bit for bit:
    the flags the previous replay left hold another dispatch's token."""
    from cuda_force_amd import _lib

    from . import gpu_util as g

    announce("graph capture: fused LoRA bf16 8192x4096x4096 r16 with shared x @ a, new x per replay")
    m, k, n, r = 8192, 4096, 4096, 16
    gen = torch.Generator(device="cuda").manual_seed(9)
    x = torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16)
    w = (0.02 * torch.randn(k, n, generator=gen, device="cuda")).to(torch.bfloat16)
    a = (torch.randn(k, r, generator=gen, device="cuda") / 64).to(torch.bfloat16)
    b = (0.02 * torch.randn(r, n, generator=gen, device="cuda")).to(torch.bfloat16)
    graph, out = capture(lambda: torch.ops.cudaforge.lora_linear(x, w, a, b, 2.0))
    want = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    for rep in range(REPLAYS):
        torch.cuda.synchronize()
        x.copy_(torch.randn(m, k, generator=gen, device="cuda").to(torch.bfloat16))
        g.call("cf_lora_linear", x.data_ptr(), w.data_ptr(), a.data_ptr(), b.data_ptr(), want.data_ptr(),
               None, _lib.CF_BF16, m, k, n, r, 2.0, g.stream())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), f"replay {rep}"

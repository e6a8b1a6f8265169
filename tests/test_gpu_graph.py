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

"""The config-4 transformer block composition on the CPU (host logic).

The block (cuda_force_amd/transformer_block.py) restates the reference's
examples/transformer_block.py:32-133 with LoRA projections. On CPU tensors every
operator takes its ATen path, so this checks the composition itself - shapes,
head split, causal mask, residual routing, LoRA wiring - against the fp32
restatement, and the operator accounting.
"""

import math

import pytest
import torch

from cuda_force_amd.transformer_block import BlockConfig, LlamaBlock


def small_config():
    return BlockConfig(hidden=64, heads=4, intermediate=96, rank=4, alpha=8.0, std=0.05)


def test_fp32_block_matches_its_restatement():
    torch.manual_seed(0)
    block = LlamaBlock(small_config(), "cpu", torch.float32, torch.Generator().manual_seed(1))
    x = torch.randn(2, 8, 64)
    residual = torch.randn(2, 8, 64)
    out, res = block.forward(x, residual)
    ref_out, ref_res = block.reference_forward(x, residual)
    assert out.shape == (2, 8, 64) and res.shape == (2, 8, 64)
    torch.testing.assert_close(res, ref_res, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(out, ref_out, rtol=1e-4, atol=1e-5)


def test_causal_mask_makes_early_positions_independent_of_later_ones():
    block = LlamaBlock(small_config(), "cpu", torch.float32, torch.Generator().manual_seed(2))
    x = torch.randn(1, 8, 64)
    residual = torch.zeros(1, 8, 64)
    out1, _ = block.forward(x, residual)
    x2 = x.clone()
    x2[:, 5:] += 3.0  # change only the later positions
    out2, _ = block.forward(x2, residual)
    torch.testing.assert_close(out1[:, :5], out2[:, :5], rtol=1e-5, atol=1e-6)
    assert not torch.allclose(out1[:, 5:], out2[:, 5:])


def test_zero_adapters_reduce_to_the_base_block():
    block = LlamaBlock(small_config(), "cpu", torch.float32, torch.Generator().manual_seed(3))
    x = torch.randn(1, 4, 64)
    residual = torch.randn(1, 4, 64)
    with_adapters, _ = block.forward(x, residual)
    for p in (block.q, block.k, block.v, block.o, block.gate, block.up, block.down):
        p.b.zero_()
    without, _ = block.forward(x, residual)
    # The same block with plain linears, written out directly.
    c = block.config
    r = x + residual
    n = r * torch.rsqrt(r.pow(2).mean(-1, keepdim=True) + c.eps) * block.attention_norm
    n = n.reshape(-1, 64)
    q, k, v = (n @ p.w for p in (block.q, block.k, block.v))
    heads = lambda t: t.view(1, 4, c.heads, c.head_dim).transpose(1, 2)
    s = heads(q) @ heads(k).transpose(-2, -1) / math.sqrt(c.head_dim)
    s = s + torch.triu(torch.full((4, 4), float("-inf")), 1)
    a = (torch.softmax(s, -1) @ heads(v)).transpose(1, 2).reshape(4, 64) @ block.o.w
    r2 = a + r.reshape(4, 64)
    n2 = r2 * torch.rsqrt(r2.pow(2).mean(-1, keepdim=True) + c.eps) * block.ffn_norm
    expect = ((torch.nn.functional.silu(n2 @ block.gate.w) * (n2 @ block.up.w)) @ block.down.w).view(1, 4, 64)
    torch.testing.assert_close(without, expect, rtol=1e-4, atol=1e-5)
    assert not torch.allclose(with_adapters, without)


def test_flop_accounting_at_config4():
    block_cfg = BlockConfig()
    block = LlamaBlock.__new__(LlamaBlock)
    block.config = block_cfg
    flops = block.gemm_flops(tokens=4096, seq=512)
    base = 4 * 2 * 4096 * 4096 * 4096 + 3 * 2 * 4096 * 4096 * 11008
    lora_base = flops["qkv_lora"] + flops["o_lora"] + flops["gate_up_lora"] + flops["down_lora"]
    adapters = 4 * (2 * 4096 * 4096 * 16 * 2) + 3 * (2 * 4096 * 16 * (4096 + 11008))
    assert lora_base == base + adapters
    assert flops["scores_matmul"] == 2 * 8 * 32 * 512 * 512 * 128


def test_heads_must_divide_hidden():
    with pytest.raises(ValueError):
        LlamaBlock(BlockConfig(hidden=65, heads=4, intermediate=8, rank=2), "cpu", torch.float32)

"""GPU parity of the config-4 transformer block through the custom operators.

The bf16 block (fused LoRA, softmax, fused residual RMSNorm and SwiGLU kernels,
hipBLASLt batched attention products) against the same block restated in fp32
torch operations from the same bf16 parameters. The chain rounds to bf16 after
every operator, so the comparison is a relative Frobenius error with the
tolerance written below (bf16 carries 8 significant bits; ~10 chained roundings
plus the bf16 attention products).
"""

import pytest
import torch

from cuda_force_amd.transformer_block import BlockConfig, LlamaBlock, timed_forward

from .gpu_util import announce

pytestmark = pytest.mark.gpu

REL_TOL_OUT = 3e-2
REL_TOL_RESIDUAL = 1e-2


def rel(a, b):
    return ((a.float() - b.float()).norm() / b.float().norm()).item()


def run_block(config, batch, seq, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    block = LlamaBlock(config, "cuda", torch.bfloat16, gen)
    x = torch.randn(batch, seq, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    residual = torch.randn(batch, seq, config.hidden, generator=gen, device="cuda").to(torch.bfloat16)
    out, res = block.forward(x, residual)
    torch.cuda.synchronize()
    ref_out, ref_res = block.reference_forward(x, residual)
    return block, x, residual, out, res, ref_out, ref_res


@pytest.mark.parametrize(
    "config,batch,seq",
    [(BlockConfig(hidden=256, heads=4, intermediate=688, rank=16, alpha=32.0), 2, 64),
     (BlockConfig(hidden=512, heads=8, intermediate=1024, rank=8, alpha=16.0), 1, 128)],
)
def test_small_block_matches_fp32(config, batch, seq):
    announce(f"block {config} batch {batch} seq {seq}")
    _, _, _, out, res, ref_out, ref_res = run_block(config, batch, seq, 41)
    assert torch.isfinite(out).all()
    assert rel(res, ref_res) < REL_TOL_RESIDUAL
    assert rel(out, ref_out) < REL_TOL_OUT


def test_config4_block_matches_fp32():
    announce("config 4 block: 8 x 512 tokens, hidden 4096, 32 heads, MLP 11008, r16")
    block, x, residual, out, res, ref_out, ref_res = run_block(BlockConfig(), 8, 512, 42)
    assert torch.isfinite(out).all()
    assert rel(res, ref_res) < REL_TOL_RESIDUAL
    assert rel(out, ref_out) < REL_TOL_OUT
    stages = timed_forward(block, x, residual)
    assert set(stages) >= {"qkv_lora", "softmax", "swiglu", "down_lora", "total"}
    assert stages["total"] > 0

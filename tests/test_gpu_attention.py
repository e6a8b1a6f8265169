"""GPU parity of the causal attention products (cf_attention.hip) through the C ABI.

cf_attention_scores_causal against oracle.attention_scores and
cf_attention_pv_causal against oracle.attention_values (both pinned against
torch's causal scaled_dot_product_attention in tests/test_attention_oracle.py):
* bit-exact on integer-valued operands, where every fp32 sum is exact in any
  order, so the kernel's bf16 result must be the oracle's value rounded once;
* within bf16 output rounding on random operands (|got - exact| <= 1e-2
  |exact| + 1e-3 max |exact|, the GEMM tolerance policy);
* the causal contract: 128 x 128 score tiles above the diagonal keep what the
  buffer held, and probabilities above the diagonal (NaN here) never reach a
  value;
* config 4's shape (8 x 512 tokens, 32 heads of 128) and the products with
  the causal softmax between them against the float64 composition.
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

SENTINEL = 0x7E7E  # a bf16 NaN pattern no kernel produces


def run_scores(q_bits, k_bits, heads, prefill=SENTINEL):
    batch, seq, _ = q_bits.shape
    qg, kg = g.to_gpu(q_bits, "bf16"), g.to_gpu(k_bits, "bf16")
    sg = torch.full((batch, heads, seq, seq), prefill, dtype=torch.int16, device=g.DEVICE).view(torch.bfloat16)
    g.call("cf_attention_scores_causal", qg.data_ptr(), kg.data_ptr(), sg.data_ptr(), g.cf("bf16"), batch, seq,
           heads, q_bits.shape[2] // heads, g.stream())
    torch.cuda.synchronize()
    return g.to_host(sg)


def run_values(p_bits, v_bits, heads):
    batch, seq, _ = v_bits.shape
    pg, vg = g.to_gpu(p_bits, "bf16"), g.to_gpu(v_bits, "bf16")
    og = torch.full(v_bits.shape, float("nan"), dtype=torch.bfloat16, device=g.DEVICE)
    g.call("cf_attention_pv_causal", pg.data_ptr(), vg.data_ptr(), og.data_ptr(), g.cf("bf16"), batch, seq, heads,
           v_bits.shape[2] // heads, g.stream())
    torch.cuda.synchronize()
    return g.to_host(og)


def within(got_bits, exact, what):
    got = g.host_values(got_bits, "bf16").astype(np.float64)
    bound = 1e-2 * np.abs(exact) + 1e-3 * np.abs(exact).max()
    bad = ~(np.abs(got - exact) <= bound)  # NaN fails
    assert not bad.any(), f"{what}: {bad.sum()} elements out of tolerance"


SHAPES = [(1, 8, 1, 32), (2, 64, 4, 64), (1, 136, 2, 32), (1, 264, 3, 128), (2, 72, 2, 96), (1, 384, 2, 128)]


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_scores_exact_on_integers_and_untouched_above_the_diagonal(shape):
    batch, seq, heads, d = shape
    g.announce(f"attention scores exact {shape}")
    r = rng(seq * 7 + d)
    q = r.integers(-3, 4, (batch, seq, heads * d)).astype(np.float32)
    k = r.integers(-3, 4, (batch, seq, heads * d)).astype(np.float32)
    got = run_scores(oracle.f32_to_bf16_bits(q), oracle.f32_to_bf16_bits(k), heads)
    want = oracle.f32_to_bf16_bits(oracle.attention_scores(q, k, heads).astype(np.float32))
    low = np.tril(np.ones((seq, seq), bool))
    np.testing.assert_array_equal(got[..., low], want[..., low])
    tiles = -(-seq // 128)
    for si in range(tiles):
        for ti in range(si + 1, tiles):
            block = got[..., si * 128:(si + 1) * 128, ti * 128:(ti + 1) * 128]
            assert (block == SENTINEL).all(), f"tile ({si}, {ti}) above the diagonal was written"


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_values_exact_and_blind_above_the_diagonal(shape):
    batch, seq, heads, d = shape
    g.announce(f"attention values exact {shape}")
    r = rng(seq * 5 + d + 1)
    v = r.integers(-3, 4, (batch, seq, heads * d)).astype(np.float32)
    probs = r.integers(0, 9, (batch, heads, seq, seq)).astype(np.float32) / 8
    low = np.tril(np.ones((seq, seq), bool))
    p_bits = oracle.f32_to_bf16_bits(probs)
    p_bits[..., ~low] = 0x7FC0  # NaN above the diagonal
    got = run_values(p_bits, oracle.f32_to_bf16_bits(v), heads)
    want = oracle.f32_to_bf16_bits(oracle.attention_values(probs * low, v, heads).astype(np.float32))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("shape", [(2, 64, 4, 64), (1, 264, 3, 128), (2, 72, 2, 96)], ids=str)
def test_products_within_bf16_rounding_on_random_operands(shape):
    batch, seq, heads, d = shape
    g.announce(f"attention products random {shape}")
    r = rng(seq + d + heads)
    q, k, v = (oracle.f32_to_bf16_bits(r.standard_normal((batch, seq, heads * d)).astype(np.float32))
               for _ in range(3))
    qv, kv, vv = (g.host_values(t, "bf16") for t in (q, k, v))
    low = np.tril(np.ones((seq, seq), bool))
    got = run_scores(q, k, heads)
    exact = oracle.attention_scores(qv, kv, heads)
    within(got[..., low], exact[..., low], "scores")
    probs = oracle.f32_to_bf16_bits(np.tril(r.random((batch, heads, seq, seq))).astype(np.float32))
    within(run_values(probs, v, heads), oracle.attention_values(g.host_values(probs, "bf16"), vv, heads), "values")


def test_config4_attention_with_the_causal_softmax():
    """Config 4 (8 x 512 tokens, 32 heads of 128): scores -> causal softmax
    (cf_softmax_scaled, period seq) -> values, against the float64
    composition on the same bf16 operands, for two of the 256 heads in full
    plus finiteness and row sums everywhere."""
    batch, seq, heads, d = 8, 512, 32, 128
    g.announce("attention products config 4")
    gen = torch.Generator(device=g.DEVICE).manual_seed(4)
    q, k, v = (torch.randn(batch, seq, heads * d, generator=gen, device=g.DEVICE).bfloat16() for _ in range(3))
    scores = g.empty((batch, heads, seq, seq), torch.bfloat16)
    g.call("cf_attention_scores_causal", q.data_ptr(), k.data_ptr(), scores.data_ptr(), g.cf("bf16"), batch, seq,
           heads, d, g.stream())
    probs = g.poison_like(scores)
    g.call("cf_softmax_scaled", scores.data_ptr(), g.cf("bf16"), probs.data_ptr(), g.cf("bf16"), batch * heads * seq,
           seq, 1 / math.sqrt(d), seq, g.stream())
    out = g.poison_like(v)
    g.call("cf_attention_pv_causal", probs.data_ptr(), v.data_ptr(), out.data_ptr(), g.cf("bf16"), batch, seq,
           heads, d, g.stream())
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    p = probs.float()
    np.testing.assert_allclose(p.sum(-1).cpu().numpy(), 1.0, atol=2e-2)
    assert (p.cpu().numpy()[..., ~np.tril(np.ones((seq, seq), bool))] == 0).all()
    for b, h in ((0, 0), (7, 31)):
        qh = q[b].float().view(seq, heads, d)[:, h].cpu().numpy().astype(np.float64)
        kh = k[b].float().view(seq, heads, d)[:, h].cpu().numpy().astype(np.float64)
        vh = v[b].float().view(seq, heads, d)[:, h].cpu().numpy().astype(np.float64)
        z = (qh @ kh.T) / math.sqrt(d)
        z = np.where(np.triu(np.ones((seq, seq), bool), 1), -np.inf, z)
        want = oracle.softmax(z) @ vh
        got = out[b].float().view(seq, heads, d)[:, h].cpu().numpy()
        # bf16 scores and probabilities (2^-9 each) feed the products.
        assert np.abs(got - want).max() <= 3e-2 * np.abs(want).max()

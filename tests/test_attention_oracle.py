"""Pins of the attention-product oracle (oracle.floatops.attention_scores /
attention_values) and of the ops-level causal attention products on the CPU.

The oracle pair, with the oracle softmax between them, must equal torch's
causal scaled_dot_product_attention in float64 (a library routine the
composition of examples/transformer_block.py:51-63 reduces to). A planted
mistake (keys and queries swapped, i.e. the upper triangle) and a mask that
is off by one both fail that check. The ops functions on CPU tensors must
equal the oracle on the causal half.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from cuda_force_amd import ops
from tests.conftest import rng


def causal_softmax(scores: np.ndarray, scale: float) -> np.ndarray:
    seq = scores.shape[-1]
    z = scale * scores
    z = np.where(np.triu(np.ones((seq, seq), bool), 1), -np.inf, z)
    return oracle.softmax(z)


def sdpa(q, k, v, heads):
    batch, seq, hidden = q.shape
    d = hidden // heads
    split = lambda t: torch.from_numpy(t).reshape(batch, seq, heads, d).transpose(1, 2)  # noqa: E731
    o = torch.nn.functional.scaled_dot_product_attention(split(q), split(k), split(v), is_causal=True)
    return o.transpose(1, 2).reshape(batch, seq, hidden).numpy()


@pytest.mark.parametrize("shape", [(2, 16, 3, 8), (1, 40, 2, 32), (3, 7, 1, 4)], ids=str)
def test_oracle_composition_is_causal_attention(shape):
    batch, seq, heads, d = shape
    r = rng(sum(shape))
    q, k, v = (r.standard_normal((batch, seq, heads * d)) for _ in range(3))
    scale = 1 / math.sqrt(d)
    probs = causal_softmax(oracle.attention_scores(q, k, heads), scale)
    got = oracle.attention_values(probs, v, heads)
    np.testing.assert_allclose(got, sdpa(q, k, v, heads), rtol=1e-10, atol=1e-12)
    # Planted mistakes fail it: scores transposed (keys attend to queries)...
    swapped = causal_softmax(oracle.attention_scores(k, q, heads), scale)
    assert np.abs(oracle.attention_values(swapped, v, heads) - got).max() > 1e-3
    # ...and a mask one column too wide.
    z = scale * oracle.attention_scores(q, k, heads)
    wide = oracle.softmax(np.where(np.triu(np.ones((seq, seq), bool), 2), -np.inf, z))
    assert np.abs(oracle.attention_values(wide, v, heads) - got).max() > 1e-3


def test_values_ignore_the_upper_triangle():
    r = rng(5)
    v = r.standard_normal((1, 6, 4))
    probs = np.tril(r.random((1, 2, 6, 6)))
    poisoned = probs + np.triu(np.full((6, 6), 1e30), 1)
    np.testing.assert_array_equal(oracle.attention_values(poisoned, v, 2), oracle.attention_values(probs, v, 2))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ops_products_on_cpu_match_the_oracle(dtype):
    batch, seq, heads, d = 2, 24, 4, 16
    r = rng(11)
    q, k, v = (torch.from_numpy(r.standard_normal((batch, seq, heads * d)).astype(np.float32)).to(dtype)
               for _ in range(3))
    scores = ops.attention_scores_causal(q, k, heads)
    assert scores.shape == (batch, heads, seq, seq) and scores.dtype == dtype
    exact = oracle.attention_scores(q.float().numpy(), k.float().numpy(), heads)
    low = np.tril(np.ones((seq, seq), bool))
    # Relative tolerance plus a floor for dot products that cancel toward 0.
    tol, floor = (1e-5, 1e-6) if dtype == torch.float32 else (1e-2, 1e-3)
    got = scores.float().numpy()
    bound = tol * np.abs(exact) + floor * np.abs(exact).max()
    assert (np.abs(got - exact) <= bound)[..., low].all()
    probs = torch.softmax(scores.float() + torch.triu(torch.full((seq, seq), -math.inf), 1), -1).to(dtype)
    out = ops.attention_pv_causal(probs, v, heads)
    assert out.shape == v.shape and out.dtype == dtype
    want = oracle.attention_values(probs.float().numpy(), v.float().numpy(), heads)
    assert (np.abs(out.float().numpy() - want) <= tol * np.abs(want) + floor * np.abs(want).max()).all()


def test_ops_products_validate_shapes():
    x = torch.zeros(2, 8, 12)
    with pytest.raises(ValueError, match="not divisible"):
        ops.attention_scores_causal(x, x, 5)
    with pytest.raises(ValueError, match="differ in shape"):
        ops.attention_scores_causal(x, torch.zeros(2, 8, 6), 3)
    with pytest.raises(ValueError, match="probs must be"):
        ops.attention_pv_causal(torch.zeros(2, 3, 8, 7), x, 3)
    with pytest.raises(ValueError, match=r"\[batch, seq, hidden\]"):
        ops.attention_pv_causal(torch.zeros(2, 3, 8, 8), torch.zeros(8, 12), 3)

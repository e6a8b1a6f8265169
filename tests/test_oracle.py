"""Pin the CPU oracle before trusting it (no GPU needed).

How each oracle function is pinned:

* quantize/dequantize (C and numpy restatements): bit-exact against golden
  vectors produced by the reference's own compiled CPU operators
  (tests/golden/quant_*.npz, see make_golden.py), bit-exact against an
  in-process ATen composition on 1M random values with outliers, and against
  each other. Planted mistakes (reciprocal multiply, the CUDA-style guard,
  half-away rounding, a NaN-dropping absmax, scale / 128) each fail a golden
  case, so the goldens can tell them apart.
* bf16 / fp16 conversions: against torch's bf16 conversion and numpy's
  float16 on random values, specials and every half value.
* rmsnorm, softmax, lora_linear, the activations, the fused residual norm and
  the sum: float64 restatements against golden outputs of the reference's
  CPU operators, plus closed forms (unit input -> weight, rows sum to one,
  B = 0 -> x @ w, linearity in scale, exact sum of ones) and planted mistakes
  (eps outside the sqrt, mean -> sum, missing weight, missing max shift,
  transposed operand, missing scale).
* lora_backward: against float64 torch autograd of the reference composition.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import quant as oq
from tests.conftest import load_golden, rng

QUANT_F32 = load_golden("quant_f32.npz")
QUANT_BF16 = load_golden("quant_bf16.npz")


# ---------------------------------------------------------------------------
# Quantisation.
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("case", sorted(QUANT_F32))
def test_c_oracle_matches_the_reference_quantiser_bit_for_bit(case):
    data = QUANT_F32[case]
    q, s = oracle.quantize_int8(data["x"])
    np.testing.assert_array_equal(q, data["q"])
    np.testing.assert_array_equal(s.view(np.uint32), data["s"].view(np.uint32))


@pytest.mark.parametrize("case", sorted(QUANT_F32))
def test_numpy_oracle_matches_the_reference_quantiser_bit_for_bit(case):
    data = QUANT_F32[case]
    q, s = oracle.quantize_int8_numpy(data["x"])
    np.testing.assert_array_equal(q, data["q"])
    np.testing.assert_array_equal(s.view(np.uint32), data["s"].view(np.uint32))


@pytest.mark.parametrize("case", sorted(QUANT_F32))
def test_c_oracle_dequantises_like_the_reference(case):
    data = QUANT_F32[case]
    deq = oracle.dequantize_int8(data["q"], data["s"])
    ref = data["deq"]
    same = (deq.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(deq) & np.isnan(ref))
    assert same.all()


@pytest.mark.parametrize("case", sorted(QUANT_BF16))
def test_bf16_quantisation_matches_the_reference(case):
    data = QUANT_BF16[case]
    q, s = oracle.quantize_int8(data["x"], "bf16")
    np.testing.assert_array_equal(q, data["q"])
    np.testing.assert_array_equal(s.view(np.uint32), data["s"].view(np.uint32))


def _aten_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The reference formula in ATen (an independent vectorised implementation)."""
    t = torch.from_numpy(x).reshape(-1).float()
    pad = (-t.numel()) % 64
    g = torch.nn.functional.pad(t, (0, pad)).view(-1, 64)
    s = g.abs().amax(dim=1) / 127.0
    s = torch.where(s > 0, s, torch.ones_like(s))
    q = torch.clamp(torch.round(g / s.unsqueeze(1)), -127, 127).reshape(-1)[: t.numel()]
    return q.to(torch.int8).numpy(), s.numpy()


def test_both_oracles_and_aten_agree_on_a_large_outlier_input():
    x = rng(1).standard_normal(1 << 20).astype(np.float32)
    idx = rng(2).choice(x.size, size=x.size // 100, replace=False)
    x[idx] *= 20.0
    q_c, s_c = oracle.quantize_int8(x)
    q_n, s_n = oracle.quantize_int8_numpy(x)
    q_t, s_t = _aten_quantize(x)
    np.testing.assert_array_equal(q_c, q_t)
    np.testing.assert_array_equal(q_n, q_t)
    np.testing.assert_array_equal(s_c.view(np.uint32), s_t.view(np.uint32))
    np.testing.assert_array_equal(s_n.view(np.uint32), s_t.view(np.uint32))


def test_round_trip_error_is_at_most_half_a_step():
    # Property from tests/python/test_ops.py:174-181.
    x = rng(3).standard_normal(100_003).astype(np.float32) * 5
    q, s = oracle.quantize_int8(x)
    back = oracle.dequantize_int8(q, s)
    step = np.repeat(s, 64)[: x.size]
    assert (np.abs(x - back) <= step / 2 + 1e-6).all()
    assert q.min() >= -127 and q.max() <= 127


def test_the_block_maximum_maps_to_127_and_zero_blocks_get_scale_one():
    x = np.full(128, 0.1, np.float32)
    x[5] = 4.0
    x[64:] = 0.0
    q, s = oracle.quantize_int8(x)
    assert q[5] == 127 and s[1] == 1.0 and (q[64:] == 0).all()


def test_fake_quantisation_equals_quantise_then_dequantise():
    x = rng(4).standard_normal(10_000).astype(np.float32) * 3
    q, s = oracle.quantize_int8(x)
    np.testing.assert_array_equal(
        oracle.quantize_dequantize(x).view(np.uint32), oracle.dequantize_int8(q, s).view(np.uint32)
    )


# Planted mistakes: each must disagree with at least one golden case.


def _variant_reciprocal(x):
    flat = x.reshape(-1)
    g = np.concatenate([flat, np.zeros((-flat.size) % 64, np.float32)]).reshape(-1, 64)
    with np.errstate(all="ignore"):
        s = np.abs(g).max(axis=1) / np.float32(127)
        s = np.where(s > 0, s, np.float32(1)).astype(np.float32)
        q = np.rint(g * (np.float32(1) / s)[:, None])
        q = np.where(np.isnan(q), 0, np.clip(q, -127, 127)).astype(np.int8)
    return q.reshape(-1)[: flat.size], s


def _variant_cuda_guard(x):
    flat = x.reshape(-1)
    g = np.concatenate([flat, np.zeros((-flat.size) % 64, np.float32)]).reshape(-1, 64)
    with np.errstate(all="ignore"):
        absmax = np.abs(g).max(axis=1)
        s = np.where(absmax > 0, absmax / np.float32(127), np.float32(1)).astype(np.float32)
        q = np.rint(g / s[:, None])
        q = np.where(np.isnan(q), 0, np.clip(q, -127, 127)).astype(np.int8)
    return q.reshape(-1)[: flat.size], s


def _variant_half_away(x):
    q, s = oracle.quantize_int8_numpy(x)
    flat = x.reshape(-1)
    with np.errstate(all="ignore"):
        v = flat / np.repeat(s, 64)[: flat.size]
        r = np.sign(v) * np.floor(np.abs(v) + 0.5)
        r = np.where(np.isnan(r), 0, np.clip(r, -127, 127)).astype(np.int8)
    return r, s


def _variant_nan_dropping_max(x):
    flat = x.reshape(-1)
    g = np.concatenate([flat, np.zeros((-flat.size) % 64, np.float32)]).reshape(-1, 64)
    with np.errstate(all="ignore"):
        s = np.nanmax(np.abs(g), axis=1) / np.float32(127)
        s = np.where(s > 0, s, np.float32(1)).astype(np.float32)
        q = np.rint(g / s[:, None])
        q = np.where(np.isnan(q), 0, np.clip(q, -127, 127)).astype(np.int8)
    return q.reshape(-1)[: flat.size], s


def _variant_128(x):
    flat = x.reshape(-1)
    g = np.concatenate([flat, np.zeros((-flat.size) % 64, np.float32)]).reshape(-1, 64)
    with np.errstate(all="ignore"):
        s = np.abs(g).max(axis=1) / np.float32(128)
        s = np.where(s > 0, s, np.float32(1)).astype(np.float32)
        q = np.rint(g / s[:, None])
        q = np.where(np.isnan(q), 0, np.clip(q, -127, 127)).astype(np.int8)
    return q.reshape(-1)[: flat.size], s


@pytest.mark.parametrize(
    "variant",
    [_variant_reciprocal, _variant_cuda_guard, _variant_half_away, _variant_nan_dropping_max, _variant_128],
)
def test_a_planted_quantiser_mistake_is_caught_by_the_goldens(variant):
    mismatched = []
    for name, data in QUANT_F32.items():
        q, s = variant(data["x"])
        if not (np.array_equal(q, data["q"]) and np.array_equal(s.view(np.uint32), data["s"].view(np.uint32))):
            mismatched.append(name)
    assert mismatched, f"{variant.__name__} agrees with every golden case"


# ---------------------------------------------------------------------------
# 16-bit conversions.
# ---------------------------------------------------------------------------


def _special_floats() -> np.ndarray:
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, 6e-5, 6.1e-5, 3.4e38, 1e-40,
            np.inf, -np.inf, np.nan]
    return np.array(vals, dtype=np.float32)


def test_bf16_rounding_matches_torch():
    x = np.concatenate([rng(5).standard_normal(200_000).astype(np.float32) * 100, _special_floats()])
    ours = oracle.f32_to_bf16_bits(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().astype(np.uint16)
    nan = np.isnan(x)
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])
    assert (ours[nan] == 0x7FC0).all()


def test_c_bf16_rounding_matches_the_numpy_one():
    x = rng(6).standard_normal(100_000).astype(np.float32)
    deq_bits = oracle.dequantize_int8(*oracle.quantize_int8(x), dtype="bf16")
    deq32 = oracle.dequantize_int8(*oracle.quantize_int8(x))
    np.testing.assert_array_equal(deq_bits, oracle.f32_to_bf16_bits(deq32))


def test_f16_conversions_match_numpy():
    x = np.concatenate([rng(7).standard_normal(200_000).astype(np.float32) * 1000,
                        rng(8).standard_normal(10_000).astype(np.float32) * 1e-6, _special_floats()])
    ours = oq.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        theirs = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])
    every_half = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    widened = oq.f16_bits_to_f32(every_half)
    expected = every_half.view(np.float16).astype(np.float32)
    finite = ~np.isnan(expected)
    np.testing.assert_array_equal(widened[finite].view(np.uint32), expected[finite].view(np.uint32))


# ---------------------------------------------------------------------------
# Floating-point ops.
# ---------------------------------------------------------------------------

RMSNORM = load_golden("rmsnorm.npz")
SOFTMAX = load_golden("softmax.npz")
LORA = load_golden("lora.npz")
MISC = load_golden("misc.npz")


def _bf16(bits: np.ndarray) -> np.ndarray:
    return oracle.bf16_bits_to_f32(bits).astype(np.float64)


def _assert_within_one_bf16_ulp(expected64: np.ndarray, got_bits: np.ndarray) -> None:
    got = _bf16(got_bits)
    ulp = np.abs(expected64) * 2.0**-7 + 1e-30
    assert (np.abs(got - expected64) <= ulp).all()


@pytest.mark.parametrize("case", sorted(RMSNORM))
def test_rmsnorm_oracle_matches_the_reference(case):
    d = RMSNORM[case]
    if case.startswith("bf16"):
        y = oracle.rmsnorm(_bf16(d["x"]), _bf16(d["w"]), 1e-6)
        _assert_within_one_bf16_ulp(y, d["y"])
    else:
        y = oracle.rmsnorm(d["x"], d["w"], 1e-6)
        np.testing.assert_allclose(d["y"], y, rtol=1e-5, atol=1e-6)


def test_rmsnorm_closed_forms():
    ones = np.ones((4, 32))
    np.testing.assert_allclose(oracle.rmsnorm(ones, np.ones(32), 0.0), ones)
    x = rng(9).standard_normal((4, 128))
    np.testing.assert_allclose(oracle.rmsnorm(x, np.ones(128), 1e-12), oracle.rmsnorm(10 * x, np.ones(128), 1e-12), rtol=1e-9)


@pytest.mark.parametrize("mistake", ["eps_outside", "sum_not_mean", "no_weight"])
def test_a_planted_rmsnorm_mistake_is_caught(mistake):
    d = RMSNORM["f32_33x1023"]
    x = d["x"].astype(np.float64)
    w = d["w"].astype(np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    if mistake == "eps_outside":
        # Only visible when eps is comparable to mean(x^2): scale the row down.
        x = x * 1e-4
        ref = oracle.rmsnorm(x, w, 1e-6)
        bad = x / (np.sqrt(np.mean(x * x, axis=-1, keepdims=True)) + 1e-6) * w
        assert not np.allclose(bad, ref, rtol=1e-5)
        return
    bad = x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + 1e-6) * w if mistake == "sum_not_mean" else x / np.sqrt(ms + 1e-6)
    assert not np.allclose(bad, d["y"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("case", sorted(SOFTMAX))
def test_softmax_oracle_matches_the_reference(case):
    d = SOFTMAX[case]
    if case.startswith("bf16"):
        _assert_within_one_bf16_ulp(oracle.softmax(_bf16(d["x"])), d["y"])
    else:
        np.testing.assert_allclose(d["y"], oracle.softmax(d["x"]), rtol=1e-5, atol=1e-7)


def test_softmax_closed_forms_and_planted_mistakes():
    x = rng(10).standard_normal((16, 128))
    p = oracle.softmax(x)
    np.testing.assert_allclose(p.sum(axis=-1), 1.0, rtol=1e-12)
    np.testing.assert_allclose(oracle.softmax(x + 12.5), p, rtol=1e-12)
    extreme = SOFTMAX["extreme"]
    with np.errstate(all="ignore"):
        naive = np.exp(extreme["x"].astype(np.float32))
        naive = naive / naive.sum(axis=-1, keepdims=True)
    assert not np.allclose(naive, extreme["y"], equal_nan=False)
    d = SOFTMAX["f32_8x256"]
    wrong_axis = np.exp(d["x"] - d["x"].max(axis=0)) / np.exp(d["x"] - d["x"].max(axis=0)).sum(axis=0)
    assert not np.allclose(wrong_axis, d["y"], rtol=1e-5)


@pytest.mark.parametrize("case", sorted(LORA))
def test_lora_oracle_matches_the_reference(case):
    d = LORA[case]
    if case.startswith("bf16"):
        y = oracle.lora_linear(_bf16(d["x"]), _bf16(d["w"]), _bf16(d["a"]), _bf16(d["b"]), 2.0, True)
        got = _bf16(d["y"])
        # The reference rounds four intermediates to bf16; compare at the
        # output's scale.
        assert np.max(np.abs(got - y)) <= 1e-2 * np.max(np.abs(y))
    else:
        y = oracle.lora_linear(d["x"], d["w"], d["a"], d["b"], 0.25, False)
        np.testing.assert_allclose(d["y"], y, rtol=1e-4, atol=1e-4 * np.abs(y).max())


def test_lora_closed_forms_and_planted_mistakes():
    g = rng(11)
    x, w = g.standard_normal((4, 32)), g.standard_normal((32, 16))
    a, b = g.standard_normal((32, 4)), g.standard_normal((4, 16))
    np.testing.assert_allclose(oracle.lora_linear(x, w, a, np.zeros((4, 16)), 1.0, False), x @ w)
    zero_w = np.zeros_like(w)
    np.testing.assert_allclose(
        oracle.lora_linear(x, zero_w, a, b, 2.0, False), 2 * oracle.lora_linear(x, zero_w, a, b, 1.0, False)
    )
    d = LORA["f32_16x256x256r16"]
    no_scale = d["x"] @ d["w"] + (d["x"] @ d["a"]) @ d["b"]
    transposed = d["x"] @ d["w"].T + 0.25 * ((d["x"] @ d["a"]) @ d["b"])
    assert not np.allclose(no_scale, d["y"], rtol=1e-4)
    assert not np.allclose(transposed, d["y"], rtol=1e-4)


def test_lora_backward_matches_float64_autograd():
    g = rng(12)
    x = torch.from_numpy(g.standard_normal((24, 40)))
    w = torch.from_numpy(g.standard_normal((40, 12)))
    a = torch.from_numpy(g.standard_normal((40, 5))).requires_grad_()
    b = torch.from_numpy(g.standard_normal((5, 12))).requires_grad_()
    dy = torch.from_numpy(g.standard_normal((24, 12)))
    y = x @ w + 0.5 * ((x @ a) @ b)
    y.backward(dy)
    xa = (x @ a).detach().numpy()
    grad_a, grad_b = oracle.lora_backward(x.numpy(), dy.numpy(), b.detach().numpy(), xa, 0.5, False)
    np.testing.assert_allclose(grad_a, a.grad.numpy(), rtol=1e-10)
    np.testing.assert_allclose(grad_b, b.grad.numpy(), rtol=1e-10)
    # A dropped scale or a swapped operand is visible.
    assert not np.allclose(grad_a / 0.5, a.grad.numpy())


def test_sum_oracle_matches_the_reference():
    for name, d in MISC.items():
        if not name.startswith("sum_"):
            continue
        exact = oracle.sum_exact(d["x"])
        tol = max(abs(exact), 1.0) * 1e-5 * math.sqrt(d["x"].size)
        assert abs(float(d["y"]) - exact) <= tol, name
    assert oracle.sum_exact(MISC["sum_ones"]["x"]) == 100_000.0


def test_activation_oracles_match_the_reference():
    np.testing.assert_allclose(MISC["silu"]["y"], oracle.silu(MISC["silu"]["x"]), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(MISC["gelu"]["y"], oracle.gelu_tanh(MISC["gelu"]["x"]), rtol=1e-5, atol=1e-6)
    sw = MISC["swiglu"]
    np.testing.assert_allclose(sw["y"], oracle.swiglu(sw["x"], sw["up"]), rtol=1e-5, atol=1e-6)
    exact_gelu = 0.5 * MISC["gelu"]["x"] * (1 + np.vectorize(math.erf)(MISC["gelu"]["x"] / math.sqrt(2)))
    assert not np.allclose(exact_gelu, MISC["gelu"]["y"], rtol=1e-5, atol=1e-6)


def test_fused_residual_rmsnorm_is_the_sum_then_rmsnorm():
    d = MISC["frn"]
    summed = d["x"] + d["res"]
    np.testing.assert_array_equal(summed, d["sum"])
    np.testing.assert_allclose(d["y"], oracle.rmsnorm(summed, d["w"], 1e-6), rtol=1e-5, atol=1e-6)

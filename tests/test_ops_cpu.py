"""The Python drop-in surface on CPU: the reference's operator tests, restated.

These mirror tests/python/test_ops.py, test_autograd.py and
test_constant_parity.py of the reference against cuda_force_amd.ops: the
same validation messages, shapes, fallbacks and properties, on CPU tensors
(dispatcher CPU key = the reference's ATen implementations). GPU behaviour is
in tests/test_gpu_ops.py.
"""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

import cuda_force_amd as cf
from cuda_force_amd import ops

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("shape", [(1, 1), (1, 64), (3, 17), (8, 128), (2, 4096), (33, 1023)])
def test_rmsnorm_matches_the_explicit_formula(shape):
    x = torch.randn(*shape)
    w = torch.randn(shape[-1])
    expected = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * w
    torch.testing.assert_close(cf.rmsnorm(x, w, 1e-6), expected, rtol=1e-5, atol=1e-6)


def test_rmsnorm_validation_messages():
    with pytest.raises(ValueError, match="does not match"):
        cf.rmsnorm(torch.randn(2, 8), torch.randn(16))
    with pytest.raises(ValueError, match="1-D"):
        cf.rmsnorm(torch.randn(2, 8), torch.randn(2, 8))


def test_rmsnorm_non_contiguous_and_half_precision():
    x = torch.randn(64, 4).t()
    assert not x.is_contiguous()
    w = torch.randn(64)
    torch.testing.assert_close(cf.rmsnorm(x, w), cf.rmsnorm(x.contiguous(), w))
    for dtype in (torch.float16, torch.bfloat16):
        big = torch.full((2, 64), 300.0, dtype=dtype)
        out = cf.rmsnorm(big, torch.ones(64, dtype=dtype))
        assert out.dtype == dtype and torch.isfinite(out).all()
        torch.testing.assert_close(out.float(), torch.ones(2, 64), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("shape", [(1, 1), (1, 32), (4, 17), (8, 256), (3, 1025)])
def test_softmax_matches_torch(shape):
    x = torch.randn(*shape)
    torch.testing.assert_close(cf.softmax(x), torch.softmax(x, dim=-1))


def test_softmax_stability_and_shift_invariance():
    x = torch.tensor([[1000.0, 1000.0, 1000.0], [-1000.0, 0.0, 1000.0]])
    out = cf.softmax(x)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out[0], torch.full((3,), 1 / 3), rtol=1e-5, atol=1e-6)
    y = torch.randn(4, 64)
    torch.testing.assert_close(cf.softmax(y), cf.softmax(y + 12.5), rtol=1e-5, atol=1e-6)
    assert cf.softmax_as(y.bfloat16(), torch.float32).dtype == torch.float32


def test_softmax_scaled_is_the_causal_attention_softmax():
    """softmax_scaled(s, scale, seq) on [batch * heads * seq, seq] scores equals
    softmax(scores * scale + causal) as examples/transformer_block.py:57-59
    composes it (per head block: row i keeps columns 0..i)."""
    batch_heads, seq = 3, 16
    scores = torch.randn(batch_heads, seq, seq) * 4
    causal = torch.triu(torch.full((seq, seq), float("-inf")), 1)
    expected = torch.softmax(scores * 0.125 + causal, dim=-1)
    got = cf.softmax_scaled(scores.reshape(-1, seq), 0.125, seq).view(batch_heads, seq, seq)
    torch.testing.assert_close(got, expected, rtol=1e-6, atol=1e-7)
    assert (got[:, 0, 1:] == 0).all() and torch.equal(got[:, 0, 0], torch.ones(batch_heads))
    # No mask: a scaled softmax; output dtype selectable; bad period refused.
    torch.testing.assert_close(cf.softmax_scaled(scores, 2.0), torch.softmax(2.0 * scores, dim=-1))
    assert cf.softmax_scaled(scores.bfloat16(), 1.0, seq, torch.float32).dtype == torch.float32
    with pytest.raises(ValueError, match="causal_period"):
        cf.softmax_scaled(scores, 1.0, -1)


@pytest.mark.parametrize(("batch", "k", "n", "r"), [(1, 8, 4, 2), (4, 64, 32, 8), (7, 129, 65, 3), (16, 256, 256, 16)])
def test_lora_linear_matches_the_definition(batch, k, n, r):
    x, w = torch.randn(batch, k), torch.randn(k, n)
    a, b = torch.randn(k, r), torch.randn(r, n)
    expected = x @ w + 0.25 * ((x @ a) @ b)
    torch.testing.assert_close(cf.lora_linear(x, w, a, b, 0.25), expected, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize(
    ("shapes", "message"),
    [
        ({"x": (4, 31), "w": (32, 16), "a": (32, 4), "b": (4, 16)}, "input features"),
        ({"x": (4, 32), "w": (32, 16), "a": (31, 4), "b": (4, 16)}, "lora_a"),
        ({"x": (4, 32), "w": (32, 16), "a": (32, 4), "b": (5, 16)}, "lora_b"),
        ({"x": (4, 32), "w": (32, 16), "a": (32, 4), "b": (4, 15)}, "lora_b"),
    ],
)
def test_lora_rejects_mismatched_shapes(shapes, message):
    with pytest.raises(ValueError, match=message):
        cf.lora_linear(*(torch.randn(*shapes[k]) for k in "xwab"))


def test_lora_zero_b_and_linear_scale_and_peft_layout():
    x, w, a = torch.randn(4, 32), torch.randn(32, 16), torch.randn(32, 4)
    torch.testing.assert_close(cf.lora_linear(x, w, a, torch.zeros(4, 16), 1.0), x @ w, rtol=1e-5, atol=1e-5)
    b = torch.randn(4, 16)
    zero_w = torch.zeros(32, 16)
    torch.testing.assert_close(cf.lora_linear(x, zero_w, a, b, 2.0), 2 * cf.lora_linear(x, zero_w, a, b, 1.0),
                               rtol=1e-4, atol=1e-4)
    # PEFT layout (W [out, in], A [r, in], B [out, r]) maps to op(x, W^T, A^T, B^T, alpha / r).
    W, A, B = torch.randn(16, 32), torch.randn(8, 32), torch.randn(16, 8)
    peft = x @ W.t() + 2.0 * (x @ A.t() @ B.t())
    torch.testing.assert_close(cf.lora_linear(x, W.t().contiguous(), A.t().contiguous(), B.t().contiguous(), 2.0),
                               peft, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("size", [1, 63, 64, 65, 1000, 4096])
def test_sum_reduce_matches_torch(size):
    x = torch.randn(size)
    torch.testing.assert_close(cf.sum_reduce(x), x.sum(), rtol=1e-4, atol=1e-4)


def test_sum_of_empty_is_zero_and_row_sum():
    assert cf.sum_reduce(torch.empty(0)).item() == 0.0
    m = torch.randn(5, 7)
    torch.testing.assert_close(cf.row_sum(m), m.sum(-1))


@pytest.mark.parametrize("size", [1, 63, 64, 65, 128, 1000])
def test_quantisation_round_trip_bound(size):
    x = torch.randn(size) * 5.0
    q, s = cf.quantize_int8(x)
    back = cf.dequantize_int8(q, s)
    assert (x - back).abs().max().item() <= s.max().item() / 2 + 1e-6


def test_quantisation_range_shape_zero_block_and_outlier():
    q, _ = cf.quantize_int8(torch.randn(1000) * 100)
    assert q.min() >= -127 and q.max() <= 127
    x = torch.randn(7, 33)
    q, s = cf.quantize_int8(x)
    assert q.shape == x.shape and s.numel() == (x.numel() + 63) // 64
    z = torch.zeros(128)
    q, s = cf.quantize_int8(z)
    assert (s > 0).all()
    torch.testing.assert_close(cf.dequantize_int8(q, s), z)
    y = torch.full((256,), 0.5)
    y[0] = 1000.0
    q, s = cf.quantize_int8(y)
    back = cf.dequantize_int8(q, s)
    assert (y[1] - back[1]).abs() > (y[200] - back[200]).abs()
    torch.testing.assert_close(back[0], y[0])


def test_dequantize_validation_and_dtypes():
    q, s = cf.quantize_int8(torch.randn(128))
    with pytest.raises(ValueError, match="block scales"):
        cf.dequantize_int8(q, torch.ones(1))
    assert cf.dequantize_int8(q, s, dtype=torch.bfloat16).dtype == torch.bfloat16
    x = torch.randn(512)
    torch.testing.assert_close(cf.quantization_error(x), (x - cf.dequantize_int8(*cf.quantize_int8(x))).abs().max())
    torch.testing.assert_close(cf.fake_quantize_int8(x), cf.dequantize_int8(*cf.quantize_int8(x)))


def test_activations_and_fused_norm():
    x = torch.randn(8, 4096)
    torch.testing.assert_close(cf.silu(x), torch.nn.functional.silu(x))
    torch.testing.assert_close(cf.gelu(x), torch.nn.functional.gelu(x, approximate="tanh"), rtol=1e-5, atol=1e-6)
    up = torch.randn_like(x)
    torch.testing.assert_close(cf.swiglu(x, up), torch.nn.functional.silu(x) * up, rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="same shape"):
        cf.swiglu(torch.randn(4, 8), torch.randn(4, 16))
    with pytest.raises(ValueError, match="same dtype"):
        cf.swiglu(torch.randn(8), torch.randn(8, dtype=torch.float64))
    res = torch.randn_like(x)
    w = torch.randn(4096)
    normed, summed = cf.fused_residual_rmsnorm(x, res, w)
    torch.testing.assert_close(summed, x + res)
    torch.testing.assert_close(normed, cf.rmsnorm(x + res, w), rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="same shape"):
        cf.fused_residual_rmsnorm(torch.randn(4, 8), torch.randn(4, 16), torch.ones(8))
    with pytest.raises(ValueError, match="weight"):
        cf.fused_residual_rmsnorm(torch.randn(4, 8), torch.randn(4, 8), torch.ones(16))
    assert cf.silu(torch.empty(0)).numel() == 0


def test_backend_report_and_dtype_support():
    report = cf.backend_report()
    assert report.extension_loaded and report.cuda_compiled
    assert report.using_custom_kernels == torch.cuda.is_available()
    assert "cudaforge" in str(report)
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        assert cf.kernel_supports(dtype)
    assert not cf.kernel_supports(torch.float64) and not cf.kernel_supports(torch.int8)


# --- autograd (reference tests/python/test_autograd.py) ------------------------


def test_differentiating_a_registered_operator_raises():
    x = torch.randn(8, requires_grad=True)
    with pytest.raises(RuntimeError, match="derivative for cudaforge::silu is not implemented"):
        torch.ops.cudaforge.silu(x).sum().backward()


def test_fused_residual_rmsnorm_is_not_guarded_like_the_reference():
    # The reference leaves fused_residual_rmsnorm off its guard list
    # (cpp/src/bindings.cpp:373-374); so does this build.
    x = torch.randn(2, 8, requires_grad=True)
    torch.ops.cudaforge.fused_residual_rmsnorm(x, torch.randn(2, 8), torch.ones(8), 1e-6)


@pytest.mark.parametrize("call", [cf.silu, cf.gelu, cf.softmax, cf.sum_reduce])
def test_the_python_wrappers_are_differentiable(call):
    x = torch.randn(4, 16, requires_grad=True)
    call(x).sum().backward()
    assert x.grad is not None and torch.isfinite(x.grad).all()


def test_a_gradient_on_the_adapter_routes_to_a_differentiable_path():
    x, w = torch.randn(4, 32), torch.randn(32, 16)
    a = torch.randn(32, 4, requires_grad=True)
    b = torch.randn(4, 16, requires_grad=True)
    cf.lora_linear(x, w, a, b, 2.0).sum().backward()
    assert a.grad is not None and b.grad is not None


def test_gradcheck_on_the_reference_path():
    x = torch.randn(6, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(cf.silu, (x,), eps=1e-6, atol=1e-4)


# --- GPU policy, exercised with a stand-in tensor ---------------------------------


class _FakeGpuTensor:
    is_cuda = True
    requires_grad = False
    dtype = torch.float32
    shape = (2, 2)


def test_a_missing_extension_raises_for_gpu_inputs(monkeypatch):
    monkeypatch.setattr(ops, "_EXTENSION_LOADED", False)
    with pytest.raises(ops.ExtensionMissingError, match="refusing to fall back"):
        ops._dispatch_available("rmsnorm", _FakeGpuTensor())


def test_strict_mode_turns_a_gpu_fallback_into_an_error(monkeypatch):
    monkeypatch.setenv("CUDAFORGE_STRICT", "1")
    with pytest.raises(NotImplementedError, match="no HIP kernel"):
        ops._refuse_gpu_fallback("softmax", _FakeGpuTensor())
    monkeypatch.setenv("CUDAFORGE_STRICT", "0")
    with pytest.warns(RuntimeWarning, match="PyTorch composition"):
        ops._refuse_gpu_fallback("softmax", _FakeGpuTensor())


# --- constant parity (reference tests/python/test_constant_parity.py) -----------


def _constant(path: Path, name: str) -> int:
    match = re.search(rf"inline\s+constexpr\s+\w+\s+{re.escape(name)}\s*=\s*(\d+)\s*;", path.read_text())
    assert match, f"{name} not found in {path}"
    return int(match.group(1))


def test_block_size_agrees_across_languages():
    header = ROOT / "cuda_force_amd" / "csrc" / "cf_common.hpp"
    assert _constant(header, "kQuantBlockSize") == cf.QUANT_BLOCK_SIZE == 64
    assert re.search(r"#define CF_QUANT_BLOCK_SIZE 64\b", (ROOT / "include" / "cudaforge_hip.h").read_text())


def test_the_wave_size_is_sixty_four():
    header = ROOT / "cuda_force_amd" / "csrc" / "cf_common.hpp"
    wave = _constant(header, "kWaveSize")
    assert wave == 64
    block = _constant(header, "kDefaultBlockSize")
    assert block % wave == 0 and block <= _constant(header, "kMaxBlockSize")

"""The drop-in boundary on a GPU: torch.ops.cudaforge.* and cuda_force_amd.ops.

Checks that the dispatcher's CUDA-key implementations are the HIP kernels (their
results equal the C ABI's bit for bit), that launches follow PyTorch's current
stream, that the autograd guard raises as the reference's does, and that
lora_linear's training path produces the reference's gradients.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import cuda_force_amd as cf
from cuda_force_amd import ops
from tests import gpu_util as g
from tests.conftest import rng

pytestmark = pytest.mark.gpu


def test_the_backend_report_names_the_hip_kernels():
    report = cf.backend_report()
    assert report.using_custom_kernels, str(report)
    assert cf.CUDA_KERNELS_AVAILABLE


def test_dispatcher_quantise_equals_the_c_abi():
    x = torch.randn(4096, 333, device=g.DEVICE)
    q, s = torch.ops.cudaforge.quantize_int8(x)
    q2 = g.empty(x.numel(), torch.int8)
    s2 = g.poison_like(s)
    g.call("cf_quantize_int8", x.data_ptr(), g.cf("f32"), q2.data_ptr(), s2.data_ptr(), x.numel(), g.stream())
    torch.cuda.synchronize()
    assert q.shape == x.shape and s.shape == ((x.numel() + 63) // 64,)
    assert torch.equal(q.reshape(-1), q2) and torch.equal(s, s2)
    back = torch.ops.cudaforge.dequantize_int8(q, s)
    assert back.dtype == torch.float32 and back.shape == x.shape


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_ops_dispatch_every_kernel_dtype(dtype):
    x = torch.randn(64, 512, device=g.DEVICE, dtype=dtype)
    w = torch.randn(512, device=g.DEVICE, dtype=dtype)
    y = ops.rmsnorm(x, w)
    ref = ops._rmsnorm_reference(x.float(), w.float(), 1e-6)
    torch.testing.assert_close(y.float(), ref, rtol=1e-2 if dtype != torch.float32 else 1e-5, atol=1e-3)
    p = ops.softmax(x)
    torch.testing.assert_close(p.float(), torch.softmax(x.float(), -1), rtol=1e-2, atol=1e-3)
    q, s = ops.quantize_int8(x)
    assert q.dtype == torch.int8
    d = ops.dequantize_int8(q, s, dtype=dtype)
    assert d.dtype == dtype
    assert (x.float() - d.float()).abs().max() <= s.max() / 2 + 1e-2


def test_ops_accept_batched_inputs():
    x = torch.randn(2, 3, 256, device=g.DEVICE, dtype=torch.bfloat16)
    w = torch.ones(256, device=g.DEVICE, dtype=torch.bfloat16)
    assert ops.rmsnorm(x, w).shape == x.shape
    assert ops.softmax(x).shape == x.shape
    wt = torch.randn(256, 128, device=g.DEVICE, dtype=torch.bfloat16) * 0.02
    a = torch.randn(256, 16, device=g.DEVICE, dtype=torch.bfloat16) / 64
    b = torch.randn(16, 128, device=g.DEVICE, dtype=torch.bfloat16) * 0.02
    assert ops.lora_linear(x, wt, a, b, 2.0).shape == (2, 3, 128)


def test_kernels_run_on_the_current_stream():
    side = torch.cuda.Stream()
    x = torch.randn(2048, 4096, device=g.DEVICE, dtype=torch.bfloat16)
    w = torch.ones(4096, device=g.DEVICE, dtype=torch.bfloat16)
    expected = ops.rmsnorm(x, w)
    torch.cuda.synchronize()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        out = ops.rmsnorm(x, w)
        again = ops.rmsnorm(out, w)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(out, expected)
    torch.testing.assert_close(again.float(), ops.rmsnorm(expected, w).float())


def test_differentiating_a_registered_operator_raises_on_the_gpu():
    x = torch.randn(8, device=g.DEVICE, requires_grad=True)
    with pytest.raises(RuntimeError, match="derivative for cudaforge::silu is not implemented"):
        torch.ops.cudaforge.silu(x).sum().backward()


def test_sum_reduce_and_row_sum_on_the_gpu():
    x = torch.randn(1 << 20, device=g.DEVICE)
    s = ops.sum_reduce(x)
    assert s.shape == () and abs(s.item() - x.double().sum().item()) < 1e-2
    m = torch.randn(17, 300, device=g.DEVICE)
    torch.testing.assert_close(ops.row_sum(m), m.sum(-1), rtol=1e-4, atol=1e-4)


def test_activations_and_fused_norm_on_the_gpu():
    x = torch.randn(8, 4096, device=g.DEVICE)
    torch.testing.assert_close(ops.silu(x), torch.nn.functional.silu(x), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ops.gelu(x), torch.nn.functional.gelu(x, approximate="tanh"), rtol=1e-5, atol=1e-6)
    up = torch.randn_like(x)
    torch.testing.assert_close(ops.swiglu(x, up), torch.nn.functional.silu(x) * up, rtol=1e-5, atol=1e-6)
    res = torch.randn_like(x)
    w = torch.randn(4096, device=g.DEVICE)
    normed, summed = ops.fused_residual_rmsnorm(x, res, w)
    torch.testing.assert_close(summed, x + res)
    torch.testing.assert_close(normed, ops.rmsnorm(x + res, w), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_lora_training_path_matches_reference_autograd(dtype):
    gen = rng(77)
    m, k, n, r = 512, 256, 384, 16
    xs = torch.from_numpy(gen.standard_normal((m, k)).astype(np.float32)).to(dtype)
    ws = torch.from_numpy((0.02 * gen.standard_normal((k, n))).astype(np.float32)).to(dtype)
    as_ = torch.from_numpy((gen.standard_normal((k, r)) / 64).astype(np.float32)).to(dtype)
    bs = torch.from_numpy((0.02 * gen.standard_normal((r, n))).astype(np.float32)).to(dtype)
    dy = torch.from_numpy(gen.standard_normal((m, n)).astype(np.float32)).to(dtype)

    a_gpu = as_.to(g.DEVICE).requires_grad_()
    b_gpu = bs.to(g.DEVICE).requires_grad_()
    y = ops.lora_linear(xs.to(g.DEVICE), ws.to(g.DEVICE), a_gpu, b_gpu, 2.0)
    y.backward(dy.to(g.DEVICE))

    # Reference gradients in float32 on the CPU (the reference composition).
    a_ref = as_.float().requires_grad_()
    b_ref = bs.float().requires_grad_()
    y_ref = xs.float() @ ws.float() + 2.0 * ((xs.float() @ a_ref) @ b_ref)
    y_ref.backward(dy.float())
    tol = dict(rtol=1e-2, atol=1e-2) if dtype == torch.bfloat16 else dict(rtol=1e-4, atol=1e-4)
    scale_a = a_ref.grad.abs().max().item()
    scale_b = b_ref.grad.abs().max().item()
    torch.testing.assert_close(a_gpu.grad.float().cpu() / scale_a, a_ref.grad / scale_a, **tol)
    torch.testing.assert_close(b_gpu.grad.float().cpu() / scale_b, b_ref.grad / scale_b, **tol)
    scale_y = y_ref.abs().max().item()
    torch.testing.assert_close(y.detach().float().cpu() / scale_y, y_ref.detach() / scale_y, **tol)


def test_strict_mode_refuses_a_gpu_fallback():
    x = torch.randn(8, 8, device=g.DEVICE, dtype=torch.float64)
    with pytest.raises(NotImplementedError, match="no HIP kernel"):
        ops.softmax(x)


def test_attention_products_reject_mixed_devices_and_dtypes():
    """The dispatcher ops check devices and dtypes before any launch: a CPU k or
    v beside a GPU q or probs, and a k whose dtype differs from q's, raise
    RuntimeError (nothing is launched)."""
    q = torch.zeros(1, 8, 64, dtype=torch.bfloat16, device=g.DEVICE)
    probs = torch.zeros(1, 2, 8, 8, dtype=torch.bfloat16, device=g.DEVICE)
    with pytest.raises(RuntimeError, match="is on"):
        torch.ops.cudaforge.attention_scores_causal(q, q.cpu(), 2)
    with pytest.raises(RuntimeError, match="dtype"):
        torch.ops.cudaforge.attention_scores_causal(q, q.half(), 2)
    with pytest.raises(RuntimeError, match="is on"):
        torch.ops.cudaforge.attention_pv_causal(probs, q.cpu(), 2)
    with pytest.raises(RuntimeError, match="dtype"):
        torch.ops.cudaforge.attention_pv_causal(probs, q.half(), 2)
    torch.cuda.synchronize()

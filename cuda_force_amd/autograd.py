"""LoRA training path: an autograd function whose adapter gradients are HIP kernels.

The reference has no backward kernels: it guards the operator
(cpp/src/bindings.cpp:369-377) and sends any grad-requiring call to the ATen
composition ``x @ w + s * ((x @ a) @ b)`` (python/cudaforge/ops.py:125-153,
178-185). Here the forward is the fused HIP kernel, which also hands back the
adapter intermediate ``x @ a`` it computes anyway, and the backward computes

    grad_a = s * x^T (dy @ b^T)      [in, r]
    grad_b = s * (x @ a)^T dy        [r, out]

with HIP kernels (cf_lora_backward). These are the gradients ATen autograd
produces for the reference composition (tests/python/test_autograd.py:81-91).
The gradients of x and w, which a LoRA layer rarely needs (the base weight is
frozen; x needs one only below the first adapted layer), are plain GEMMs and
go to the vendor BLAS through torch.
"""

from __future__ import annotations

import torch


class _LoRALinearFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, lora_a, lora_b, scale):  # type: ignore[override]
        y, xa = torch.ops.cudaforge.lora_linear_fwd(x, weight, lora_a, lora_b, float(scale))
        ctx.save_for_backward(x, weight, lora_a, lora_b, xa)
        ctx.scale = float(scale)
        return y

    @staticmethod
    def backward(ctx, grad_y):  # type: ignore[override]
        x, weight, lora_a, lora_b, xa = ctx.saved_tensors
        grad_y = grad_y.contiguous()
        grad_x = grad_w = grad_a = grad_b = None
        if ctx.needs_input_grad[2] or ctx.needs_input_grad[3]:
            grad_a, grad_b = torch.ops.cudaforge.lora_linear_bwd(x, grad_y, lora_b, xa, ctx.scale)
        if ctx.needs_input_grad[0]:
            adapter = (grad_y @ lora_b.t()) @ lora_a.t()
            grad_x = grad_y @ weight.t() + ctx.scale * adapter
        if ctx.needs_input_grad[1]:
            grad_w = x.t() @ grad_y
        return grad_x, grad_w, grad_a, grad_b, None


def lora_linear_autograd(
    x: torch.Tensor, weight: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scale: float
) -> torch.Tensor:
    """Differentiable fused LoRA linear (op layout, 2-D contiguous operands)."""
    return _LoRALinearFunction.apply(x, weight, lora_a, lora_b, scale)

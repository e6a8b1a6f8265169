"""Public operators: the drop-in for ``cudaforge.ops``.

Same names, signatures, argument meaning, validation errors and fallback rules
as the reference module (python/cudaforge/ops.py:41-488). What changes is what
runs underneath: on a GPU tensor every operator here dispatches to
``torch.ops.cudaforge.*``, whose CUDA-key implementation calls the gfx950 HIP
kernels in ``libcudaforge_hip.so``.

Dispatch rules (reference ops.py:125-153, widened):

* GPU tensors go to the HIP kernels for float32, bfloat16 and float16 (the
  reference dispatches float32 only, so every bf16 configuration ran ATen).
  lora_linear takes float32 and bfloat16.
* If the compiled extension is missing, a GPU call raises instead of silently
  running PyTorch: a GPU result that did not come from these kernels is never
  returned. CPU tensors without the extension use the reference semantics in
  plain PyTorch, as the reference does.
* When a backward pass is expected, rmsnorm/softmax/sum/activations/quant take
  the differentiable PyTorch composition, as the reference does; lora_linear
  takes its own autograd function whose adapter gradients are HIP kernels
  (``cuda_force_amd.autograd``).
"""

from __future__ import annotations

import importlib.util
import logging
import os
import warnings
from dataclasses import dataclass

import torch

_LOG = logging.getLogger(__name__)

# Elements per quantisation scale; equals kQuantBlockSize in
# cuda_force_amd/csrc/cf_common.hpp and CF_QUANT_BLOCK_SIZE in the C header.
QUANT_BLOCK_SIZE = 64


def _load_extension() -> tuple[bool, bool, str]:
    """(extension_loaded, hip_kernels_compiled, explanation)."""
    if importlib.util.find_spec("cuda_force_amd._C") is None:
        return False, False, "extension not built; run cuda_force_amd.build"
    try:
        from cuda_force_amd import _C  # type: ignore[attr-defined]
    except ImportError as error:
        return False, False, f"extension present but failed to load: {error}"
    compiled = bool(getattr(_C, "cuda_kernels_available", lambda: False)())
    if compiled:
        return True, True, "extension loaded with HIP kernels for gfx950"
    return True, False, "extension loaded without HIP kernels"


_EXTENSION_LOADED, _CUDA_COMPILED, _LOAD_MESSAGE = _load_extension()

#: True when the HIP kernels are compiled in *and* a GPU is visible.
CUDA_KERNELS_AVAILABLE: bool = _CUDA_COMPILED and torch.cuda.is_available()

#: Storage dtypes with a HIP kernel path.
KERNEL_DTYPES: frozenset[torch.dtype] = frozenset({torch.float32, torch.float16, torch.bfloat16})

#: lora_linear's kernels cover these.
LORA_KERNEL_DTYPES: frozenset[torch.dtype] = frozenset({torch.float32, torch.bfloat16})

if not CUDA_KERNELS_AVAILABLE:
    _LOG.info("cuda_force_amd: %s", _LOAD_MESSAGE)


class ExtensionMissingError(RuntimeError):
    """A GPU tensor reached an operator whose HIP extension is not loaded."""


@dataclass(frozen=True)
class BackendReport:
    """Which backend serves GPU calls here, and the facts that decided it."""

    extension_loaded: bool
    cuda_compiled: bool
    cuda_device_available: bool
    device_name: str | None
    message: str

    @property
    def using_custom_kernels(self) -> bool:
        return self.extension_loaded and self.cuda_compiled and self.cuda_device_available

    def __str__(self) -> str:
        path = "custom HIP kernels" if self.using_custom_kernels else "PyTorch reference"
        return f"cudaforge: {path} on {self.device_name or 'cpu'} ({self.message})"


def kernel_supports(dtype: torch.dtype) -> bool:
    """True when a HIP kernel exists for this storage dtype."""
    return dtype in KERNEL_DTYPES


def backend_report() -> BackendReport:
    """Describe the active implementation path."""
    available = torch.cuda.is_available()
    return BackendReport(
        extension_loaded=_EXTENSION_LOADED,
        cuda_compiled=_CUDA_COMPILED,
        cuda_device_available=available,
        device_name=torch.cuda.get_device_name(0) if available else None,
        message=_LOAD_MESSAGE,
    )


def _needs_autograd(*tensors: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)


def _on_gpu(tensors: tuple[torch.Tensor, ...]) -> bool:
    return any(t.is_cuda for t in tensors)


def _require_extension(name: str, tensors: tuple[torch.Tensor, ...]) -> None:
    if _on_gpu(tensors) and not (_EXTENSION_LOADED and _CUDA_COMPILED):
        raise ExtensionMissingError(
            f"cudaforge.{name}: GPU tensors need the HIP extension ({_LOAD_MESSAGE}). "
            "Build it with `python -m cuda_force_amd.build`; refusing to fall back to PyTorch."
        )


def _dispatch_available(name: str, *tensors: torch.Tensor) -> bool:
    """True when torch.ops.cudaforge.<name> should handle these tensors."""
    _require_extension(name, tensors)
    if not _EXTENSION_LOADED:
        return False
    if not hasattr(torch.ops.cudaforge, name):
        return False
    if _needs_autograd(*tensors):
        return False
    if tensors and tensors[0].is_cuda:
        return _CUDA_COMPILED
    return True


def _same_dtype(*tensors: torch.Tensor) -> bool:
    return all(t.dtype == tensors[0].dtype for t in tensors)


# ---------------------------------------------------------------------------
# Reference semantics in plain PyTorch (CPU without the extension, and the
# differentiable path). These follow python/cudaforge/ops.py:164-240.
# ---------------------------------------------------------------------------


def _rmsnorm_reference(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    wide = x.float()
    inv_rms = torch.rsqrt(wide.pow(2).mean(dim=-1, keepdim=True) + eps)
    return ((wide * inv_rms) * weight.float()).to(x.dtype)


def _softmax_reference(x: torch.Tensor) -> torch.Tensor:
    return torch.softmax(x, dim=-1)


def _lora_linear_reference(
    x: torch.Tensor, weight: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scale: float
) -> torch.Tensor:
    return x @ weight + scale * ((x @ lora_a) @ lora_b)


def _fused_residual_rmsnorm_reference(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    summed = x + residual
    return _rmsnorm_reference(summed, weight, eps), summed


def _swiglu_reference(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    if gate.dtype in (torch.float16, torch.bfloat16):
        return (torch.nn.functional.silu(gate.float()) * up.float()).to(gate.dtype)
    return torch.nn.functional.silu(gate) * up


def _quantize_int8_reference(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    count = x.numel()
    flat = x.reshape(-1).float()
    pad = (-count) % QUANT_BLOCK_SIZE
    blocks = torch.nn.functional.pad(flat, (0, pad)).view(-1, QUANT_BLOCK_SIZE)
    scales = blocks.abs().amax(dim=1) / 127.0
    scales = torch.where(scales > 0, scales, torch.ones_like(scales))
    codes = torch.clamp(torch.round(blocks / scales.unsqueeze(1)), -127, 127)
    return codes.reshape(-1)[:count].to(torch.int8).view_as(x), scales


def _dequantize_int8_reference(quantised: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    count = quantised.numel()
    flat = quantised.reshape(-1).float()
    pad = (-count) % QUANT_BLOCK_SIZE
    blocks = torch.nn.functional.pad(flat, (0, pad)).view(-1, QUANT_BLOCK_SIZE)
    return (blocks * scales.unsqueeze(1)).reshape(-1)[:count].view_as(quantised)


# ---------------------------------------------------------------------------
# Public operators.
# ---------------------------------------------------------------------------


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Root-mean-square normalisation over the last dimension.

    ``y = x * rsqrt(mean(x^2) + eps) * weight`` in fp32, cast back to x's
    dtype. ``weight`` is ``[hidden]``; non-contiguous inputs are copied.

    Raises:
        ValueError: if ``weight`` is not 1-D or does not match the last dim.
    """
    if weight.ndim != 1:
        raise ValueError(f"weight must be 1-D, got shape {tuple(weight.shape)}")
    if x.shape[-1] != weight.shape[0]:
        raise ValueError(
            f"weight length {weight.shape[0]} does not match the last dimension "
            f"of x, which is {x.shape[-1]}"
        )
    if x.numel() == 0:
        return x.clone()
    x = x.contiguous()
    weight = weight.contiguous()
    if (
        _dispatch_available("rmsnorm", x, weight)
        and x.dtype in KERNEL_DTYPES
        and _same_dtype(x, weight)
    ):
        rows = x.reshape(-1, x.shape[-1])
        return torch.ops.cudaforge.rmsnorm(rows, weight, eps).view(x.shape)
    _refuse_gpu_fallback("rmsnorm", x, weight)
    return _rmsnorm_reference(x, weight, eps)


def softmax(x: torch.Tensor) -> torch.Tensor:
    """Row softmax over the last dimension (max-subtracted, fp32 arithmetic)."""
    if x.numel() == 0:
        return x.clone()
    x = x.contiguous()
    if _dispatch_available("softmax", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.softmax(x.reshape(-1, x.shape[-1])).view(x.shape)
    _refuse_gpu_fallback("softmax", x)
    return _softmax_reference(x)


def softmax_as(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Softmax over the last dim with the result in ``dtype`` (fp32 arithmetic).

    Not in the reference: lets bf16 logits produce fp32 probabilities in one
    pass (torch.softmax(x.float(), -1).to(dtype) otherwise)."""
    if x.numel() == 0:
        return x.to(dtype).clone()
    x = x.contiguous()
    if (
        _dispatch_available("softmax_as", x)
        and x.dtype in KERNEL_DTYPES
        and dtype in KERNEL_DTYPES
    ):
        return torch.ops.cudaforge.softmax_as(x.reshape(-1, x.shape[-1]), dtype).view(x.shape)
    _refuse_gpu_fallback("softmax_as", x)
    return torch.softmax(x.float(), dim=-1).to(dtype)


def _softmax_scaled_reference(x: torch.Tensor, scale: float, causal_period: int) -> torch.Tensor:
    rows = x.reshape(-1, x.shape[-1]).float() * scale
    if causal_period > 0:
        cols = torch.arange(rows.shape[1], device=x.device)[None, :]
        limit = (torch.arange(rows.shape[0], device=x.device) % causal_period)[:, None]
        rows = rows.masked_fill(cols > limit, float("-inf"))
    return torch.softmax(rows, dim=-1).view(x.shape)


def softmax_scaled(
    x: torch.Tensor, scale: float, causal_period: int = 0, dtype: torch.dtype | None = None
) -> torch.Tensor:
    """Softmax over the last dim of ``scale * x`` with an optional causal mask.

    Row ``r`` of the flattened ``[-1, cols]`` view keeps columns
    ``0 .. r % causal_period`` and gives the rest probability 0 (no mask when
    ``causal_period`` is 0). For attention scores ``[batch, heads, seq, seq]``,
    ``softmax_scaled(q @ k^T, 1 / sqrt(d), seq)`` is the causal softmax that
    examples/transformer_block.py:57-59 composes from ``scores / sqrt(d) +
    causal`` and ``softmax``, in one pass that does not read the masked
    scores. Result in ``dtype`` (default: the input's); fp32 arithmetic. Not
    in the reference's API."""
    dtype = x.dtype if dtype is None else dtype
    if causal_period < 0:
        raise ValueError(f"causal_period must be >= 0, got {causal_period}")
    if x.numel() == 0:
        return x.to(dtype).clone()
    x = x.contiguous()
    if (
        _dispatch_available("softmax_scaled", x)
        and x.dtype in KERNEL_DTYPES
        and dtype in KERNEL_DTYPES
    ):
        rows = x.reshape(-1, x.shape[-1])
        return torch.ops.cudaforge.softmax_scaled(rows, float(scale), int(causal_period), dtype).view(x.shape)
    _refuse_gpu_fallback("softmax_scaled", x)
    return _softmax_scaled_reference(x, scale, causal_period).to(dtype)


#: Head sizes the causal attention kernels take (sequence lengths: multiples of 8).
ATTENTION_HEAD_DIMS = (32, 64, 96, 128)


def _attention_kernel_shape(rows: torch.Tensor, heads: int, *others: torch.Tensor) -> bool:
    """True when the bf16 attention kernels take [batch, seq, heads * head_dim]
    (and the tensors are 16-byte aligned, as the kernels' loads need)."""
    return (
        rows.dtype == torch.bfloat16
        and rows.shape[-1] // heads in ATTENTION_HEAD_DIMS
        and rows.shape[1] % 8 == 0
        and all(t.data_ptr() % 16 == 0 for t in (rows, *others))
    )


def _check_attention_rows(rows: torch.Tensor, heads: int, name: str) -> None:
    if rows.dim() != 3:
        raise ValueError(f"{name} must be [batch, seq, hidden], got {tuple(rows.shape)}")
    if heads <= 0 or rows.shape[-1] % heads:
        raise ValueError(f"hidden {rows.shape[-1]} is not divisible by heads {heads}")


def attention_scores_causal(q: torch.Tensor, k: torch.Tensor, heads: int) -> torch.Tensor:
    """``q @ k^T`` per head for causal attention: q, k ``[batch, seq, hidden]``
    (the projections' output, ``hidden = heads * head_dim``) give scores
    ``[batch, heads, seq, seq]``.

    The product of examples/transformer_block.py:54 without the head
    transposes. Only the causal half is defined: entries above the diagonal
    are unspecified (the HIP kernel skips the 128 x 128 tiles above it), so
    follow it with ``softmax_scaled(..., causal_period=seq)``, which never
    reads them. bf16 with head_dim 32/64/96/128 and seq a multiple of 8 runs
    the MFMA kernel on a GPU. Not in the reference's API."""
    _check_attention_rows(q, heads, "q")
    if k.shape != q.shape:
        raise ValueError(f"q and k differ in shape: {tuple(q.shape)} and {tuple(k.shape)}")
    q, k = q.contiguous(), k.contiguous()
    if (
        _dispatch_available("attention_scores_causal", q, k)
        and _same_dtype(q, k)
        and (not q.is_cuda or _attention_kernel_shape(q, heads, k))
    ):
        return torch.ops.cudaforge.attention_scores_causal(q, k, int(heads))
    _refuse_gpu_fallback("attention_scores_causal", q, k)
    batch, seq, hidden = q.shape
    qh = q.view(batch, seq, heads, hidden // heads).transpose(1, 2).float()
    kh = k.view(batch, seq, heads, hidden // heads).transpose(1, 2).float()
    return (qh @ kh.transpose(-2, -1)).to(q.dtype)


def attention_pv_causal(probs: torch.Tensor, v: torch.Tensor, heads: int) -> torch.Tensor:
    """``probs @ v`` per head for causal attention, back in the
    ``[batch, seq, hidden]`` layout: probs ``[batch, heads, seq, seq]``, v
    ``[batch, seq, hidden]``. Row s of probs contributes keys 0 .. s only;
    entries above the diagonal are never read as values.

    The product of examples/transformer_block.py:63 with its transpose and
    reshape folded in. Same kernel rules as ``attention_scores_causal``. Not
    in the reference's API."""
    _check_attention_rows(v, heads, "v")
    batch, seq, hidden = v.shape
    if probs.shape != (batch, heads, seq, seq):
        raise ValueError(f"probs must be {(batch, heads, seq, seq)}, got {tuple(probs.shape)}")
    probs, v = probs.contiguous(), v.contiguous()
    if (
        _dispatch_available("attention_pv_causal", probs, v)
        and probs.dtype == v.dtype
        and (not v.is_cuda or _attention_kernel_shape(v, heads, probs))
    ):
        return torch.ops.cudaforge.attention_pv_causal(probs, v, int(heads))
    _refuse_gpu_fallback("attention_pv_causal", probs, v)
    vh = v.view(batch, seq, heads, hidden // heads).transpose(1, 2).float()
    out = torch.tril(probs.float()) @ vh
    return out.transpose(1, 2).reshape(batch, seq, hidden).to(v.dtype)


def lora_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    lora_a: torch.Tensor,
    lora_b: torch.Tensor,
    scale: float = 1.0,
) -> torch.Tensor:
    """``y = x @ weight + scale * (x @ lora_a) @ lora_b`` (operator layout).

    Shapes, with M rows, K input and N output features and adapter rank r:
    ``x`` is ``[M, K]``; the frozen ``weight`` is ``[K, N]`` (columns are output
    features); the down-projection ``lora_a`` is ``[K, r]`` and the
    up-projection ``lora_b`` is ``[r, N]``. ``scale`` multiplies the adapter
    term only; LoRA training sets it to alpha / r.

    A PEFT-layout layer (W ``[out, in]``, A ``[r, in]``, B ``[out, r]``) maps to
    ``lora_linear(x, W.t().contiguous(), A.t().contiguous(), B.t().contiguous(), alpha / r)``.
    """
    if x.shape[-1] != weight.shape[0]:
        raise ValueError(f"x has {x.shape[-1]} input features but weight expects {weight.shape[0]}")
    if lora_a.shape[0] != weight.shape[0]:
        raise ValueError(
            f"lora_a must be [in_features, rank] with in_features={weight.shape[0]}, "
            f"got {tuple(lora_a.shape)}"
        )
    if lora_b.shape[0] != lora_a.shape[1] or lora_b.shape[1] != weight.shape[1]:
        raise ValueError(
            f"lora_b must be [rank, out_features] = "
            f"[{lora_a.shape[1]}, {weight.shape[1]}], got {tuple(lora_b.shape)}"
        )
    x = x.contiguous()
    weight = weight.contiguous()
    lora_a = lora_a.contiguous()
    lora_b = lora_b.contiguous()
    operands = (x, weight, lora_a, lora_b)
    kernel_shape = x.ndim >= 2 and x.dtype in LORA_KERNEL_DTYPES and _same_dtype(*operands)
    rows = x.reshape(-1, x.shape[-1]) if x.ndim >= 2 else x
    out_shape = (*x.shape[:-1], weight.shape[1])
    if _needs_autograd(*operands):
        _require_extension("lora_linear", operands)
        if x.is_cuda and kernel_shape and _EXTENSION_LOADED:
            from cuda_force_amd.autograd import lora_linear_autograd

            return lora_linear_autograd(rows, weight, lora_a, lora_b, scale).view(out_shape)
        _refuse_gpu_fallback("lora_linear", *operands)
        return _lora_linear_reference(x, weight, lora_a, lora_b, scale)
    if _dispatch_available("lora_linear", *operands) and kernel_shape:
        return torch.ops.cudaforge.lora_linear(rows, weight, lora_a, lora_b, scale).view(out_shape)
    _refuse_gpu_fallback("lora_linear", *operands)
    return _lora_linear_reference(x, weight, lora_a, lora_b, scale)


def fused_residual_rmsnorm(
    x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6
) -> tuple[torch.Tensor, torch.Tensor]:
    """``h = x + residual``, then RMSNorm of ``h``, both from one pass.

    Returns ``(rmsnorm(h, weight, eps), h)``; a ``ValueError`` is raised when
    ``x`` and ``residual`` differ in shape or ``weight`` does not match their
    last dimension.
    """
    if x.shape != residual.shape:
        raise ValueError(
            f"x and residual must have the same shape, got {tuple(x.shape)} "
            f"and {tuple(residual.shape)}"
        )
    if weight.ndim != 1 or weight.shape[0] != x.shape[-1]:
        raise ValueError(f"weight must be 1-D of length {x.shape[-1]}, got {tuple(weight.shape)}")
    if x.numel() == 0:
        return x.clone(), residual.clone()
    x = x.contiguous()
    residual = residual.contiguous()
    weight = weight.contiguous()
    if (
        _dispatch_available("fused_residual_rmsnorm", x, residual, weight)
        and not _needs_autograd(x, residual, weight)
        and x.ndim == 2
        and x.dtype in KERNEL_DTYPES
        and _same_dtype(x, residual, weight)
    ):
        normalised, summed = torch.ops.cudaforge.fused_residual_rmsnorm(x, residual, weight, eps)
        return normalised, summed
    _refuse_gpu_fallback("fused_residual_rmsnorm", x, residual, weight)
    return _fused_residual_rmsnorm_reference(x, residual, weight, eps)


def silu(x: torch.Tensor) -> torch.Tensor:
    """SiLU (swish): ``x * sigmoid(x)``."""
    if x.numel() == 0:
        return x.clone()
    x = x.contiguous()
    if _dispatch_available("silu", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.silu(x)
    _refuse_gpu_fallback("silu", x)
    return torch.nn.functional.silu(x)


def gelu(x: torch.Tensor) -> torch.Tensor:
    """GELU, tanh approximation."""
    if x.numel() == 0:
        return x.clone()
    x = x.contiguous()
    if _dispatch_available("gelu", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.gelu(x)
    _refuse_gpu_fallback("gelu", x)
    return torch.nn.functional.gelu(x, approximate="tanh")


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """``silu(gate) * up`` elementwise (fp32 arithmetic for 16-bit inputs).

    ``gate`` and ``up`` must agree in shape and dtype; otherwise a
    ``ValueError`` is raised before anything runs.
    """
    if gate.shape != up.shape:
        raise ValueError(
            f"gate and up must have the same shape, got {tuple(gate.shape)} and {tuple(up.shape)}"
        )
    if gate.dtype != up.dtype:
        raise ValueError(f"gate and up must have the same dtype, got {gate.dtype} and {up.dtype}")
    if gate.numel() == 0:
        return gate.clone()
    gate = gate.contiguous()
    up = up.contiguous()
    if _dispatch_available("swiglu", gate, up) and gate.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.swiglu(gate, up)
    _refuse_gpu_fallback("swiglu", gate, up)
    return _swiglu_reference(gate, up)


def sum_reduce(x: torch.Tensor) -> torch.Tensor:
    """Sum of every element, as a 0-D tensor (deterministic on the GPU)."""
    if x.numel() == 0:
        return torch.zeros((), dtype=x.dtype, device=x.device)
    x = x.contiguous()
    if _dispatch_available("sum", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.sum(x)
    _refuse_gpu_fallback("sum", x)
    return x.sum()


def row_sum(x: torch.Tensor) -> torch.Tensor:
    """Per-row fp32 sums of a 2-D tensor (the reference's launch_row_sum)."""
    if x.ndim != 2:
        raise ValueError(f"row_sum takes a 2-D tensor, got shape {tuple(x.shape)}")
    x = x.contiguous()
    if x.numel() == 0:
        return torch.zeros(x.shape[0], dtype=torch.float32, device=x.device)
    if _dispatch_available("row_sum", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.row_sum(x)
    _refuse_gpu_fallback("row_sum", x)
    return x.float().sum(dim=-1)


def quantize_int8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Block-wise symmetric int8 quantisation.

    Returns:
        ``(quantised, scales)``: int8 codes shaped like ``x`` and one fp32
        scale per ``QUANT_BLOCK_SIZE`` elements of the flattened input.
    """
    x = x.contiguous()
    if _dispatch_available("quantize_int8", x) and x.dtype in KERNEL_DTYPES:
        quantised, scales = torch.ops.cudaforge.quantize_int8(x)
        return quantised, scales
    _refuse_gpu_fallback("quantize_int8", x)
    return _quantize_int8_reference(x)


def dequantize_int8(
    quantised: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype | None = None
) -> torch.Tensor:
    """Inverse of :func:`quantize_int8`. Lossy by construction.

    ``dtype`` (not in the reference) selects the output type; by default it is
    the scales' dtype, float32. A half dtype equals the float32 result
    followed by ``.to(dtype)``, computed in one pass.
    """
    expected = (quantised.numel() + QUANT_BLOCK_SIZE - 1) // QUANT_BLOCK_SIZE
    if scales.numel() != expected:
        raise ValueError(
            f"expected {expected} block scales for {quantised.numel()} elements, "
            f"got {scales.numel()}"
        )
    quantised = quantised.contiguous()
    scales = scales.contiguous()
    target = scales.dtype if dtype is None else dtype
    if _dispatch_available("dequantize_int8", quantised, scales) and scales.dtype == torch.float32:
        if target == scales.dtype:
            return torch.ops.cudaforge.dequantize_int8(quantised, scales)
        if target in KERNEL_DTYPES:
            return torch.ops.cudaforge.dequantize_int8_to(quantised, scales, target)
    _refuse_gpu_fallback("dequantize_int8", quantised, scales)
    return _dequantize_int8_reference(quantised, scales).to(target)


def fake_quantize_int8(x: torch.Tensor) -> torch.Tensor:
    """Quantise and dequantise in one pass, in x's dtype (the reference's
    launch_quantize_dequantize, which it never exposed as an operator)."""
    if x.numel() == 0:
        return x.clone()
    x = x.contiguous()
    if _dispatch_available("quantize_dequantize", x) and x.dtype in KERNEL_DTYPES:
        return torch.ops.cudaforge.quantize_dequantize(x)
    _refuse_gpu_fallback("quantize_dequantize", x)
    codes, scales = _quantize_int8_reference(x)
    return _dequantize_int8_reference(codes, scales).to(x.dtype)


def quantization_error(x: torch.Tensor) -> torch.Tensor:
    """Maximum absolute round-trip error of int8 quantisation (<= scale / 2)."""
    quantised, scales = quantize_int8(x)
    restored = dequantize_int8(quantised, scales)
    return (x - restored).abs().max()


def _refuse_gpu_fallback(name: str, *tensors: torch.Tensor) -> None:
    """Account for a GPU call that could not take a kernel.

    Reached with the extension loaded (a missing extension already raised in
    _dispatch_available) for a dtype with no kernel (float64, mixed dtypes) or
    a backward pass through an inference-only operator. Backward passes take
    the differentiable composition silently, as in the reference; a dtype
    without a kernel falls back like the reference's ops.py does, but with a
    RuntimeWarning, or a NotImplementedError when CUDAFORGE_STRICT is set.
    """
    if not _on_gpu(tensors) or _needs_autograd(*tensors):
        return
    dtypes = sorted({str(t.dtype) for t in tensors})
    shapes = [tuple(t.shape) for t in tensors]
    message = f"cudaforge.{name}: no HIP kernel for dtypes {dtypes} and shapes {shapes}"
    if os.environ.get("CUDAFORGE_STRICT", "") not in ("", "0"):
        raise NotImplementedError(message)
    warnings.warn(message + "; running the PyTorch composition", RuntimeWarning, stacklevel=3)

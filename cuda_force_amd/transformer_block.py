"""A Llama-style transformer block composed from the custom operators (config 4).

The reference shows where its operators sit in a real architecture with
examples/transformer_block.py (:32-133): a pre-norm block whose residual adds
are fused into the following RMSNorm, attention with the softmax over the
materialised score matrix, and a SwiGLU feed-forward. This module is that
composition for the MI355X build, at the configuration the benchmark names:
every projection is a LoRA-adapted linear (rank 16, alpha 32) through the fused
bf16 MFMA kernel, so one block runs

    fused_residual_rmsnorm -> lora_linear Q, K, V -> scores = Q K^T ->
    softmax(scores / sqrt(d) + causal mask) in one kernel -> P V ->
    lora_linear O -> fused_residual_rmsnorm
    -> lora_linear gate, up -> swiglu -> lora_linear down

The two batched attention products run the causal HIP kernels
(ops.attention_scores_causal / attention_pv_causal): the reference composes
them from torch matmuls over the full [seq, seq] block, these compute its lower
triangle only and read the heads in place.

`reference_forward` restates the same block in fp32 torch operations (from the
same bf16 parameters) for parity checks; `timed_forward` reports each
operator's share of a forward pass.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from cuda_force_amd import ops


@dataclass
class LoRAProjection:
    """One LoRA-adapted projection in the operator layout of `ops.lora_linear`:
    w ``[in, out]``, a ``[in, rank]``, b ``[rank, out]``, y = x w + scale (x a) b."""

    w: torch.Tensor
    a: torch.Tensor
    b: torch.Tensor
    scale: float

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return ops.lora_linear(x, self.w, self.a, self.b, self.scale)

    def reference(self, x: torch.Tensor) -> torch.Tensor:
        """fp32: x w + scale (x a) b, from the stored (bf16) parameters."""
        w, a, b = self.w.float(), self.a.float(), self.b.float()
        return x @ w + self.scale * ((x @ a) @ b)


@dataclass(frozen=True)
class BlockConfig:
    hidden: int = 4096
    heads: int = 32
    intermediate: int = 11008
    rank: int = 16
    alpha: float = 32.0
    eps: float = 1e-6
    std: float = 0.02

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


def _init(shape, std, gen, device, dtype):
    return (std * torch.randn(*shape, generator=gen, device=device)).to(dtype)


class LlamaBlock:
    """One pre-norm block with LoRA projections; parameters drawn N(0, std)
    (norm weights 1 + N(0, std)) from `gen`."""

    def __init__(self, config: BlockConfig, device, dtype=torch.bfloat16, gen=None):
        if config.hidden % config.heads:
            raise ValueError(f"hidden {config.hidden} is not divisible by heads {config.heads}")
        self.config = config
        gen = gen if gen is not None else torch.Generator(device=device).manual_seed(0)
        h, m, r = config.hidden, config.intermediate, config.rank
        scale = config.alpha / r

        def projection(n_in, n_out):
            return LoRAProjection(_init((n_in, n_out), config.std, gen, device, dtype),
                                  _init((n_in, r), config.std, gen, device, dtype),
                                  _init((r, n_out), config.std, gen, device, dtype), scale)

        self.attention_norm = (1 + _init((h,), config.std, gen, device, torch.float32)).to(dtype)
        self.ffn_norm = (1 + _init((h,), config.std, gen, device, torch.float32)).to(dtype)
        self.q, self.k, self.v, self.o = (projection(h, h) for _ in range(4))
        self.gate, self.up = projection(h, m), projection(h, m)
        self.down = projection(m, h)

    # -- the block through the custom operators ------------------------------

    def _attention(self, normed: torch.Tensor, batch: int, seq: int, hook=None) -> torch.Tensor:
        c = self.config
        mark = hook or (lambda name: None)
        q, k, v = self.q(normed), self.k(normed), self.v(normed)
        mark("qkv_lora")

        # The causal products read q, k and v in the projections' [batch,
        # seq, hidden] layout (no head transposes) and compute only the
        # lower triangle; the softmax reads only that triangle too.
        rows = (batch, seq, c.hidden)
        scores = ops.attention_scores_causal(q.view(rows), k.view(rows), c.heads)
        mark("scores_matmul")
        # softmax(scores / sqrt(d) + causal) in one pass: row r of each
        # head's [seq, seq] block keeps columns 0 .. r; the masked scores
        # are never read.
        weights = ops.softmax_scaled(scores.view(-1, seq), 1.0 / math.sqrt(c.head_dim), seq).view_as(scores)
        mark("softmax")
        attended = ops.attention_pv_causal(weights, v.view(rows), c.heads).view(batch * seq, c.hidden)
        mark("pv_matmul")
        out = self.o(attended)
        mark("o_lora")
        return out

    def forward(self, x: torch.Tensor, residual: torch.Tensor, hook=None):
        """x, residual: ``[batch, seq, hidden]``. Returns (output, residual)."""
        batch, seq, hidden = x.shape
        mark = hook or (lambda name: None)
        normed, residual2 = ops.fused_residual_rmsnorm(
            x.reshape(-1, hidden), residual.reshape(-1, hidden), self.attention_norm, self.config.eps)
        mark("residual_rmsnorm_1")
        attended = self._attention(normed, batch, seq, hook)
        normed, residual2 = ops.fused_residual_rmsnorm(attended, residual2, self.ffn_norm, self.config.eps)
        mark("residual_rmsnorm_2")
        gate, up = self.gate(normed), self.up(normed)
        mark("gate_up_lora")
        activated = ops.swiglu(gate, up)
        mark("swiglu")
        out = self.down(activated)
        mark("down_lora")
        return out.view(batch, seq, hidden), residual2.view(batch, seq, hidden)

    # -- fp32 restatement --------------------------------------------------

    def reference_forward(self, x: torch.Tensor, residual: torch.Tensor):
        """The same block in fp32 torch operations (parity reference)."""
        c = self.config
        batch, seq, hidden = x.shape

        def rmsnorm(t, w):
            return t * torch.rsqrt(t.pow(2).mean(-1, keepdim=True) + c.eps) * w.float()

        residual2 = (x.float() + residual.float()).reshape(-1, hidden)
        normed = rmsnorm(residual2, self.attention_norm)
        q, k, v = self.q.reference(normed), self.k.reference(normed), self.v.reference(normed)

        def heads(t):
            return t.view(batch, seq, c.heads, c.head_dim).transpose(1, 2).contiguous()

        scores = heads(q) @ heads(k).transpose(-2, -1).contiguous() / math.sqrt(c.head_dim)
        causal = torch.triu(torch.full((seq, seq), float("-inf"), device=x.device), 1)
        weights = torch.softmax(scores + causal, dim=-1)
        attended = (weights @ heads(v)).transpose(1, 2).reshape(batch * seq, hidden)
        attended = self.o.reference(attended)
        residual2 = attended + residual2
        normed = rmsnorm(residual2, self.ffn_norm)
        gate, up = self.gate.reference(normed), self.up.reference(normed)
        out = self.down.reference(torch.nn.functional.silu(gate) * up)
        return out.view(batch, seq, hidden), residual2.view(batch, seq, hidden)

    # -- accounting ----------------------------------------------------------

    def gemm_flops(self, tokens: int, seq: int) -> dict[str, int]:
        """Algorithmic FLOPs of the projections and the attention products."""
        c = self.config
        h, m, r = c.hidden, c.intermediate, c.rank

        def lora(n_in, n_out):
            return 2 * tokens * n_in * n_out + 2 * tokens * n_in * r + 2 * tokens * r * n_out

        batch_heads = tokens // seq * c.heads
        return {
            "qkv_lora": 3 * lora(h, h),
            "o_lora": lora(h, h),
            "gate_up_lora": 2 * lora(h, m),
            "down_lora": lora(m, h),
            "scores_matmul": 2 * batch_heads * seq * seq * c.head_dim,
            "pv_matmul": 2 * batch_heads * seq * seq * c.head_dim,
        }


def timed_forward(block: LlamaBlock, x: torch.Tensor, residual: torch.Tensor) -> dict[str, float]:
    """One forward pass with a HIP event after each stage; milliseconds per
    stage (GPU tensors only)."""
    events = [("start", torch.cuda.Event(enable_timing=True))]
    events[0][1].record()

    def hook(name):
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        events.append((name, event))

    block.forward(x, residual, hook)
    torch.cuda.synchronize()
    out = {}
    for (_, previous), (name, event) in zip(events, events[1:]):
        out[name] = out.get(name, 0.0) + previous.elapsed_time(event)
    out["total"] = events[0][1].elapsed_time(events[-1][1])
    return out

"""float64 restatements of the floating-point ops (test infrastructure only).

Each function takes the values the kernel receives (16-bit inputs already
widened from their stored bits) and returns the float64 result before the
final rounding to the output type, so a test can apply its tolerance - or,
for bf16 outputs, compare against the same value rounded once. Citations are
to the reference semantics each follows.
"""

from __future__ import annotations

import math

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even, NaN -> 0x7FC0."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, np.uint16(0x7FC0), rounded).astype(np.uint16)


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round (via fp32) to the nearest bf16 value; returned as float64."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32))).astype(np.float64)


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """(x * rsqrt(mean(x^2) + eps)) * w per row (python/cudaforge/ops.py:164-171).

    eps is added in fp32 by the reference (variance + eps on a float32
    tensor); it is taken here as the fp32 value of eps."""
    x64 = np.asarray(x, dtype=np.float64)
    mean = np.mean(x64 * x64, axis=-1, keepdims=True)
    inv = 1.0 / np.sqrt(mean + float(np.float32(eps)))
    return (x64 * inv) * np.asarray(weight, dtype=np.float64)


def softmax(x: np.ndarray) -> np.ndarray:
    """exp(x - max) / sum per row (torch.softmax, python/cudaforge/ops.py:174-175)."""
    x64 = np.asarray(x, dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        shifted = x64 - np.max(x64, axis=-1, keepdims=True)
        e = np.exp(shifted)
        return e / np.sum(e, axis=-1, keepdims=True)


def sum_exact(x: np.ndarray) -> float:
    """Correctly rounded sum of the values (math.fsum)."""
    return math.fsum(np.asarray(x, dtype=np.float64).reshape(-1).tolist())


def lora_linear(
    x: np.ndarray,
    w: np.ndarray,
    a: np.ndarray,
    b: np.ndarray,
    scale: float,
    round_intermediate: bool,
) -> np.ndarray:
    """x @ w + scale * ((x @ a) @ b), op layout (python/cudaforge/ops.py:178-185).

    With round_intermediate the adapter intermediate x @ a is rounded to bf16
    first, as the reference's bf16 ATen path materialises it as a bf16 tensor."""
    x64 = np.asarray(x, dtype=np.float64)
    xa = x64 @ np.asarray(a, dtype=np.float64)
    if round_intermediate:
        xa = round_bf16(xa)
    return x64 @ np.asarray(w, dtype=np.float64) + scale * (xa @ np.asarray(b, dtype=np.float64))


def lora_backward(
    x: np.ndarray,
    dy: np.ndarray,
    b: np.ndarray,
    xa: np.ndarray,
    scale: float,
    round_intermediate: bool,
) -> tuple[np.ndarray, np.ndarray]:
    """Adapter gradients of x @ w + s * (x @ a) @ b in op layout:
    grad_a = s * x^T (dy @ b^T), grad_b = s * (x @ a)^T dy
    (tests/python/test_autograd.py:81-91 checks the reference produces them).

    With round_intermediate, dy @ b^T and x @ a are rounded to bf16, the
    tensors ATen's bf16 autograd sees."""
    x64 = np.asarray(x, dtype=np.float64)
    dy64 = np.asarray(dy, dtype=np.float64)
    g = dy64 @ np.asarray(b, dtype=np.float64).T
    p = np.asarray(xa, dtype=np.float64)
    if round_intermediate:
        g = round_bf16(g)
        p = round_bf16(p)
    return scale * (x64.T @ g), scale * (p.T @ dy64)


def silu(x: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) (python/cudaforge/ops.py:195-196)."""
    x64 = np.asarray(x, dtype=np.float64)
    with np.errstate(over="ignore"):
        return x64 / (1.0 + np.exp(-x64))


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) (python/cudaforge/ops.py:208-212)."""
    x64 = np.asarray(x, dtype=np.float64)
    return 0.5 * x64 * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x64 + 0.044715 * x64**3)))


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """silu(gate) * up (python/cudaforge/ops.py:199-205)."""
    return silu(gate) * np.asarray(up, dtype=np.float64)


def paged_attention(
    query: np.ndarray,
    k_cache: np.ndarray,
    v_cache: np.ndarray,
    block_tables: np.ndarray,
    context_lens: np.ndarray,
    scale: float,
) -> np.ndarray:
    """One decode step of attention through a paged KV cache, float64
    (cuda/include/cudaforge/paged_attention.cuh:10-61; the host reference of
    tests/cuda/test_paged_attention.cu:45-103 computes the same).

    query [S, H, D]; k_cache / v_cache [blocks, block_size, KVH, D];
    block_tables [S, max_blocks]; context_lens [S]. Token t of sequence s is
    k_cache[block_tables[s, t // block_size], t % block_size]; query head h reads
    KV head h // (H // KVH). out[s, h] = softmax(scale * q K^T) V over the first
    context_lens[s] tokens, zeros for an empty context.
    """
    q = np.asarray(query, dtype=np.float64)
    kc = np.asarray(k_cache, dtype=np.float64)
    vc = np.asarray(v_cache, dtype=np.float64)
    sequences, heads, dim = q.shape
    block_size, kv_heads = kc.shape[1], kc.shape[2]
    group = heads // kv_heads
    out = np.zeros((sequences, heads, dim), dtype=np.float64)
    for s in range(sequences):
        n = int(context_lens[s])
        if n <= 0:
            continue
        tokens = np.arange(n)
        blocks = np.asarray(block_tables[s], dtype=np.int64)[tokens // block_size]
        keys = kc[blocks, tokens % block_size]  # [n, KVH, D]
        values = vc[blocks, tokens % block_size]
        for h in range(heads):
            scores = keys[:, h // group, :] @ q[s, h] * scale
            weights = np.exp(scores - scores.max())
            out[s, h] = weights @ values[:, h // group, :] / weights.sum()
    return out


def attention_scores(q: np.ndarray, k: np.ndarray, heads: int) -> np.ndarray:
    """query @ key^T per head (examples/transformer_block.py:51-54, before the
    1/sqrt(d) and the mask): q, k [batch, seq, heads * d] -> [batch, heads,
    seq, seq], float64, every entry (the kernels define the lower triangle)."""
    batch, seq, hidden = q.shape
    d = hidden // heads
    qh = np.asarray(q, dtype=np.float64).reshape(batch, seq, heads, d).transpose(0, 2, 1, 3)
    kh = np.asarray(k, dtype=np.float64).reshape(batch, seq, heads, d).transpose(0, 2, 1, 3)
    return qh @ kh.transpose(0, 1, 3, 2)


def attention_values(probs: np.ndarray, v: np.ndarray, heads: int) -> np.ndarray:
    """(weights @ value).transpose(1, 2).reshape(batch, seq, hidden) of
    examples/transformer_block.py:63, with row s of the weights taking keys
    0 .. s only (the causal lower triangle): probs [batch, heads, seq, seq],
    v [batch, seq, heads * d] -> [batch, seq, heads * d], float64."""
    batch, seq, hidden = v.shape
    d = hidden // heads
    vh = np.asarray(v, dtype=np.float64).reshape(batch, seq, heads, d).transpose(0, 2, 1, 3)
    lower = np.tril(np.asarray(probs, dtype=np.float64))
    return (lower @ vh).transpose(0, 2, 1, 3).reshape(batch, seq, hidden)


def e4m3fn_to_f64(codes: np.ndarray) -> np.ndarray:
    """Decode OCP fp8 e4m3fn codes (OCP 8-bit floating point specification
    v1.0, E4M3: sign, 4 exponent bits with bias 7, 3 mantissa bits; exponent
    0 is subnormal, m * 2^-9; S.1111.111 is NaN; no infinities). The reference
    has no fp8 type; this is the format the fp8 matmul consumes."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    exponent = (c >> 3) & 0xF
    mantissa = c & 0x7
    normal = np.ldexp(1.0 + mantissa / 8.0, exponent - 7)
    subnormal = np.ldexp(mantissa.astype(np.float64), -9)
    value = sign * np.where(exponent == 0, subnormal, normal)
    return np.where((c & 0x7F) == 0x7F, np.nan, value)


def matmul_fp8(x_codes: np.ndarray, w_codes: np.ndarray, scale: float) -> np.ndarray:
    """scale * (x @ w) for e4m3fn codes x [M, K] and w [K, N], float64 (every
    fp8 product is exact; the sum is float64). The fp8 half of the MFMA matmul
    that replaces the TF32 demonstration (cuda/include/cudaforge/
    tensor_core_matmul.cuh:40-41 keeps C = A B row-major with fp32 operands)."""
    return float(scale) * (e4m3fn_to_f64(x_codes) @ e4m3fn_to_f64(w_codes))

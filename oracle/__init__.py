"""CPU oracle for the custom-op hot path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything from this package, and only as the checker (or the timed CPU
baseline), never as the thing measured or shipped. The product path
(cuda_force_amd) never imports it and fails loudly without its HIP extension.

Contents:
  quant.py      block-wise INT8 quantise/dequantise/fake-quant: a C
                restatement (cf_oracle.c, bit-exact by construction) and an
                independent numpy restatement, cross-checked in the tests.
  floatops.py   float64 restatements of RMSNorm, softmax, the sum, the LoRA
                linear and its adapter gradients, the activations,
                paged-attention decode, the fp8 (e4m3fn) matmul, and the
                block's two attention products.
  ref_runner.py runs the reference's own CPU operators (cpp/src/bindings.cpp,
                compiled by `make -C oracle ref` into oracle/_ref/) in a child
                process, for golden vectors and the "reference" CPU baseline.

How each function is pinned (golden vectors from oracle/_ref, closed forms,
invariants, planted mistakes) is listed in tests/test_oracle.py.
"""

from oracle.floatops import (  # noqa: F401
    attention_scores,
    attention_values,
    bf16_bits_to_f32,
    e4m3fn_to_f64,
    f32_to_bf16_bits,
    gelu_tanh,
    lora_backward,
    lora_linear,
    matmul_fp8,
    paged_attention,
    rmsnorm,
    round_bf16,
    silu,
    softmax,
    sum_exact,
    swiglu,
)
from oracle.quant import (  # noqa: F401
    dequantize_int8,
    dequantize_int8_numpy,
    quantize_dequantize,
    quantize_int8,
    quantize_int8_numpy,
)

/*
 * cf_oracle.c - CPU restatement of the reference's block-wise INT8
 * quantisation, used ONLY as the checker in tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg. Nothing in the product links or loads it.
 *
 * Follows the reference's CPU semantics:
 *   python/cudaforge/ops.py:215-229   _quantize_int8_reference
 *   python/cudaforge/ops.py:232-240   _dequantize_int8_reference
 *   cpp/src/bindings.cpp:298-329      quantize_int8_cpu / dequantize_int8_cpu
 *   cuda/src/quantization.cu:61-76    quantize_dequantize (fake quant)
 *
 * Per 64-element block of the flattened input (zero-padded at the end):
 *   s = absmax / 127         fp32 IEEE divide; a NaN anywhere in the block
 *                            makes absmax NaN (torch.amax propagates it)
 *   s = (s > 0) ? s : 1      after the divide; NaN > 0 is false, so a NaN
 *                            block also gets scale 1
 *   q = clamp(rint(x / s), -127, 127)   round half to even (rintf under the
 *                            default rounding mode); a NaN quotient -> 0,
 *                            what ATen's float->int8 conversion gives
 * Dequantise: y = (float)q * s, then rounded to bf16/fp16 when asked (RNE),
 * as `.to(dtype)` after the fp32 result does.
 *
 * Written as plain scalar loops on purpose: each line is one step of the
 * formula above. Build: see oracle/Makefile (gcc -O2, no fast-math, no FMA
 * contraction).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2 };
enum { BLOCK = 64 };

static uint32_t bits_of(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

static float float_of(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* bf16 -> fp32 is exact: the bf16 bits are the high half of the fp32 bits. */
float oracle_bf16_to_f32(uint16_t h) { return float_of((uint32_t)h << 16); }

/* fp32 -> bf16, round to nearest even; NaN -> 0x7FC0 (c10::BFloat16's rule). */
uint16_t oracle_f32_to_bf16(float f) {
    uint32_t u = bits_of(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

/* IEEE binary16 -> fp32, exact. */
float oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    if (exponent == 0) {
        const float magnitude = (float)mantissa * 5.9604644775390625e-08f; /* 2^-24 */
        return sign ? -magnitude : magnitude;
    }
    if (exponent == 31) return float_of(sign | 0x7F800000u | (mantissa << 13));
    return float_of(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* fp32 -> IEEE binary16, round to nearest even. */
uint16_t oracle_f32_to_f16(float f) {
    const uint32_t u = bits_of(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t magnitude = u & 0x7FFFFFFFu;
    if (magnitude > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);
    if (magnitude >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 -> inf */
    if (magnitude < 0x38800000u) {
        /* Below 2^-14: a multiple of 2^-24. Scaling by 2^24 is exact, rintf
         * rounds half to even; 1024 lands on the smallest normal's encoding. */
        const float scaled = float_of(magnitude) * 16777216.0f;
        return (uint16_t)(sign | (uint16_t)rintf(scaled));
    }
    const uint32_t rounded = magnitude + 0xFFFu + ((magnitude >> 13) & 1u);
    return (uint16_t)(sign | (uint16_t)((rounded >> 13) - (112u << 10)));
}

static float load_element(const void* x, int dtype, int64_t i) {
    switch (dtype) {
        case ORACLE_F32:
            return ((const float*)x)[i];
        case ORACLE_BF16:
            return oracle_bf16_to_f32(((const uint16_t*)x)[i]);
        default:
            return oracle_f16_to_f32(((const uint16_t*)x)[i]);
    }
}

static void store_element(void* y, int dtype, int64_t i, float v) {
    switch (dtype) {
        case ORACLE_F32:
            ((float*)y)[i] = v;
            break;
        case ORACLE_BF16:
            ((uint16_t*)y)[i] = oracle_f32_to_bf16(v);
            break;
        default:
            ((uint16_t*)y)[i] = oracle_f32_to_f16(v);
            break;
    }
}

int64_t oracle_scale_count(int64_t n) { return n <= 0 ? 0 : (n + BLOCK - 1) / BLOCK; }

/* Scale of block b: absmax / 127, NaN-propagating, then the > 0 guard. */
static float block_scale(const void* x, int dtype, int64_t n, int64_t b) {
    float absmax = 0.0f;
    int saw_nan = 0;
    for (int j = 0; j < BLOCK; ++j) {
        const int64_t i = b * BLOCK + j;
        const float a = i < n ? fabsf(load_element(x, dtype, i)) : 0.0f;
        if (isnan(a)) {
            saw_nan = 1;
        } else if (a > absmax) {
            absmax = a;
        }
    }
    float s = saw_nan ? NAN : absmax / 127.0f;
    if (!(s > 0.0f)) s = 1.0f;
    return s;
}

static int8_t code_of(float v, float s) {
    const float r = rintf(v / s);
    if (isnan(r)) return 0;
    if (r > 127.0f) return 127;
    if (r < -127.0f) return -127;
    return (int8_t)r;
}

void oracle_quantize_int8(const void* x, int dtype, int64_t n, int8_t* q, float* scales) {
    const int64_t blocks = oracle_scale_count(n);
    for (int64_t b = 0; b < blocks; ++b) {
        const float s = block_scale(x, dtype, n, b);
        scales[b] = s;
        for (int j = 0; j < BLOCK; ++j) {
            const int64_t i = b * BLOCK + j;
            if (i < n) q[i] = code_of(load_element(x, dtype, i), s);
        }
    }
}

void oracle_dequantize_int8(const int8_t* q, const float* scales, int64_t n, void* y,
                            int dtype) {
    for (int64_t i = 0; i < n; ++i) {
        store_element(y, dtype, i, (float)q[i] * scales[i / BLOCK]);
    }
}

void oracle_quantize_dequantize(const void* x, int dtype, int64_t n, void* y) {
    const int64_t blocks = oracle_scale_count(n);
    for (int64_t b = 0; b < blocks; ++b) {
        const float s = block_scale(x, dtype, n, b);
        for (int j = 0; j < BLOCK; ++j) {
            const int64_t i = b * BLOCK + j;
            if (i < n) store_element(y, dtype, i, (float)code_of(load_element(x, dtype, i), s) * s);
        }
    }
}

void oracle_to_bf16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_bf16(x[i]);
}

void oracle_to_f16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f32_to_f16(x[i]);
}

void oracle_from_f16(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f16_to_f32(x[i]);
}

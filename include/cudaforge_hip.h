/*
 * cudaforge_hip.h - C ABI of the MI355X (gfx950) custom-op library
 * `libcudaforge_hip.so`.
 *
 * This is the drop-in boundary for CudaForge's custom-op hot path. Every entry
 * point replaces one host launcher of the reference's CUDA library
 * (the headers under cuda/include/cudaforge/) and keeps its argument meaning, but with a
 * plain C signature that any FFI can bind (ctypes, cgo, JNI, N-API):
 *
 *   - raw device pointers and element counts (int64_t instead of the
 *     reference's `int count`, so tensors above 2^31 elements are legal);
 *   - an explicit dtype tag where the reference had one function per storage
 *     type (launch_rmsnorm / launch_rmsnorm_half / launch_rmsnorm_bf16);
 *   - `stream` is a hipStream_t passed as `void*` (NULL = the null stream), so
 *     this header needs no HIP include. Every launch is asynchronous on that
 *     stream and nothing here synchronises, except when the environment
 *     variable CUDAFORGE_DEBUG_SYNC is set (then every entry point waits for
 *     its stream and reports kernel faults synchronously);
 *   - no exceptions cross the ABI: each entry point returns a cf_status and
 *     leaves a message for cf_last_error() (thread-local). The reference threw
 *     cudaforge::CudaError (cuda/include/cudaforge/cuda_error.cuh:15-69) and
 *     std::invalid_argument (cuda/src/lora_linear.cu:263-265).
 *
 * Empty inputs (count <= 0, rows <= 0 or cols <= 0) return CF_OK without
 * launching anything, as every reference launcher does.
 *
 * No operator entry point allocates device memory. Those that need scratch
 * space take a caller-provided `workspace` and publish its size through a
 * *_workspace_bytes() query, like the reference's lora_workspace_bytes
 * (cuda/include/cudaforge/lora_linear.cuh:62). Only the runtime section at the
 * end (stream scheduler, caching pools) allocates, which is its purpose.
 */
#ifndef CUDAFORGE_HIP_H
#define CUDAFORGE_HIP_H

#include <stddef.h>
#include <stdint.h>

/* The library is built with -fvisibility=hidden: the entry points below are
 * its only exported symbols, so two builds loaded into one process share no
 * internal C++ symbol. */
#pragma GCC visibility push(default)

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status, dtypes, library facts ------------------------------------ */

typedef enum cf_status {
    CF_OK = 0,
    CF_ERR_INVALID_ARGUMENT = 1, /* shape, pointer, alignment or size error  */
    CF_ERR_UNSUPPORTED = 2,      /* dtype or shape combination with no kernel */
    CF_ERR_HIP = 3,              /* the HIP runtime reported an error         */
    CF_ERR_OUT_OF_MEMORY = 4,    /* a pool backend could not supply a block   */
} cf_status;

typedef enum cf_dtype {
    CF_F32 = 0,
    CF_F16 = 1,
    CF_BF16 = 2,
} cf_dtype;

/* Elements per quantisation block. Same value as kQuantBlockSize
 * (cuda/include/cudaforge/quantization.cuh:18) and QUANT_BLOCK_SIZE
 * (python/cudaforge/ops.py:41). */
#define CF_QUANT_BLOCK_SIZE 64

/* Message describing the most recent failure on the calling thread; the text
 * the reference put in CudaError::what() (cuda/include/cudaforge/cuda_error.cuh:44-51). */
const char* cf_last_error(void);

/* hipError_t value behind the most recent CF_ERR_HIP on this thread (0 if the
 * last failure was not a HIP error). Replaces CudaError::status()
 * (cuda/include/cudaforge/cuda_error.cuh:21). */
int cf_last_hip_error(void);

/* True when the hipError_t names a fault that has poisoned the context
 * (illegal address, launch failure, ...). Replaces CudaError::is_sticky()
 * (cuda/include/cudaforge/cuda_error.cuh:25-39). */
int cf_hip_error_is_sticky(int hip_error);

/* ABI version of this header; bumped on any incompatible change. It has no
 * counterpart in the reference (a C++ API needs none). */
int cf_abi_version(void);

/* ---- block-wise INT8 quantisation -------------------------------------- */

/* Number of block scales `count` elements need: ceil(count / 64), 0 for
 * count <= 0. Replaces quant_scale_count (cuda/include/cudaforge/quantization.cuh:54,
 * cuda/src/quantization.cu:80-82). */
int64_t cf_quant_scale_count(int64_t count);

/* Symmetric absmax INT8 quantisation over 64-element blocks of the flattened
 * input:  s_b = absmax_b / 127 (IEEE fp32 divide; 1 when that is not > 0),
 *         q_i = clamp(rint(x_i / s_b), -127, 127)  (round half to even;
 *               NaN codes to 0).
 * `x` is fp32, fp16 or bf16 (`x_dtype`); half inputs are widened exactly to
 * fp32 first. `q` holds `count` int8 codes, `scales` cf_quant_scale_count(count)
 * fp32 scales. Bit-identical to the reference's CPU semantics
 * (python/cudaforge/ops.py:215-229, cpp/src/bindings.cpp:298-318).
 * Replaces launch_quantize_int8 (cuda/include/cudaforge/quantization.cuh:40-41). */
cf_status cf_quantize_int8(const void* x, cf_dtype x_dtype, int8_t* q, float* scales,
                           int64_t count, void* stream);

/* y_i = (fp32)q_i * s_{i/64}, one IEEE multiply, then rounded to `y_dtype`
 * (round to nearest even) when that is fp16/bf16.
 * Replaces launch_dequantize_int8 (cuda/include/cudaforge/quantization.cuh:45-46);
 * fp32 output is the reference's dequantize_int8 (python/cudaforge/ops.py:232-240),
 * half output equals that followed by `.to(dtype)`. */
cf_status cf_dequantize_int8(const int8_t* q, const float* scales, void* y, cf_dtype y_dtype,
                             int64_t count, void* stream);

/* Tensors per launch of the grouped entry points below. */
#define CF_QUANT_GROUP_MAX 48

/* Quantises `n_tensors` tensors as cf_quantize_int8(x[i], x_dtype, q[i],
 * scales[i], counts[i], stream) would each (bit-identical), but with up to
 * CF_QUANT_GROUP_MAX tensors per launch: the start-up and drain of a launch
 * (about 1.8 us on MI355X, a fifth of a [4096, 4096] bf16 tensor's time) are
 * paid once per group instead of once per tensor - bulk quantisation of a
 * model's weight set. `x`, `q`, `scales` and `counts` are host arrays of
 * n_tensors entries (device pointers, element counts), read before the call
 * returns; tensors with counts[i] <= 0 are skipped. A tensor whose x is not
 * 16-byte aligned or whose q is not aligned to 4 (fp32) / 8 (16-bit) bytes
 * gets a launch of its own. Outputs may not overlap any input or each other.
 * It has no counterpart in the reference, whose callers quantise one tensor
 * per call (python/cudaforge/ops.py:449-460). */
cf_status cf_quantize_int8_group(const void* const* x, cf_dtype x_dtype, int8_t* const* q,
                                 float* const* scales, const int64_t* counts, int64_t n_tensors,
                                 void* stream);

/* Dequantises `n_tensors` tensors as cf_dequantize_int8(q[i], scales[i],
 * y[i], y_dtype, counts[i], stream) would each, up to CF_QUANT_GROUP_MAX per
 * launch; same conventions as cf_quantize_int8_group (q aligned to 4 / 8
 * bytes and y to 16 bytes, or the tensor gets a launch of its own). It has no
 * counterpart in the reference (python/cudaforge/ops.py:463-476 dequantises
 * one tensor per call). */
cf_status cf_dequantize_int8_group(const int8_t* const* q, const float* const* scales,
                                   void* const* y, cf_dtype y_dtype, const int64_t* counts,
                                   int64_t n_tensors, void* stream);

/* Quantise then dequantise in registers ("fake quantisation"); `y` has the
 * dtype of `x`. Equals cf_quantize_int8 followed by cf_dequantize_int8.
 * Replaces launch_quantize_dequantize (cuda/include/cudaforge/quantization.cuh:51). */
cf_status cf_quantize_dequantize(const void* x, void* y, cf_dtype dtype, int64_t count,
                                 void* stream);

/* ---- RMSNorm ------------------------------------------------------------ */

/* y = (x * rsqrt(mean(x^2) + eps)) * w per row of a row-major [rows, cols]
 * matrix; fp32 arithmetic for every storage dtype; eps inside the sqrt.
 * `x`, `w`, `y` share `dtype`. Replaces launch_rmsnorm / launch_rmsnorm_half /
 * launch_rmsnorm_bf16 (cuda/include/cudaforge/rmsnorm.cuh:35-62); semantics of
 * _rmsnorm_reference (python/cudaforge/ops.py:164-171). launch_rmsnorm's
 * `RMSNormKernel variant` (Naive, Vectorised: rmsnorm.cuh:9-19) chose between
 * two implementations of this same function; the kernel here is chosen from
 * the shape and alignment, so a caller drops the argument. */
cf_status cf_rmsnorm(const void* x, const void* w, void* y, cf_dtype dtype, int64_t rows,
                     int64_t cols, float eps, void* stream);

/* r = x + residual; y = rmsnorm(r) * w. Writes both `y` and `residual_out`.
 * Replaces launch_fused_residual_rmsnorm (cuda/include/cudaforge/fused_norm.cuh:38-40);
 * semantics of _fused_residual_rmsnorm_reference (python/cudaforge/ops.py:188-192). */
cf_status cf_fused_residual_rmsnorm(const void* x, const void* residual, const void* w, void* y,
                                    void* residual_out, cf_dtype dtype, int64_t rows,
                                    int64_t cols, float eps, void* stream);

/* ---- softmax ------------------------------------------------------------ */

/* Numerically stable softmax over the last dim of a row-major [rows, cols]
 * matrix, fp32 arithmetic: y = exp(x - max) * (1 / sum exp(x - max)).
 * `y_dtype` may differ from `x_dtype` (e.g. bf16 logits -> fp32 probabilities).
 * `x` and `y` may alias when the dtypes match. Replaces launch_softmax /
 * launch_softmax_half / launch_softmax_bf16 (cuda/include/cudaforge/softmax.cuh:43-65);
 * semantics of torch.softmax(x, -1) (python/cudaforge/ops.py:174-175).
 * launch_softmax's `SoftmaxKernel variant` (Naive, SharedMemory, Online:
 * softmax.cuh:9-24) chose between implementations of this same function; the
 * kernel here is chosen from the shape, so a caller drops the argument. */
cf_status cf_softmax(const void* x, cf_dtype x_dtype, void* y, cf_dtype y_dtype, int64_t rows,
                     int64_t cols, void* stream);

/* Row softmax of scale * x with an optional causal mask: column c of row r is
 * -inf (probability 0) when causal_period > 0 and c > r mod causal_period;
 * causal_period 0 masks nothing. fp32 arithmetic as cf_softmax; masked
 * 16-byte vectors of x are not read. This is the attention-score softmax of
 * examples/transformer_block.py:57-59 (softmax(scores / sqrt(d) + causal))
 * in one pass: the reference composes it from a scale-and-mask pass and
 * launch_softmax (cuda/include/cudaforge/softmax.cuh:43-65). */
cf_status cf_softmax_scaled(const void* x, cf_dtype x_dtype, void* y, cf_dtype y_dtype,
                            int64_t rows, int64_t cols, float scale, int64_t causal_period,
                            void* stream);

/* ---- reductions --------------------------------------------------------- */

/* Bytes of workspace cf_reduce_sum needs for `count` elements (the stage-1
 * partial sums). The reference needs none because it reduces with atomics
 * into the zeroed output (cuda/src/reduction.cu:60-89). */
size_t cf_reduce_sum_workspace_bytes(int64_t count);

/* Sum of `count` elements (fp32 accumulation) into the single fp32 `*out`.
 * With accumulate != 0 the sum is added to `*out` (the reference launcher's
 * contract: cuda/include/cudaforge/reduction.cuh:36-42); with 0 it overwrites.
 * Deterministic: a fixed two-stage tree whose shape depends only on `count`.
 * Replaces launch_reduce_sum (cuda/include/cudaforge/reduction.cuh:43-44): its
 * contract (add into a zeroed *out) is accumulate = 1. Its `ReductionKernel
 * variant` (Naive, SharedMemory, WarpOptimised: reduction.cuh:14-34) chose
 * between implementations of the same sum, and reduction_grid_size
 * (reduction.cuh:55, the launch grid those variants used) has no counterpart:
 * the grid here is a function of `count` alone, at most 4096 stage-1
 * workgroups, i.e. cf_reduce_sum_workspace_bytes(count) / 4. */
cf_status cf_reduce_sum(const void* x, cf_dtype x_dtype, float* out, int64_t count,
                        void* workspace, size_t workspace_bytes, int accumulate, void* stream);

/* cf_reduce_sum without a workspace and without allocating: the stage-1
 * partial sums go to a static device array of 16 KiB (4096 floats, the most
 * any count needs; a count whose partials would not fit is
 * CF_ERR_INVALID_ARGUMENT), which each device holds until the process ends.
 * Same kernels, same result bits as cf_reduce_sum. Calls no hipMalloc /
 * hipFree. Every call on one device shares that device's array: calls that
 * overlap on one device (two streams, or two threads without ordering) race
 * and must be serialised by the caller. It has no counterpart in the
 * reference; it is for callers that cannot allocate: code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc. */
cf_status cf_reduce_sum_noalloc(const void* x, cf_dtype x_dtype, float* out, int64_t count,
                                int accumulate, void* stream);

/* Per-row sums of a row-major [rows, cols] matrix into fp32 `out[rows]`.
 * Replaces launch_row_sum (cuda/include/cudaforge/reduction.cuh:48). */
cf_status cf_row_sum(const void* x, cf_dtype x_dtype, float* out, int64_t rows, int64_t cols,
                     void* stream);

/* ---- LoRA linear -------------------------------------------------------- */

/* Bytes of workspace cf_lora_linear needs: the batch x rank adapter
 * intermediate (fp32). Replaces lora_workspace_bytes
 * (cuda/include/cudaforge/lora_linear.cuh:62). */
size_t cf_lora_workspace_bytes(int64_t batch, int64_t rank);

/* y = x @ w + scale * ((x @ a) @ b), the reference's operator layout
 * (cuda/include/cudaforge/lora_linear.cuh:26-31, python/cudaforge/ops.py:289-332):
 *   x [batch, in]   w [in, out]   a [in, rank]   b [rank, out]   y [batch, out]
 * all row-major and of one dtype (fp32 or bf16). fp32 accumulation; for bf16 the
 * adapter intermediate x @ a is rounded to bf16 before the up-projection, as the
 * reference's ATen path does. When `xa_out` is non-NULL the fp32 adapter
 * intermediate x @ a ([batch, rank], before that rounding) is also written
 * there (the autograd path keeps it for the backward). Any rank >= 0: bf16
 * problems with an even rank <= 16 run the fused MFMA kernel, fp32 problems
 * with rank <= 16 and in_features, out_features multiples of 4 the fp32 MFMA
 * kernel of cf_lora_linear_ws (one slice), every other case the unfused path
 * (cf_lora_workspace_bytes of xa_out required).
 * Replaces launch_lora_linear (cuda/include/cudaforge/lora_linear.cuh:49-51):
 * its `workspace` (batch x rank floats for the unfused variant) is `xa_out`,
 * and its `LoRAKernel variant` (Unfused, Fused: lora_linear.cuh:9-20) has no
 * counterpart - the path is chosen from dtype, shape and alignment. */
cf_status cf_lora_linear(const void* x, const void* w, const void* a, const void* b, void* y,
                         float* xa_out, cf_dtype dtype, int64_t batch, int64_t in_features,
                         int64_t out_features, int64_t rank, float scale, void* stream);

/* Workspace bytes cf_lora_linear_ws can use. fp32: to split the reduction of
 * a small problem across workgroups (0 when it would not split: large
 * outputs, shapes the fp32 MFMA kernel does not take). bf16 (shapes of the
 * fused MFMA kernel with rank > 0): a flag block and 8 KiB per 256 rows of x,
 * through which the output tiles that start late take x @ a from the first
 * tile of their rows instead of forming it again. It has no counterpart in
 * the reference, whose launcher's workspace is the batch x rank intermediate
 * (cuda/include/cudaforge/lora_linear.cuh:62). */
size_t cf_lora_linear_ws_bytes(cf_dtype dtype, int64_t batch, int64_t in_features,
                               int64_t out_features, int64_t rank);

/* cf_lora_linear with a workspace of cf_lora_linear_ws_bytes(...) bytes
 * (16-byte aligned, in any state; NULL when that is 0). fp32 problems with
 * rank <= 16 and in_features, out_features multiples of 4 run on the MFMA
 * units with each operand split into bf16 high and low parts (three products
 * per term, about 2^-16 relative error per product; fp32 accumulation), and a
 * small problem splits its reduction range across workgroups, partial results
 * summed in a fixed order (deterministic). bf16 problems on the fused kernel
 * share x @ a between output tiles through it; the output is bit-identical
 * to cf_lora_linear's. cf_lora_linear runs the same kernels without the split
 * and the sharing. Calls that overlap (other streams) need workspaces of
 * their own. Replaces launch_lora_linear
 * (cuda/include/cudaforge/lora_linear.cuh:49-51) for callers that can give
 * it a workspace. */
cf_status cf_lora_linear_ws(const void* x, const void* w, const void* a, const void* b, void* y,
                            float* xa_out, cf_dtype dtype, int64_t batch, int64_t in_features,
                            int64_t out_features, int64_t rank, float scale, void* workspace,
                            size_t workspace_bytes, void* stream);

/* c[m, n] = a[m, k] @ b[k, n], row-major, one dtype (fp32 or bf16), fp32
 * accumulation. Replaces launch_matmul (cuda/include/cudaforge/lora_linear.cuh:57-58). */
cf_status cf_matmul(const void* a, const void* b, void* c, cf_dtype dtype, int64_t m, int64_t n,
                    int64_t k, void* stream);

/* Bytes of workspace cf_lora_backward needs. The reference has no backward
 * kernel to size (cpp/src/bindings.cpp:369-377 guards the operator instead). */
size_t cf_lora_backward_workspace_bytes(int64_t batch, int64_t in_features, int64_t out_features,
                                        int64_t rank);

/* Adapter gradients of y = x @ w + scale * (x @ a) @ b, op layout:
 *   grad_a [in, rank]  = scale * x^T (dy @ b^T)
 *   grad_b [rank, out] = scale * (x @ a)^T dy
 * `xa` is the fp32 adapter intermediate x @ a [batch, rank] from the forward
 * (cf_lora_linear's xa_out); the bf16 path rounds it to bf16 first, as the
 * reference's ATen autograd sees the bf16 tensor. Gradients are written in
 * `dtype` (fp32 or bf16) after fp32 accumulation. These are the derivatives
 * ATen autograd produces for _lora_linear_reference (python/cudaforge/ops.py:178-185,
 * tests/python/test_autograd.py:81-91); the reference has no backward kernel
 * and guards the operator instead (cpp/src/bindings.cpp:369-377). */
cf_status cf_lora_backward(const void* x, const void* dy, const void* b, const float* xa,
                           void* grad_a, void* grad_b, cf_dtype dtype, int64_t batch,
                           int64_t in_features, int64_t out_features, int64_t rank, float scale,
                           void* workspace, size_t workspace_bytes, void* stream);

/* ---- elementwise activations ------------------------------------------- */

/* silu(x) = x * sigmoid(x), fp32 arithmetic for every dtype.
 * Replaces launch_silu (cuda/include/cudaforge/activations.cuh:25). */
cf_status cf_silu(const void* x, void* y, cf_dtype dtype, int64_t count, void* stream);

/* GELU, tanh approximation, fp32 arithmetic.
 * Replaces launch_gelu (cuda/include/cudaforge/activations.cuh:77). */
cf_status cf_gelu(const void* x, void* y, cf_dtype dtype, int64_t count, void* stream);

/* silu(gate) * up, fp32 arithmetic, one rounding to the storage type.
 * Replaces launch_swiglu / launch_swiglu_half / launch_swiglu_bf16
 * (cuda/include/cudaforge/activations.cuh:47-70). */
cf_status cf_swiglu(const void* gate, const void* up, void* y, cf_dtype dtype, int64_t count,
                    void* stream);

/* ---- fp32 matmul on the matrix cores --------------------------------------- */

/* 1: this build's fp32 matmul runs on the bf16 MFMA units (every gfx950 device
 * has them). Replaces tensor_cores_available
 * (cuda/include/cudaforge/tensor_core_matmul.cuh:44). */
int cf_tensor_cores_available(void);

/* 1 when cf_matmul_tensor_core takes this shape: m, k >= 1 and n a positive
 * multiple of 8 (the reference also required m, n multiples of 16 and k of 8).
 * Replaces tensor_core_shape_supported
 * (cuda/include/cudaforge/tensor_core_matmul.cuh:51). */
int cf_matmul_tensor_core_shape_supported(int64_t m, int64_t n, int64_t k);

/* Workspace for the bf16 operand parts and, for small outputs, the fp32
 * partial products of the split reduction range (2-8 slices); the size covers
 * whichever of the two kernels below the call takes (0 for an unsupported
 * shape). It has no counterpart in the reference, whose TF32 kernel read fp32
 * directly. */
size_t cf_matmul_tensor_core_workspace_bytes(int64_t m, int64_t n, int64_t k);

/* c[m, n] = a[m, k] b[k, n], row-major fp32, on the bf16 MFMA units: each
 * operand is split into bf16 high and low parts and the three significant
 * cross products are accumulated in fp32 (about 16 significant bits per
 * product; the reference's TF32 kept 11). Outputs of fewer than 64 256 x 256
 * tiles with a 16-byte aligned and k a multiple of 4 split the operands while
 * staging them (one launch, or two with a split reduction range); the rest
 * write the bf16 parts to the workspace and run one bf16 GEMM over them. b, c
 * and the workspace 16-byte aligned. An unsupported shape is CF_ERR_UNSUPPORTED
 * without launching, where the reference returned false.
 * Replaces launch_matmul_tensor_core (cuda/include/cudaforge/tensor_core_matmul.cuh:40-41). */
cf_status cf_matmul_tensor_core(const float* a, const float* b, float* c, int64_t m, int64_t n,
                                int64_t k, void* workspace, size_t workspace_bytes, void* stream);

/* ---- fp8 matmul on the matrix cores ------------------------------------- */

/* 1 when cf_matmul_fp8 takes this shape: m >= 1, k a positive multiple of
 * 128, n a positive multiple of 16, k * n < 2^31. It has no counterpart in
 * the reference (no fp8 path there); it is the fp8 half of the MFMA matmul that
 * replaces the TF32 demonstration (cuda/include/cudaforge/tensor_core_matmul.cuh:40-41). */
int cf_matmul_fp8_shape_supported(int64_t m, int64_t n, int64_t k);

/* y[m, n] = bf16(scale * (x[m, k] w[k, n])) for row-major OCP e4m3fn codes x
 * and w (one byte each), fp32 accumulation on the fp8 MFMA units, bf16 y; scale
 * is the product of the operands' per-tensor dequantisation scales. x, w and y
 * 16-byte aligned. An unsupported shape is CF_ERR_UNSUPPORTED without
 * launching. No workspace, no allocation. It has no counterpart in the
 * reference, which has no fp8 path. */
cf_status cf_matmul_fp8(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k,
                        float scale, void* stream);

/* 1 when cf_matmul_fp8_wt takes this shape: m >= 1, k a positive multiple of
 * 128, n a positive multiple of 16, 256 k < 2^31. It has no counterpart in
 * the reference (no fp8 path there). */
int cf_matmul_fp8_wt_shape_supported(int64_t m, int64_t n, int64_t k);

/* cf_matmul_fp8 with the right operand K-major: y[m, n] = bf16(scale * (x[m, k]
 * w_t[n, k]^T)), w_t row-major [n, k] (the weight layout of a torch Linear and
 * the operand order fp8 GEMM libraries take). Both operands then stream into
 * LDS as whole row lines and need no transposing reads. Same numerics,
 * alignment and error behaviour as cf_matmul_fp8; no workspace, no
 * allocation. It has no counterpart in the reference, which has no fp8 path. */
cf_status cf_matmul_fp8_wt(const void* x, const void* w_t, void* y, int64_t m, int64_t n, int64_t k,
                           float scale, void* stream);

/* ---- paged-attention decode ---------------------------------------------- */

/* Workspace bytes cf_paged_attention uses to split long contexts across
 * workgroups (0 when it would not split). max_context is
 * max_blocks_per_sequence * block_size. It has no counterpart in the reference,
 * whose kernel is one workgroup per (sequence, head) with no split. */
size_t cf_paged_attention_workspace_bytes(int64_t num_sequences, int64_t num_heads,
                                          int64_t num_kv_heads, int64_t head_dim,
                                          int64_t block_size, int64_t max_blocks_per_sequence);

/* Attention for one decode step over a paged KV cache: query / out
 * [num_sequences, num_heads, head_dim], k_cache / v_cache [num_blocks,
 * block_size, num_kv_heads, head_dim], block_tables [num_sequences,
 * max_blocks_per_sequence] (uint32), context_lens [num_sequences] (int32);
 * dtype CF_F32 (the reference's type) or CF_BF16 for all four tensors, fp32
 * scores and softmax. Query head h reads KV head h / (num_heads / num_kv_heads).
 * An empty context writes zeros. Contexts longer than the table holds are read
 * only as far as the table reaches. `workspace` may be NULL (no context split)
 * or hold cf_paged_attention_workspace_bytes(...) bytes, 16-byte aligned.
 * num_heads not a multiple of num_kv_heads, or head_dim > 1024, is
 * CF_ERR_INVALID_ARGUMENT (the reference returned without launching).
 * Replaces launch_paged_attention (cuda/include/cudaforge/paged_attention.cuh:61-65). */
cf_status cf_paged_attention(const void* query, const void* k_cache, const void* v_cache,
                             const uint32_t* block_tables, const int32_t* context_lens, void* out,
                             cf_dtype dtype, int64_t num_sequences, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                             int64_t max_blocks_per_sequence, float scale, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---- causal attention products ------------------------------------------ */

/* scores[b, h, s, t] = sum_d q[b, s, h, d] * k[b, t, h, d] for t <= s: the
 * query @ key^T of examples/transformer_block.py:54 with the head transposes
 * folded into the addressing. q and k are [batch, seq, heads * head_dim] (the
 * projections' output), scores [batch, heads, seq, seq]; bfloat16, fp32
 * accumulation, one rounding. Only the causal half is computed: 128 x 128
 * tiles wholly above the diagonal are not written, and entries above the
 * diagonal inside a written tile hold their dot products. A causal softmax
 * (cf_softmax_scaled with causal_period = seq) reads none of them. head_dim
 * 32, 64, 96 or 128 and seq a multiple of 8; other shapes and dtypes are
 * CF_ERR_UNSUPPORTED. Tensors 16-byte aligned. It has no counterpart in the
 * reference, whose block runs this product through torch. */
cf_status cf_attention_scores_causal(const void* q, const void* k, void* scores, cf_dtype dtype,
                                     int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                                     void* stream);

/* out[b, s, h, d] = sum over t <= s of probs[b, h, s, t] * v[b, t, h, d]:
 * the weights @ value of examples/transformer_block.py:63, written straight
 * into the [batch, seq, heads * head_dim] layout the output projection takes.
 * probs [batch, heads, seq, seq]; entries above the diagonal are never read
 * as values. Same dtype, shape and alignment rules as
 * cf_attention_scores_causal. It has no counterpart in the reference. */
cf_status cf_attention_pv_causal(const void* probs, const void* v, void* out, cf_dtype dtype,
                                 int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                                 void* stream);

/* ---- measurement helper ------------------------------------------------- */

/* Plain device-to-device copy of `bytes` bytes through a streaming kernel
 * (16-byte loads and stores). It has no counterpart in the reference: it is
 * the known-size kernel used to calibrate hardware byte counters and to
 * measure the achievable HBM bandwidth next to the ops above. */
cf_status cf_copy_bytes(const void* src, void* dst, int64_t bytes, void* stream);

/* Reads `read_bytes` from `src` and writes read_bytes / `divisor` bytes
 * derived from them to `dst` (divisor 1, 2 or 4), with the fp32 quantiser's
 * access pattern (four 16-byte loads per lane, then the stores; one-shot
 * grid). Divisor 0 only reads (dst receives one 4-byte word per 16 KiB
 * read); divisor -1 only writes read_bytes bytes to dst with the same store
 * pattern (src unused, may be NULL); divisors -2 .. -5 also only write, one
 * 16-byte store per lane, with the non-temporal (-2), device-scope (-3),
 * both (-4) or no (-5) cache-policy bits (read_bytes under 4 GiB).
 * read_bytes must be a multiple of 16 KiB and the pointers used 16-byte
 * aligned. It has no counterpart in the
 * reference: it measures the streaming ceiling of a traffic mix (divisor 4
 * is the fp32 quantiser's 4 : 1) and of its read and write halves next to
 * the kernels that move them. */
cf_status cf_stream_bytes(const void* src, void* dst, int64_t read_bytes, int divisor, void* stream);

/* Arms the calling thread's next operator call into this library: its
 * kernel dispatches record their own timestamps on `start_event` and
 * `stop_event` (hipEvent_t, created by the caller with timing enabled), so
 * hipEventElapsedTime(start, stop) is the kernel execution time as a kernel
 * trace reports it, without the queue packets of an event pair recorded around
 * the call. Every kernel of the library launches through this hook; for an
 * entry point that launches several kernels (the two-stage sum, the adapter
 * backward, split-K matmuls and LoRA, context-split paged attention) the
 * interval runs from the first kernel's start to the last one's completion,
 * the gaps between them included. The events belong to the next operator
 * entry point the thread calls: one that returns without launching (empty
 * input, an invalid argument, an unsupported shape) disarms them, so they
 * never time a later, unrelated launch. Runtime calls (scheduler, pools) leave them armed. Both
 * NULL disarms. It has no counterpart in the reference, whose benchmarks
 * bracket each launch with an event pair (benchmarks/benchmark_kernels.cu:59-79). */
cf_status cf_time_next_launch(void* start_event, void* stop_event);

/* 1 while cf_time_next_launch() has events armed on the calling thread, else
 * 0. A diagnostic for the hook above; no counterpart in the reference. */
int cf_time_next_launch_armed(void);

/* ---- runtime: stream scheduler and caching pools ------------------------
 *
 * The C form of the reference's GpuScheduler / StreamLease
 * (cuda/include/cudaforge/gpu_scheduler.cuh:16-142, cuda/src/gpu_scheduler.cu)
 * and MemoryPool with its backends (cpp/include/cudaforge/memory_pool.hpp:76-216,
 * gpu_scheduler.cuh:150-258). C++ callers can use the same classes directly
 * from include/cudaforge_runtime.hpp and include/cudaforge_pool.hpp. A lease
 * is named by its stream index; the hipStream_t comes back as `void*`. Every
 * stream is non-blocking and at the default priority. Handles are not
 * reference counted: destroy each exactly once, after its last use. */

typedef struct cf_scheduler cf_scheduler;
typedef struct cf_pool cf_pool;

typedef struct cf_stream_stats {
    uint64_t batches_dispatched;
    uint64_t bytes_to_device;
    uint64_t bytes_to_host;
} cf_stream_stats;

typedef struct cf_pool_stats {
    uint64_t bytes_reserved;
    uint64_t bytes_in_use;
    uint64_t peak_bytes_in_use;
    uint64_t allocation_count;
    uint64_t backend_allocations;
    uint64_t reuse_count;
    uint64_t free_count;
    uint64_t free_block_count;
} cf_pool_stats;

typedef enum cf_pool_backend {
    CF_POOL_HOST = 0,         /* malloc / free ("host")                     */
    CF_POOL_DEVICE = 1,       /* hipMalloc / hipFree ("device")             */
    CF_POOL_DEVICE_ASYNC = 2, /* hipMallocAsync / hipFreeAsync on a stream ("device-async") */
    CF_POOL_PINNED = 3,       /* hipHostMalloc / hipHostFree ("pinned")     */
} cf_pool_backend;

/* A scheduler owning `stream_count` (>= 1) streams on `device`; 0 streams is
 * CF_ERR_INVALID_ARGUMENT, as the reference's std::invalid_argument.
 * Replaces GpuScheduler::GpuScheduler (cuda/src/gpu_scheduler.cu:10-33). */
cf_status cf_scheduler_create(int64_t stream_count, int device, cf_scheduler** out);

/* Waits for every stream, then releases them.
 * Replaces GpuScheduler::~GpuScheduler (cuda/src/gpu_scheduler.cu:35-43). */
cf_status cf_scheduler_destroy(cf_scheduler* scheduler);

/* Next stream in round-robin order: its index and hipStream_t. Never blocks.
 * Replaces GpuScheduler::acquire (cuda/src/gpu_scheduler.cu:45-49). */
cf_status cf_scheduler_acquire(cf_scheduler* scheduler, int64_t* index, void** stream);

/* hipStream_t of stream `index`.
 * Replaces StreamLease::stream (cuda/include/cudaforge/gpu_scheduler.cuh:41). */
cf_status cf_scheduler_stream(const cf_scheduler* scheduler, int64_t index, void** stream);

/* Number of streams. Replaces GpuScheduler::stream_count
 * (cuda/include/cudaforge/gpu_scheduler.cuh:127). */
int64_t cf_scheduler_stream_count(const cf_scheduler* scheduler);

/* Asynchronous host-to-device / device-to-host copy on stream `index`,
 * counted in that stream's statistics; 0 bytes is a no-op. Replaces
 * GpuScheduler::copy_to_device / copy_to_host (cuda/src/gpu_scheduler.cu:51-73). */
cf_status cf_scheduler_copy_to_device(cf_scheduler* scheduler, int64_t index, void* device,
                                      const void* host, size_t bytes);
cf_status cf_scheduler_copy_to_host(cf_scheduler* scheduler, int64_t index, void* host,
                                    const void* device, size_t bytes);

/* Records stream `index`'s completion event on it.
 * Replaces StreamLease::record_completion (cuda/include/cudaforge/gpu_scheduler.cuh:47). */
cf_status cf_scheduler_record_completion(cf_scheduler* scheduler, int64_t index);

/* Stream `waiter` waits (on the device) for the last completion recorded on
 * stream `signaller`. Replaces GpuScheduler::chain (cuda/src/gpu_scheduler.cu:75-77). */
cf_status cf_scheduler_chain(cf_scheduler* scheduler, int64_t waiter, int64_t signaller);

/* Counts one dispatched batch on stream `index`.
 * Replaces GpuScheduler::note_dispatch (cuda/src/gpu_scheduler.cu:79-82). */
cf_status cf_scheduler_note_dispatch(cf_scheduler* scheduler, int64_t index);

/* Blocks until stream `index` is idle. Replaces StreamLease::synchronize
 * (cuda/include/cudaforge/gpu_scheduler.cuh:51). */
cf_status cf_scheduler_synchronize(cf_scheduler* scheduler, int64_t index);

/* *complete = 1 once everything issued to stream `index` has finished
 * (StreamLease::complete, gpu_scheduler.cuh:53), or, for the event query, once
 * its last recorded completion event has (CudaEvent::query via
 * StreamLease::completion_event, gpu_scheduler.cuh:42). */
cf_status cf_scheduler_query(cf_scheduler* scheduler, int64_t index, int* complete);
cf_status cf_scheduler_event_query(cf_scheduler* scheduler, int64_t index, int* complete);

/* Blocks until every stream is idle (shutdown, not per batch).
 * Replaces GpuScheduler::synchronize_all (cuda/src/gpu_scheduler.cu:84-91). */
cf_status cf_scheduler_synchronize_all(cf_scheduler* scheduler);

/* Copies up to `capacity` per-stream records into `per_stream` (may be NULL
 * when capacity is 0) and their sums into `totals` (batches_dispatched holds
 * the total dispatch count). Replaces GpuScheduler::stats
 * (cuda/src/gpu_scheduler.cu:93-105). */
cf_status cf_scheduler_stats(const cf_scheduler* scheduler, cf_stream_stats* per_stream,
                             int64_t capacity, cf_stream_stats* totals);

/* 1 when the current device backs hipMallocAsync with a memory pool.
 * Replaces supports_stream_ordered_allocation
 * (cuda/include/cudaforge/gpu_scheduler.cuh:175-186). */
int cf_stream_ordered_allocation_supported(void);

/* A caching pool over `backend`; `stream` is used by CF_POOL_DEVICE_ASYNC only
 * (its allocations and frees are ordered on it). Sizes round up to a power of
 * two, never below `min_block_bytes` (0 is CF_ERR_INVALID_ARGUMENT).
 * Replaces MemoryPool::MemoryPool (cpp/include/cudaforge/memory_pool.hpp:78-84)
 * with DeviceAllocatorBackend, StreamOrderedAllocatorBackend,
 * PinnedAllocatorBackend (gpu_scheduler.cuh:150-258) or HostAllocatorBackend
 * (memory_pool.hpp:209-216). */
cf_status cf_pool_create(cf_pool_backend backend, void* stream, size_t min_block_bytes,
                         cf_pool** out);

/* Returns every block, cached or checked out, to the backend.
 * Replaces MemoryPool::~MemoryPool (cpp/include/cudaforge/memory_pool.hpp:94). */
cf_status cf_pool_destroy(cf_pool* pool);

/* *out = a block of at least `bytes` bytes (NULL for 0 bytes). CF_ERR_OUT_OF_MEMORY
 * where the reference threw std::bad_alloc; the pool stays usable (trim and
 * retry). Replaces MemoryPool::allocate (cpp/include/cudaforge/memory_pool.hpp:96-123). */
cf_status cf_pool_allocate(cf_pool* pool, size_t bytes, void** out);

/* Returns a block to its free list; NULL is a no-op, a pointer the pool did not
 * hand out is CF_ERR_INVALID_ARGUMENT. Replaces MemoryPool::deallocate
 * (cpp/include/cudaforge/memory_pool.hpp:128-145). */
cf_status cf_pool_deallocate(cf_pool* pool, void* pointer);

/* Hands cached blocks back to the backend.
 * Replaces MemoryPool::trim (cpp/include/cudaforge/memory_pool.hpp:150-160). */
cf_status cf_pool_trim(cf_pool* pool);

/* Replaces MemoryPool::stats (cpp/include/cudaforge/memory_pool.hpp:162-165). */
cf_status cf_pool_get_stats(const cf_pool* pool, cf_pool_stats* out);

/* "host", "device", "device-async" or "pinned" (NULL for an unknown value).
 * Replaces MemoryPool::backend_name (cpp/include/cudaforge/memory_pool.hpp:167). */
const char* cf_pool_backend_name(cf_pool_backend backend);

#ifdef __cplusplus
}
#endif

#pragma GCC visibility pop

#endif /* CUDAFORGE_HIP_H */

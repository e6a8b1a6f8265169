// fp32 matmul on the bf16 MFMA units: C[m, n] = A[m, k] B[k, n], row-major.
//
// The reference's launch_matmul_tensor_core (cuda/include/cudaforge/
// tensor_core_matmul.cuh:7-53, cuda/src/tensor_core_matmul.cu) keeps an fp32
// interface and runs TF32 WMMA (10 mantissa bits per operand). gfx950 has no
// TF32 matrix instruction; its fast matrix path is bf16 (8 bits). So each
// operand is split into two bf16 parts, a = hi + lo with hi = bf16(a) and
// lo = bf16(a - hi), and
//
//     A B ~= A_hi B_hi + A_hi B_lo + A_lo B_hi
//
// (the dropped A_lo B_lo term and the split residue are ~2^-16 relative), which
// is one bf16 GEMM over a reduction three times as long:
//
//     A' = [A_hi | A_hi | A_lo]   [m, 3 kp]      B' = [B_hi; B_lo; B_hi]   [3 kp, n]
//
// with each third zero-padded from k to kp = ceil(k / 64) * 64, the K-step of
// the fused MFMA kernel (cf_lora_fused.hip, fp32-output variant). The result
// is more accurate than TF32 (about 16 significant bits per product against
// 11) at three bf16 MFMA passes; A' and B' live in a caller workspace.
//
// Shapes: any m and k; n a multiple of 8 (16-byte output rows), and the
// tensors 16-byte aligned. The reference accepted m, n multiples of 16 and k
// a multiple of 8; every shape it took is taken here.
#include "cf_common.hpp"
#include "cf_lora_fused.hpp"

namespace cf {
namespace {

constexpr int64_t kPad = 64;  // K granule of the MFMA kernel

int64_t padded_k(int64_t k) { return ceil_div<int64_t>(k, kPad) * kPad; }

__device__ __forceinline__ void split_bf16(float a, uint32_t& hi, uint32_t& lo) {
    hi = f32_to_bf16_bits(a);
    lo = f32_to_bf16_bits(a - __uint_as_float(hi << 16));
}

/// A' [m][3 kp]: thread -> 4 consecutive columns of one row.
__global__ void split_rows_kernel(const float* __restrict__ a, uint16_t* __restrict__ out, int64_t m,
                                  int64_t k, int64_t kp) {
    const int64_t quads_per_row = 3 * kp / 4;
    const int64_t total = m * quads_per_row;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = idx / quads_per_row;
        const int64_t col = (idx % quads_per_row) * 4;
        const int64_t part = col / kp;  // 0, 1: hi; 2: lo
        const int64_t j = col % kp;
        uint32_t bits[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = j + e < k ? a[row * k + j + e] : 0.0f;
            uint32_t hi;
            uint32_t lo;
            split_bf16(v, hi, lo);
            bits[e] = part == 2 ? lo : hi;
        }
        uint2 packed;
        packed.x = bits[0] | (bits[1] << 16);
        packed.y = bits[2] | (bits[3] << 16);
        *reinterpret_cast<uint2*>(out + row * 3 * kp + col) = packed;
    }
}

/// B' [3 kp][n]: thread -> 4 consecutive columns of one row.
__global__ void split_cols_kernel(const float* __restrict__ b, uint16_t* __restrict__ out, int64_t k,
                                  int64_t n, int64_t kp) {
    const int64_t quads_per_row = n / 4;
    const int64_t total = 3 * kp * quads_per_row;
    for (int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = idx / quads_per_row;  // 0 .. 3 kp - 1
        const int64_t col = (idx % quads_per_row) * 4;
        const int64_t part = row / kp;  // 0, 2: hi; 1: lo
        const int64_t j = row % kp;
        float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
        if (j < k) v = *reinterpret_cast<const float4*>(b + j * n + col);
        const float vals[4] = {v.x, v.y, v.z, v.w};
        uint32_t bits[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            uint32_t hi;
            uint32_t lo;
            split_bf16(vals[e], hi, lo);
            bits[e] = part == 1 ? lo : hi;
        }
        uint2 packed;
        packed.x = bits[0] | (bits[1] << 16);
        packed.y = bits[2] | (bits[3] << 16);
        *reinterpret_cast<uint2*>(out + row * n + col) = packed;
    }
}

int split_grid(int64_t quads) {
    const int64_t blocks = ceil_div<int64_t>(quads, kDefaultBlockSize);
    const int64_t cap = static_cast<int64_t>(cu_count()) * 16;
    return static_cast<int>(blocks < cap ? blocks : cap);
}

}  // namespace
}  // namespace cf

extern "C" {

int cf_tensor_cores_available(void) { return 1; }

int cf_matmul_tensor_core_shape_supported(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 8 != 0) return 0;
    const int64_t kk = 3 * cf::padded_k(k);
    // The MFMA kernel's 32-bit buffer offsets: B' and one 256-row panel of A'.
    return kk * n * 2 < (1LL << 31) && 256 * kk * 2 < (1LL << 31) ? 1 : 0;
}

size_t cf_matmul_tensor_core_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (!cf_matmul_tensor_core_shape_supported(m, n, k)) return 0;
    const int64_t kk = 3 * cf::padded_k(k);
    const size_t a_bytes = static_cast<size_t>(m * kk) * 2;
    return ((a_bytes + 255) / 256) * 256 + static_cast<size_t>(kk * n) * 2;
}

cf_status cf_matmul_tensor_core(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                                void* workspace, size_t workspace_bytes, void* stream) {
    if (!cf_matmul_tensor_core_shape_supported(m, n, k)) {
        return cf::fail(CF_ERR_UNSUPPORTED,
                        "cf_matmul_tensor_core: shape %lld x %lld x %lld is not tiled (n must be a "
                        "positive multiple of 8)",
                        static_cast<long long>(m), static_cast<long long>(n), static_cast<long long>(k));
    }
    if (a == nullptr || b == nullptr || c == nullptr || workspace == nullptr) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT, "cf_matmul_tensor_core: null pointer");
    }
    if (!cf::host_aligned(b, 16) || !cf::host_aligned(c, 16) || !cf::host_aligned(workspace, 16)) {
        return cf::fail(CF_ERR_UNSUPPORTED, "cf_matmul_tensor_core: b, c and the workspace must be 16-byte aligned");
    }
    if (workspace_bytes < cf_matmul_tensor_core_workspace_bytes(m, n, k)) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT, "cf_matmul_tensor_core: workspace of %zu bytes, %zu needed",
                        workspace_bytes, cf_matmul_tensor_core_workspace_bytes(m, n, k));
    }
    const int64_t kp = cf::padded_k(k);
    const size_t a_bytes = static_cast<size_t>(m * 3 * kp) * 2;
    auto* a_split = static_cast<uint16_t*>(workspace);
    auto* b_split = reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(workspace) + ((a_bytes + 255) / 256) * 256);
    auto s = static_cast<hipStream_t>(stream);
    cf::split_rows_kernel<<<cf::split_grid(m * 3 * kp / 4), cf::kDefaultBlockSize, 0, s>>>(a, a_split, m, k, kp);
    cf::split_cols_kernel<<<cf::split_grid(3 * kp * n / 4), cf::kDefaultBlockSize, 0, s>>>(b, b_split, k, n, kp);
    const cf_status split = cf::check_launch("splitting the fp32 operands into bf16 parts", s);
    if (split != CF_OK) return split;
    return cf::launch_matmul_bf16_f32out(a_split, b_split, c, m, n, 3 * kp, s);
}

}  // extern "C"

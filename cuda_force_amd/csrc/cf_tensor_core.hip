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
// Small outputs (fewer than 64 of these 256 x 256 tiles) with 16-byte aligned
// operands and k a multiple of 4 take the kernel of cf_matmul_f32.hip
// instead: 128 x 128 tiles that split the operands on their way into LDS, no
// split pass, fixed-order split K. Otherwise small outputs split K here: with
// few 256 x 256 output tiles (1024 x 1024 is 16 tiles, 16 of 256 CUs), the K'
// range is cut into up to 8 slices (at most 256 workgroups); each slice
// writes an fp32 partial product into the workspace and sum_splits_kernel
// adds them in slice order (the result is deterministic and independent of
// the device). Both operand splits run as one launch.
//
// Shapes: any m and k; n a multiple of 8 (16-byte output rows), and the
// tensors 16-byte aligned. The reference accepted m, n multiples of 16 and k
// a multiple of 8; every shape it took is taken here.
#include "cf_common.hpp"
#include "cf_lora_fused.hpp"
#include "cf_matmul_f32.hpp"

namespace cf {
namespace {

constexpr int64_t kPad = 64;          // K granule of the MFMA kernel
constexpr int64_t kTile = 256;        // output tile edge of the MFMA kernel
// Measured on MI355X: 1024^3 runs fastest with 8 slices (128 workgroups;
// 16 slices: 10% slower), 2048^3 with 4 (256 workgroups; 2 slices: 17%
// slower).
constexpr int64_t kSplitTarget = 256;  // workgroups split K may fill
constexpr int kMaxSplits = 8;

int64_t padded_k(int64_t k) { return ceil_div<int64_t>(k, kPad) * kPad; }

/// Slices of the K' = 3 kp range: the largest power of two up to 8 that
/// divides K' into whole granules and keeps tiles x slices <= 256. A
/// function of the shape alone.
int k_splits(int64_t m, int64_t n, int64_t kk) {
    const int64_t tiles = ceil_div<int64_t>(m, kTile) * ceil_div<int64_t>(n, kTile);
    const int64_t granules = kk / kPad;
    int splits = 1;
    for (int s = 2; s <= kMaxSplits; s *= 2) {
        if (tiles * s <= kSplitTarget && granules % s == 0) splits = s;
    }
    return splits;
}

/// True when the split-while-staging kernel (128 x 128 tiles, cf_matmul_f32.hip)
/// is the faster path: fewer than 64 of this path's 256 x 256 output tiles.
/// Measured (us): 1024^3 36.5 -> 24.7-26.7, 128 x 4096 x 4096 93 -> 39,
/// 512^3 25 -> 15; from 2048^3 (64 tiles: 92 against 94-98) and 8192 x 1024 x
/// 4096 (128 tiles: 316 against 327) up, and at 4096^3 (406 against 613),
/// this path is.
bool tensor_core_prefers_staged(int64_t m, int64_t n) {
    return ceil_div<int64_t>(m, kTile) * ceil_div<int64_t>(n, kTile) < 64;
}

/// c = sum over slices of part[s] (s = 0, 1, ...), four floats per thread.
__global__ void sum_splits_kernel(const float4* __restrict__ part, float4* __restrict__ c,
                                  int64_t quads, int splits) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < quads;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        float4 total = part[i];
        for (int s = 1; s < splits; ++s) {
            const float4 v = part[s * quads + i];
            total.x += v.x;
            total.y += v.y;
            total.z += v.z;
            total.w += v.w;
        }
        c[i] = total;
    }
}

/// A' [m][3 kp] element quad q (4 consecutive columns of one row).
__device__ __forceinline__ void split_row_quad(const float* __restrict__ a, uint16_t* __restrict__ out,
                                               int64_t k, int64_t kp, int64_t q) {
    const int64_t quads_per_row = 3 * kp / 4;
    const int64_t row = q / quads_per_row;
    const int64_t col = (q % quads_per_row) * 4;
    const int64_t part = col / kp;  // 0, 1: hi; 2: lo
    const int64_t j = col % kp;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = j + e < k ? a[row * k + j + e] : 0.0f;
    uint2 hi;
    uint2 lo;
    split_pk4(v[0], v[1], v[2], v[3], hi, lo);
    *reinterpret_cast<uint2*>(out + row * 3 * kp + col) = part == 2 ? lo : hi;
}

/// B' [3 kp][n] element quad q (4 consecutive columns of one row).
__device__ __forceinline__ void split_col_quad(const float* __restrict__ b, uint16_t* __restrict__ out,
                                               int64_t k, int64_t n, int64_t kp, int64_t q) {
    const int64_t quads_per_row = n / 4;
    const int64_t row = q / quads_per_row;  // 0 .. 3 kp - 1
    const int64_t col = (q % quads_per_row) * 4;
    const int64_t part = row / kp;  // 0, 2: hi; 1: lo
    const int64_t j = row % kp;
    float4 v = float4{0.0f, 0.0f, 0.0f, 0.0f};
    if (j < k) v = *reinterpret_cast<const float4*>(b + j * n + col);
    uint2 hi;
    uint2 lo;
    split_pk4(v.x, v.y, v.z, v.w, hi, lo);
    *reinterpret_cast<uint2*>(out + row * n + col) = part == 1 ? lo : hi;
}

/// Both operand splits in one launch: quads [0, a_quads) of the grid-stride
/// range are A', the rest B'.
__global__ void split_operands_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                      uint16_t* __restrict__ a_out, uint16_t* __restrict__ b_out,
                                      int64_t m, int64_t n, int64_t k, int64_t kp) {
    const int64_t a_quads = m * 3 * kp / 4;
    const int64_t total = a_quads + 3 * kp * n / 4;
    for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; q < total;
         q += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (q < a_quads) {
            split_row_quad(a, a_out, k, kp, q);
        } else {
            split_col_quad(b, b_out, k, n, kp, q - a_quads);
        }
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
    const size_t b_bytes = static_cast<size_t>(kk * n) * 2;
    const int splits = cf::k_splits(m, n, kk);
    const size_t part_bytes = splits > 1 ? static_cast<size_t>(splits) * m * n * 4 : 0;
    const size_t split_path = ((a_bytes + 255) / 256) * 256 + ((b_bytes + 255) / 256) * 256 + part_bytes;
    // The split-while-staging kernel (taken for small outputs with 16-byte
    // aligned operands and k a multiple of 4) needs only its slices' partial
    // outputs; the query covers whichever path the call takes.
    const size_t staged_path = cf::matmul_f32_workspace_bytes(m, n, cf::matmul_f32_splits(m, n, k));
    return split_path > staged_path ? split_path : staged_path;
}

cf_status cf_matmul_tensor_core(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                                void* workspace, size_t workspace_bytes, void* stream) {
    CF_ENTRY();
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
    auto s = static_cast<hipStream_t>(stream);
    if (cf::matmul_f32_eligible(a, b, c, m, n, k) && cf::tensor_core_prefers_staged(m, n)) {
        return cf::launch_matmul_f32(a, b, c, m, n, k, cf::matmul_f32_splits(m, n, k), workspace, s);
    }
    const int64_t kp = cf::padded_k(k);
    const size_t a_bytes = static_cast<size_t>(m * 3 * kp) * 2;
    const size_t b_bytes = static_cast<size_t>(3 * kp * n) * 2;
    auto* a_split = static_cast<uint16_t*>(workspace);
    auto* b_split = reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(workspace) + ((a_bytes + 255) / 256) * 256);
    auto* partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + ((a_bytes + 255) / 256) * 256 +
                                              ((b_bytes + 255) / 256) * 256);
    const int splits = cf::k_splits(m, n, 3 * kp);
    cf::launch(cf::split_operands_kernel, dim3(cf::split_grid(m * 3 * kp / 4 + 3 * kp * n / 4)),
               dim3(cf::kDefaultBlockSize), 0, s, a, b, a_split, b_split, m, n, k, kp);
    const cf_status split = cf::check_launch("splitting the fp32 operands into bf16 parts", s);
    if (split != CF_OK) return split;
    if (splits == 1) return cf::launch_matmul_bf16_f32out(a_split, b_split, c, m, n, 3 * kp, 1, s);
    const cf_status gemm = cf::launch_matmul_bf16_f32out(a_split, b_split, partials, m, n, 3 * kp, splits, s);
    if (gemm != CF_OK) return gemm;
    const int64_t quads = m * n / 4;  // n is a multiple of 8
    cf::launch(cf::sum_splits_kernel, dim3(cf::split_grid(quads)), dim3(cf::kDefaultBlockSize), 0, s,
               reinterpret_cast<const float4*>(partials), reinterpret_cast<float4*>(c), quads, splits);
    return cf::check_launch("summing the split-K partial products", s);
}

}  // extern "C"

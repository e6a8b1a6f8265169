// LoRA linear (forward and adapter backward) and plain matmul for gfx950.
//
// Operator layout, as the reference's (cuda/include/cudaforge/lora_linear.cuh:26-31,
// python/cudaforge/ops.py:289-332), all row-major:
//   x [M, K]   w [K, N]   a [K, r]   b [r, N]   y [M, N]
//   y = x @ w + scale * ((x @ a) @ b)
//
// Fast path (bf16, K % 64 == 0, N % 8 == 0, r <= 16, 16-byte aligned): the
// fused MFMA kernel in cf_lora_fused.hip, one launch.
//
// fp32 (r <= 16, K and N multiples of 4, 16-byte aligned): the MFMA kernel of
// cf_lora_f32.hip, operands split into bf16 high and low parts on the way
// into LDS, one launch (plus a fixed-order sum when a workspace lets it split
// the reduction).
//
// Generic path (shapes neither fast path takes): x @ a into a fp32 [M, r]
// workspace (one wave per row), then a 64x64-tiled fp32 FMA GEMM whose
// epilogue adds scale * (xa @ b).
//
// Backward (adapter only, op layout):
//   G      = dy @ b^T            [M, r]
//   grad_b = scale * xa^T @ dy   [r, N]   column reduction over M
//   grad_a = scale * x^T @ G     [K, r]   column reduction over M
// bf16 with rank <= 16 runs the MFMA kernels of cf_lora_bwd.hip. The generic
// path here (fp32, other shapes): G one wave per row of dy, the column
// reductions in row chunks into an fp32 workspace and a second kernel summing
// the chunks in a fixed order (deterministic).
#include "cf_common.hpp"
#include "cf_lora_bwd.hpp"
#include "cf_lora_f32.hpp"
#include "cf_lora_fused.hpp"

namespace cf {
namespace {

// ---------------------------------------------------------------------------
// Generic path.
// ---------------------------------------------------------------------------

/// out[m, q] = sum_k x[m, k] * p[k * k_stride + q * q_stride] for q < rank,
/// fp32, one wave per row. Used for x @ a (k_stride = r, q_stride = 1) and
/// for dy @ b^T (k_stride = 1, q_stride = N).
template <typename T>
__global__ __launch_bounds__(kDefaultBlockSize) void row_dot_kernel(
    const T* __restrict__ x, const T* __restrict__ p, float* __restrict__ out, int64_t rows,
    int64_t inner, int64_t rank, int64_t k_stride, int64_t q_stride) {
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (kDefaultBlockSize / kWaveSize) +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * (kDefaultBlockSize / kWaveSize);
    for (int64_t row = wave; row < rows; row += waves) {
        const T* xr = x + row * inner;
        for (int64_t q0 = 0; q0 < rank; q0 += 16) {
            float acc[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
            for (int64_t k = lane; k < inner; k += kWaveSize) {
                const float xv = Storage<T>::load(xr + k);
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    if (q0 + q < rank) {
                        acc[q] += xv * Storage<T>::load(p + k * k_stride + (q0 + q) * q_stride);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float total = wave_reduce_f32<AddF32>(acc[q]);
                if (lane == 0 && q0 + q < rank) out[row * rank + q0 + q] = total;
            }
        }
    }
}

/// Round a float through the storage type T (identity for fp32).
template <typename T>
__device__ __forceinline__ float round_to(float v) {
    if constexpr (sizeof(typename Storage<T>::elem) == 4) {
        return v;
    } else {
        return Storage<T>::from_bits(Storage<T>::to_bits(v));
    }
}

constexpr int kGT = 64;   // generic output tile edge
constexpr int kGK = 16;   // generic K step

/// y = x @ w (+ scale * (round_T(xa) @ b) when xa != nullptr), 64x64 tile per
/// workgroup, 4x4 outputs per thread, fp32 FMA accumulation.
template <typename T>
__global__ __launch_bounds__(kDefaultBlockSize) void tiled_gemm_kernel(
    const T* __restrict__ x, const T* __restrict__ w, const float* __restrict__ xa,
    const T* __restrict__ b, T* __restrict__ y, int64_t M, int64_t N, int64_t K, int64_t rank,
    float scale) {
    __shared__ float as[kGK][kGT + 4];
    __shared__ float bs[kGK][kGT + 4];
    const int tid = static_cast<int>(threadIdx.x);
    const int ty = tid / 16;
    const int tx = tid % 16;
    const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kGT;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kGT;

    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    }

    for (int64_t k0 = 0; k0 < K; k0 += kGK) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = i * kDefaultBlockSize + tid;
            const int am = e / kGK;
            const int ak = e % kGK;
            const int64_t gm = m0 + am;
            const int64_t gk = k0 + ak;
            as[ak][am] = (gm < M && gk < K) ? Storage<T>::load(x + gm * K + gk) : 0.0f;
            const int bk = e / kGT;
            const int bn = e % kGT;
            const int64_t gk2 = k0 + bk;
            const int64_t gn = n0 + bn;
            bs[bk][bn] = (gk2 < K && gn < N) ? Storage<T>::load(w + gk2 * N + gn) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kGK; ++k) {
            float av[4];
            float bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = as[k][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = bs[k][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] += av[i] * bv[j];
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gm = m0 + ty * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gn = n0 + tx * 4 + j;
            if (gn >= N) continue;
            float v = acc[i][j];
            if (xa != nullptr) {
                float adapter = 0.0f;
                for (int64_t q = 0; q < rank; ++q) {
                    adapter += round_to<T>(xa[gm * rank + q]) * Storage<T>::load(b + q * N + gn);
                }
                v += scale * adapter;
            }
            Storage<T>::store(y + gm * N + gn, v);
        }
    }
}

// ---------------------------------------------------------------------------
// Backward: column reductions.
// ---------------------------------------------------------------------------

constexpr int kColThreads = 256;
constexpr int kColRowsPerChunk = 256;

/// part[chunk, q, n] = sum_{m in chunk} round_T(p[m, q]) * v[m, n] for
/// q < rank (<= 16 per launch slice q0). Each wave takes a quarter of the
/// chunk's rows for the same 64 columns per lane-group; the four waves are
/// combined through LDS.
template <typename T>
__global__ __launch_bounds__(kColThreads) void column_reduce_kernel(
    const float* __restrict__ p, const T* __restrict__ v, float* __restrict__ part, int64_t rows,
    int64_t cols, int64_t rank, int64_t q0) {
    __shared__ float red[kColThreads / kWaveSize][16][kWaveSize];
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int wave = static_cast<int>(threadIdx.x) / kWaveSize;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * kWaveSize + lane;
    const int64_t chunk = blockIdx.y;
    const int64_t row_begin = chunk * kColRowsPerChunk;
    const int64_t row_end =
        row_begin + kColRowsPerChunk < rows ? row_begin + kColRowsPerChunk : rows;
    float acc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.0f;
    if (n < cols) {
        for (int64_t m = row_begin + wave; m < row_end; m += kColThreads / kWaveSize) {
            const float vv = Storage<T>::load(v + m * cols + n);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                if (q0 + q < rank) acc[q] += round_to<T>(p[m * rank + q0 + q]) * vv;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) red[wave][q][lane] = acc[q];
    __syncthreads();
    if (wave == 0 && n < cols) {
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            if (q0 + q < rank) {
                const float total = (red[0][q][lane] + red[1][q][lane]) +
                                    (red[2][q][lane] + red[3][q][lane]);
                part[(chunk * rank + q0 + q) * cols + n] = total;
            }
        }
    }
}

/// out = scale * sum over chunks of part, written as [rank, cols] or, with
/// kTransposed, as [cols, rank].
template <typename T, bool kTransposed>
__global__ __launch_bounds__(kDefaultBlockSize) void column_finish_kernel(
    const float* __restrict__ part, T* __restrict__ out, int64_t chunks, int64_t rank,
    int64_t cols, float scale) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rank * cols) return;
    const int64_t q = i / cols;
    const int64_t n = i % cols;
    float total = 0.0f;
    for (int64_t c = 0; c < chunks; ++c) total += part[(c * rank + q) * cols + n];
    const int64_t dst = kTransposed ? n * rank + q : q * cols + n;
    Storage<T>::store(out + dst, scale * total);
}

template <typename T>
cf_status column_reduce(const float* p, const void* v, void* out, bool transposed, int64_t rows,
                        int64_t cols, int64_t rank, float scale, float* part, hipStream_t stream) {
    const int64_t chunks = ceil_div<int64_t>(rows, kColRowsPerChunk);
    const dim3 grid(static_cast<unsigned>(ceil_div<int64_t>(cols, kWaveSize)),
                    static_cast<unsigned>(chunks));
    for (int64_t q0 = 0; q0 < rank; q0 += 16) {
        launch(column_reduce_kernel<T>, dim3(grid), dim3(kColThreads), 0, stream, p,
               static_cast<const T*>(v), part, rows, cols, rank, q0);
    }
    const int64_t total = rank * cols;
    const unsigned fgrid = static_cast<unsigned>(ceil_div<int64_t>(total, kDefaultBlockSize));
    if (transposed) {
        launch(column_finish_kernel<T, true>, dim3(fgrid), dim3(kDefaultBlockSize), 0, stream, part,
               static_cast<T*>(out), chunks, rank, cols, scale);
    } else {
        launch(column_finish_kernel<T, false>, dim3(fgrid), dim3(kDefaultBlockSize), 0, stream,
               part, static_cast<T*>(out), chunks, rank, cols, scale);
    }
    return check_launch("launching the LoRA backward column reduction", stream);
}

template <typename T>
cf_status zero_gradients(void* grad_a, void* grad_b, int64_t in_features, int64_t out_features,
                         int64_t rank, hipStream_t stream) {
    if (in_features > 0) {
        const unsigned grid =
            static_cast<unsigned>(ceil_div<int64_t>(rank * in_features, kDefaultBlockSize));
        launch(column_finish_kernel<T, true>, dim3(grid), dim3(kDefaultBlockSize), 0, stream,
               nullptr, static_cast<T*>(grad_a), 0, rank, in_features, 1.0f);
    }
    if (out_features > 0) {
        const unsigned grid =
            static_cast<unsigned>(ceil_div<int64_t>(rank * out_features, kDefaultBlockSize));
        launch(column_finish_kernel<T, false>, dim3(grid), dim3(kDefaultBlockSize), 0, stream,
               nullptr, static_cast<T*>(grad_b), 0, rank, out_features, 1.0f);
    }
    return check_launch("zeroing the LoRA gradients", stream);
}

template <typename T>
void launch_row_dot(const void* x, const void* p, float* out, int64_t rows, int64_t inner,
                    int64_t rank, int64_t k_stride, int64_t q_stride, hipStream_t stream) {
    const int64_t max_waves = static_cast<int64_t>(cu_count()) * 16;
    const int64_t waves = rows < max_waves ? rows : max_waves;
    const int64_t grid = ceil_div<int64_t>(waves, kDefaultBlockSize / kWaveSize);
    launch(row_dot_kernel<T>, dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize), 0, stream,
           static_cast<const T*>(x), static_cast<const T*>(p), out, rows, inner, rank, k_stride,
           q_stride);
}

template <typename T>
cf_status launch_generic(const void* x, const void* w, const void* a, const void* b, void* y,
                         float* xa, int64_t M, int64_t N, int64_t K, int64_t rank, float scale,
                         hipStream_t stream) {
    if (rank > 0) {
        launch_row_dot<T>(x, a, xa, M, K, rank, rank, 1, stream);
    }
    const dim3 grid(static_cast<unsigned>(ceil_div<int64_t>(N, kGT)),
                    static_cast<unsigned>(ceil_div<int64_t>(M, kGT)));
    launch(tiled_gemm_kernel<T>, dim3(grid), dim3(kDefaultBlockSize), 0, stream,
           static_cast<const T*>(x), static_cast<const T*>(w),
           rank > 0 ? xa : nullptr, static_cast<const T*>(b), static_cast<T*>(y), M, N, K, rank, scale);
    return check_launch("launching the tiled LoRA GEMM", stream);
}

}  // namespace
}  // namespace cf

extern "C" {

size_t cf_lora_workspace_bytes(int64_t batch, int64_t rank) {
    if (batch <= 0 || rank <= 0) return 0;
    return static_cast<size_t>(batch) * static_cast<size_t>(rank) * sizeof(float);
}

cf_status cf_lora_linear(const void* x, const void* w, const void* a, const void* b, void* y,
                         float* xa_out, cf_dtype dtype, int64_t batch, int64_t in_features,
                         int64_t out_features, int64_t rank, float scale, void* stream) {
    CF_ENTRY();
    if (batch <= 0 || out_features <= 0) return CF_OK;
    CF_REQUIRE(in_features >= 0 && rank >= 0, "cf_lora_linear: negative dimension");
    CF_REQUIRE(x != nullptr && w != nullptr && y != nullptr, "cf_lora_linear: null pointer");
    CF_REQUIRE(rank == 0 || (a != nullptr && b != nullptr), "cf_lora_linear: null adapter");
    CF_REQUIRE(dtype == CF_F32 || dtype == CF_BF16,
               "cf_lora_linear: dtype %s has no kernel (float32 or bfloat16)",
               cf::dtype_name(dtype));
    auto s = static_cast<hipStream_t>(stream);
    if (dtype == CF_BF16 &&
        cf::lora_fused_eligible(x, w, a, b, batch, out_features, in_features, rank)) {
        return cf::launch_lora_fused(x, w, a, b, y, xa_out, batch, out_features, in_features, rank,
                                scale, nullptr, s);
    }
    if (dtype == CF_F32 &&
        cf::lora_f32_eligible(x, w, a, b, y, batch, out_features, in_features, rank)) {
        return cf::launch_lora_f32(static_cast<const float*>(x), static_cast<const float*>(w),
                                   static_cast<const float*>(a), static_cast<const float*>(b),
                                   static_cast<float*>(y), xa_out, batch, out_features, in_features,
                                   rank, scale, 1, nullptr, s);
    }
    CF_REQUIRE(rank == 0 || xa_out != nullptr,
               "cf_lora_linear: this shape takes the unfused path, which needs xa_out "
               "(cf_lora_workspace_bytes(batch, rank) bytes) as its workspace");
    if (dtype == CF_F32) {
        return cf::launch_generic<float>(x, w, a, b, y, xa_out, batch, out_features, in_features,
                                         rank, scale, s);
    }
    return cf::launch_generic<cf::bf16_t>(x, w, a, b, y, xa_out, batch, out_features, in_features,
                                          rank, scale, s);
}

size_t cf_lora_linear_ws_bytes(cf_dtype dtype, int64_t batch, int64_t in_features,
                               int64_t out_features, int64_t rank) {
    if (dtype == CF_BF16) {
        // The fused kernel's shapes (its pointer checks aside): x @ a shared
        // between the column tiles of a row tile.
        const bool fused_shape = batch > 0 && out_features > 0 && in_features > 0 &&
                                 in_features % 64 == 0 && out_features % 8 == 0 && rank > 0 &&
                                 rank <= 16 && rank % 2 == 0;
        return fused_shape ? cf::lora_fused_workspace_bytes(batch, rank) : 0;
    }
    if (dtype != CF_F32 || batch <= 0 || in_features <= 0 || out_features <= 0 || rank < 0 ||
        rank > 16 || in_features % 4 != 0 || out_features % 4 != 0) {
        return 0;
    }
    const int splits = cf::lora_f32_splits(batch, out_features, in_features);
    return cf::lora_f32_workspace_bytes(batch, out_features, rank, splits);
}

cf_status cf_lora_linear_ws(const void* x, const void* w, const void* a, const void* b, void* y,
                            float* xa_out, cf_dtype dtype, int64_t batch, int64_t in_features,
                            int64_t out_features, int64_t rank, float scale, void* workspace,
                            size_t workspace_bytes, void* stream) {
    CF_ENTRY();
    if (batch <= 0 || out_features <= 0) return CF_OK;
    CF_REQUIRE(in_features >= 0 && rank >= 0, "cf_lora_linear_ws: negative dimension");
    const size_t needed = cf_lora_linear_ws_bytes(dtype, batch, in_features, out_features, rank);
    if (needed > 0 && dtype == CF_BF16 &&
        cf::lora_fused_eligible(x, w, a, b, batch, out_features, in_features, rank)) {
        CF_REQUIRE(x != nullptr && w != nullptr && y != nullptr && a != nullptr && b != nullptr,
                   "cf_lora_linear_ws: null pointer");
        CF_REQUIRE(workspace != nullptr && workspace_bytes >= needed,
                   "cf_lora_linear_ws: workspace of %zu bytes given, %zu needed", workspace_bytes,
                   needed);
        CF_REQUIRE(cf::host_aligned(workspace, 16), "cf_lora_linear_ws: workspace must be 16-byte aligned");
        return cf::launch_lora_fused(x, w, a, b, y, xa_out, batch, out_features, in_features, rank,
                                     scale, workspace, static_cast<hipStream_t>(stream));
    }
    if (needed > 0 && dtype == CF_F32 &&
        cf::lora_f32_eligible(x, w, a, b, y, batch, out_features, in_features, rank)) {
        CF_REQUIRE(x != nullptr && w != nullptr && y != nullptr && (rank == 0 || (a != nullptr && b != nullptr)),
                   "cf_lora_linear_ws: null pointer");
        CF_REQUIRE(workspace != nullptr && workspace_bytes >= needed,
                   "cf_lora_linear_ws: workspace of %zu bytes given, %zu needed", workspace_bytes,
                   needed);
        CF_REQUIRE(cf::host_aligned(workspace, 16), "cf_lora_linear_ws: workspace must be 16-byte aligned");
        return cf::launch_lora_f32(static_cast<const float*>(x), static_cast<const float*>(w),
                                   static_cast<const float*>(a), static_cast<const float*>(b),
                                   static_cast<float*>(y), xa_out, batch, out_features, in_features,
                                   rank, scale, cf::lora_f32_splits(batch, out_features, in_features),
                                   workspace, static_cast<hipStream_t>(stream));
    }
    return cf_lora_linear(x, w, a, b, y, xa_out, dtype, batch, in_features, out_features, rank,
                          scale, stream);
}

cf_status cf_matmul(const void* a, const void* b, void* c, cf_dtype dtype, int64_t m, int64_t n,
                    int64_t k, void* stream) {
    CF_ENTRY();
    if (m <= 0 || n <= 0) return CF_OK;
    CF_REQUIRE(a != nullptr && b != nullptr && c != nullptr, "cf_matmul: null pointer");
    CF_REQUIRE(dtype == CF_F32 || dtype == CF_BF16, "cf_matmul: dtype %s has no kernel",
               cf::dtype_name(dtype));
    auto s = static_cast<hipStream_t>(stream);
    if (dtype == CF_BF16 && cf::lora_fused_eligible(a, b, nullptr, nullptr, m, n, k, 0)) {
        return cf::launch_lora_fused(a, b, nullptr, nullptr, c, nullptr, m, n, k, 0, 0.0f, nullptr, s);
    }
    if (dtype == CF_F32 && cf::lora_f32_eligible(a, b, nullptr, nullptr, c, m, n, k, 0)) {
        return cf::launch_lora_f32(static_cast<const float*>(a), static_cast<const float*>(b), nullptr,
                                   nullptr, static_cast<float*>(c), nullptr, m, n, k, 0, 0.0f, 1,
                                   nullptr, s);
    }
    if (dtype == CF_F32) {
        return cf::launch_generic<float>(a, b, nullptr, nullptr, c, nullptr, m, n, k, 0, 0.0f, s);
    }
    return cf::launch_generic<cf::bf16_t>(a, b, nullptr, nullptr, c, nullptr, m, n, k, 0, 0.0f, s);
}

size_t cf_lora_backward_workspace_bytes(int64_t batch, int64_t in_features, int64_t out_features,
                                        int64_t rank) {
    if (batch <= 0 || rank <= 0) return 0;
    const int64_t chunks = cf::ceil_div<int64_t>(batch, cf::kColRowsPerChunk);
    const int64_t widest = in_features > out_features ? in_features : out_features;
    const size_t g = static_cast<size_t>(batch * rank) * sizeof(float);
    const size_t part = static_cast<size_t>(chunks * rank * widest) * sizeof(float);
    const size_t generic = ((g + 255) / 256) * 256 + part;
    // Enough for either path: which one runs depends on dtype and alignment.
    const size_t fast = cf::lora_backward_fast_workspace_bytes(batch, in_features, out_features);
    return generic > fast ? generic : fast;
}

cf_status cf_lora_backward(const void* x, const void* dy, const void* b, const float* xa,
                           void* grad_a, void* grad_b, cf_dtype dtype, int64_t batch,
                           int64_t in_features, int64_t out_features, int64_t rank, float scale,
                           void* workspace, size_t workspace_bytes, void* stream) {
    CF_ENTRY();
    if (rank <= 0) return CF_OK;
    CF_REQUIRE(batch >= 0 && in_features >= 0 && out_features >= 0,
               "cf_lora_backward: negative dimension");
    CF_REQUIRE(dtype == CF_F32 || dtype == CF_BF16, "cf_lora_backward: dtype %s has no kernel",
               cf::dtype_name(dtype));
    CF_REQUIRE(grad_a != nullptr && grad_b != nullptr, "cf_lora_backward: null gradient output");
    if (batch == 0) {
        // Empty batch: both gradients are zero (a finish pass over zero chunks
        // writes them without reading anything).
        auto s0 = static_cast<hipStream_t>(stream);
        return dtype == CF_F32 ? cf::zero_gradients<float>(grad_a, grad_b, in_features,
                                                           out_features, rank, s0)
                               : cf::zero_gradients<cf::bf16_t>(grad_a, grad_b, in_features,
                                                                out_features, rank, s0);
    }
    CF_REQUIRE(x != nullptr && dy != nullptr && b != nullptr && xa != nullptr,
               "cf_lora_backward: null input");
    const size_t needed = cf_lora_backward_workspace_bytes(batch, in_features, out_features, rank);
    CF_REQUIRE(workspace != nullptr && workspace_bytes >= needed,
               "cf_lora_backward: workspace of %zu bytes given, %zu needed", workspace_bytes,
               needed);
    CF_REQUIRE(cf::host_aligned(workspace, 16), "cf_lora_backward: workspace must be 16-byte aligned");
    auto s = static_cast<hipStream_t>(stream);
    if (dtype == CF_BF16 && cf::lora_backward_fast_eligible(x, dy, b, batch, in_features,
                                                            out_features, rank)) {
        return cf::launch_lora_backward_fast(x, dy, b, xa, grad_a, grad_b, batch, in_features,
                                             out_features, rank, scale, workspace, s);
    }
    float* g = static_cast<float*>(workspace);
    const size_t g_bytes = ((static_cast<size_t>(batch * rank) * sizeof(float) + 255) / 256) * 256;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + g_bytes);
    if (dtype == CF_F32) {
        cf::launch_row_dot<float>(dy, b, g, batch, out_features, rank, 1, out_features, s);
        cf_status st = cf::column_reduce<float>(xa, dy, grad_b, false, batch, out_features, rank,
                                                scale, part, s);
        if (st != CF_OK) return st;
        return cf::column_reduce<float>(g, x, grad_a, true, batch, in_features, rank, scale, part,
                                        s);
    }
    cf::launch_row_dot<cf::bf16_t>(dy, b, g, batch, out_features, rank, 1, out_features, s);
    cf_status st = cf::column_reduce<cf::bf16_t>(xa, dy, grad_b, false, batch, out_features, rank,
                                                 scale, part, s);
    if (st != CF_OK) return st;
    return cf::column_reduce<cf::bf16_t>(g, x, grad_a, true, batch, in_features, rank, scale, part,
                                         s);
}

}  // extern "C"

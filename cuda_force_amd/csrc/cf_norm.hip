// RMSNorm and residual-add + RMSNorm for gfx950.
//
// Semantics: _rmsnorm_reference (python/cudaforge/ops.py:164-171),
//   y = (x * rsqrt(mean(x^2) + eps)) * w      fp32 arithmetic, eps inside the
//                                             sqrt, rounded once to the
//                                             storage type at the end,
// and _fused_residual_rmsnorm_reference (ops.py:188-192): r = x + residual in
// the storage type, then rmsnorm(r). rsqrt is taken as 1 / sqrt with IEEE
// sqrt and divide, the way ATen's CPU rsqrt computes it.
//
// Design (fast path for rows of 256, 512 or 1024 16-byte vectors with many
// rows): rmsnorm_tile_kernel, where a workgroup of 256 or 512 threads owns
// whole rows, each thread holds one to four 16-byte vectors, and each load
// instruction of the workgroup reads 4 or 8 KiB of contiguous memory; row
// sums meet in LDS. Otherwise one wavefront owns a row. The row is loaded once with
// 16-byte loads into registers (a 4096-wide bf16 row is 8 loads per lane),
// the sum of squares reduces with DPP inside the wave (no LDS, no barrier),
// and the row is scaled and stored from the same registers, so HBM sees one
// read and one write per element. The weight vector is staged once per
// workgroup in LDS (or, for ragged rows, read through the cache by each
// wave). The reference instead uses a
// block per row with a 32-lane shuffle tree and an LDS exchange, and re-reads
// the row for the normalising pass (cuda/src/rmsnorm.cu:46-83).
//
// Fallback: rows that do not fit the register tile, unaligned pointers or a
// row length that is not a whole number of 16-byte vectors use a workgroup per
// row that reads the row twice (the second pass hits L2).
#include "cf_common.hpp"

#include <type_traits>

namespace cf {
namespace {

constexpr int kWavesPerBlock = kDefaultBlockSize / kWaveSize;

/// rsqrt(mean + eps) from the row's sum of squares.
__device__ __forceinline__ float inv_rms(float sum_squares, int64_t cols, float eps) {
    const float mean = sum_squares / static_cast<float>(cols);
    return 1.0f / sqrtf(mean + eps);
}

/// One wave per kRows consecutive rows, one-shot grid: every load of the
/// wave's rows is issued before any arithmetic, rows and outputs stream with
/// nontemporal hints, the weight (reused by every wave) goes through the cache.
/// Loads are never conditional on data: a row past the end is loaded from
/// the last row (and not stored), and with kFullCols (the row is exactly
/// kVecs vectors per lane) no column is tested either; otherwise the
/// missing columns are zero-filled after the load. With kFullCols the weight
/// is staged once per workgroup in LDS instead of being re-read from L2 by
/// every wave.
template <typename T, int kVecs, int kRows, bool kResidual, bool kFullCols>
__global__ __launch_bounds__(kDefaultBlockSize) void rmsnorm_wave_kernel(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ w,
    T* __restrict__ y, T* __restrict__ residual_out, int64_t rows, int64_t cols, float eps) {
    constexpr int kPer = Storage<T>::kPerVec;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t vec_cols = cols / kPer;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const int64_t row0 = wave * kRows;
    __shared__ uint4 w_lds[kFullCols ? kVecs * kWaveSize : 1];
    // With kFullCols the weight is staged in LDS: its loads go out first so
    // that the LDS store below waits for them alone, not for the row loads.
    // (Unguarded when the weight is a whole number of workgroup-wide
    // vectors: a guarded index makes the compiler move the staging array
    // into memory and wait for it.)
    constexpr int kWeightVecs = kVecs * kWaveSize;
    constexpr bool kStageGuard = kWeightVecs % kDefaultBlockSize != 0;
    constexpr int kStage = kFullCols ? ceil_div(kWeightVecs, kDefaultBlockSize) : 1;
    uint4 wstage[kStage];
    if constexpr (kFullCols) {
#pragma unroll
        for (int k = 0; k < kStage; ++k) {
            const int i = k * kDefaultBlockSize + static_cast<int>(threadIdx.x);
            if (!kStageGuard || i < kWeightVecs) wstage[k] = reinterpret_cast<const uint4*>(w)[i];
        }
    }

    uint4 xv[kRows][kVecs];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t v = static_cast<int64_t>(j) * kWaveSize + lane;
            const int64_t vc = kFullCols || v < vec_cols ? v : vec_cols - 1;
            xv[r][j] = load_stream16(x + row * cols + vc * kPer);
        }
    }
    // Stage the weight while the row loads are in flight (a wave past the
    // last row still takes part in the barrier, then leaves).
    if constexpr (kFullCols) {
#pragma unroll
        for (int k = 0; k < kStage; ++k) {
            const int i = k * kDefaultBlockSize + static_cast<int>(threadIdx.x);
            if (!kStageGuard || i < kWeightVecs) w_lds[i] = wstage[k];
        }
        lds_barrier();
    }
    if (row0 >= rows) return;  // wave-uniform
    uint4 wv[kVecs];
#pragma unroll
    for (int j = 0; j < kVecs; ++j) {
        const int64_t v = static_cast<int64_t>(j) * kWaveSize + lane;
        if constexpr (kFullCols) {
            wv[j] = w_lds[v];
        } else {
            wv[j] = reinterpret_cast<const uint4*>(w)[v < vec_cols ? v : vec_cols - 1];
        }
    }
    if constexpr (!kFullCols) {
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t v = static_cast<int64_t>(j) * kWaveSize + lane;
            if (v >= vec_cols) {
#pragma unroll
                for (int r = 0; r < kRows; ++r) xv[r][j] = make_uint4(0, 0, 0, 0);
            }
        }
    }

    if constexpr (kResidual) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int64_t row = row0 + r;
#pragma unroll
            for (int j = 0; j < kVecs; ++j) {
                const int64_t v = static_cast<int64_t>(j) * kWaveSize + lane;
                if (row < rows && (kFullCols || v < vec_cols)) {
                    float a[kPer];
                    float b[kPer];
                    unpack16<T>(xv[r][j], a);
                    unpack16<T>(load_stream16(residual + row * cols + v * kPer), b);
#pragma unroll
                    for (int i = 0; i < kPer; ++i) a[i] = a[i] + b[i];
                    // The sum is rounded to the storage type before the norm,
                    // as `x + residual` is in the reference.
                    xv[r][j] = pack16<T>(a);
                    store_stream16(residual_out + row * cols + v * kPer, xv[r][j]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r;
        float partial[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            float a[kPer];
            unpack16<T>(xv[r][j], a);
#pragma unroll
            for (int i = 0; i < kPer; ++i) partial[i & 3] += a[i] * a[i];
        }
        const float total =
            wave_reduce_f32<AddF32>((partial[0] + partial[1]) + (partial[2] + partial[3]));
        const float scale = inv_rms(total, cols, eps);
        if (row >= rows) continue;  // wave-uniform
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t v = static_cast<int64_t>(j) * kWaveSize + lane;
            if (kFullCols || v < vec_cols) {
                float a[kPer];
                float g[kPer];
                unpack16<T>(xv[r][j], a);
                unpack16<T>(wv[j], g);
#pragma unroll
                for (int i = 0; i < kPer; ++i) a[i] = (a[i] * scale) * g[i];
                store_stream16(y + row * cols + v * kPer, pack16<T>(a));
            }
        }
    }
}

/// Sum of squares of one 16-byte vector. bf16 pairs go through
/// v_dot2_f32_bf16 (the products of bf16 values are exact in fp32), which
/// keeps the row in its packed registers.
template <typename T>
__device__ __forceinline__ float sum_squares16(const uint4& v) {
    if constexpr (std::is_same_v<T, bf16_t>) {
        typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
        const bf16x2_v a = __builtin_bit_cast(bf16x2_v, v.x);
        const bf16x2_v b = __builtin_bit_cast(bf16x2_v, v.y);
        const bf16x2_v c = __builtin_bit_cast(bf16x2_v, v.z);
        const bf16x2_v d = __builtin_bit_cast(bf16x2_v, v.w);
        const float p = __builtin_amdgcn_fdot2_f32_bf16(c, c, __builtin_amdgcn_fdot2_f32_bf16(a, a, 0.0f, false),
                                                        false);
        const float q = __builtin_amdgcn_fdot2_f32_bf16(d, d, __builtin_amdgcn_fdot2_f32_bf16(b, b, 0.0f, false),
                                                        false);
        return p + q;
    } else {
        constexpr int kPer = Storage<T>::kPerVec;
        float a[kPer];
        unpack16<T>(v, a);
        float p[2] = {0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < kPer; ++i) p[i & 1] += a[i] * a[i];
        return p[0] + p[1];
    }
}

/// (x * scale) * g for one 16-byte vector, rounded to T. For bf16 with
/// `finite` (the row's sum of squares and this weight vector are finite, so
/// no product is NaN) the rounding is v_cvt_pk_bf16_f32, which then equals
/// f32_to_bf16_bits bit for bit.
template <typename T>
__device__ __forceinline__ uint4 scale16(const uint4& x, const uint4& g, float scale, bool finite) {
    if constexpr (std::is_same_v<T, bf16_t>) {
        if (finite) {
            auto pair = [&](uint32_t xw, uint32_t gw) {
                const float x0 = __uint_as_float(xw << 16);
                const float x1 = __uint_as_float(xw & 0xffff0000u);
                const float g0 = __uint_as_float(gw << 16);
                const float g1 = __uint_as_float(gw & 0xffff0000u);
                return f32x2_to_bf16x2_bits((x0 * scale) * g0, (x1 * scale) * g1);
            };
            return make_uint4(pair(x.x, g.x), pair(x.y, g.y), pair(x.z, g.z), pair(x.w, g.w));
        }
    }
    constexpr int kPer = Storage<T>::kPerVec;
    float a[kPer];
    float w[kPer];
    unpack16<T>(x, a);
    unpack16<T>(g, w);
#pragma unroll
    for (int i = 0; i < kPer; ++i) a[i] = (a[i] * scale) * w[i];
    return pack16<T>(a);
}

/// True when all values of a 16-byte vector of T are finite.
template <typename T>
__device__ __forceinline__ bool finite16(const uint4& v) {
    if constexpr (std::is_same_v<T, float>) {
        const uint32_t m = 0x7f800000u;
        return (v.x & m) != m && (v.y & m) != m && (v.z & m) != m && (v.w & m) != m;
    } else {
        const uint32_t m = std::is_same_v<T, bf16_t> ? 0x7f807f80u : 0x7c007c00u;
        auto ok = [&](uint32_t w) { return (w & (m & 0xffffu)) != (m & 0xffffu) && (w & (m & 0xffff0000u)) != (m & 0xffff0000u); };
        return ok(v.x) && ok(v.y) && ok(v.z) && ok(v.w);
    }
}

/// Rows of exactly kV 16-byte vectors, kV in {256, 512, 1024}: a workgroup
/// of kThreads (256 or 512, dividing kV) threads owns kThreads * kLoads / kV
/// consecutive rows, and each of its kLoads load instructions reads
/// kThreads * 16 bytes of contiguous memory (thread t of the workgroup takes
/// vector kThreads * u + t of the workgroup's span). Few loads per lane run
/// fastest on MI355X: with 16-byte loads, 1-2 per lane before the first
/// store stream at 77-79% of HBM peak, 4 at 76%, 8 at 50-70%. Row sums are
/// reduced in each wave (DPP), then across the waves through LDS in a fixed
/// order. A workgroup that reaches past the last row loads the last row
/// again in place of the missing ones and stores nothing for them.
template <typename T, int kV, int kLoads, int kThreads, bool kResidual>
__global__ __launch_bounds__(kThreads) void rmsnorm_tile_kernel(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ w,
    T* __restrict__ y, T* __restrict__ residual_out, int64_t rows, int64_t cols, float eps) {
    static_assert(kV == 256 || kV == 512 || kV == 1024, "row of 256, 512 or 1024 vectors");
    static_assert(kThreads == 256 || kThreads == 512, "four or eight waves");
    static_assert(kV % kThreads == 0, "an instruction's vectors lie in one row");
    static_assert((kThreads * kLoads) % kV == 0, "whole rows per workgroup");
    constexpr int kPer = Storage<T>::kPerVec;
    constexpr int kWaves = kThreads / kWaveSize;
    constexpr int kRows = kThreads * kLoads / kV;  // rows per workgroup
    constexpr int kWeights = kV / kThreads;        // weight vectors per thread
    const int tid = static_cast<int>(threadIdx.x);
    const int wave = tid / kWaveSize;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows;
    const bool whole = row0 + kRows <= rows;       // workgroup-uniform
    __shared__ float partials[kWaves][kRows];

    uint4 v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        const int64_t r = row0 + (u * kThreads) / kV;
        const int64_t row = whole || r < rows ? r : rows - 1;
        v[u] = load_stream16(x + row * cols + static_cast<int64_t>((u * kThreads) % kV + tid) * kPer);
    }
    uint4 g[kWeights];
    bool finite = true;
#pragma unroll
    for (int i = 0; i < kWeights; ++i) {
        g[i] = reinterpret_cast<const uint4*>(w)[i * kThreads + tid];
        finite = finite && finite16<T>(g[i]);
    }
    if constexpr (kResidual) {
#pragma unroll
        for (int u = 0; u < kLoads; ++u) {
            const int64_t r = row0 + (u * kThreads) / kV;
            const int64_t off = (whole || r < rows ? r : rows - 1) * cols +
                                static_cast<int64_t>((u * kThreads) % kV + tid) * kPer;
            float a[kPer];
            float b[kPer];
            unpack16<T>(v[u], a);
            unpack16<T>(load_stream16(residual + off), b);
#pragma unroll
            for (int i = 0; i < kPer; ++i) a[i] = a[i] + b[i];
            // The sum is rounded to the storage type before the norm, as
            // `x + residual` is in the reference.
            v[u] = pack16<T>(a);
            if (whole || r < rows) store_stream16(residual_out + off, v[u]);
        }
    }

    float part[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) part[r] = 0.0f;
#pragma unroll
    for (int u = 0; u < kLoads; ++u) part[(u * kThreads) / kV] += sum_squares16<T>(v[u]);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        part[r] = wave_reduce_f32<AddF32>(part[r]);
        if ((tid & (kWaveSize - 1)) == 0) partials[wave][r] = part[r];
    }
    __syncthreads();
    float scale[kRows];
    bool row_finite[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        float total = (partials[0][r] + partials[1][r]) + (partials[2][r] + partials[3][r]);
        if constexpr (kWaves == 8) {
            total = total + ((partials[4][r] + partials[5][r]) + (partials[6][r] + partials[7][r]));
        }
        scale[r] = inv_rms(total, cols, eps);
        row_finite[r] = finite && __builtin_isfinite(total);
    }
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        const int r = (u * kThreads) / kV;
        if (whole || row0 + r < rows) {
            const int64_t off =
                (row0 + r) * cols + static_cast<int64_t>((u * kThreads) % kV + tid) * kPer;
            store_stream16(y + off, scale16<T>(v[u], g[u % kWeights], scale[r], row_finite[r]));
        }
    }
}

/// Launch shape of the tile kernel for one row width.
template <int V, int L, int Th>
struct TileShape {
    static constexpr int kV = V;
    static constexpr int kLoads = L;
    static constexpr int kThreads = Th;
    static constexpr int kRows = Th * L / V;
};
/// Shapes measured on MI355X ([16384, 4096] and [32768, 2048] bf16): plain
/// RMSNorm is fastest with two row vectors per lane in 256-thread
/// workgroups (77.8% of HBM peak against 76.1% with four; one per lane in
/// 512-thread workgroups 69%); the fused residual form, which loads x and
/// the residual for each vector, with one vector per lane (80.1% in
/// 512-thread workgroups against 76.3% with four per lane). Rows of 1024
/// vectors keep four per lane.
template <int kV, bool kResidual>
struct TileFor;
template <bool kResidual>
struct TileFor<256, kResidual> {
    using type = TileShape<256, kResidual ? 1 : 2, 256>;
};
template <bool kResidual>
struct TileFor<512, kResidual> {
    using type = std::conditional_t<kResidual, TileShape<512, 1, 512>, TileShape<512, 2, 256>>;
};
template <bool kResidual>
struct TileFor<1024, kResidual> {
    using type = TileShape<1024, 4, 256>;
};

/// Any shape and alignment: one workgroup per row, two passes over the row.
template <typename T, bool kResidual>
__global__ __launch_bounds__(kDefaultBlockSize) void rmsnorm_block_kernel(
    const T* __restrict__ x, const T* __restrict__ residual, const T* __restrict__ w,
    T* __restrict__ y, T* __restrict__ residual_out, int64_t rows, int64_t cols, float eps) {
    __shared__ float slot[kWavesPerBlock];
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const T* xr = x + row * cols;
        float partial = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            float a = Storage<T>::load(xr + c);
            if constexpr (kResidual) {
                a = a + Storage<T>::load(residual + row * cols + c);
                Storage<T>::store(residual_out + row * cols + c, a);
                a = Storage<T>::load(residual_out + row * cols + c);
            }
            partial += a * a;
        }
        const float total = block_reduce_f32<kWavesPerBlock, AddF32>(partial, slot);
        const float scale = inv_rms(total, cols, eps);
        const T* src = kResidual ? residual_out + row * cols : xr;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            const float a = Storage<T>::load(src + c);
            Storage<T>::store(y + row * cols + c, (a * scale) * Storage<T>::load(w + c));
        }
    }
}

/// Rows per wave: at least 4 16-byte loads in flight per lane for short
/// rows, one row per wave from 4 vectors per lane up. The wave kernel serves
/// the matrices below the tile kernel's threshold (a few waves per CU, one
/// round), where more waves with fewer rows each cover the memory latency
/// better: fp32 [4096, 1024] 7.84 -> 7.44 us and [2048, 4096] 13.2 -> 12.6 us
/// against two rows per wave at 4 vectors per lane.
constexpr int rows_per_wave(int vecs) { return vecs >= 4 ? 1 : 4 / vecs; }

template <typename T, int kVecs, bool kResidual>
void launch_wave(const void* x, const void* residual, const void* w, void* y, void* residual_out,
                 int64_t rows, int64_t cols, float eps, hipStream_t stream) {
    constexpr int kRows = rows_per_wave(kVecs);
    const int64_t waves = ceil_div<int64_t>(rows, kRows);
    const int64_t grid = ceil_div<int64_t>(waves, kWavesPerBlock);
    const bool full_cols = cols / Storage<T>::kPerVec == static_cast<int64_t>(kVecs) * kWaveSize;
    if (full_cols) {
        launch(rmsnorm_wave_kernel<T, kVecs, kRows, kResidual, true>,
               dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize), 0, stream,
               static_cast<const T*>(x), static_cast<const T*>(residual), static_cast<const T*>(w),
               static_cast<T*>(y), static_cast<T*>(residual_out), rows, cols, eps);
    } else {
        launch(rmsnorm_wave_kernel<T, kVecs, kRows, kResidual, false>,
               dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize), 0, stream,
               static_cast<const T*>(x), static_cast<const T*>(residual), static_cast<const T*>(w),
               static_cast<T*>(y), static_cast<T*>(residual_out), rows, cols, eps);
    }
}

template <typename T, bool kResidual>
cf_status dispatch(const void* x, const void* residual, const void* w, void* y,
                   void* residual_out, int64_t rows, int64_t cols, float eps,
                   hipStream_t stream) {
    constexpr int kPer = Storage<T>::kPerVec;
    bool vec = cols % kPer == 0 && host_aligned(x, 16) && host_aligned(w, 16) &&
               host_aligned(y, 16);
    if (kResidual) vec = vec && host_aligned(residual, 16) && host_aligned(residual_out, 16);
    const int64_t vectors_per_lane = ceil_div<int64_t>(cols / kPer, kWaveSize);
    const int64_t row_vectors = cols / kPer;
    // The tiled kernel wins once the matrix holds at least 16 x 1024
    // 16-byte vectors per CU, several rounds of workgroups (measured on [16384,
    // 2048 / 4096 / 8192] bf16: 1-3 points of HBM peak); below that
    // ([4096, 4096] bf16) the wave kernel is faster.
    using Tile256 = typename TileFor<256, kResidual>::type;
    using Tile512 = typename TileFor<512, kResidual>::type;
    using Tile1024 = typename TileFor<1024, kResidual>::type;
    const int64_t tile_rows = row_vectors == 256    ? Tile256::kRows
                              : row_vectors == 512  ? Tile512::kRows
                              : row_vectors == 1024 ? Tile1024::kRows
                                                    : 0;  // rows per tile workgroup
    const int64_t tile_groups = tile_rows > 0 ? ceil_div<int64_t>(rows, tile_rows) : 0;
    if (vec && tile_rows > 0 && rows * row_vectors >= 16 * 1024 * static_cast<int64_t>(cu_count())) {
        const auto grid = static_cast<unsigned>(tile_groups);
        auto run = [&](auto shape) {
            using S = decltype(shape);
            launch(rmsnorm_tile_kernel<T, S::kV, S::kLoads, S::kThreads, kResidual>, dim3(grid),
                   dim3(S::kThreads), 0, stream, static_cast<const T*>(x),
                   static_cast<const T*>(residual), static_cast<const T*>(w), static_cast<T*>(y),
                   static_cast<T*>(residual_out), rows, cols, eps);
        };
        if (row_vectors == 256) {
            run(Tile256{});
        } else if (row_vectors == 512) {
            run(Tile512{});
        } else {
            run(Tile1024{});
        }
    } else if (vec && vectors_per_lane <= 16) {
        if (vectors_per_lane <= 1) {
            launch_wave<T, 1, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, stream);
        } else if (vectors_per_lane <= 2) {
            launch_wave<T, 2, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, stream);
        } else if (vectors_per_lane <= 4) {
            launch_wave<T, 4, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, stream);
        } else if (vectors_per_lane <= 8) {
            launch_wave<T, 8, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, stream);
        } else {
            launch_wave<T, 16, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, stream);
        }
    } else {
        const int64_t max_blocks = static_cast<int64_t>(cu_count()) * 8;
        const int64_t grid = rows < max_blocks ? rows : max_blocks;
        launch(rmsnorm_block_kernel<T, kResidual>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x),
               static_cast<const T*>(residual), static_cast<const T*>(w), static_cast<T*>(y),
               static_cast<T*>(residual_out), rows, cols, eps);
    }
    return check_launch(kResidual ? "launching fused_residual_rmsnorm" : "launching rmsnorm",
                        stream);
}

template <bool kResidual>
cf_status run(const void* x, const void* residual, const void* w, void* y, void* residual_out,
              cf_dtype dtype, int64_t rows, int64_t cols, float eps, void* stream) {
    auto s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case CF_F32:
            return dispatch<float, kResidual>(x, residual, w, y, residual_out, rows, cols, eps, s);
        case CF_BF16:
            return dispatch<bf16_t, kResidual>(x, residual, w, y, residual_out, rows, cols, eps,
                                               s);
        case CF_F16:
            return dispatch<f16_t, kResidual>(x, residual, w, y, residual_out, rows, cols, eps,
                                              s);
    }
    return fail(CF_ERR_UNSUPPORTED, "rmsnorm: unknown dtype %d", static_cast<int>(dtype));
}

}  // namespace
}  // namespace cf

extern "C" {

cf_status cf_rmsnorm(const void* x, const void* w, void* y, cf_dtype dtype, int64_t rows,
                     int64_t cols, float eps, void* stream) {
    CF_ENTRY();
    if (rows <= 0 || cols <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && w != nullptr && y != nullptr, "cf_rmsnorm: null pointer");
    return cf::run<false>(x, nullptr, w, y, nullptr, dtype, rows, cols, eps, stream);
}

cf_status cf_fused_residual_rmsnorm(const void* x, const void* residual, const void* w, void* y,
                                    void* residual_out, cf_dtype dtype, int64_t rows,
                                    int64_t cols, float eps, void* stream) {
    CF_ENTRY();
    if (rows <= 0 || cols <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && residual != nullptr && w != nullptr && y != nullptr &&
                   residual_out != nullptr,
               "cf_fused_residual_rmsnorm: null pointer");
    return cf::run<true>(x, residual, w, y, residual_out, dtype, rows, cols, eps, stream);
}

}  // extern "C"

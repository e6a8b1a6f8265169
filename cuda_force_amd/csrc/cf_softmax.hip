// Row softmax for gfx950.
//
// Semantics: torch.softmax(x, dim=-1) (python/cudaforge/ops.py:174-175): fp32
// arithmetic for every storage type, y = exp(x - max) * (1 / sum), which is
// the order ATen's vectorised CPU softmax uses. A row whose entries are all
// -inf yields NaN, as torch does; the causal-masked configuration always has a
// finite entry in column 0. exp is the hardware base-2 exponential of
// (x - max) * log2(e) (__expf, as the reference's kernel uses): for the
// non-positive arguments here its relative error is below 1e-7 * |x - max|,
// inside the 1e-5 fp32 tolerance.
//
// Design (fast path): one wavefront per row with the row held in registers:
// one 16-byte-vector read, a DPP max reduction, exp and a DPP sum reduction
// from registers, then one write - one HBM read and one write per element.
// The reference's bound kernel is the online variant that reads the row twice
// (cuda/src/softmax.cu:102-138); the register tile makes the second read and
// the online rescaling unnecessary. Input and output may have different
// storage types (bf16 logits -> fp32 probabilities) and may alias when equal:
// a wave reads its whole row before it writes any of it.
//
// Fallback: long rows, unaligned pointers or ragged widths use a workgroup per
// row with three passes over the row (max, sum, normalise).
#include "cf_common.hpp"

namespace cf {
namespace {

constexpr int kWavesPerBlock = kDefaultBlockSize / kWaveSize;

/// Store `n` (4 or 8) floats as Tout at `p` with 16- or 8-byte streaming stores.
template <typename Tout, int kN>
__device__ __forceinline__ void store_vec(Tout* p, const float* v) {
    constexpr int kOutPer = Storage<Tout>::kPerVec;
    if constexpr (kN == kOutPer) {
        store_stream16(p, pack16<Tout>(v));
    } else if constexpr (kN == 2 * kOutPer) {
        store_stream16(p, pack16<Tout>(v));
        store_stream16(p + kOutPer, pack16<Tout>(v + kOutPer));
    } else {
        // 4 values into a 16-bit type: one 8-byte store.
        static_assert(kN == 4 && kOutPer == 8, "unsupported store width");
        uint2 w;
        w.x = Storage<Tout>::to_bits(v[0]) | (Storage<Tout>::to_bits(v[1]) << 16);
        w.y = Storage<Tout>::to_bits(v[2]) | (Storage<Tout>::to_bits(v[3]) << 16);
        store_stream8(p, w);
    }
}

/// One wave per kRows consecutive rows, one-shot grid; all of the wave's
/// loads are issued before the first reduction. No load depends on a
/// condition (which would make the compiler wait for each one before the
/// next): rows past the end are loaded from the last row and not stored,
/// and with kFullCols every lane's vectors are inside the row; otherwise
/// the missing columns are replaced by -inf after the load.
template <typename Tin, typename Tout, int kVecs, int kRows, bool kFullCols>
__global__ __launch_bounds__(kDefaultBlockSize) void softmax_wave_kernel(const Tin* x, Tout* y,
                                                                         int64_t rows,
                                                                         int64_t cols) {
    constexpr int kPer = Storage<Tin>::kPerVec;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t vec_cols = cols / kPer;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const int64_t row0 = wave * kRows;
    if (row0 >= rows) return;  // wave-uniform
    const float neg_inf = -__builtin_inff();

    uint4 raw[kRows][kVecs];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            const int64_t ic = kFullCols || idx < vec_cols ? idx : vec_cols - 1;
            raw[r][j] = load_stream16(x + row * cols + ic * kPer);
        }
    }
    // Keep all of the wave's loads ahead of the first reduction.
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r;
        if (row >= rows) continue;  // wave-uniform
        float v[kVecs][kPer];
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            if (kFullCols || idx < vec_cols) {
                unpack16<Tin>(raw[r][j], v[j]);
            } else {
#pragma unroll
                for (int i = 0; i < kPer; ++i) v[j][i] = neg_inf;
            }
        }

        float local_max = neg_inf;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
#pragma unroll
            for (int i = 0; i < kPer; ++i) local_max = fmaxf(local_max, v[j][i]);
        }
        const float row_max = wave_reduce_f32<MaxF32>(local_max);

        float partial[2] = {0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                v[j][i] = __expf(v[j][i] - row_max);
                partial[i & 1] += v[j][i];
            }
        }
        const float row_sum = wave_reduce_f32<AddF32>(partial[0] + partial[1]);
        const float inv_sum = 1.0f / row_sum;

#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            if (kFullCols || idx < vec_cols) {
#pragma unroll
                for (int i = 0; i < kPer; ++i) v[j][i] = v[j][i] * inv_sum;
                store_vec<Tout, kPer>(y + row * cols + idx * kPer, v[j]);
            }
        }
    }
}

/// Any shape: one workgroup per row, three passes.
template <typename Tin, typename Tout>
__global__ __launch_bounds__(kDefaultBlockSize) void softmax_block_kernel(const Tin* x, Tout* y,
                                                                          int64_t rows,
                                                                          int64_t cols) {
    __shared__ float slot[kWavesPerBlock];
    const float neg_inf = -__builtin_inff();
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const Tin* xr = x + row * cols;
        float local_max = neg_inf;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            local_max = fmaxf(local_max, Storage<Tin>::load(xr + c));
        }
        const float row_max = block_reduce_f32<kWavesPerBlock, MaxF32>(local_max, slot);
        float local_sum = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            local_sum += __expf(Storage<Tin>::load(xr + c) - row_max);
        }
        const float inv_sum = 1.0f / block_reduce_f32<kWavesPerBlock, AddF32>(local_sum, slot);
        // When x and y alias, every thread must finish reading before any
        // writes: the reductions above end in a barrier, and this pass reads
        // and writes the same element in the same thread.
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            const float e = __expf(Storage<Tin>::load(xr + c) - row_max);
            Storage<Tout>::store(y + row * cols + c, e * inv_sum);
        }
    }
}

template <typename Tin, typename Tout, int kVecs>
void launch_wave(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t stream) {
    // Rows per wave: two for rows of one 16-byte vector per lane, else one.
    // More loads in flight per lane are slower, not faster: on [131072, 512]
    // bf16 eight rows per wave (eight 16-byte loads per lane before the
    // first store) ran at 70% of HBM peak, one or two at 78.7%; a plain
    // copy shows the same (8 loads per lane 50%, 1-2 loads 77-79%). Never
    // so many rows per wave that fewer waves than SIMDs (4 per CU) would run.
    constexpr int kRows = kVecs >= 2 ? 1 : 2;
    const int64_t simds = static_cast<int64_t>(cu_count()) * 4;
    const int64_t grid_rows = ceil_div<int64_t>(rows, kRows) >= simds ? kRows : 1;
    const int64_t waves = ceil_div<int64_t>(rows, grid_rows);
    const int64_t grid = ceil_div<int64_t>(waves, kWavesPerBlock);
    const bool full = cols / Storage<Tin>::kPerVec == static_cast<int64_t>(kVecs) * kWaveSize;
    const auto* xin = static_cast<const Tin*>(x);
    auto* out = static_cast<Tout*>(y);
    const unsigned g = static_cast<unsigned>(grid);
    if (grid_rows == 1) {
        if (full) {
            launch(softmax_wave_kernel<Tin, Tout, kVecs, 1, true>, dim3(g), dim3(kDefaultBlockSize),
                   0, stream, xin, out, rows, cols);
        } else {
            launch(softmax_wave_kernel<Tin, Tout, kVecs, 1, false>, dim3(g),
                   dim3(kDefaultBlockSize), 0, stream, xin, out, rows, cols);
        }
        return;
    }
    if (full) {
        launch(softmax_wave_kernel<Tin, Tout, kVecs, kRows, true>, dim3(g), dim3(kDefaultBlockSize),
               0, stream, xin, out, rows, cols);
    } else {
        launch(softmax_wave_kernel<Tin, Tout, kVecs, kRows, false>, dim3(g),
               dim3(kDefaultBlockSize), 0, stream, xin, out, rows, cols);
    }
}

template <typename Tin, typename Tout>
cf_status dispatch(const void* x, void* y, int64_t rows, int64_t cols, hipStream_t stream) {
    constexpr int kPer = Storage<Tin>::kPerVec;
    const bool vec = cols % kPer == 0 && host_aligned(x, 16) && host_aligned(y, 16);
    const int64_t vectors_per_lane = ceil_div<int64_t>(cols / kPer, kWaveSize);
    if (vec && vectors_per_lane <= 16) {
        if (vectors_per_lane <= 1) {
            launch_wave<Tin, Tout, 1>(x, y, rows, cols, stream);
        } else if (vectors_per_lane <= 2) {
            launch_wave<Tin, Tout, 2>(x, y, rows, cols, stream);
        } else if (vectors_per_lane <= 4) {
            launch_wave<Tin, Tout, 4>(x, y, rows, cols, stream);
        } else if (vectors_per_lane <= 8) {
            launch_wave<Tin, Tout, 8>(x, y, rows, cols, stream);
        } else {
            launch_wave<Tin, Tout, 16>(x, y, rows, cols, stream);
        }
    } else {
        const int64_t max_blocks = static_cast<int64_t>(cu_count()) * 8;
        const int64_t grid = rows < max_blocks ? rows : max_blocks;
        launch(softmax_block_kernel<Tin, Tout>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const Tin*>(x),
               static_cast<Tout*>(y), rows, cols);
    }
    return check_launch("launching softmax", stream);
}

template <typename Tin>
cf_status dispatch_out(const void* x, void* y, cf_dtype y_dtype, int64_t rows, int64_t cols,
                       hipStream_t stream) {
    switch (y_dtype) {
        case CF_F32:
            return dispatch<Tin, float>(x, y, rows, cols, stream);
        case CF_BF16:
            return dispatch<Tin, bf16_t>(x, y, rows, cols, stream);
        case CF_F16:
            return dispatch<Tin, f16_t>(x, y, rows, cols, stream);
    }
    return fail(CF_ERR_UNSUPPORTED, "cf_softmax: unknown output dtype %d",
                static_cast<int>(y_dtype));
}

}  // namespace
}  // namespace cf

extern "C" {

cf_status cf_softmax(const void* x, cf_dtype x_dtype, void* y, cf_dtype y_dtype, int64_t rows,
                     int64_t cols, void* stream) {
    CF_ENTRY();
    if (rows <= 0 || cols <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_softmax: null pointer");
    CF_REQUIRE(x != y || x_dtype == y_dtype,
               "cf_softmax: input and output may alias only when their dtypes match");
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::dispatch_out<float>(x, y, y_dtype, rows, cols, s);
        case CF_BF16:
            return cf::dispatch_out<cf::bf16_t>(x, y, y_dtype, rows, cols, s);
        case CF_F16:
            return cf::dispatch_out<cf::f16_t>(x, y, y_dtype, rows, cols, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_softmax: unknown input dtype %d",
                    static_cast<int>(x_dtype));
}

}  // extern "C"

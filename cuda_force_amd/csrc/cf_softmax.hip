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
// Rows too long for one wave's registers (more than 1024 16-byte vectors: fp32
// rows past 4096 columns, 16-bit rows past 8192) take a workgroup of 1024
// threads per row, the row again in registers (up to 8 vectors per thread),
// with the two reductions across the workgroup through LDS.
//
// Fallback: longer rows, unaligned pointers or ragged widths use a workgroup
// per row with three passes over the row (max, sum, normalise).
//
// cf_softmax_scaled is the same kernel on scale * x with an optional causal
// mask (column c of row r hidden when c > r mod period): the attention-score
// softmax of a causal block, softmax(scores / sqrt(d) + causal), in one pass
// instead of a scale-and-mask pass followed by a softmax. A 16-byte vector
// of a row that lies wholly past the row's last visible column is not read
// at all (buffer load with an out-of-range offset: zeros, no memory access),
// so a causal score matrix is read about half, and written whole.
#include "cf_common.hpp"

#include <type_traits>

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
        w.x = Storage<Tout>::to_bits2(v[0], v[1]);
        w.y = Storage<Tout>::to_bits2(v[2], v[3]);
        store_stream8(p, w);
    }
}

/// Scale and causal mask of cf_softmax_scaled (kMasked kernels only):
/// logits are scale * x, and column c of row r is -inf when period > 0 and
/// c > r mod period.
struct Masking {
    float scale;
    int64_t period;
};

/// Last visible column of `row` (cols - 1 when there is no mask).
__device__ __forceinline__ int64_t last_visible(const Masking& m, int64_t row, int64_t cols) {
    return m.period > 0 ? row % m.period : cols - 1;
}

/// The same for the wave kernel, whose x spans fewer than 2^31 bytes (so
/// row, period and cols fit in 32 bits): a 32-bit remainder.
__device__ __forceinline__ int last_visible32(const Masking& m, int64_t row, int64_t cols) {
    return m.period > 0 ? static_cast<int>(static_cast<uint32_t>(row) % static_cast<uint32_t>(m.period))
                        : static_cast<int>(cols) - 1;
}

/// 16-byte streaming load through a buffer resource: an offset past the
/// resource's range returns zeros without touching memory.
__device__ __forceinline__ uint4 buffer_load_stream16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, 0, 2 /* nt */);
    return make_uint4(v.x, v.y, v.z, v.w);
}

/// One wave per kRows consecutive rows, one-shot grid; all of the wave's
/// loads are issued before the first reduction. No load depends on a
/// condition (which would make the compiler wait for each one before the
/// next): rows past the end are loaded from the last row and not stored,
/// and with kFullCols every lane's vectors are inside the row; otherwise
/// the missing columns are replaced by -inf after the load.
/// store_vec for a row's probabilities e * (1 / sum). Each e is in [0, 1]
/// unless one of them is NaN, and then the sum is NaN and so is every value of
/// the row; otherwise the sum is at least 1 (the maximum gives e = 1) and no
/// value is NaN. So for bf16 a row whose 1 / sum is finite is rounded by
/// v_cvt_pk_bf16_f32 alone, and a NaN row stores the canonical 0x7FC0: the
/// bits of f32_to_bf16_bits either way, with no per-value NaN test.
template <typename Tout, int kN>
__device__ __forceinline__ void store_probs(Tout* p, const float* v, bool row_nan) {
    if constexpr (std::is_same_v<Tout, bf16_t> && (kN == 8 || kN == 4)) {
        uint32_t w[kN / 2];
#pragma unroll
        for (int i = 0; i < kN / 2; ++i) {
            w[i] = row_nan ? 0x7FC07FC0u : f32x2_to_bf16x2_bits(v[2 * i], v[2 * i + 1]);
        }
        if constexpr (kN == 8) {
            store_stream16(p, make_uint4(w[0], w[1], w[2], w[3]));
        } else {
            store_stream8(p, make_uint2(w[0], w[1]));
        }
    } else {
        store_vec<Tout, kN>(p, v);
    }
}

template <typename Tin, typename Tout, int kVecs, int kRows, bool kFullCols, bool kMasked>
__global__ __launch_bounds__(kDefaultBlockSize) void softmax_wave_kernel(const Tin* x, Tout* y,
                                                                         int64_t rows,
                                                                         int64_t cols,
                                                                         Masking mask) {
    constexpr int kPer = Storage<Tin>::kPerVec;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t vec_cols = cols / kPer;
    // Wave-uniform (readfirstlane tells the compiler): the row index and
    // the mask's remainder are computed once per wave.
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                         __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWaveSize);
    const int64_t row0 = wave * kRows;
    if (row0 >= rows) return;  // wave-uniform
    const float neg_inf = -__builtin_inff();

    // kMasked: x spans fewer than 2^31 bytes (checked on the host).
    const __amdgpu_buffer_rsrc_t xbuf =
        make_buffer(x, kMasked ? static_cast<uint32_t>(rows * cols * sizeof(Tin)) : 0u);
    uint4 raw[kRows][kVecs];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            const int64_t ic = kFullCols || idx < vec_cols ? idx : vec_cols - 1;
            if constexpr (kMasked) {
                const bool read = static_cast<int>(ic) * kPer <= last_visible32(mask, row, cols);
                raw[r][j] = buffer_load_stream16(
                    xbuf, read ? static_cast<uint32_t>((row * cols + ic * kPer) * sizeof(Tin))
                               : 0x80000000u);
            } else {
                raw[r][j] = load_stream16(x + row * cols + ic * kPer);
            }
        }
    }
    // Keep all of the wave's loads ahead of the first reduction.
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t row = row0 + r;
        if (row >= rows) continue;  // wave-uniform
        float v[kVecs][kPer];
        const int visible = kMasked ? last_visible32(mask, row, cols) : 0;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            if (kFullCols || idx < vec_cols) {
                unpack16<Tin>(raw[r][j], v[j]);
                if constexpr (kMasked) {
                    const int first = static_cast<int>(idx) * kPer;
#pragma unroll
                    for (int i = 0; i < kPer; ++i) {
                        v[j][i] = first + i <= visible ? mask.scale * v[j][i] : neg_inf;
                    }
                }
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
        const bool row_nan = inv_sum != inv_sum;

#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kWaveSize + lane;
            if (kFullCols || idx < vec_cols) {
#pragma unroll
                for (int i = 0; i < kPer; ++i) v[j][i] = v[j][i] * inv_sum;
                store_probs<Tout, kPer>(y + row * cols + idx * kPer, v[j], row_nan);
            }
        }
    }
}

/// One workgroup of kThreads threads per row (grid-stride over rows), the
/// row in registers: thread t holds vectors t, t + kThreads, ... of it.
/// Every thread reads its vectors before the first reduction's barrier, so
/// x and y may alias. Rows wider than a wave's registers take 1024 threads;
/// latency-bound shapes (no more rows than SIMDs, 257-1024 vectors a row)
/// take 512 or 1024 threads of one vector each, so the row's serial
/// arithmetic (unpack, exp, scale, pack) is spread over more lanes, for two
/// cross-wave reductions through LDS.
constexpr int kRowThreads = 1024;

template <typename Tin, typename Tout, int kVecs, bool kFullCols, bool kMasked, int kThreads = kRowThreads>
__global__ __launch_bounds__(kThreads) void softmax_row_kernel(const Tin* x, Tout* y, int64_t rows,
                                                               int64_t cols, Masking mask) {
    constexpr int kPer = Storage<Tin>::kPerVec;
    __shared__ float slot[kThreads / kWaveSize];
    const int tid = static_cast<int>(threadIdx.x);
    const int64_t vec_cols = cols / kPer;
    const float neg_inf = -__builtin_inff();
    // kMasked: x spans fewer than 2^31 bytes (checked on the host).
    const __amdgpu_buffer_rsrc_t xbuf =
        make_buffer(x, kMasked ? static_cast<uint32_t>(rows * cols * sizeof(Tin)) : 0u);
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int visible = kMasked ? last_visible32(mask, row, cols) : 0;
        uint4 raw[kVecs];
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kThreads + tid;
            const int64_t ic = kFullCols || idx < vec_cols ? idx : vec_cols - 1;
            if constexpr (kMasked) {
                const bool read = static_cast<int>(ic) * kPer <= visible;
                raw[j] = buffer_load_stream16(
                    xbuf, read ? static_cast<uint32_t>((row * cols + ic * kPer) * sizeof(Tin)) : 0x80000000u);
            } else {
                raw[j] = load_stream16(x + row * cols + ic * kPer);
            }
        }
        float v[kVecs][kPer];
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kThreads + tid;
            if (kFullCols || idx < vec_cols) {
                unpack16<Tin>(raw[j], v[j]);
                if constexpr (kMasked) {
                    const int first = static_cast<int>(idx) * kPer;
#pragma unroll
                    for (int i = 0; i < kPer; ++i) v[j][i] = first + i <= visible ? mask.scale * v[j][i] : neg_inf;
                }
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
        const float row_max = block_reduce_f32<kThreads / kWaveSize, MaxF32>(local_max, slot);
        float partial[2] = {0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                v[j][i] = __expf(v[j][i] - row_max);
                partial[i & 1] += v[j][i];
            }
        }
        const float inv_sum =
            1.0f / block_reduce_f32<kThreads / kWaveSize, AddF32>(partial[0] + partial[1], slot);
        const bool row_nan = inv_sum != inv_sum;
#pragma unroll
        for (int j = 0; j < kVecs; ++j) {
            const int64_t idx = static_cast<int64_t>(j) * kThreads + tid;
            if (kFullCols || idx < vec_cols) {
#pragma unroll
                for (int i = 0; i < kPer; ++i) v[j][i] = v[j][i] * inv_sum;
                store_probs<Tout, kPer>(y + row * cols + idx * kPer, v[j], row_nan);
            }
        }
    }
}

template <typename Tin, typename Tout, int kVecs, bool kMasked, int kThreads = kRowThreads>
void launch_row(const void* x, void* y, int64_t rows, int64_t cols, const Masking& mask, hipStream_t stream) {
    const bool full = cols / Storage<Tin>::kPerVec == static_cast<int64_t>(kVecs) * kThreads;
    const unsigned grid = static_cast<unsigned>(rows < (1 << 20) ? rows : (1 << 20));
    const auto* xin = static_cast<const Tin*>(x);
    auto* out = static_cast<Tout*>(y);
    if (full) {
        launch(softmax_row_kernel<Tin, Tout, kVecs, true, kMasked, kThreads>, dim3(grid), dim3(kThreads), 0, stream,
               xin, out, rows, cols, mask);
    } else {
        launch(softmax_row_kernel<Tin, Tout, kVecs, false, kMasked, kThreads>, dim3(grid), dim3(kThreads), 0, stream,
               xin, out, rows, cols, mask);
    }
}

/// Any shape: one workgroup per row, three passes.
template <typename Tin, typename Tout, bool kMasked>
__global__ __launch_bounds__(kDefaultBlockSize) void softmax_block_kernel(const Tin* x, Tout* y,
                                                                          int64_t rows,
                                                                          int64_t cols,
                                                                          Masking mask) {
    __shared__ float slot[kWavesPerBlock];
    const float neg_inf = -__builtin_inff();
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const Tin* xr = x + row * cols;
        // Columns past `visible` are -inf (never read); the rest are scaled.
        const int64_t visible = kMasked ? last_visible(mask, row, cols) : cols - 1;
        auto logit = [&](int64_t c) {
            return kMasked ? (c <= visible ? mask.scale * Storage<Tin>::load(xr + c) : neg_inf)
                           : Storage<Tin>::load(xr + c);
        };
        float local_max = neg_inf;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            local_max = fmaxf(local_max, logit(c));
        }
        const float row_max = block_reduce_f32<kWavesPerBlock, MaxF32>(local_max, slot);
        float local_sum = 0.0f;
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            local_sum += __expf(logit(c) - row_max);
        }
        const float inv_sum = 1.0f / block_reduce_f32<kWavesPerBlock, AddF32>(local_sum, slot);
        // When x and y alias, every thread must finish reading before any
        // writes: the reductions above end in a barrier, and this pass reads
        // and writes the same element in the same thread.
        for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
            const float e = __expf(logit(c) - row_max);
            Storage<Tout>::store(y + row * cols + c, e * inv_sum);
        }
    }
}

template <typename Tin, typename Tout, int kVecs, bool kMasked>
void launch_wave(const void* x, void* y, int64_t rows, int64_t cols, const Masking& mask,
                 hipStream_t stream) {
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
            launch(softmax_wave_kernel<Tin, Tout, kVecs, 1, true, kMasked>, dim3(g), dim3(kDefaultBlockSize),
                   0, stream, xin, out, rows, cols, mask);
        } else {
            launch(softmax_wave_kernel<Tin, Tout, kVecs, 1, false, kMasked>, dim3(g),
                   dim3(kDefaultBlockSize), 0, stream, xin, out, rows, cols, mask);
        }
        return;
    }
    if (full) {
        launch(softmax_wave_kernel<Tin, Tout, kVecs, kRows, true, kMasked>, dim3(g), dim3(kDefaultBlockSize),
               0, stream, xin, out, rows, cols, mask);
    } else {
        launch(softmax_wave_kernel<Tin, Tout, kVecs, kRows, false, kMasked>, dim3(g),
               dim3(kDefaultBlockSize), 0, stream, xin, out, rows, cols, mask);
    }
}

template <typename Tin, typename Tout, bool kMasked>
cf_status dispatch(const void* x, void* y, int64_t rows, int64_t cols, const Masking& mask,
                   hipStream_t stream) {
    constexpr int kPer = Storage<Tin>::kPerVec;
    // The masked wave kernel addresses x through a buffer resource with
    // 32-bit offsets and 0x80000000 as its "skip" offset.
    const bool offsets_fit = !kMasked || rows * cols * static_cast<int64_t>(sizeof(Tin)) < (1LL << 31);
    const bool vec = cols % kPer == 0 && host_aligned(x, 16) && host_aligned(y, 16) && offsets_fit;
    const int64_t vectors_per_lane = ceil_div<int64_t>(cols / kPer, kWaveSize);
    const int64_t simds = static_cast<int64_t>(cu_count()) * 4;
    if (vec && rows <= simds && vectors_per_lane > 4 && vectors_per_lane <= 16) {
        // At most one wave per SIMD with 5-16 vectors per lane: the one-wave
        // form's per-lane arithmetic is the latency, so each row is spread
        // over 64 threads per vector per lane ([256, 4096] bf16: 4.05 -> 3.4
        // us by kernel trace). With 2-4 vectors per lane the two LDS
        // reductions cost more than they save ([1024, 2048] bf16 3.7 -> 4.2
        // us), and those shapes keep the one-wave form.
        if (vectors_per_lane <= 8) {
            launch_row<Tin, Tout, 1, kMasked, 512>(x, y, rows, cols, mask, stream);
        } else {
            launch_row<Tin, Tout, 1, kMasked, 1024>(x, y, rows, cols, mask, stream);
        }
    } else if (vec && vectors_per_lane <= 16) {
        if (vectors_per_lane <= 1) {
            launch_wave<Tin, Tout, 1, kMasked>(x, y, rows, cols, mask, stream);
        } else if (vectors_per_lane <= 2) {
            launch_wave<Tin, Tout, 2, kMasked>(x, y, rows, cols, mask, stream);
        } else if (vectors_per_lane <= 4) {
            launch_wave<Tin, Tout, 4, kMasked>(x, y, rows, cols, mask, stream);
        } else if (vectors_per_lane <= 8) {
            launch_wave<Tin, Tout, 8, kMasked>(x, y, rows, cols, mask, stream);
        } else {
            launch_wave<Tin, Tout, 16, kMasked>(x, y, rows, cols, mask, stream);
        }
    } else if (vec && vectors_per_lane <= 8 * kRowThreads / kWaveSize) {
        const int64_t per_thread = ceil_div<int64_t>(cols / kPer, kRowThreads);
        if (per_thread <= 2) {
            launch_row<Tin, Tout, 2, kMasked>(x, y, rows, cols, mask, stream);
        } else if (per_thread <= 4) {
            launch_row<Tin, Tout, 4, kMasked>(x, y, rows, cols, mask, stream);
        } else {
            launch_row<Tin, Tout, 8, kMasked>(x, y, rows, cols, mask, stream);
        }
    } else {
        const int64_t max_blocks = static_cast<int64_t>(cu_count()) * 8;
        const int64_t grid = rows < max_blocks ? rows : max_blocks;
        launch(softmax_block_kernel<Tin, Tout, kMasked>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const Tin*>(x),
               static_cast<Tout*>(y), rows, cols, mask);
    }
    return check_launch("launching softmax", stream);
}

template <typename Tin, bool kMasked>
cf_status dispatch_out(const void* x, void* y, cf_dtype y_dtype, int64_t rows, int64_t cols,
                       const Masking& mask, hipStream_t stream) {
    switch (y_dtype) {
        case CF_F32:
            return dispatch<Tin, float, kMasked>(x, y, rows, cols, mask, stream);
        case CF_BF16:
            return dispatch<Tin, bf16_t, kMasked>(x, y, rows, cols, mask, stream);
        case CF_F16:
            return dispatch<Tin, f16_t, kMasked>(x, y, rows, cols, mask, stream);
    }
    return fail(CF_ERR_UNSUPPORTED, "softmax: unknown output dtype %d", static_cast<int>(y_dtype));
}

template <bool kMasked>
cf_status dispatch_in(const void* x, cf_dtype x_dtype, void* y, cf_dtype y_dtype, int64_t rows,
                      int64_t cols, const Masking& mask, hipStream_t stream) {
    switch (x_dtype) {
        case CF_F32:
            return dispatch_out<float, kMasked>(x, y, y_dtype, rows, cols, mask, stream);
        case CF_BF16:
            return dispatch_out<bf16_t, kMasked>(x, y, y_dtype, rows, cols, mask, stream);
        case CF_F16:
            return dispatch_out<f16_t, kMasked>(x, y, y_dtype, rows, cols, mask, stream);
    }
    return fail(CF_ERR_UNSUPPORTED, "softmax: unknown input dtype %d", static_cast<int>(x_dtype));
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
    return cf::dispatch_in<false>(x, x_dtype, y, y_dtype, rows, cols, cf::Masking{1.0f, 0},
                                  static_cast<hipStream_t>(stream));
}

cf_status cf_softmax_scaled(const void* x, cf_dtype x_dtype, void* y, cf_dtype y_dtype,
                            int64_t rows, int64_t cols, float scale, int64_t causal_period,
                            void* stream) {
    CF_ENTRY();
    if (rows <= 0 || cols <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_softmax_scaled: null pointer");
    CF_REQUIRE(x != y || x_dtype == y_dtype,
               "cf_softmax_scaled: input and output may alias only when their dtypes match");
    CF_REQUIRE(causal_period >= 0, "cf_softmax_scaled: negative causal period %lld",
               static_cast<long long>(causal_period));
    // A period of rows or more gives row % period == row for every row, as
    // rows does: clamping keeps the mask and lets the wave kernel take the
    // period as a 32-bit value (it runs only for rows below 2^31).
    if (causal_period > rows) causal_period = rows;
    return cf::dispatch_in<true>(x, x_dtype, y, y_dtype, rows, cols,
                                 cf::Masking{scale, causal_period}, static_cast<hipStream_t>(stream));
}

}  // extern "C"

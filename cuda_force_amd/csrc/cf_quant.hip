// Block-wise symmetric INT8 quantisation for gfx950.
//
// Semantics (bit-exact target): the reference's CPU path,
// python/cudaforge/ops.py:215-229 and cpp/src/bindings.cpp:298-318:
//
//   s_b = absmax_b / 127          IEEE fp32 divide
//   s_b = s_b > 0 ? s_b : 1       applied after the divide (a NaN absmax also
//                                 lands on 1, since NaN > 0 is false)
//   q_i = clamp(rint(x_i / s_b), -127, 127), round half to even, NaN -> 0
//
// The reference's CUDA kernel (cuda/src/quantization.cu:18-47) tests
// `absmax > 0` before dividing instead; the two disagree when absmax/127
// underflows to zero, and this file follows the CPU path.
//
// Mapping to CDNA4: a 64-element block is 256 bytes of fp32, so 16 lanes load
// it with one 16-byte load each; 16 lanes are exactly one DPP row, and the
// absmax reduces inside the row in 4 DPP steps - no LDS, no barrier, and each
// wave quantises 4 blocks (8 for 16-bit inputs, 8 lanes per block) per step.
// The absmax is reduced over the integer bit patterns of |x|, which orders
// non-negative floats correctly and propagates NaN the way torch.amax does.
//
// The per-element divide is the only expensive arithmetic. With inv the
// correctly rounded 1/s (one IEEE divide per block) and q0 = fl(x * inv), one
// Markstein step, q1 = fma(fma(-q0, s, x), inv, q0), recovers fl(x/s) itself
// (Markstein's correctly-rounded-quotient theorem for a correctly rounded
// reciprocal), and rint(q1) rounds half to even exactly as rint(x / s) does -
// no divide, no branch. The theorem needs the residual to stay clear of the
// subnormal range, which holds for s >= 2^-100; blocks with a smaller scale
// use the IEEE divide.
//
// In a block with a finite absmax and such a scale (every block of ordinary
// data) |x / s| <= 127 + tiny and no element is NaN, so the code needs no
// clamp, and one add rounds it: for |q| < 2^22 the sum q + 3 * 2^22 lies in
// [2^23, 2^24), where floats are spaced 1, so the IEEE add itself rounds q
// half to even and the sum's low mantissa byte is rint(q) modulo 256, the
// int8 code's byte (checked exhaustively on the host for every float with
// |q| <= 127.75). Byte permutes pack four of them into the output word.
// Other blocks (absmax NaN or infinite, or a scale below 2^-100) take
// clamp_code per element.
#include "cf_common.hpp"

namespace cf {
namespace {

// 16-byte loads per lane before the first store: 4 for one tensor per launch
// (config 1's fp32 [4096, 4096] ran 15.6 us against 16.1 with 8), 8 for the
// grouped launches of bulk quantisation (bf16 [4096, 4096] x 48 per launch:
// quantise 68% -> 75.5%, dequantise 65.5% -> 74% of HBM peak against 4).
// Grouped dequantisation reads 8 codes per lane and step and takes 2 steps,
// finding its tensor with one ballot (group_member_ballot): config 5's
// grouped dequantise 74.6-74.9% -> 77.5-77.7% of HBM peak against 12 steps
// with a binary search, bit-identical. A bare read-8-bytes / write-16-bytes
// stream favours few steps (one: 84.6%, twelve: 73.4% at 48 x 16M codes),
// but with the binary search, six dependent loads of the kernel arguments
// per wave, fewer steps lost (2 steps 43.6%); with the ballot 1 step gave
// 62.5%, 4 steps 75.4%, 12 steps 71.5-71.9%. The grouped quantiser keeps the
// binary search (75.6-75.9% with the ballot against 76.7-77.4%). Single
// tensors: fp32 [4096, 4096] dequantise 4 steps 15.1 us, 2 steps 15.3,
// 1 step 18.6.
constexpr int kUnroll = 4;
constexpr int kDequantUnroll = 4;
constexpr int kGroupUnroll = 8;
constexpr int kDequantGroupUnroll = 2;
constexpr float kTieMargin = 6.0e-5f;
constexpr float kMinFastScale = 7.88860905e-31f;  // 2^-100
constexpr float kRoundShift = 12582912.0f;        // 3 * 2^22

struct BlockScale {
    float s;
    float inv;
    bool exact;
};

__device__ __forceinline__ BlockScale block_scale(uint32_t absmax_bits) {
    const float absmax = __uint_as_float(absmax_bits);
    float s = absmax / 127.0f;
    s = (s > 0.0f) ? s : 1.0f;
    BlockScale b;
    b.s = s;
    b.inv = 1.0f / s;
    b.exact = !(s >= kMinFastScale);
    return b;
}

/// The scales of kU blocks whose absmax bit patterns every lane holds in
/// mx[0 .. kU) (kU a multiple of 4). Each block's two IEEE divides (absmax /
/// 127 and 1 / s) are the bulk of the quantiser's arithmetic, and the lanes
/// of a block compute them alike; here lane l of each quad divides for block
/// c + l % 4 and quad-permute DPP moves hand the four results to every lane
/// of the quad: one divide sequence per four blocks instead of one per
/// block, the same values (block_scale on the same bits). All 64 lanes must
/// be active.
template <int kU>
__device__ __forceinline__ void block_scales(const uint32_t (&mx)[kU], BlockScale (&bs)[kU]) {
    static_assert(kU % 4 == 0, "blocks are taken four at a time");
    // Lane bits 0 and 1 as all-ones masks. The pick is written as masked xors:
    // a chain of selects is turned into an indexed load from a stack copy.
    const uint32_t b0 = 0u - (threadIdx.x & 1u);
    const uint32_t b1 = 0u - ((threadIdx.x >> 1) & 1u);
#pragma unroll
    for (int c = 0; c < kU; c += 4) {
        const uint32_t a01 = mx[c] ^ ((mx[c] ^ mx[c + 1]) & b0);
        const uint32_t a23 = mx[c + 2] ^ ((mx[c + 2] ^ mx[c + 3]) & b0);
        const uint32_t mine = a01 ^ ((a01 ^ a23) & b1);
        const BlockScale b = block_scale(mine);
        auto take = [&](auto kk) {
            constexpr int k = decltype(kk)::value;
            constexpr int kCtrl = k | (k << 2) | (k << 4) | (k << 6);  // quad_perm [k, k, k, k]
            BlockScale& out = bs[c + k];
            out.s = dpp_f32<kCtrl>(b.s);
            out.inv = dpp_f32<kCtrl>(b.inv);
            out.exact = !(out.s >= kMinFastScale);
        };
        take(std::integral_constant<int, 0>{});
        take(std::integral_constant<int, 1>{});
        take(std::integral_constant<int, 2>{});
        take(std::integral_constant<int, 3>{});
    }
}

/// A rounded quotient clamped to [-127, 127]; NaN gives 0 (what ATen's
/// float->int8 conversion of a NaN yields after torch.clamp propagates it).
__device__ __forceinline__ int clamp_code(float r) {
    if (r != r) return 0;
    return static_cast<int>(fminf(fmaxf(r, -127.0f), 127.0f));
}

/// rint(x / s), round half to even, via the reciprocal and, next to a
/// half-integer, one Markstein correction (valid unless b.exact).
__device__ __forceinline__ int fast_code(float x, const BlockScale& b) {
    const float q0 = x * b.inv;
    const float r0 = rintf(q0);
    const float q1 = fmaf(fmaf(-q0, b.s, x), b.inv, q0);  // fl(x / s)
    return clamp_code(fabsf(q0 - r0) > 0.5f - kTieMargin ? rintf(q1) : r0);
}

/// Four codes of an ordinary block (finite absmax, s >= 2^-100) packed into
/// one word; see the file comment.
__device__ __forceinline__ uint32_t pack4_ordinary(const float* v, const BlockScale& b) {
    uint32_t t[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float q0 = v[i] * b.inv;
        const float q1 = fmaf(fmaf(-q0, b.s, v[i]), b.inv, q0);  // fl(v / s)
        t[i] = __float_as_uint(q1 + kRoundShift);                 // low byte: int8(rint(q1))
    }
    // v_perm_b32 byte selects: 0-3 take the second operand's bytes, 4-7 the
    // first's, 0x0c gives zero.
    const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], 0x0c0c0400u);  // codes 0, 1
    const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], 0x0c0c0400u);  // codes 2, 3
    return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

/// rint(x / s) with the IEEE divide.
__device__ __forceinline__ int exact_code(float x, const BlockScale& b) {
    return clamp_code(rintf(x / b.s));
}

__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

/// Load the kPer elements of this lane (zero beyond `count`). kFull: the
/// caller guarantees the whole vector is in range and aligned, so the load
/// is unconditional (no branch, no select on the loaded data, which would
/// make the compiler wait for each load before issuing the next).
template <typename T, bool kVec, bool kFull>
__device__ __forceinline__ void load_lane(const T* __restrict__ x, int64_t e, int64_t count,
                                          float* v) {
    constexpr int kPer = Storage<T>::kPerVec;
    if (kFull) {
        unpack16<T>(load_stream16(x + e), v);
    } else if (kVec && e + kPer <= count) {
        unpack16<T>(load_stream16(x + e), v);
    } else {
#pragma unroll
        for (int i = 0; i < kPer; ++i) v[i] = (e + i < count) ? Storage<T>::load(x + e + i) : 0.0f;
    }
}

/// The loads of one step of quant_body: this lane's kPer elements of each of
/// the kU block groups of step `wave` (zeros past `count`).
template <typename T, bool kVec, bool kFull, int kU>
__device__ __forceinline__ void quant_load(const T* __restrict__ x, int64_t count, int64_t wave,
                                           float (&v)[kU][Storage<T>::kPerVec]) {
    constexpr int kPer = Storage<T>::kPerVec;
    constexpr int kLanesPerBlock = kQuantBlockSize / kPer;
    constexpr int kBlocksPerStep = kWaveSize / kLanesPerBlock;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t base_block = wave * (kBlocksPerStep * kU);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t block = base_block + u * kBlocksPerStep + lane / kLanesPerBlock;
        load_lane<T, kVec, kFull>(x, block * kQuantBlockSize + (lane % kLanesPerBlock) * kPer, count, v[u]);
    }
}

/// Quantise (kMode 0: codes + scales) or fake-quantise (kMode 1: q * s in T)
/// the elements quant_load brought in for step `wave`. kFull: every element
/// of the step is inside `count` and the pointers are vector-aligned, so
/// stores need no bounds tests. Every lane of the wave must be active.
template <typename T, bool kVec, int kMode, bool kFull, int kU>
__device__ __forceinline__ void quant_process(float (&v)[kU][Storage<T>::kPerVec], int8_t* __restrict__ q,
                                              float* __restrict__ scales, T* __restrict__ y, int64_t count,
                                              int64_t wave) {
    constexpr int kPer = Storage<T>::kPerVec;                  // 4 (fp32) or 8 (16-bit)
    constexpr int kLanesPerBlock = kQuantBlockSize / kPer;     // 16 or 8
    constexpr int kBlocksPerStep = kWaveSize / kLanesPerBlock; // 4 or 8

    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t base_block = wave * (kBlocksPerStep * kU);
    const int sub = lane / kLanesPerBlock;
    const int part = lane % kLanesPerBlock;

    uint32_t mx[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const uint32_t a = abs_bits(v[u][i]);
            m = a > m ? a : m;
        }
        mx[u] = group_reduce_u32<kLanesPerBlock, MaxU32>(m);
    }
    BlockScale bs[kU];
    block_scales<kU>(mx, bs);

#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const uint32_t m = mx[u];
        const BlockScale& b = bs[u];

        const int64_t block = base_block + u * kBlocksPerStep + sub;
        const int64_t e = block * kQuantBlockSize + part * kPer;
        if (!kFull && e >= count) continue;

        if constexpr (kMode == 0) {
            const bool ordinary = m < 0x7F800000u && !b.exact;
            uint32_t w[kPer / 4];
            if (ordinary) {
#pragma unroll
                for (int j = 0; j < kPer / 4; ++j) w[j] = pack4_ordinary(&v[u][4 * j], b);
            } else {
                int c[kPer];
#pragma unroll
                for (int i = 0; i < kPer; ++i) c[i] = b.exact ? exact_code(v[u][i], b) : fast_code(v[u][i], b);
#pragma unroll
                for (int j = 0; j < kPer / 4; ++j) {
                    w[j] = (static_cast<uint32_t>(c[4 * j]) & 0xFFu) |
                           ((static_cast<uint32_t>(c[4 * j + 1]) & 0xFFu) << 8) |
                           ((static_cast<uint32_t>(c[4 * j + 2]) & 0xFFu) << 16) |
                           ((static_cast<uint32_t>(c[4 * j + 3]) & 0xFFu) << 24);
                }
            }
            // A plain store: the 4-byte scales of neighbouring waves merge into
            // whole lines in L2 (a non-temporal store of each costs ~7% of the
            // kernel). The codes and inputs stay non-temporal.
            if (part == 0) scales[block] = b.s;
            if (kFull || (kVec && e + kPer <= count)) {
                if constexpr (kPer == 4) {
                    store_stream4(q + e, w[0]);
                } else {
                    store_stream8(q + e, make_uint2(w[0], w[1]));
                }
            } else {
#pragma unroll
                for (int i = 0; i < kPer; ++i) {
                    if (e + i < count) q[e + i] = static_cast<int8_t>((w[i / 4] >> (8 * (i % 4))) & 0xFFu);
                }
            }
            continue;
        }

        // Fake quantisation: the reciprocal path for every element; blocks with
        // a scale below 2^-100 (rare: only when the whole block is that small)
        // divide.
        int codes[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) codes[i] = fast_code(v[u][i], b);
        if (__any(b.exact)) {
            if (b.exact) {
#pragma unroll
                for (int i = 0; i < kPer; ++i) codes[i] = exact_code(v[u][i], b);
            }
        }

        float out[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) out[i] = static_cast<float>(codes[i]) * b.s;
        if (kFull || (kVec && e + kPer <= count)) {
            store_stream16(y + e, pack16<T>(out));
        } else {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                if (e + i < count) Storage<T>::store(y + e + i, out[i]);
            }
        }
    }
}

/// One step of quantise / fake-quantise: the loads, then the arithmetic and
/// stores. kFull: every element of step `wave` is inside `count` and the
/// pointers are vector-aligned (all waves but the last).
template <typename T, bool kVec, int kMode, bool kFull, int kU = kUnroll>
__device__ __forceinline__ void quant_body(const T* __restrict__ x, int8_t* __restrict__ q,
                                           float* __restrict__ scales, T* __restrict__ y,
                                           int64_t count, int64_t wave) {
    float v[kU][Storage<T>::kPerVec];
    quant_load<T, kVec, kFull, kU>(x, count, wave, v);
    // Keep every load of the step ahead of the first use: without this the
    // scheduler starts on block 0 after two of the four loads.
    __builtin_amdgcn_sched_barrier(0);
    quant_process<T, kVec, kMode, kFull, kU>(v, q, scales, y, count, wave);
}

/// Index of the calling wave in the grid (wave-uniform).
__device__ __forceinline__ int64_t grid_wave() {
    return static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWaveSize) +
           static_cast<int64_t>(threadIdx.x) / kWaveSize;
}

/// Quantisation blocks one wave covers.
template <typename T, int kU = kUnroll>
constexpr int64_t quant_blocks_per_wave() {
    return (kWaveSize / (kQuantBlockSize / Storage<T>::kPerVec)) * kU;
}

/// True when every element of wave `wave`'s quantisation blocks is below
/// `count` (wave-uniform).
template <typename T, int kU = kUnroll>
__device__ __forceinline__ bool wave_is_full(int64_t count, int64_t wave) {
    return (wave + 1) * quant_blocks_per_wave<T, kU>() * kQuantBlockSize <= count;
}

template <typename T, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void quantize_kernel(const T* __restrict__ x,
                                                                     int8_t* __restrict__ q,
                                                                     float* __restrict__ scales,
                                                                     int64_t count) {
    const int64_t wave = grid_wave();
    if (kVec && wave_is_full<T>(count, wave)) {
        quant_body<T, kVec, 0, true>(x, q, scales, nullptr, count, wave);
    } else {
        quant_body<T, kVec, 0, false>(x, q, scales, nullptr, count, wave);
    }
}

template <typename T, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void fake_quant_kernel(const T* __restrict__ x,
                                                                       T* __restrict__ y,
                                                                       int64_t count) {
    const int64_t wave = grid_wave();
    if (kVec && wave_is_full<T>(count, wave)) {
        quant_body<T, kVec, 1, true>(x, nullptr, nullptr, y, count, wave);
    } else {
        quant_body<T, kVec, 1, false>(x, nullptr, nullptr, y, count, wave);
    }
}

/// y = float(q) * s, one multiply, rounded to Tout. Each lane owns kPer
/// consecutive elements (always inside one block); codes come in by
/// non-temporal loads and a wave stores 1 KiB per step with 16-byte
/// non-temporal stores. (Plain code loads measured 70% against 71% of HBM
/// peak at config 1 once no launch could find its codes in the Infinity
/// Cache; device-scope (sc1) output stores, 62%.) kFull: the wave's whole
/// range is below `count` and aligned, so nothing is bounds-tested.
template <typename Tout, bool kVec, bool kFull, int kU = kUnroll>
__device__ __forceinline__ void dequantize_body(const int8_t* __restrict__ q,
                                                const float* __restrict__ scales,
                                                Tout* __restrict__ y, int64_t count,
                                                int64_t wave) {
    constexpr int kPer = Storage<Tout>::kPerVec;
    constexpr int64_t kStep = static_cast<int64_t>(kWaveSize) * kPer;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t base = wave * kStep * kU + static_cast<int64_t>(lane) * kPer;

    int codes[kU][kPer];
    float scale[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t e = base + u * kStep;
        scale[u] = (kFull || e < count) ? scales[e / kQuantBlockSize] : 0.0f;
        if (kFull || (kVec && e + kPer <= count)) {
            if constexpr (kPer == 4) {
                const uint32_t w = load_stream4(q + e);
#pragma unroll
                for (int i = 0; i < 4; ++i) codes[u][i] = static_cast<int8_t>((w >> (8 * i)) & 0xFFu);
            } else {
                const uint2 w = load_stream8(q + e);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    codes[u][i] = static_cast<int8_t>((w.x >> (8 * i)) & 0xFFu);
                    codes[u][4 + i] = static_cast<int8_t>((w.y >> (8 * i)) & 0xFFu);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kPer; ++i) codes[u][i] = (e + i < count) ? q[e + i] : 0;
        }
    }

#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t e = base + u * kStep;
        if (!kFull && e >= count) continue;
        float out[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) out[i] = static_cast<float>(codes[u][i]) * scale[u];
        if (kFull || (kVec && e + kPer <= count)) {
            store_stream16(y + e, pack16<Tout>(out));
        } else {
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                if (e + i < count) Storage<Tout>::store(y + e + i, out[i]);
            }
        }
    }
}

/// Elements one dequantising wave covers.
template <typename Tout, int kU = kUnroll>
constexpr int64_t dequant_elements_per_wave() {
    return static_cast<int64_t>(kWaveSize) * Storage<Tout>::kPerVec * kU;
}

template <typename Tout, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void dequantize_kernel(
    const int8_t* __restrict__ q, const float* __restrict__ scales, Tout* __restrict__ y,
    int64_t count) {
    const int64_t wave = grid_wave();
    if (kVec && (wave + 1) * dequant_elements_per_wave<Tout, kDequantUnroll>() <= count) {
        dequantize_body<Tout, kVec, true, kDequantUnroll>(q, scales, y, count, wave);
    } else {
        dequantize_body<Tout, kVec, false, kDequantUnroll>(q, scales, y, count, wave);
    }
}

/// Workgroups needed so that every block (or element step) has a wave.
template <typename T>
int64_t quant_grid(int64_t count) {
    constexpr int kPer = Storage<T>::kPerVec;
    constexpr int64_t kBlocksPerWave = (kWaveSize / (kQuantBlockSize / kPer)) * kUnroll;
    const int64_t blocks = ceil_div<int64_t>(count, kQuantBlockSize);
    const int64_t waves = ceil_div<int64_t>(blocks, kBlocksPerWave);
    return ceil_div<int64_t>(waves, kDefaultBlockSize / kWaveSize);
}

template <typename T>
int64_t dequant_grid(int64_t count) {
    const int64_t waves = ceil_div<int64_t>(count, dequant_elements_per_wave<T, kDequantUnroll>());
    return ceil_div<int64_t>(waves, kDefaultBlockSize / kWaveSize);
}

constexpr int64_t kMaxGrid = 2147483647;

// ---------------------------------------------------------------------------
// Grouped launches: up to CF_QUANT_GROUP_MAX tensors per kernel, described in
// the kernel arguments (no device-side staging, nothing allocated). Tensor t
// owns grid waves [first_wave[t], first_wave[t + 1]); each wave finds its
// tensor in first_wave (a binary search of scalar loads from the kernel
// argument segment for quantisation, one ballot over a vector load for
// dequantisation) and then runs the single-tensor body with its index inside
// that tensor. Every tensor of a group is vector-aligned.
// ---------------------------------------------------------------------------

constexpr int kGroupMax = CF_QUANT_GROUP_MAX;

struct QuantGroupArgs {
    const void* x[kGroupMax];
    int8_t* q[kGroupMax];
    float* scales[kGroupMax];
    int64_t count[kGroupMax];
    int64_t first_wave[kGroupMax + 1];
    int n;
};

struct DequantGroupArgs {
    const int8_t* q[kGroupMax];
    const float* scales[kGroupMax];
    void* y[kGroupMax];
    int64_t count[kGroupMax];
    int64_t first_wave[kGroupMax + 1];
    int n;
};

/// Index t with first_wave[t] <= wave < first_wave[t + 1] (wave-uniform;
/// the caller has checked wave < first_wave[n]).
__device__ __forceinline__ int group_member(const int64_t* first_wave, int n, int64_t wave) {
    int lo = 0;
    int hi = n;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (first_wave[mid] <= wave) {
            lo = mid;
        } else {
            hi = mid;
        }
    }
    return lo;
}

/// The same index t in one round trip: lane l reads tensor l's first wave
/// (n <= 48 < 64 lanes) and a ballot counts the tensors that start at or
/// before `wave` (first_wave is increasing and first_wave[0] = 0). Every lane
/// of the wave must be active; the caller has checked wave < first_wave[n].
__device__ __forceinline__ int group_member_ballot(const int64_t* first_wave, int n, int64_t wave) {
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t fw = lane < n ? first_wave[lane] : INT64_MAX;
    return __popcll(__ballot(fw <= wave)) - 1;
}

template <typename T>
__global__ __launch_bounds__(kDefaultBlockSize) void quantize_group_kernel(QuantGroupArgs args) {
    const int64_t gw = grid_wave();
    if (gw >= args.first_wave[args.n]) return;  // wave-uniform
    const int t = group_member(args.first_wave, args.n, gw);
    const int64_t wave = gw - args.first_wave[t];
    const T* x = static_cast<const T*>(args.x[t]);
    const int64_t count = args.count[t];
    if (wave_is_full<T, kGroupUnroll>(count, wave)) {
        quant_body<T, true, 0, true, kGroupUnroll>(x, args.q[t], args.scales[t], nullptr, count, wave);
    } else {
        quant_body<T, true, 0, false, kGroupUnroll>(x, args.q[t], args.scales[t], nullptr, count, wave);
    }
}

template <typename Tout>
__global__ __launch_bounds__(kDefaultBlockSize) void dequantize_group_kernel(DequantGroupArgs args) {
    const int64_t gw = grid_wave();
    if (gw >= args.first_wave[args.n]) return;  // wave-uniform
    const int t = group_member_ballot(args.first_wave, args.n, gw);
    const int64_t wave = gw - args.first_wave[t];
    Tout* y = static_cast<Tout*>(args.y[t]);
    const int64_t count = args.count[t];
    if ((wave + 1) * dequant_elements_per_wave<Tout, kDequantGroupUnroll>() <= count) {
        dequantize_body<Tout, true, true, kDequantGroupUnroll>(args.q[t], args.scales[t], y, count, wave);
    } else {
        dequantize_body<Tout, true, false, kDequantGroupUnroll>(args.q[t], args.scales[t], y, count, wave);
    }
}

template <typename T>
cf_status launch_quantize(const void* x, int8_t* q, float* scales, int64_t count,
                          hipStream_t stream) {
    const int64_t grid = quant_grid<T>(count);
    CF_REQUIRE(grid <= kMaxGrid, "cf_quantize_int8: %lld elements exceed the launch limit",
               static_cast<long long>(count));
    constexpr int kPer = Storage<T>::kPerVec;
    const bool vec = host_aligned(x, 16) && host_aligned(q, kPer);
    if (vec) {
        launch(quantize_kernel<T, true>, dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize),
               0, stream, static_cast<const T*>(x), q, scales, count);
    } else {
        launch(quantize_kernel<T, false>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x), q, scales, count);
    }
    return check_launch("launching quantize_int8", stream);
}

template <typename T>
cf_status launch_fake_quant(const void* x, void* y, int64_t count, hipStream_t stream) {
    const int64_t grid = quant_grid<T>(count);
    CF_REQUIRE(grid <= kMaxGrid, "cf_quantize_dequantize: %lld elements exceed the launch limit",
               static_cast<long long>(count));
    const bool vec = host_aligned(x, 16) && host_aligned(y, 16);
    if (vec) {
        launch(fake_quant_kernel<T, true>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x), static_cast<T*>(y),
               count);
    } else {
        launch(fake_quant_kernel<T, false>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x), static_cast<T*>(y),
               count);
    }
    return check_launch("launching quantize_dequantize", stream);
}

template <typename T>
cf_status launch_dequantize(const int8_t* q, const float* scales, void* y, int64_t count,
                            hipStream_t stream) {
    const int64_t grid = dequant_grid<T>(count);
    CF_REQUIRE(grid <= kMaxGrid, "cf_dequantize_int8: %lld elements exceed the launch limit",
               static_cast<long long>(count));
    constexpr int kPer = Storage<T>::kPerVec;
    const bool vec = host_aligned(q, kPer) && host_aligned(y, 16);
    if (vec) {
        launch(dequantize_kernel<T, true>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, q, scales, static_cast<T*>(y), count);
    } else {
        launch(dequantize_kernel<T, false>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, q, scales, static_cast<T*>(y), count);
    }
    return check_launch("launching dequantize_int8", stream);
}

/// Send one group (if any) and empty it.
template <typename Kernel, typename Args>
cf_status flush_group(Kernel kernel, Args& args, int64_t& waves, const char* what,
                      hipStream_t stream) {
    if (args.n == 0) return CF_OK;
    args.first_wave[args.n] = waves;
    const int64_t grid = ceil_div<int64_t>(waves, kDefaultBlockSize / kWaveSize);
    CF_REQUIRE(grid <= kMaxGrid, "%s: a group exceeds the launch limit", what);
    launch(kernel, dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize), 0, stream, args);
    args.n = 0;
    waves = 0;
    return check_launch(what, stream);
}

template <typename T>
cf_status launch_quantize_group(const void* const* x, int8_t* const* q, float* const* scales,
                                const int64_t* counts, int64_t n, hipStream_t stream) {
    constexpr int kPer = Storage<T>::kPerVec;
    constexpr const char* kWhat = "launching the grouped quantize_int8";
    QuantGroupArgs args;
    args.n = 0;
    int64_t waves = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t count = counts[i];
        if (count <= 0) continue;
        CF_REQUIRE(x[i] != nullptr && q[i] != nullptr && scales[i] != nullptr,
                   "cf_quantize_int8_group: null pointer in tensor %lld", static_cast<long long>(i));
        if (!host_aligned(x[i], 16) || !host_aligned(q[i], kPer)) {
            const cf_status status = launch_quantize<T>(x[i], q[i], scales[i], count, stream);
            if (status != CF_OK) return status;
            continue;
        }
        const int64_t blocks = ceil_div<int64_t>(count, kQuantBlockSize);
        args.x[args.n] = x[i];
        args.q[args.n] = q[i];
        args.scales[args.n] = scales[i];
        args.count[args.n] = count;
        args.first_wave[args.n] = waves;
        waves += ceil_div<int64_t>(blocks, quant_blocks_per_wave<T, kGroupUnroll>());
        if (++args.n == kGroupMax) {
            const cf_status status = flush_group(quantize_group_kernel<T>, args, waves, kWhat, stream);
            if (status != CF_OK) return status;
        }
    }
    return flush_group(quantize_group_kernel<T>, args, waves, kWhat, stream);
}

template <typename T>
cf_status launch_dequantize_group(const int8_t* const* q, const float* const* scales,
                                  void* const* y, const int64_t* counts, int64_t n,
                                  hipStream_t stream) {
    constexpr int kPer = Storage<T>::kPerVec;
    constexpr const char* kWhat = "launching the grouped dequantize_int8";
    DequantGroupArgs args;
    args.n = 0;
    int64_t waves = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t count = counts[i];
        if (count <= 0) continue;
        CF_REQUIRE(q[i] != nullptr && scales[i] != nullptr && y[i] != nullptr,
                   "cf_dequantize_int8_group: null pointer in tensor %lld", static_cast<long long>(i));
        if (!host_aligned(q[i], kPer) || !host_aligned(y[i], 16)) {
            const cf_status status = launch_dequantize<T>(q[i], scales[i], y[i], count, stream);
            if (status != CF_OK) return status;
            continue;
        }
        args.q[args.n] = q[i];
        args.scales[args.n] = scales[i];
        args.y[args.n] = y[i];
        args.count[args.n] = count;
        args.first_wave[args.n] = waves;
        waves += ceil_div<int64_t>(count, dequant_elements_per_wave<T, kDequantGroupUnroll>());
        if (++args.n == kGroupMax) {
            const cf_status status =
                flush_group(dequantize_group_kernel<T>, args, waves, kWhat, stream);
            if (status != CF_OK) return status;
        }
    }
    return flush_group(dequantize_group_kernel<T>, args, waves, kWhat, stream);
}

}  // namespace
}  // namespace cf

extern "C" {

cf_status cf_quantize_int8_group(const void* const* x, cf_dtype x_dtype, int8_t* const* q,
                                 float* const* scales, const int64_t* counts, int64_t n_tensors,
                                 void* stream) {
    CF_ENTRY();
    if (n_tensors <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && q != nullptr && scales != nullptr && counts != nullptr,
               "cf_quantize_int8_group: null array");
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::launch_quantize_group<float>(x, q, scales, counts, n_tensors, s);
        case CF_BF16:
            return cf::launch_quantize_group<cf::bf16_t>(x, q, scales, counts, n_tensors, s);
        case CF_F16:
            return cf::launch_quantize_group<cf::f16_t>(x, q, scales, counts, n_tensors, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_quantize_int8_group: unknown input dtype %d",
                    static_cast<int>(x_dtype));
}

cf_status cf_dequantize_int8_group(const int8_t* const* q, const float* const* scales,
                                   void* const* y, cf_dtype y_dtype, const int64_t* counts,
                                   int64_t n_tensors, void* stream) {
    CF_ENTRY();
    if (n_tensors <= 0) return CF_OK;
    CF_REQUIRE(q != nullptr && scales != nullptr && y != nullptr && counts != nullptr,
               "cf_dequantize_int8_group: null array");
    auto s = static_cast<hipStream_t>(stream);
    switch (y_dtype) {
        case CF_F32:
            return cf::launch_dequantize_group<float>(q, scales, y, counts, n_tensors, s);
        case CF_BF16:
            return cf::launch_dequantize_group<cf::bf16_t>(q, scales, y, counts, n_tensors, s);
        case CF_F16:
            return cf::launch_dequantize_group<cf::f16_t>(q, scales, y, counts, n_tensors, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_dequantize_int8_group: unknown output dtype %d",
                    static_cast<int>(y_dtype));
}

int64_t cf_quant_scale_count(int64_t count) {
    return count <= 0 ? 0 : cf::ceil_div<int64_t>(count, cf::kQuantBlockSize);
}

cf_status cf_quantize_int8(const void* x, cf_dtype x_dtype, int8_t* q, float* scales,
                           int64_t count, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && q != nullptr && scales != nullptr,
               "cf_quantize_int8: null pointer (x=%p q=%p scales=%p)", x,
               static_cast<void*>(q), static_cast<void*>(scales));
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::launch_quantize<float>(x, q, scales, count, s);
        case CF_BF16:
            return cf::launch_quantize<cf::bf16_t>(x, q, scales, count, s);
        case CF_F16:
            return cf::launch_quantize<cf::f16_t>(x, q, scales, count, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_quantize_int8: unknown input dtype %d",
                    static_cast<int>(x_dtype));
}

cf_status cf_dequantize_int8(const int8_t* q, const float* scales, void* y, cf_dtype y_dtype,
                             int64_t count, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(q != nullptr && scales != nullptr && y != nullptr,
               "cf_dequantize_int8: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    switch (y_dtype) {
        case CF_F32:
            return cf::launch_dequantize<float>(q, scales, y, count, s);
        case CF_BF16:
            return cf::launch_dequantize<cf::bf16_t>(q, scales, y, count, s);
        case CF_F16:
            return cf::launch_dequantize<cf::f16_t>(q, scales, y, count, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_dequantize_int8: unknown output dtype %d",
                    static_cast<int>(y_dtype));
}

cf_status cf_quantize_dequantize(const void* x, void* y, cf_dtype dtype, int64_t count,
                                 void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_quantize_dequantize: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case CF_F32:
            return cf::launch_fake_quant<float>(x, y, count, s);
        case CF_BF16:
            return cf::launch_fake_quant<cf::bf16_t>(x, y, count, s);
        case CF_F16:
            return cf::launch_fake_quant<cf::f16_t>(x, y, count, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_quantize_dequantize: unknown dtype %d",
                    static_cast<int>(dtype));
}

}  // extern "C"

// Attention over a paged KV cache for one decode step (one query token per
// sequence), the operator the reference's block tables exist for
// (cuda/include/cudaforge/paged_attention.cuh:10-61, cuda/src/paged_attention.cu).
//
// Layouts (the reference's): query / out [S, H, D]; k_cache / v_cache
// [num_blocks, block_size, KVH, D]; block_tables [S, max_blocks] (uint32);
// context_lens [S]. Token t of sequence s lives in physical block
// block_tables[s][t / block_size] at offset t % block_size. H is a multiple of
// KVH (grouped-query attention: head h reads KV head h / (H / KVH)). fp32
// scores, online softmax, zeros for an empty context.
//
// Design on gfx950 (HBM-bound: every K and V element of a context is read once
// per KV head, 2 * context * D * sizeof(T) bytes per (sequence, KV head)):
//   * One workgroup (4 waves) per (sequence, KV head, group of up to 4 query
//     heads, context split): the query heads of a GQA group are served from
//     one pass over K and V, instead of re-reading the KV head per query head.
//     Larger groups take several workgroups per KV head (each reads K and V;
//     the per-head state of 8 heads held the kernel to 2 waves per SIMD and
//     ran slower: group 8 fp32 32 -> 36%, bf16 25 -> 29% of HBM peak).
//   * A token's K (and V) row is read by D/4 lanes (fp32) or D/8 lanes (bf16),
//     16 bytes each, several tokens per wave instruction: whole rows,
//     coalesced. Each lane keeps its 4 (8) query values and output
//     accumulators per head; a score is a butterfly sum over the token's lanes.
//   * The block table is held as a 64-entry window in lane registers, so a
//     token's address costs a lane shuffle, not a dependent memory load, and
//     the K/V loads of the next chunk of tokens are in flight while the
//     current chunk is consumed.
//   * Online softmax per head per token slot, rescaled once per chunk; slots,
//     then waves, then splits are merged with the (max, sum, accumulator)
//     rescaling rule.
//   * Long contexts are split across workgroups so short batches still fill
//     256 CUs; a second small kernel combines the splits (caller workspace).
//     Without a workspace every (sequence, KV head) runs unsplit.
// Head sizes the 16-byte lane pieces do not tile (fp32: 4 * 2^j <= 256,
// bf16: 8 * 2^j <= 512), or unaligned tensors, take a wave-per-head kernel
// (one token per step, lanes over the head dimension, up to 1024).
#include <cfloat>
#include <type_traits>

#include "cf_common.hpp"

namespace cf {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWaveSize;
constexpr int kMaxGroup = 4;          // query heads per workgroup
constexpr int kMinSplitTokens = 256;  // tokens per split, at least
constexpr int kTargetWorkgroups = 1024;

struct PagedArgs {
    const void* query;
    const void* k_cache;
    const void* v_cache;
    const uint32_t* tables;
    const int32_t* context;
    void* out;
    float* partial;  // [S][H][splits][D + 2] (m, l, acc[D]) when splits > 1
    int64_t heads;
    int64_t kv_heads;
    int64_t head_dim;
    int64_t block_size;
    int64_t max_blocks;
    int64_t split_tokens;
    int splits;
    int head_groups;  // workgroups per KV head (ceil(group / GS))
    float scale;
};

/// Values of T in one 16-byte load: a lane's share of a K or V row.
template <typename T>
constexpr int vals_per_lane() { return 16 / static_cast<int>(sizeof(T)); }

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4_t load16(const void* base, int64_t byte_offset) {
    return *reinterpret_cast<const u32x4_t*>(static_cast<const uint8_t*>(base) + byte_offset);
}

/// A 16-byte piece of a K or V row of cache type T. fp32 caches are read
/// with the non-temporal hint and 16-bit caches without: at the benchmark
/// shapes the hint moved fp32 decode 6-12% up (5.2 -> 5.8 TB/s for 16
/// sequences x 512 tokens, 32 heads) and bf16 decode 4-10% down.
template <typename T>
__device__ __forceinline__ u32x4_t load16_kv(const void* base, int64_t byte_offset) {
    const auto* p = reinterpret_cast<const u32x4_t*>(static_cast<const uint8_t*>(base) + byte_offset);
    if constexpr (std::is_same<T, float>::value) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}

/// The kVals values of a raw 16-byte piece, widened to fp32.
template <typename T>
__device__ __forceinline__ void widen(const u32x4_t& raw, float (&v)[vals_per_lane<T>()]) {
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(raw[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(raw[e] << 16);
            v[2 * e + 1] = __uint_as_float(raw[e] & 0xffff0000u);
        }
    }
}

template <typename T>
__device__ __forceinline__ void store_piece(T* base, int64_t index, const float (&v)[vals_per_lane<T>()]) {
    u32x4_t raw;
    if constexpr (std::is_same<T, float>::value) {
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[e] = __float_as_uint(v[e]);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[e] = f32_to_bf16_bits(v[2 * e]) | (f32_to_bf16_bits(v[2 * e + 1]) << 16);
    }
    *reinterpret_cast<u32x4_t*>(base + index) = raw;
}

/// Sum over aligned groups of kLanes lanes (DPP within 16-lane rows, lane
/// permutes across rows); every lane of a group gets the group's sum. All 64
/// lanes must be active.
template <int kLanes>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (kLanes == 2) {
        v += dpp_f32<kDppQuadXor1>(v);
    } else if constexpr (kLanes == 4 || kLanes == 8 || kLanes == 16) {
        v = group_reduce_f32<kLanes, AddF32>(v);
    } else if constexpr (kLanes >= 32) {
        v = group_reduce_f32<16, AddF32>(v);
        v += __shfl_xor(v, 16);
        if constexpr (kLanes == 64) v += __shfl_xor(v, 32);
    }
    return v;
}

/// Online-softmax state of one query head over kVals output dimensions.
template <int kVals>
struct HeadState {
    float m;
    float l;
    float acc[kVals];
};

/// Folds (m2, l2, acc2) into s: both are partial softmax sums over disjoint
/// token sets; an empty one has m = -inf and l = 0 and contributes nothing.
template <int kVals>
__device__ __forceinline__ void merge_into(HeadState<kVals>& s, float m2, float l2, const float (&acc2)[kVals]) {
    const float m = fmaxf(s.m, m2);
    const float c1 = s.m == -INFINITY ? 0.0f : __expf(s.m - m);
    const float c2 = m2 == -INFINITY ? 0.0f : __expf(m2 - m);
    s.l = s.l * c1 + l2 * c2;
#pragma unroll
    for (int e = 0; e < kVals; ++e) s.acc[e] = s.acc[e] * c1 + acc2[e] * c2;
    s.m = m;
}

/// One wave's walk over the block table of a (sequence, split). A wave takes
/// chunks of consecutive tokens c0, c0 + stride, ...; lane-relative token k of
/// a chunk (k < kSpan) is token c0 + k. The block and in-block position of c0
/// (q0, r0; wave uniform) advance by whole strides, so no lane divides by the
/// block size: token c0 + k is in block q0 + dq with dq = (r0 + k) / block
/// size, where r0 + k < block size + kSpan. For blocks of kSpan tokens or more
/// dq is 0 or 1; below that it is the quotient of two numbers under 2 kSpan
/// (<= 128), exact from a float reciprocal and one upward correction (the
/// float product is within 2^-23 of r / block size, which is at least
/// 1 / block size from the next integer unless it is one). Token positions
/// are below 2^31 (int32 context lengths), so q0, r0 and r0 + k fit 32 bits
/// for any block size; comparisons use the block size saturated to 32 bits.
/// 64 block-table entries sit in lane registers, so a token's block is a lane
/// shuffle, not a dependent load. The matrix-core kernels use it. The
/// streaming kernel keeps a per-token (32-bit) division: with the cursor its
/// fp32 group-4 form needed 141 VGPRs instead of 118, one wave per SIMD fewer,
/// and ran at 54% of HBM peak instead of 61% (128 x 256 tokens).
template <int kSpan>
struct TokenCursor {
    static_assert(kSpan >= 1 && kSpan <= kWaveSize, "span");
    const uint32_t* table;  // this sequence's block-table row
    int64_t max_blocks;
    int64_t block_size;
    uint32_t bs;            // block size saturated to 32 bits
    float inv_bs;
    uint32_t q0, r0;        // block and position of the chunk's first token
    uint32_t step_q, step_r;
    int64_t window_base;
    int window;             // table[window_base + lane]

    __device__ void load_window(int64_t base, int lane) {
        const int64_t entry = base + lane < max_blocks ? base + lane : max_blocks - 1;
        window_base = base;
        window = static_cast<int>(table[entry]);
    }
    __device__ void start(const uint32_t* row, int64_t blocks, int64_t size, int64_t first, int64_t stride,
                          int lane) {
        table = row;
        max_blocks = blocks;
        block_size = size;
        bs = size < int64_t{0xFFFFFFFF} ? static_cast<uint32_t>(size) : 0xFFFFFFFFu;
        inv_bs = 1.0f / static_cast<float>(bs);
        q0 = static_cast<uint32_t>(first / size);
        r0 = static_cast<uint32_t>(first % size);
        step_q = static_cast<uint32_t>(stride / size);
        step_r = static_cast<uint32_t>(stride % size);
        load_window(q0, lane);
    }
    /// Move q0, r0 on by one stride.
    __device__ void advance() {
        q0 += step_q;
        r0 += step_r;
        if (r0 >= bs) {
            r0 -= bs;
            ++q0;
        }
    }
    /// Make the window cover the blocks of tokens c0 .. c0 + kSpan - 1.
    __device__ void cover(int lane) {
        if (static_cast<int64_t>(q0) + kSpan > window_base + kWaveSize || static_cast<int64_t>(q0) < window_base) {
            load_window(q0, lane);
        }
    }
    /// Cache row (block * block size + position) of token c0 + k, or of c0
    /// itself when c0 + k is not below t_hi (such tokens are masked).
    __device__ int64_t row(int64_t c0, int k, int64_t t_hi) const {
        uint32_t blk = q0;
        uint32_t pos = r0;
        if (c0 + k < t_hi) {
            const uint32_t r = r0 + static_cast<uint32_t>(k);
            uint32_t dq;
            if (bs >= static_cast<uint32_t>(kSpan)) {
                dq = r >= bs ? 1u : 0u;
            } else {
                dq = static_cast<uint32_t>(static_cast<float>(r) * inv_bs);
                if ((dq + 1) * bs <= r) ++dq;
            }
            blk = q0 + dq;
            pos = r - dq * bs;
        }
        const int64_t block = static_cast<uint32_t>(__shfl(window, static_cast<int>(blk - window_base)));
        return block * block_size + pos;
    }
};

/// kLanes = D / kVals lanes per token (kVals = 16 bytes of T), kGroup query
/// heads per workgroup.
///
/// 16-bit caches are held to 128 VGPRs (4 waves per SIMD instead of 3; up
/// to 2 registers spill): at the usual grids (1024-2048 workgroups of 4
/// waves) every workgroup is then resident at once instead of leaving a
/// second partial round, and each wave's short token range no longer waits
/// on the previous round. Measured on bf16 D = 128: GQA group 4 41.5 ->
/// 50.0% and 38.8 -> 45.3% of HBM peak (64 x 1024 and 128 x 256 tokens),
/// group 1 unchanged. fp32 keeps the compiler's choice (4-6 waves).
template <typename T, int kLanes, int kGroup>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 ? 4 : 1, 8))) void paged_decode_kernel(PagedArgs a) {
    constexpr int kVals = vals_per_lane<T>();
    constexpr int kTokensPerStep = kWaveSize / kLanes;
    constexpr int kDim = kVals * kLanes;
    // Token steps whose loads are issued together (two buffers of them in
    // flight). Two rather than four for groups of one or two heads: the
    // staging registers then leave room for 4-6 waves per SIMD (fp32 GQA
    // group 2: 59 -> 74% of HBM peak; group 1 unchanged).
    constexpr int kStepsPerLoad = 2;
    constexpr int kChunk = kStepsPerLoad * kTokensPerStep;  // tokens per load batch
    __shared__ float lds_m[kWaves][kGroup];
    __shared__ float lds_l[kWaves][kGroup];
    __shared__ float lds_acc[kWaves][kGroup][kDim];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWaveSize - 1);
    const int wave = tid / kWaveSize;
    const int slot = lane / kLanes;   // token slot of this lane within a step
    const int piece = lane % kLanes;  // dimensions kVals piece .. kVals piece + kVals - 1

    // Workgroup -> (sequence, KV head, head group, split).
    int64_t id = blockIdx.x;
    const int split = static_cast<int>(id % a.splits);
    id /= a.splits;
    const int hgroup = static_cast<int>(id % a.head_groups);
    id /= a.head_groups;
    const int64_t kv_head = id % a.kv_heads;
    const int64_t seq = id / a.kv_heads;

    const int64_t group = a.heads / a.kv_heads;
    const int64_t head0 = kv_head * group + static_cast<int64_t>(hgroup) * kGroup;
    const int n_heads = static_cast<int>(group - static_cast<int64_t>(hgroup) * kGroup < kGroup
                                             ? group - static_cast<int64_t>(hgroup) * kGroup
                                             : kGroup);

    // fp32: q is widened and pre-scaled. bf16: q stays as packed pairs and
    // a score is four v_dot2_f32_bf16 on the raw K piece (products of bf16
    // values are exact in fp32, sums in fp32), scaled after the lane sum -
    // no widening of K, a quarter of the multiply instructions.
    constexpr bool kPacked = !std::is_same<T, float>::value;
    float q[kGroup][kPacked ? 1 : kVals];
    u32x4_t qp[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
        const int64_t head = head0 + (g < n_heads ? g : 0);  // in range even when unused
        const u32x4_t raw = load16(a.query, ((seq * a.heads + head) * kDim + kVals * piece) * sizeof(T));
        if constexpr (kPacked) {
            qp[g] = g < n_heads ? raw : u32x4_t{0u, 0u, 0u, 0u};
        } else {
            widen<T>(raw, q[g]);
#pragma unroll
            for (int e = 0; e < kVals; ++e) q[g][e] = g < n_heads ? q[g][e] * a.scale : 0.0f;
        }
    }

    HeadState<kVals> st[kGroup];
#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
        st[g].m = -INFINITY;
        st[g].l = 0.0f;
#pragma unroll
        for (int e = 0; e < kVals; ++e) st[g].acc[e] = 0.0f;
    }

    // Tokens of this split, then of this wave (a contiguous share in whole steps).
    const int64_t capacity = a.max_blocks * a.block_size;  // never read past the table
    const int64_t stored = a.context[seq] > 0 ? a.context[seq] : 0;
    const int64_t context = stored < capacity ? stored : capacity;
    const int64_t t_lo = static_cast<int64_t>(split) * a.split_tokens;
    const int64_t t_hi = context < t_lo + a.split_tokens ? context : t_lo + a.split_tokens;
    const int64_t count = t_hi > t_lo ? t_hi - t_lo : 0;
    const int64_t steps_total = (count + kTokensPerStep - 1) / kTokensPerStep;
    const int64_t steps_per_wave = (steps_total + kWaves - 1) / kWaves;
    const int64_t w_lo = t_lo + static_cast<int64_t>(wave) * steps_per_wave * kTokensPerStep;
    const int64_t w_hi_raw = w_lo + steps_per_wave * kTokensPerStep;
    const int64_t w_hi = w_hi_raw < t_hi ? w_hi_raw : t_hi;
    const int64_t row_bytes = a.kv_heads * kDim * static_cast<int64_t>(sizeof(T));
    const int64_t piece_bytes = (kv_head * kDim + kVals * piece) * static_cast<int64_t>(sizeof(T));
    const uint32_t* table = a.tables + seq * a.max_blocks;

    // A window of 64 block-table entries, one per lane, so the K/V addresses
    // of a chunk need a lane shuffle rather than a dependent memory load.
    // Token positions are below 2^31 (int32 context lengths): 32-bit
    // quotients are exact, with the block size saturated to 32 bits.
    const uint32_t bs32 = a.block_size < int64_t{0xFFFFFFFF} ? static_cast<uint32_t>(a.block_size) : 0xFFFFFFFFu;
    int64_t window_base = static_cast<uint32_t>(w_lo) / bs32;
    auto load_window = [&](int64_t base) {
        const int64_t entry = base + lane < a.max_blocks ? base + lane : a.max_blocks - 1;
        return static_cast<int>(table[entry]);
    };
    int window = w_lo < w_hi ? load_window(window_base) : 0;

    auto fetch = [&](int64_t t0, u32x4_t (&raw)[kStepsPerLoad][2]) {
        // Uniform decisions: every lane sees the same chunk. A chunk spanning
        // more blocks than the window holds (tiny blocks) reads the table
        // directly.
        const int64_t first_block = static_cast<uint32_t>(t0) / bs32;
        const int64_t last_block = static_cast<uint32_t>(t0 + kChunk - 1 < w_hi - 1 ? t0 + kChunk - 1 : w_hi - 1) / bs32;
        const bool windowed = last_block - first_block < kWaveSize;
        if (windowed && last_block - window_base >= kWaveSize) {
            window_base = first_block;
            window = load_window(window_base);
        }
#pragma unroll
        for (int u = 0; u < kStepsPerLoad; ++u) {
            const int64_t t = t0 + u * kTokensPerStep + slot;
            const int64_t tc = t < w_hi ? t : w_hi - 1;  // a valid token even past the end
            const uint32_t bq = static_cast<uint32_t>(tc) / bs32;
            const uint32_t br = static_cast<uint32_t>(tc) - bq * bs32;
            const int64_t block =
                windowed ? static_cast<uint32_t>(__shfl(window, static_cast<int>(bq - window_base)))
                         : table[bq];
            const int64_t offset = (block * a.block_size + br) * row_bytes + piece_bytes;
            raw[u][0] = load16_kv<T>(a.k_cache, offset);
            raw[u][1] = load16_kv<T>(a.v_cache, offset);
        }
    };

    // Scores of a chunk first, then one rescale per head per chunk.
    auto consume = [&](int64_t t0, const u32x4_t (&raw)[kStepsPerLoad][2]) {
        float score[kGroup][kStepsPerLoad];
#pragma unroll
        for (int u = 0; u < kStepsPerLoad; ++u) {
            float k[kPacked ? 1 : kVals];
            if constexpr (!kPacked) widen<T>(raw[u][0], k);
            const bool valid = t0 + u * kTokensPerStep + slot < w_hi;
#pragma unroll
            for (int g = 0; g < kGroup; ++g) {
                float part;
                if constexpr (kPacked) {
                    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
                    part = 0.0f;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // Through plain words: a bit_cast of a vector element
                        // subscript read element 0 for every e.
                        const uint32_t qw = qp[g][e];
                        const uint32_t kw = raw[u][0][e];
                        part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, qw),
                                                              __builtin_bit_cast(bf16x2_v, kw), part, false);
                    }
                    part = lanes_sum<kLanes>(part) * a.scale;
                } else {
                    part = q[g][0] * k[0];
#pragma unroll
                    for (int e = 1; e < kVals; ++e) part = fmaf(q[g][e], k[e], part);
                    part = lanes_sum<kLanes>(part);
                }
                score[g][u] = valid ? part : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            float m = st[g].m;
#pragma unroll
            for (int u = 0; u < kStepsPerLoad; ++u) m = fmaxf(m, score[g][u]);
            if (m == -INFINITY) continue;  // nothing valid for this slot yet
            const float c = __expf(st[g].m - m);  // 0 when the state was empty
            st[g].l *= c;
#pragma unroll
            for (int e = 0; e < kVals; ++e) st[g].acc[e] *= c;
            st[g].m = m;
        }
#pragma unroll
        for (int u = 0; u < kStepsPerLoad; ++u) {
            float v[kVals];
            widen<T>(raw[u][1], v);
#pragma unroll
            for (int g = 0; g < kGroup; ++g) {
                const float p = score[g][u] == -INFINITY ? 0.0f : __expf(score[g][u] - st[g].m);
                st[g].l += p;
#pragma unroll
                for (int e = 0; e < kVals; ++e) st[g].acc[e] = fmaf(p, v[e], st[g].acc[e]);
            }
        }
    };

    // Loads of the next chunk are in flight while this one is consumed.
    u32x4_t buf_a[kStepsPerLoad][2];
    u32x4_t buf_b[kStepsPerLoad][2];
    int64_t t0 = w_lo;
    if (t0 < w_hi) fetch(t0, buf_a);
    while (t0 < w_hi) {
        const int64_t t1 = t0 + kChunk;
        if (t1 < w_hi) fetch(t1, buf_b);
        consume(t0, buf_a);
        if (t1 >= w_hi) break;
        const int64_t t2 = t1 + kChunk;
        if (t2 < w_hi) fetch(t2, buf_a);
        consume(t1, buf_b);
        t0 = t2;
    }

    // Merge the token slots of the wave (lanes piece, piece + kLanes, ...).
#pragma unroll
    for (int mask = kLanes; mask < kWaveSize; mask <<= 1) {
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            const float m2 = __shfl_xor(st[g].m, mask);
            const float l2 = __shfl_xor(st[g].l, mask);
            float acc2[kVals];
#pragma unroll
            for (int e = 0; e < kVals; ++e) acc2[e] = __shfl_xor(st[g].acc[e], mask);
            merge_into(st[g], m2, l2, acc2);
        }
    }
    if (slot == 0) {
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            if (piece == 0) {
                lds_m[wave][g] = st[g].m;
                lds_l[wave][g] = st[g].l;
            }
#pragma unroll
            for (int e = 0; e < kVals; ++e) lds_acc[wave][g][kVals * piece + e] = st[g].acc[e];
        }
    }
    __syncthreads();
    if (wave != 0 || slot != 0) return;

#pragma unroll
    for (int g = 0; g < kGroup; ++g) {
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            float acc2[kVals];
#pragma unroll
            for (int e = 0; e < kVals; ++e) acc2[e] = lds_acc[w][g][kVals * piece + e];
            merge_into(st[g], lds_m[w][g], lds_l[w][g], acc2);
        }
        if (g >= n_heads) continue;
        const int64_t head = head0 + g;
        if (a.splits == 1) {
            float o[kVals];
            const float inv = st[g].l > 0.0f ? 1.0f / st[g].l : 0.0f;
#pragma unroll
            for (int e = 0; e < kVals; ++e) o[e] = st[g].acc[e] * inv;
            store_piece<T>(static_cast<T*>(a.out), (seq * a.heads + head) * kDim + kVals * piece, o);
        } else {
            float* part = a.partial + ((seq * a.heads + head) * a.splits + split) * (kDim + 2);
            if (piece == 0) {
                part[0] = st[g].m;
                part[1] = st[g].l;
            }
#pragma unroll
            for (int e = 0; e < kVals; ++e) part[2 + kVals * piece + e] = st[g].acc[e];
        }
    }
}

/// Combines the splits of one (sequence, head): one wave, lanes over D.
template <typename T>
__global__ __launch_bounds__(kWaveSize) void paged_combine_kernel(PagedArgs a) {
    const int64_t row = blockIdx.x;  // seq * heads + head
    const int64_t dim = a.head_dim;
    const float* part = a.partial + row * a.splits * (dim + 2);
    float m = -INFINITY;
    for (int j = 0; j < a.splits; ++j) m = fmaxf(m, part[j * (dim + 2)]);
    T* out = static_cast<T*>(a.out) + row * dim;
    for (int64_t d = threadIdx.x; d < dim; d += kWaveSize) {
        float num = 0.0f;
        float den = 0.0f;
        for (int j = 0; j < a.splits; ++j) {
            const float* pj = part + j * (dim + 2);
            const float c = pj[0] == -INFINITY ? 0.0f : __expf(pj[0] - m);
            den = fmaf(pj[1], c, den);
            num = fmaf(pj[2 + d], c, num);
        }
        const float v = den > 0.0f ? num / den : 0.0f;
        if constexpr (std::is_same<T, float>::value) {
            out[d] = v;
        } else {
            out[d] = static_cast<uint16_t>(f32_to_bf16_bits(v));
        }
    }
}

/// Any head size up to 1024: one wave per (sequence, head), lanes over the
/// head dimension (kPer values each), one token per step.
template <typename T, int kPer>
__global__ __launch_bounds__(kWaveSize) void paged_decode_wide_kernel(PagedArgs a) {
    const int lane = static_cast<int>(threadIdx.x);
    const int64_t row = blockIdx.x;  // seq * heads + head
    const int64_t seq = row / a.heads;
    const int64_t head = row % a.heads;
    const int64_t kv_head = head / (a.heads / a.kv_heads);
    const int64_t dim = a.head_dim;
    const T* query = static_cast<const T*>(a.query);
    const T* k_cache = static_cast<const T*>(a.k_cache);
    const T* v_cache = static_cast<const T*>(a.v_cache);

    auto read = [](const T* p, int64_t i) -> float {
        if constexpr (std::is_same<T, float>::value) {
            return p[i];
        } else {
            return __uint_as_float(static_cast<uint32_t>(p[i]) << 16);
        }
    };
    float q[kPer];
    float acc[kPer];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int64_t d = lane + kWaveSize * r;
        q[r] = d < dim ? read(query, row * dim + d) * a.scale : 0.0f;
        acc[r] = 0.0f;
    }
    float m = -INFINITY;
    float l = 0.0f;
    const int64_t capacity = a.max_blocks * a.block_size;
    const int64_t stored = a.context[seq] > 0 ? a.context[seq] : 0;
    const int64_t context = stored < capacity ? stored : capacity;
    const uint32_t* table = a.tables + seq * a.max_blocks;
    for (int64_t t = 0; t < context; ++t) {
        const int64_t block = table[t / a.block_size];
        const int64_t base = ((block * a.block_size + t % a.block_size) * a.kv_heads + kv_head) * dim;
        float part = 0.0f;
        float v[kPer];
#pragma unroll
        for (int r = 0; r < kPer; ++r) {
            const int64_t d = lane + kWaveSize * r;
            const bool in = d < dim;
            part = fmaf(q[r], in ? read(k_cache, base + d) : 0.0f, part);
            v[r] = in ? read(v_cache, base + d) : 0.0f;
        }
        const float score = wave_reduce_f32<AddF32>(part);
        const float mn = fmaxf(m, score);
        const float c = __expf(m - mn);
        const float p = __expf(score - mn);
        l = l * c + p;
#pragma unroll
        for (int r = 0; r < kPer; ++r) acc[r] = fmaf(p, v[r], acc[r] * c);
        m = mn;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int64_t d = lane + kWaveSize * r;
        if (d >= dim) continue;
        const float o = acc[r] * inv;
        if constexpr (std::is_same<T, float>::value) {
            static_cast<float*>(a.out)[row * dim + d] = o;
        } else {
            static_cast<uint16_t*>(a.out)[row * dim + d] = static_cast<uint16_t>(f32_to_bf16_bits(o));
        }
    }
}

/// 16-bit caches on the matrix cores: one workgroup (4 waves) per (sequence,
/// KV head, context split) serves every query head of the GQA group (up to
/// kMfmaHeads). Each wave takes chunks of 16 tokens (chunks wave, wave + 4,
/// ... of the split) and, per chunk, computes
///   S^T [16 tokens x 16 heads] = K [16 x D] Q^T [D x 16]
/// with D / 32 v_mfma_f32_16x16x32_bf16: the A fragments are the tokens' K
/// rows straight from memory (lane j % 16 = token, 16 bytes of dims), Q^T
/// stays in registers, and lane (g = lane / 16, j = lane % 16) receives the
/// scores of tokens 4 g .. 4 g + 3 for head j. After the online-softmax
/// update of head j (one cross-lane max per chunk),
///   O^T [D x 16 heads] += V^T [D x 16 tokens] P^T [16 tokens x 16 heads]
/// with D / 16 v_mfma_f32_16x16x16_bf16: the B operand is the lane's own four
/// probabilities as bf16 (exactly the score layout), the A operand is V^T
/// read transposed (ds_read_b64_tr_b16) out of a per-wave LDS copy of the
/// chunk's V rows. The next chunk's K and V loads are in flight while a chunk
/// is computed. The waves' states merge through LDS at the end. Four waves
/// serve one (sequence, KV head, split), or two when a one-round grid allows
/// (two per workgroup, half the workgroups, each wave twice the tokens).
constexpr int kMfmaHeads = 16;
constexpr int kMfmaChunk = 16;

typedef __bf16 bf16x8_m __attribute__((ext_vector_type(8)));
typedef short s16x4_m __attribute__((ext_vector_type(4)));
typedef float f32x4_m __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_m lds_s16x4_m;
typedef __attribute__((address_space(3))) uint8_t lds_u8_m;

template <int kD, int kSubs, int kPW>
__global__ __launch_bounds__(kThreads) void paged_mfma_kernel(PagedArgs a) {
    // kSubs 16-token sub-chunks per step (one or two): two keep twice the
    // bytes in flight per wave. kPW waves (4 or 2) serve one (sequence, KV
    // head, split); a workgroup holds kWaves / kPW of them.
    constexpr int kTok = kMfmaChunk * kSubs;                // tokens per step
    constexpr int kS = kD / 32;                             // score MFMAs per sub-chunk
    constexpr int kB = kD / 16;                             // P.V output blocks
    constexpr int kRowBytes = kD * 2;                       // one token's K or V row
    constexpr int kPiecesPerRow = kRowBytes / 16;
    constexpr int kVPieces = kTok * kPiecesPerRow / kWaveSize;  // V 16-byte pieces per lane
    constexpr int kVBytes = kTok * kRowBytes;               // one wave's V buffer
    static_assert(kD % 32 == 0 && kD <= 256 && kVPieces >= 1 && (kSubs == 1 || kSubs == 2), "shape");
    // Two V buffers per wave; after the loop the same bytes hold the waves'
    // output accumulators for the merge ([wave][head][dim] fp32).
    constexpr int kLdsBytes = kWaves * 2 * kVBytes;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    static_assert(kLdsBytes >= kWaves * kMfmaHeads * kD * 4, "merge area");
    __shared__ float lds_m[kWaves][kMfmaHeads];
    __shared__ float lds_l[kWaves][kMfmaHeads];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWaveSize - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize);  // uniform: scalar wave-level state
    const int g = lane >> 4;
    const int j = lane & 15;

    const int sub = wave / kPW;  // this wave's (sequence, KV head, split) in the workgroup
    const int wv = wave % kPW;   // and its place among the kPW waves serving it
    int64_t id = static_cast<int64_t>(blockIdx.x) * (kWaves / kPW) + sub;
    const int split = static_cast<int>(id % a.splits);
    id /= a.splits;
    const int64_t kv_head = id % a.kv_heads;
    const int64_t seq = id / a.kv_heads;
    const int64_t group = a.heads / a.kv_heads;  // <= kMfmaHeads (checked on the host)
    const int64_t head0 = kv_head * group;

    // Q^T fragments: lane holds q[head j][dims 32 s + 8 g .. +7]; heads past
    // the group are zero (their scores are never used).
    bf16x8_m qfrag[kS];
#pragma unroll
    for (int s = 0; s < kS; ++s) {
        u32x4_t raw = {0u, 0u, 0u, 0u};
        if (j < group) raw = load16(a.query, ((seq * a.heads + head0 + j) * kD + 32 * s + 8 * g) * 2);
        qfrag[s] = __builtin_bit_cast(bf16x8_m, raw);
    }

    const int64_t capacity = a.max_blocks * a.block_size;
    const int64_t stored = a.context[seq] > 0 ? a.context[seq] : 0;
    const int64_t context = stored < capacity ? stored : capacity;
    const int64_t t_lo = static_cast<int64_t>(split) * a.split_tokens;
    const int64_t t_hi = context < t_lo + a.split_tokens ? context : t_lo + a.split_tokens;
    const int64_t row_stride = a.kv_heads * kRowBytes;
    const int64_t head_bytes = kv_head * kRowBytes;
    const uint32_t* table = a.tables + seq * a.max_blocks;

    // Lane (g, j) loads the K and V rows of token 16 u + j of each sub-chunk:
    // K dims 32 s + 8 g .. +7, V 16-byte pieces 4 i + g.
    TokenCursor<kTok> cur;
    bf16x8_m kfrag[kSubs][kS];
    u32x4_t vraw[kVPieces];
    auto fetch = [&](int64_t c0) {
        cur.cover(lane);
#pragma unroll
        for (int u = 0; u < kSubs; ++u) {
            const int64_t off = cur.row(c0, kMfmaChunk * u + j, t_hi) * row_stride + head_bytes;
#pragma unroll
            for (int s = 0; s < kS; ++s) {
                kfrag[u][s] = __builtin_bit_cast(bf16x8_m, load16_kv<uint16_t>(a.k_cache, off + (32 * s + 8 * g) * 2));
            }
#pragma unroll
            for (int i = 0; i < kPiecesPerRow / 4; ++i) {
                vraw[u * (kPiecesPerRow / 4) + i] = load16_kv<uint16_t>(a.v_cache, off + (4 * i + g) * 16);
            }
        }
    };
    // Physical 16-byte piece of piece pc of V row rw in a wave's buffer:
    // rotated by the row, so the 16 rows one store instruction writes fall in
    // different banks.
    auto v_piece = [](int rw, int pc) { return (pc + (rw & 15)) % kPiecesPerRow; };
    auto stage_v = [&](int buf) {
        uint8_t* base = lds + (wave * 2 + buf) * kVBytes;
#pragma unroll
        for (int u = 0; u < kSubs; ++u) {
            const int rw = kMfmaChunk * u + j;
#pragma unroll
            for (int i = 0; i < kPiecesPerRow / 4; ++i) {
                *reinterpret_cast<u32x4_t*>(base + rw * kRowBytes + v_piece(rw, 4 * i + g) * 16) =
                    vraw[u * (kPiecesPerRow / 4) + i];
            }
        }
    };

    float m = -INFINITY;   // running max of head j (the same in all four lane groups)
    float l = 0.0f;        // this lane's share of head j's running sum (tokens 4 g .. 4 g + 3)
    f32x4_m acc[kB];       // O^T[dim 16 b + 4 g + t][head j]
#pragma unroll
    for (int b = 0; b < kB; ++b) acc[b] = f32x4_m{0.0f, 0.0f, 0.0f, 0.0f};

    const int64_t first = t_lo + static_cast<int64_t>(wv) * kTok;
    constexpr int64_t kStride = static_cast<int64_t>(kPW) * kTok;
    int buf = 0;
    if (first < t_hi) {
        cur.start(table, a.max_blocks, a.block_size, first, kStride, lane);
        fetch(first);
        stage_v(0);
    }
    for (int64_t c0 = first; c0 < t_hi; c0 += kStride) {
        // The scores take this step's K fragments before the next step's
        // loads reuse their registers.
        f32x4_m sc[kSubs];
#pragma unroll
        for (int u = 0; u < kSubs; ++u) {
            sc[u] = f32x4_m{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < kS; ++s) sc[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kfrag[u][s], qfrag[s], sc[u], 0, 0, 0);
        }
        const int64_t next = c0 + kStride;
        cur.advance();
        if (next < t_hi) fetch(next);

        float cmax = -INFINITY;
#pragma unroll
        for (int u = 0; u < kSubs; ++u) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                sc[u][t] = c0 + kMfmaChunk * u + 4 * g + t < t_hi ? sc[u][t] * a.scale : -INFINITY;
                cmax = fmaxf(cmax, sc[u][t]);
            }
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        // Every step holds at least one valid token, so cmax is finite.
        const float m_new = fmaxf(m, cmax);
        const float c = m == -INFINITY ? 0.0f : __expf(m - m_new);
        m = m_new;
        // Probabilities rounded to bf16 two at a time (v_cvt_pk_bf16_f32; a
        // NaN keeps its payload here and the output rounding canonicalises
        // it).
        s16x4_m pb[kSubs];
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < kSubs; ++u) {
            float pt[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                pt[t] = sc[u][t] == -INFINITY ? 0.0f : __expf(sc[u][t] - m_new);
                psum += pt[t];
            }
            pb[u] = __builtin_bit_cast(s16x4_m, make_uint2(f32x2_to_bf16x2_bits(pt[0], pt[1]),
                                                           f32x2_to_bf16x2_bits(pt[2], pt[3])));
        }
        l = l * c + psum;
#pragma unroll
        for (int b = 0; b < kB; ++b) acc[b] *= c;

        // V^T fragments: lane (g, j) reads 8 bytes of token row 4 g + j / 4 (of
        // each sub-chunk) at dims 16 b + 4 (j % 4) .. +3 and receives
        // V[tokens 4 g .. 4 g + 3][dim 16 b + j]. With two sub-chunks the MFMA's
        // k index 8 g + t is token 4 g + t % 4 of sub-chunk t / 4, in both the
        // V^T and the P^T operand. This wave's own writes of the buffer must
        // have landed.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
        asm volatile("" ::: "memory");
        const uint8_t* vb = lds + (wave * 2 + buf) * kVBytes;
#pragma unroll
        for (int b = 0; b < kB; ++b) {
            const int rw = 4 * g + (j >> 2);
            const int off = rw * kRowBytes + v_piece(rw, 2 * b + ((j & 3) >> 1)) * 16 + (j & 1) * 8;
            const s16x4_m v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4_m*)((lds_u8_m*)(const_cast<uint8_t*>(vb)) + off));
            if constexpr (kSubs == 1) {
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v0, pb[0], acc[b], 0, 0, 0);
            } else {
                // Row rw + 16 has the rotation of row rw.
                const s16x4_m v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4_m*)((lds_u8_m*)(const_cast<uint8_t*>(vb)) + off + kMfmaChunk * kRowBytes));
                const bf16x8_m vv = __builtin_bit_cast(bf16x8_m, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
                const bf16x8_m pp =
                    __builtin_bit_cast(bf16x8_m, __builtin_shufflevector(pb[0], pb[1], 0, 1, 2, 3, 4, 5, 6, 7));
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, pp, acc[b], 0, 0, 0);
            }
        }
        if (next < t_hi) {
            buf ^= 1;
            stage_v(buf);
        }
    }

    // Head j's sum over the wave's tokens: add the four lane groups.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    __syncthreads();  // every wave is done with its V buffers
    float* macc = reinterpret_cast<float*>(lds);  // [wave][head][dim]
#pragma unroll
    for (int b = 0; b < kB; ++b) {
#pragma unroll
        for (int t = 0; t < 4; ++t) macc[(wave * kMfmaHeads + j) * kD + 16 * b + 4 * g + t] = acc[b][t];
    }
    if (g == 0) {
        lds_m[wave][j] = m;
        lds_l[wave][j] = l;
    }
    __syncthreads();

    // Merge the kPW waves w0 .. w0 + kPW - 1: their threads take (head, dim)
    // pairs in turn.
    const int w0 = sub * kPW;
    for (int pair = tid % (kPW * kWaveSize); pair < kMfmaHeads * kD; pair += kPW * kWaveSize) {
        const int h = pair / kD;
        const int d = pair % kD;
        if (h >= group) continue;
        float mm = -INFINITY;
#pragma unroll
        for (int w = w0; w < w0 + kPW; ++w) mm = fmaxf(mm, lds_m[w][h]);
        float ll = 0.0f;
        float oo = 0.0f;
#pragma unroll
        for (int w = w0; w < w0 + kPW; ++w) {
            const float cw = lds_m[w][h] == -INFINITY ? 0.0f : __expf(lds_m[w][h] - mm);
            ll = fmaf(lds_l[w][h], cw, ll);
            oo = fmaf(macc[(w * kMfmaHeads + h) * kD + d], cw, oo);
        }
        const int64_t head = head0 + h;
        if (a.splits == 1) {
            const float v = ll > 0.0f ? oo / ll : 0.0f;
            static_cast<uint16_t*>(a.out)[(seq * a.heads + head) * kD + d] = static_cast<uint16_t>(f32_to_bf16_bits(v));
        } else {
            float* part = a.partial + ((seq * a.heads + head) * a.splits + split) * (kD + 2);
            if (d == 0) {
                part[0] = mm;
                part[1] = ll;
            }
            part[2 + d] = oo;
        }
    }
}

/// fp32 caches on the matrix cores (v_mfma_f32_16x16x4_f32: fp32 products,
/// fp32 sums, the accuracy of the streaming kernel). Same organisation as
/// paged_mfma_kernel (workgroup per sequence, KV head and split; 16-token
/// chunks per wave; waves merged through LDS), with these operand layouts:
///   scores, step 4 u + e (u < D / 16, e < 4): A = K[token j][dim 16 u + 4 g + e]
///     (lane (g, j) holds dims 16 u + 4 g .. +3 from one 16-byte load), B =
///     Q[head j][the same dim] (registers), so MFMA slot g of every step pairs
///     one dim of K with the same dim of Q; lane (g, j) receives the scores of
///     tokens 4 g .. 4 g + 3 for head j;
///   P.V, step c < 4 of output block b: slot g stands for token 4 g + c, so the
///     B operand is the lane's own probability p[c] and the A operand is
///     V[token 4 g + c][dim 16 b + j], one ds_read_b32 from a per-wave LDS copy
///     of the chunk's V rows (rows padded by 16 bytes, so rows 4 apart start
///     64 bytes apart in the banks and the four lane groups of a read use
///     different banks).
template <int kD>
__global__ __launch_bounds__(kThreads) void paged_mfma_f32_kernel(PagedArgs a) {
    constexpr int kU = kD / 16;                             // 16-dim blocks
    constexpr int kRowBytes = kD * 4;
    constexpr int kLdsRow = kRowBytes + 16;                 // padded V row in LDS
    constexpr int kPiecesPerRow = kRowBytes / 16;
    constexpr int kVPieces = kMfmaChunk * kPiecesPerRow / kWaveSize;
    constexpr int kVBytes = kMfmaChunk * kLdsRow;           // one wave's V buffer
    static_assert(kD % 16 == 0 && kD <= 128 && kVPieces >= 1, "head size");
    constexpr int kLdsBytes = kWaves * 2 * kVBytes;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
    static_assert(kLdsBytes >= kWaves * kMfmaHeads * kD * 4, "merge area");
    __shared__ float lds_m[kWaves][kMfmaHeads];
    __shared__ float lds_l[kWaves][kMfmaHeads];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWaveSize - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWaveSize);  // uniform: scalar wave-level state
    const int g = lane >> 4;
    const int j = lane & 15;

    int64_t id = blockIdx.x;
    const int split = static_cast<int>(id % a.splits);
    id /= a.splits;
    const int64_t kv_head = id % a.kv_heads;
    const int64_t seq = id / a.kv_heads;
    const int64_t group = a.heads / a.kv_heads;  // <= kMfmaHeads (checked on the host)
    const int64_t head0 = kv_head * group;

    // q[head j][dims 16 u + 4 g .. +3], pre-scaled; heads past the group are zero.
    f32x4_m qv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        u32x4_t raw = {0u, 0u, 0u, 0u};
        if (j < group) raw = load16(a.query, ((seq * a.heads + head0 + j) * kD + 16 * u + 4 * g) * 4);
        qv[u] = f32x4_m{__uint_as_float(raw[0]), __uint_as_float(raw[1]), __uint_as_float(raw[2]),
                        __uint_as_float(raw[3])} * a.scale;
    }

    const int64_t capacity = a.max_blocks * a.block_size;
    const int64_t stored = a.context[seq] > 0 ? a.context[seq] : 0;
    const int64_t context = stored < capacity ? stored : capacity;
    const int64_t t_lo = static_cast<int64_t>(split) * a.split_tokens;
    const int64_t t_hi = context < t_lo + a.split_tokens ? context : t_lo + a.split_tokens;
    const int64_t row_stride = a.kv_heads * kRowBytes;
    const int64_t head_bytes = kv_head * kRowBytes;
    const uint32_t* table = a.tables + seq * a.max_blocks;

    // Lane (g, j) loads the K and V rows of token j: K dims 16 u + 4 g .. +3,
    // V 16-byte pieces 4 i + g.
    TokenCursor<kMfmaChunk> cur;
    u32x4_t kraw[kU];
    u32x4_t vraw[kVPieces];
    auto fetch = [&](int64_t c0) {
        cur.cover(lane);
        const int64_t off = cur.row(c0, j, t_hi) * row_stride + head_bytes;
#pragma unroll
        for (int u = 0; u < kU; ++u) kraw[u] = load16_kv<float>(a.k_cache, off + (16 * u + 4 * g) * 4);
#pragma unroll
        for (int i = 0; i < kVPieces; ++i) vraw[i] = load16_kv<float>(a.v_cache, off + (4 * i + g) * 16);
    };
    auto stage_v = [&](int buf) {
        uint8_t* base = lds + (wave * 2 + buf) * kVBytes;
#pragma unroll
        for (int i = 0; i < kVPieces; ++i) {
            *reinterpret_cast<u32x4_t*>(base + j * kLdsRow + (4 * i + g) * 16) = vraw[i];
        }
    };

    float m = -INFINITY;
    float l = 0.0f;
    f32x4_m acc[kU];  // O^T[dim 16 b + 4 g + t][head j]
#pragma unroll
    for (int b = 0; b < kU; ++b) acc[b] = f32x4_m{0.0f, 0.0f, 0.0f, 0.0f};

    const int64_t first = t_lo + static_cast<int64_t>(wave) * kMfmaChunk;
    constexpr int64_t kStride = static_cast<int64_t>(kWaves) * kMfmaChunk;
    int buf = 0;
    if (first < t_hi) {
        cur.start(table, a.max_blocks, a.block_size, first, kStride, lane);
        fetch(first);
        stage_v(0);
    }
    for (int64_t c0 = first; c0 < t_hi; c0 += kStride) {
        // The scores take this step's K before the next step's loads reuse
        // its registers.
        f32x4_m sc = f32x4_m{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < kU; ++u) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kraw[u][e]), qv[u][e], sc, 0, 0, 0);
            }
        }
        const int64_t next = c0 + kStride;
        cur.advance();
        if (next < t_hi) fetch(next);

        float cmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sc[t] = c0 + 4 * g + t < t_hi ? sc[t] : -INFINITY;
            cmax = fmaxf(cmax, sc[t]);
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m, cmax);  // finite: every chunk has a valid token
        const float c = m == -INFINITY ? 0.0f : __expf(m - m_new);
        m = m_new;
        float p[4];
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            p[t] = sc[t] == -INFINITY ? 0.0f : __expf(sc[t] - m_new);
            psum += p[t];
        }
        l = l * c + psum;
#pragma unroll
        for (int b = 0; b < kU; ++b) acc[b] *= c;

        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
        asm volatile("" ::: "memory");
        const uint8_t* vb = lds + (wave * 2 + buf) * kVBytes;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            const float* vrow = reinterpret_cast<const float*>(vb + (4 * g + cc) * kLdsRow);
#pragma unroll
            for (int b = 0; b < kU; ++b) {
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * b + j], p[cc], acc[b], 0, 0, 0);
            }
        }
        if (next < t_hi) {
            buf ^= 1;
            stage_v(buf);
        }
    }

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);

    __syncthreads();
    float* macc = reinterpret_cast<float*>(lds);  // [wave][head][dim]
#pragma unroll
    for (int b = 0; b < kU; ++b) {
#pragma unroll
        for (int t = 0; t < 4; ++t) macc[(wave * kMfmaHeads + j) * kD + 16 * b + 4 * g + t] = acc[b][t];
    }
    if (g == 0) {
        lds_m[wave][j] = m;
        lds_l[wave][j] = l;
    }
    __syncthreads();

    for (int pair = tid; pair < kMfmaHeads * kD; pair += kThreads) {
        const int h = pair / kD;
        const int d = pair % kD;
        if (h >= group) continue;
        float mm = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, lds_m[w][h]);
        float ll = 0.0f;
        float oo = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float cw = lds_m[w][h] == -INFINITY ? 0.0f : __expf(lds_m[w][h] - mm);
            ll = fmaf(lds_l[w][h], cw, ll);
            oo = fmaf(macc[(w * kMfmaHeads + h) * kD + d], cw, oo);
        }
        const int64_t head = head0 + h;
        if (a.splits == 1) {
            static_cast<float*>(a.out)[(seq * a.heads + head) * kD + d] = ll > 0.0f ? oo / ll : 0.0f;
        } else {
            float* part = a.partial + ((seq * a.heads + head) * a.splits + split) * (kD + 2);
            if (d == 0) {
                part[0] = mm;
                part[1] = ll;
            }
            part[2 + d] = oo;
        }
    }
}

/// Lanes per token for the streaming kernel (16 bytes per lane), or 0 when D
/// needs the wide one.
int lanes_for(int64_t head_dim, int64_t elem_bytes) {
    const int64_t per_lane = 16 / elem_bytes;
    if (head_dim % per_lane != 0) return 0;
    const int64_t lanes = head_dim / per_lane;
    if (lanes < 1 || lanes > kWaveSize || (lanes & (lanes - 1)) != 0) return 0;
    return static_cast<int>(lanes);
}

int group_size_for(int64_t group) {
    int gs = 1;
    while (gs < group && gs < kMaxGroup) gs *= 2;
    return gs;
}

struct Plan {
    int lanes;
    int gs;
    int head_groups;
    int splits;
    int64_t split_tokens;
};

/// Plan.lanes values that select paged_mfma_kernel (16-bit caches) and
/// paged_mfma_f32_kernel (fp32 caches).
constexpr int kMfmaPlan = -1;
constexpr int kMfmaF32Plan = -2;

Plan plan_for(int64_t sequences, int64_t heads, int64_t kv_heads, int64_t head_dim,
              int64_t block_size, int64_t max_blocks, int64_t elem_bytes, bool may_split) {
    Plan p{};
    p.lanes = lanes_for(head_dim, elem_bytes);
    const int64_t group = heads / kv_heads;
    p.gs = group_size_for(group);
    p.head_groups = static_cast<int>((group + p.gs - 1) / p.gs);
    // The matrix-core kernel for 16-bit caches with up to 16 query heads per
    // KV head, except groups of 2, where the streaming kernel is faster (bf16
    // D = 128, 64 x 1024 tokens: 69.0% of HBM peak against 66.8%). MHA 51.6
    // -> 56.3%, group 4 47.3 -> 61.3%, group 8 29.8 -> 60.7%.
    if (elem_bytes == 2 && head_dim % 32 == 0 && head_dim <= 256 && group != 2 && group <= kMfmaHeads) {
        p.lanes = kMfmaPlan;
        p.gs = kMfmaHeads;
        p.head_groups = 1;
    }
    // fp32 caches on the matrix cores where that is faster (fp32 D = 128):
    // groups of 8 or more (64 x 1024 tokens, 8 KV heads: 35.9 -> 64.6% of HBM
    // peak), and groups of 4 when one round of two workgroups per CU holds
    // every (sequence, KV head) (64 x 1024: 60.6 -> 65.1%; with 128 x 256,
    // two rounds: 59.8 -> 51.6%, so not). MHA (64.4 against 60.2%) and
    // groups of 2 (75.3 against 70.9%) stay on the streaming kernel.
    const bool one_round = sequences * kv_heads <= 2 * static_cast<int64_t>(cu_count());
    if (elem_bytes == 4 && head_dim % 16 == 0 && head_dim <= 128 && group <= kMfmaHeads &&
        (group >= 8 || (group >= 4 && one_round))) {
        p.lanes = kMfmaF32Plan;
        p.gs = kMfmaHeads;
        p.head_groups = 1;
    }
    const int64_t max_context = max_blocks * block_size;
    p.splits = 1;
    p.split_tokens = max_context > 0 ? max_context : 1;
    if (p.lanes == 0 || !may_split) return p;
    const int64_t base = sequences * kv_heads * p.head_groups;
    // The matrix-core kernel's workgroups take 33-66 KiB of LDS, two per CU:
    // split only as far as one round of them fills the GPU.
    const int64_t target =
        p.lanes == kMfmaPlan || p.lanes == kMfmaF32Plan ? 2 * static_cast<int64_t>(cu_count()) : kTargetWorkgroups;
    int64_t splits = (target + base - 1) / base;
    const int64_t by_length = (max_context + kMinSplitTokens - 1) / kMinSplitTokens;
    if (splits > by_length) splits = by_length;
    if (splits < 1) splits = 1;
    if (splits > 64) splits = 64;
    p.splits = static_cast<int>(splits);
    p.split_tokens = (max_context + splits - 1) / splits;
    return p;
}

size_t partial_bytes(const Plan& p, int64_t sequences, int64_t heads, int64_t head_dim) {
    if (p.splits <= 1) return 0;
    return static_cast<size_t>(sequences) * static_cast<size_t>(heads) * static_cast<size_t>(p.splits) *
           static_cast<size_t>(head_dim + 2) * sizeof(float);
}

template <typename T, int kLanes>
void launch_streaming(const PagedArgs& args, int gs, int64_t workgroups, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(workgroups));
    switch (gs) {
        case 1: launch(paged_decode_kernel<T, kLanes, 1>, dim3(grid), dim3(kThreads), 0, stream, args); break;
        case 2: launch(paged_decode_kernel<T, kLanes, 2>, dim3(grid), dim3(kThreads), 0, stream, args); break;
        default: launch(paged_decode_kernel<T, kLanes, 4>, dim3(grid), dim3(kThreads), 0, stream, args); break;
    }
}

template <typename T>
void launch_typed(const PagedArgs& args, const Plan& plan, int64_t sequences, hipStream_t stream) {
    if (plan.lanes == 0) {
        const int64_t per = (args.head_dim + kWaveSize - 1) / kWaveSize;
        const dim3 grid(static_cast<unsigned>(sequences * args.heads));
        if (per <= 1) {
            launch(paged_decode_wide_kernel<T, 1>, dim3(grid), dim3(kWaveSize), 0, stream, args);
        } else if (per <= 2) {
            launch(paged_decode_wide_kernel<T, 2>, dim3(grid), dim3(kWaveSize), 0, stream, args);
        } else if (per <= 4) {
            launch(paged_decode_wide_kernel<T, 4>, dim3(grid), dim3(kWaveSize), 0, stream, args);
        } else if (per <= 8) {
            launch(paged_decode_wide_kernel<T, 8>, dim3(grid), dim3(kWaveSize), 0, stream, args);
        } else {
            launch(paged_decode_wide_kernel<T, 16>, dim3(grid), dim3(kWaveSize), 0, stream, args);
        }
        return;
    }
    const int64_t workgroups = sequences * args.kv_heads * plan.head_groups * plan.splits;
    if constexpr (std::is_same<T, float>::value) {
        if (plan.lanes == kMfmaF32Plan) {
            const dim3 grid(static_cast<unsigned>(workgroups));
            switch (args.head_dim / 16) {
                case 1: launch(paged_mfma_f32_kernel<16>, grid, dim3(kThreads), 0, stream, args); break;
                case 2: launch(paged_mfma_f32_kernel<32>, grid, dim3(kThreads), 0, stream, args); break;
                case 3: launch(paged_mfma_f32_kernel<48>, grid, dim3(kThreads), 0, stream, args); break;
                case 4: launch(paged_mfma_f32_kernel<64>, grid, dim3(kThreads), 0, stream, args); break;
                case 5: launch(paged_mfma_f32_kernel<80>, grid, dim3(kThreads), 0, stream, args); break;
                case 6: launch(paged_mfma_f32_kernel<96>, grid, dim3(kThreads), 0, stream, args); break;
                case 7: launch(paged_mfma_f32_kernel<112>, grid, dim3(kThreads), 0, stream, args); break;
                default: launch(paged_mfma_f32_kernel<128>, grid, dim3(kThreads), 0, stream, args); break;
            }
            if (plan.splits > 1) {
                launch(paged_combine_kernel<T>, dim3(static_cast<unsigned>(sequences * args.heads)), dim3(kWaveSize),
                       0, stream, args);
            }
            return;
        }
    }
    if constexpr (!std::is_same<T, float>::value) {
      if (plan.lanes == kMfmaPlan) {
        // Two waves per (sequence, KV head, split) for GQA when one round of
        // two workgroups per CU holds them all: each wave then takes twice the
        // tokens and the grid halves (bf16 D = 128, 64 x 1024 tokens: group 4
        // 63.8 -> 68.1% of HBM peak, group 8 63.4 -> 66.5%). With two rounds
        // (128 x 256 tokens, 54.2 -> 52.8%) and for MHA (16 x 512 tokens, 58.8
        // -> 57.5%) it was slower.
        const bool pair_waves = args.heads > args.kv_heads && workgroups % 2 == 0 &&
                                workgroups <= 2 * static_cast<int64_t>(cu_count());
        const dim3 grid(static_cast<unsigned>(pair_waves ? workgroups / 2 : workgroups));
        // Two sub-chunks per step up to D = 128 (64 KiB of LDS), one above.
        constexpr int kSubsSmall = 2;
        auto go = [&](auto k4, auto k2) {
            if (pair_waves) {
                launch(k2, grid, dim3(kThreads), 0, stream, args);
            } else {
                launch(k4, grid, dim3(kThreads), 0, stream, args);
            }
        };
        switch (args.head_dim / 32) {
            case 1: go(paged_mfma_kernel<32, kSubsSmall, 4>, paged_mfma_kernel<32, kSubsSmall, 2>); break;
            case 2: go(paged_mfma_kernel<64, kSubsSmall, 4>, paged_mfma_kernel<64, kSubsSmall, 2>); break;
            case 3: go(paged_mfma_kernel<96, kSubsSmall, 4>, paged_mfma_kernel<96, kSubsSmall, 2>); break;
            case 4: go(paged_mfma_kernel<128, kSubsSmall, 4>, paged_mfma_kernel<128, kSubsSmall, 2>); break;
            case 5: go(paged_mfma_kernel<160, 1, 4>, paged_mfma_kernel<160, 1, 2>); break;
            case 6: go(paged_mfma_kernel<192, 1, 4>, paged_mfma_kernel<192, 1, 2>); break;
            case 7: go(paged_mfma_kernel<224, 1, 4>, paged_mfma_kernel<224, 1, 2>); break;
            default: go(paged_mfma_kernel<256, 1, 4>, paged_mfma_kernel<256, 1, 2>); break;
        }
        if (plan.splits > 1) {
            launch(paged_combine_kernel<T>, dim3(static_cast<unsigned>(sequences * args.heads)), dim3(kWaveSize), 0,
                   stream, args);
        }
        return;
      }
    }
    switch (plan.lanes) {
        case 1: launch_streaming<T, 1>(args, plan.gs, workgroups, stream); break;
        case 2: launch_streaming<T, 2>(args, plan.gs, workgroups, stream); break;
        case 4: launch_streaming<T, 4>(args, plan.gs, workgroups, stream); break;
        case 8: launch_streaming<T, 8>(args, plan.gs, workgroups, stream); break;
        case 16: launch_streaming<T, 16>(args, plan.gs, workgroups, stream); break;
        case 32: launch_streaming<T, 32>(args, plan.gs, workgroups, stream); break;
        default: launch_streaming<T, 64>(args, plan.gs, workgroups, stream); break;
    }
    if (plan.splits > 1) {
        launch(paged_combine_kernel<T>, dim3(dim3(static_cast<unsigned>(sequences * args.heads))),
               dim3(kWaveSize), 0, stream, args);
    }
}

}  // namespace
}  // namespace cf

extern "C" {

size_t cf_paged_attention_workspace_bytes(int64_t num_sequences, int64_t num_heads, int64_t num_kv_heads,
                                          int64_t head_dim, int64_t block_size,
                                          int64_t max_blocks_per_sequence) {
    if (num_sequences <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
        max_blocks_per_sequence <= 0 || num_heads % num_kv_heads != 0) {
        return 0;
    }
    // The split plan depends on the element size (16-byte lane pieces): size
    // for whichever of fp32 and bf16 needs more.
    size_t bytes = 0;
    for (int64_t elem : {4, 2}) {
        const cf::Plan plan = cf::plan_for(num_sequences, num_heads, num_kv_heads, head_dim, block_size,
                                           max_blocks_per_sequence, elem, true);
        const size_t need = cf::partial_bytes(plan, num_sequences, num_heads, head_dim);
        bytes = need > bytes ? need : bytes;
    }
    return bytes;
}

cf_status cf_paged_attention(const void* query, const void* k_cache, const void* v_cache,
                             const uint32_t* block_tables, const int32_t* context_lens, void* out,
                             cf_dtype dtype, int64_t num_sequences, int64_t num_heads,
                             int64_t num_kv_heads, int64_t head_dim, int64_t block_size,
                             int64_t max_blocks_per_sequence, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
    CF_ENTRY();
    if (num_sequences <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
        max_blocks_per_sequence <= 0) {
        return CF_OK;
    }
    if (num_heads % num_kv_heads != 0) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT,
                        "paged attention: num_heads %lld is not a multiple of num_kv_heads %lld",
                        static_cast<long long>(num_heads), static_cast<long long>(num_kv_heads));
    }
    if (head_dim > 1024) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT, "paged attention: head_dim %lld exceeds 1024",
                        static_cast<long long>(head_dim));
    }
    if (dtype != CF_F32 && dtype != CF_BF16) {
        return cf::fail(CF_ERR_UNSUPPORTED, "paged attention: fp32 or bf16 only");
    }
    if (query == nullptr || k_cache == nullptr || v_cache == nullptr || block_tables == nullptr ||
        context_lens == nullptr || out == nullptr) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT, "paged attention: null pointer");
    }
    const int64_t elem = dtype == CF_F32 ? 4 : 2;
    const bool aligned = cf::host_aligned(query, 16) && cf::host_aligned(k_cache, 16) &&
                         cf::host_aligned(v_cache, 16) && cf::host_aligned(out, 16);
    cf::Plan plan = cf::plan_for(num_sequences, num_heads, num_kv_heads, head_dim, block_size,
                                 max_blocks_per_sequence, elem, workspace != nullptr);
    if (plan.lanes != 0 && !aligned) plan = cf::Plan{0, 1, 1, 1, max_blocks_per_sequence * block_size};
    const size_t needed = cf::partial_bytes(plan, num_sequences, num_heads, head_dim);
    if (needed > 0 && (workspace_bytes < needed || !cf::host_aligned(workspace, 16))) {
        plan = cf::plan_for(num_sequences, num_heads, num_kv_heads, head_dim, block_size,
                            max_blocks_per_sequence, elem, false);
    }
    cf::PagedArgs args;
    args.query = query;
    args.k_cache = k_cache;
    args.v_cache = v_cache;
    args.tables = block_tables;
    args.context = context_lens;
    args.out = out;
    args.partial = static_cast<float*>(workspace);
    args.heads = num_heads;
    args.kv_heads = num_kv_heads;
    args.head_dim = head_dim;
    args.block_size = block_size;
    args.max_blocks = max_blocks_per_sequence;
    args.split_tokens = plan.split_tokens;
    args.splits = plan.splits;
    args.head_groups = plan.head_groups;
    args.scale = scale;
    auto s = static_cast<hipStream_t>(stream);
    if (dtype == CF_F32) {
        cf::launch_typed<float>(args, plan, num_sequences, s);
    } else {
        cf::launch_typed<uint16_t>(args, plan, num_sequences, s);
    }
    return cf::check_launch("launching paged attention", s);
}

}  // extern "C"

// fp32 LoRA linear on the bf16 MFMA units of gfx950:
//
//   y[M, N] = x[M, K] @ w[K, N] + scale * (x @ a)[M, r] @ b[r, N]
//
// operator layout of the reference (cuda/include/cudaforge/lora_linear.cuh:26-31),
// fp32 inputs and output, r <= 16 - the dtype the reference's own kernel runs
// (python/cudaforge/ops.py:326-330, cpp/src/bindings.cpp:94-127,
// cuda/src/lora_linear.cu:138-203).
//
// gfx950 has no fast fp32 matrix instruction to match its bf16 MFMA, so every
// fp32 operand element v is split on its way into LDS into two bf16 parts,
// hi = bf16(v) and lo = bf16(v - hi), and each product takes three MFMAs,
// a_hi b_hi + a_hi b_lo + a_lo b_hi, accumulated in fp32 (the dropped
// lo * lo term and the split residue are ~2^-16 of the product; TF32, which
// the reference's tensor-core path accepts, keeps 2^-11).
//
// Shape of the kernel:
//   * 64 x 64 output tile per workgroup of 4 waves; wave w owns rows
//     16 w .. +15 and all 64 columns as four 16 x 16 blocks, computed
//     transposed (C^T = w^T x^T) so each lane holds 4 consecutive columns of
//     one row (16-byte stores), as in the bf16 kernel of cf_lora_fused.hip.
//   * K-step 32: each thread loads 16-byte pieces of x, w and a (fp32) into
//     registers one step ahead, splits them and writes both bf16 planes to
//     one of two LDS stages; one barrier per step. Rows past M, columns past
//     N and k past K read as zero.
//   * The adapter's x @ a rides in the same loop: a^T fragments (transposed
//     out of LDS) meet the wave's x^T fragments in three more MFMAs per step,
//     so the x @ a of a wave's 16 rows lands in registers in exactly the
//     layout the epilogue's 16x16x16 MFMA takes as its B operand: no LDS
//     exchange. The epilogue adds scale * (x @ a) @ b with u = scale * (x @ a)
//     and b split the same way.
//   * Small problems split the reduction: slice s of `splits` covers K-steps
//     [s * steps, (s + 1) * steps) and writes its partial output (and
//     partial x @ a), adapter term included - the sum over slices is the
//     whole result, as the adapter term is linear in x @ a - into a
//     workspace that a second launch sums in slice order (deterministic).
#include "cf_lora_f32.hpp"

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kTM = 64;        // rows per workgroup
constexpr int kTN = 64;        // columns per workgroup
constexpr int kTK = 32;        // K-step
constexpr int kThreads = 256;  // 4 waves
constexpr int kRankSlots = 16;

// One LDS stage: bf16 high and low planes of x [64 m][32 k] (64-byte rows),
// w [32 k][64 n] (128-byte rows) and a [32 k][16 j] (32-byte rows).
constexpr int kXPlane = kTM * kTK * 2;          // 4 KiB
constexpr int kWPlane = kTK * kTN * 2;          // 4 KiB
constexpr int kAPlane = kTK * kRankSlots * 2;   // 1 KiB
constexpr int kOffXHi = 0;
constexpr int kOffXLo = kOffXHi + kXPlane;
constexpr int kOffWHi = kOffXLo + kXPlane;
constexpr int kOffWLo = kOffWHi + kWPlane;
constexpr int kOffAHi = kOffWLo + kWPlane;
constexpr int kOffALo = kOffAHi + kAPlane;
constexpr int kStageBytes = kOffALo + kAPlane;  // 18 KiB
// b planes for the epilogue ([16 j][64 n], 128-byte rows) after two stages.
constexpr int kBPlane = kRankSlots * kTN * 2;   // 2 KiB
constexpr int kOffBHi = 2 * kStageBytes;
constexpr int kOffBLo = kOffBHi + kBPlane;
constexpr int kLdsBytes = kOffBLo + kBPlane;    // 40 KiB

struct F32Args {
    const float* x;
    const float* w;
    const float* a;
    const float* b;
    float* y;        // output (one slice) or nullptr
    float* part;     // [splits][M][N] partial outputs (several slices)
    float* xa_out;   // [M][rank] x @ a (one slice) or nullptr
    float* xa_part;  // [splits][M][16] partial x @ a (several slices)
    int64_t M;
    int64_t N;
    int64_t K;
    int64_t rank;
    float scale;
    int steps;    // K-steps per slice
    int n_tiles;
    int want_xa;  // write x @ a (to xa_out or xa_part)
};

__device__ __forceinline__ s16x4_t lds_read_tr(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

__device__ __forceinline__ bf16x8_t concat(s16x4_t lo, s16x4_t hi) {
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

/// x plane: 16-byte chunk c of row r at chunk c ^ ((r >> 2) & 3), so the 8
/// rows one ds_read_b128 octet reads spread over all banks.
__device__ __forceinline__ int x_offset(int row, int k) {
    return row * (kTK * 2) + ((((k >> 3) ^ (row >> 2)) & 3) << 4) + (k & 7) * 2;
}

/// a plane ([32 k][16 j], 32-byte rows): rows 8-15 and 24-31 swap 128-byte
/// halves so the two 16-lane groups of a transposed read use other banks.
__device__ __forceinline__ int a_offset(int row, int byte) {
    return (row * 32 + byte) ^ (((row >> 3) & 1) << 7);
}

/// Registers one thread carries from global memory to LDS per K-step: two
/// 16-byte pieces of x, two of w, two elements of a.
struct Staged {
    float4 x[2];
    float4 w[2];
    float a[2];
};

__global__ __launch_bounds__(kThreads) void lora_f32_kernel(F32Args args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int jl = lane & 15;
    const int tn = static_cast<int>(blockIdx.x) % args.n_tiles;
    const int tm = static_cast<int>(blockIdx.x) / args.n_tiles;
    const int slice = static_cast<int>(blockIdx.y);
    const int64_t m0 = static_cast<int64_t>(tm) * kTM;
    const int64_t n0 = static_cast<int64_t>(tn) * kTN;
    const int64_t M = args.M;
    const int64_t N = args.N;
    const int64_t K = args.K;
    const int64_t rank = args.rank;
    const int64_t k_begin = static_cast<int64_t>(slice) * args.steps * kTK;

    // Buffer resources: loads past the end read zero. x rows past M fall
    // outside x's range; columns past N and k past K are masked below (a
    // row's tail would otherwise read the next row).
    const __amdgpu_buffer_rsrc_t xbuf = make_buffer(args.x, static_cast<uint32_t>(M * K * 4));
    const __amdgpu_buffer_rsrc_t wbuf = make_buffer(args.w, static_cast<uint32_t>(K * N * 4));
    const __amdgpu_buffer_rsrc_t abuf = make_buffer(args.a, static_cast<uint32_t>(K * rank * 4));

    // Load roles. x piece i: row (tid + 256 i) / 8 of the tile, k 4 ((tid +
    // 256 i) % 8); w piece i: k row (tid + 256 i) / 16, columns 4 ((tid + 256
    // i) % 16); a element i: k row (tid + 256 i) / 16, column (tid + 256 i) % 16.
    auto load = [&](Staged& st, int64_t k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx >> 3;
            const int64_t k = k0 + 4 * (idx & 7);
            const int64_t grow = m0 + row;
            const bool ok = k < K && grow < M;
            const uint4 v = buffer_load16(xbuf, ok ? static_cast<uint32_t>((grow * K + k) * 4) : 0x80000000u, 0);
            st.x[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                                  __uint_as_float(v.w));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int64_t k = k0 + (idx >> 4);
            const int64_t col = n0 + 4 * (idx & 15);
            const bool ok = k < K && col < N;
            const uint4 v = buffer_load16(wbuf, ok ? static_cast<uint32_t>((k * N + col) * 4) : 0x80000000u, 0);
            st.w[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                                  __uint_as_float(v.w));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int64_t k = k0 + (idx >> 4);
            const int j = idx & 15;
            const bool ok = k < K && j < rank;
            st.a[i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                abuf, ok ? static_cast<uint32_t>((k * rank + j) * 4) : 0x80000000u, 0, 0));
        }
    };
    auto store = [&](const Staged& st, int stage) {
        uint8_t* base = lds + stage * kStageBytes;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx >> 3;
            const int k = 4 * (idx & 7);
            uint2 hi;
            uint2 lo;
            split_pk_as<false>(st.x[i].x, st.x[i].y, hi.x, lo.x);
            split_pk_as<false>(st.x[i].z, st.x[i].w, hi.y, lo.y);
            const int off = x_offset(row, k);
            *reinterpret_cast<uint2*>(base + kOffXHi + off) = hi;
            *reinterpret_cast<uint2*>(base + kOffXLo + off) = lo;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int krow = idx >> 4;
            const int col = 4 * (idx & 15);
            uint2 hi;
            uint2 lo;
            split_pk_as<false>(st.w[i].x, st.w[i].y, hi.x, lo.x);
            split_pk_as<false>(st.w[i].z, st.w[i].w, hi.y, lo.y);
            const int off = krow * (kTN * 2) + col * 2;
            *reinterpret_cast<uint2*>(base + kOffWHi + off) = hi;
            *reinterpret_cast<uint2*>(base + kOffWLo + off) = lo;
        }
        uint32_t ahi;
        uint32_t alo;
        split_pk_as<false>(st.a[0], st.a[1], ahi, alo);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            const int off = a_offset(idx >> 4, (idx & 15) * 2);
            *reinterpret_cast<uint16_t*>(base + kOffAHi + off) = static_cast<uint16_t>(ahi >> (16 * i));
            *reinterpret_cast<uint16_t*>(base + kOffALo + off) = static_cast<uint16_t>(alo >> (16 * i));
        }
    };


    // Fragment roles (16x16x32 MFMA, C^T = w^T x^T):
    //   B (x^T): lane holds x[16 wave + jl][k 8 g .. +7], one ds_read_b128;
    //   A (w^T) of column block jb: lane holds w[k 8 g .. +7][16 jb + jl], two
    //     transposed reads of rows 8 g .. +3 and +4 .. +7;
    //   A (a^T): lane holds a[k 8 g .. +7][j = jl], the same from the a plane.
    const int x_rd = x_offset(16 * wave + jl, 8 * g);
    int w_rd[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int row = 8 * g + (jl >> 2);
        w_rd[jb] = row * (kTN * 2) + (2 * jb + ((jl & 3) >> 1)) * 16 + (jl & 1) * 8;
    }
    const int a_rd0 = a_offset(8 * g + (jl >> 2), (jl & 3) * 8);
    const int a_rd1 = a_offset(8 * g + 4 + (jl >> 2), (jl & 3) * 8);

    f32x4_t acc[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) acc[jb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4_t xacc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](int stage) {
        const uint8_t* base = lds + stage * kStageBytes;
        const bf16x8_t xh = *reinterpret_cast<const bf16x8_t*>(base + kOffXHi + x_rd);
        const bf16x8_t xl = *reinterpret_cast<const bf16x8_t*>(base + kOffXLo + x_rd);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const bf16x8_t wh = concat(lds_read_tr(base + kOffWHi, w_rd[jb]),
                                       lds_read_tr(base + kOffWHi, w_rd[jb] + 4 * kTN * 2));
            const bf16x8_t wl = concat(lds_read_tr(base + kOffWLo, w_rd[jb]),
                                       lds_read_tr(base + kOffWLo, w_rd[jb] + 4 * kTN * 2));
            acc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, xh, acc[jb], 0, 0, 0);
            acc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh, xl, acc[jb], 0, 0, 0);
            acc[jb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl, xh, acc[jb], 0, 0, 0);
        }
        const bf16x8_t ah = concat(lds_read_tr(base + kOffAHi, a_rd0), lds_read_tr(base + kOffAHi, a_rd1));
        const bf16x8_t al = concat(lds_read_tr(base + kOffALo, a_rd0), lds_read_tr(base + kOffALo, a_rd1));
        xacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, xh, xacc, 0, 0, 0);
        xacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, xl, xacc, 0, 0, 0);
        xacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, xh, xacc, 0, 0, 0);
    };

    // Stage j % 2 is written at the top of step j: every wave finished
    // reading it in step j - 2, before the barrier of step j - 1.
    // Stage j % 2 is written at the top of step j: every wave finished
    // reading it in step j - 2, before the barrier of step j - 1.
    Staged st;
    load(st, k_begin);
    for (int j = 0; j < args.steps; ++j) {
        store(st, j & 1);
        __syncthreads();
        if (j + 1 < args.steps) load(st, k_begin + static_cast<int64_t>(j + 1) * kTK);
        compute(j & 1);
    }

    // The split above is exact for values within bf16's range. A value
    // outside it (inf, NaN, |v| > 0x7F7F) in this tile's x, w or a always
    // leaves some accumulator of the tile (or of x @ a) non-finite under that
    // split, and so does an fp32 overflow. Such a tile (a rare one; the vote
    // costs two barriers and uses the b planes, idle until the epilogue) is
    // summed again in plain fp32 arithmetic, the reference's own, from global
    // memory: slow, and exact in its inf / NaN / overflow behaviour.
    {
        float probe = (xacc[0] + xacc[1]) + (xacc[2] + xacc[3]);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) probe += (acc[jb][0] + acc[jb][1]) + (acc[jb][2] + acc[jb][3]);
        if (workgroup_any<kThreads / 64>(!__builtin_isfinite(probe), reinterpret_cast<int*>(lds + kOffBHi))) {
            const int64_t row = m0 + 16 * wave + jl;
            const int64_t k_end = k_begin + static_cast<int64_t>(args.steps) * kTK < K
                                      ? k_begin + static_cast<int64_t>(args.steps) * kTK
                                      : K;
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) acc[jb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            xacc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            if (row < M) {
                for (int64_t k = k_begin; k < k_end; ++k) {
                    const float xv = args.x[row * K + k];
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int64_t col = n0 + 16 * jb + 4 * g + e;
                            if (col < N) acc[jb][e] = __builtin_fmaf(xv, args.w[k * N + col], acc[jb][e]);
                        }
                    }
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (4 * g + t < rank) xacc[t] = __builtin_fmaf(xv, args.a[k * rank + 4 * g + t], xacc[t]);
                    }
                }
            }
        }
    }

    // Epilogue: b's tile split into planes, then acc += u b with
    // u = scale * (x @ a): xacc lane holds (x @ a)^T[j = 4 g + t][m = 16 wave + jl],
    // the B operand of the 16x16x16 MFMA; b is its A operand (b^T[n][j]),
    // read transposed: lane jl of group g receives b[4 g .. 4 g + 3][16 jb + jl].
    {
        const int j = tid >> 4;
        const int64_t col = n0 + 4 * (tid & 15);
        const bool ok = j < rank && col < N;
        const __amdgpu_buffer_rsrc_t bbuf = make_buffer(args.b, static_cast<uint32_t>(rank * N * 4));
        const uint4 v = buffer_load16(bbuf, ok ? static_cast<uint32_t>((j * N + col) * 4) : 0x80000000u, 0);
        uint2 hi;
        uint2 lo;
        split_pk4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w), hi, lo);
        const int off = j * (kTN * 2) + 8 * (tid & 15);
        *reinterpret_cast<uint2*>(lds + kOffBHi + off) = hi;
        *reinterpret_cast<uint2*>(lds + kOffBLo + off) = lo;
    }
    __syncthreads();
    // Adapter columns past the rank are padding (a reads zero there): an
    // infinite x makes them inf * 0 = NaN, which must not reach y through
    // b's zero rows.
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        if (4 * g + t >= rank) xacc[t] = 0.0f;
    }
    uint2 uhw;
    uint2 ulw;
    split_pk4(args.scale * xacc[0], args.scale * xacc[1], args.scale * xacc[2], args.scale * xacc[3], uhw, ulw);
    const s16x4_t uh = __builtin_bit_cast(s16x4_t, uhw);
    const s16x4_t ul = __builtin_bit_cast(s16x4_t, ulw);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int row = 4 * g + (jl >> 2);
        const int off = row * (kTN * 2) + (2 * jb + ((jl & 3) >> 1)) * 16 + (jl & 1) * 8;
        const s16x4_t bh = lds_read_tr(lds + kOffBHi, off);
        const s16x4_t bl = lds_read_tr(lds + kOffBLo, off);
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bh, uh, acc[jb], 0, 0, 0);
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bh, ul, acc[jb], 0, 0, 0);
        acc[jb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bl, uh, acc[jb], 0, 0, 0);
    }

    // acc[jb] lane holds y[m0 + 16 wave + jl][n0 + 16 jb + 4 g .. +3]; N is a
    // multiple of 4, so the four columns are all inside or all outside.
    const int64_t row = m0 + 16 * wave + jl;
    if (row < M) {
        float* dst = args.y != nullptr ? args.y : args.part + static_cast<int64_t>(slice) * M * N;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const int64_t col = n0 + 16 * jb + 4 * g;
            if (col < N) *reinterpret_cast<f32x4_t*>(dst + row * N + col) = acc[jb];
        }
        if (args.want_xa && tn == 0) {
            if (args.xa_out != nullptr) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if (4 * g + t < rank) args.xa_out[row * rank + 4 * g + t] = xacc[t];
                }
            } else {
                *reinterpret_cast<f32x4_t*>(args.xa_part + (static_cast<int64_t>(slice) * M + row) * kRankSlots +
                                            4 * g) = xacc;
            }
        }
    }
}

/// y = sum over slices of part (slice order), four outputs per thread; the
/// threads past M * N / 4 sum x @ a likewise into xa_out.
__global__ __launch_bounds__(kThreads) void lora_f32_sum_kernel(const float4* __restrict__ part,
                                                                float4* __restrict__ y,
                                                                const float* __restrict__ xa_part,
                                                                float* __restrict__ xa_out, int64_t quads,
                                                                int64_t M, int64_t rank, int splits) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < quads) {
        float4 total = part[i];
        for (int s = 1; s < splits; ++s) {
            const float4 v = part[s * quads + i];
            total.x += v.x;
            total.y += v.y;
            total.z += v.z;
            total.w += v.w;
        }
        y[i] = total;
        return;
    }
    const int64_t e = i - quads;
    if (xa_out == nullptr || e >= M * rank) return;
    const int64_t row = e / rank;
    const int64_t j = e % rank;
    float total = 0.0f;
    for (int s = 0; s < splits; ++s) total += xa_part[(s * M + row) * kRankSlots + j];
    xa_out[e] = total;
}

size_t align256(size_t bytes) { return (bytes + 255) / 256 * 256; }

}  // namespace

bool lora_f32_eligible(const void* x, const void* w, const void* a, const void* b, const void* y,
                       int64_t M, int64_t N, int64_t K, int64_t rank) {
    // 32-bit buffer offsets with 0x80000000 as the "zero" offset.
    const bool fits = M * K * 4 < (1LL << 31) && K * N * 4 < (1LL << 31) &&
                      K * rank * 4 < (1LL << 31) && rank * N * 4 < (1LL << 31);
    const bool adapter_ok = rank == 0 || (host_aligned(a, 4) && host_aligned(b, 16));
    return M > 0 && N > 0 && K > 0 && rank <= kRankSlots && N % 4 == 0 && K % 4 == 0 && fits &&
           adapter_ok && host_aligned(x, 16) && host_aligned(w, 16) && host_aligned(y, 16) &&
           ceil_div<int64_t>(M, kTM) * ceil_div<int64_t>(N, kTN) < (1LL << 31);
}

int lora_f32_splits(int64_t M, int64_t N, int64_t K) {
    // Enough workgroups for two per CU, and at least four K-steps per slice.
    const int64_t tiles = ceil_div<int64_t>(M, kTM) * ceil_div<int64_t>(N, kTN);
    const int64_t steps = ceil_div<int64_t>(K, kTK);
    const int64_t target = 2 * static_cast<int64_t>(cu_count());
    int64_t splits = ceil_div<int64_t>(target, tiles);
    const int64_t most = steps / 4 > 1 ? steps / 4 : 1;
    if (splits > most) splits = most;
    // At most 8 slices: 64 x 2048 x 2048 took 13.2 us against 14.4 with 16
    // (the reference's other two shapes unchanged).
    if (splits > 8) splits = 8;
    return static_cast<int>(splits < 1 ? 1 : splits);
}

size_t lora_f32_workspace_bytes(int64_t M, int64_t N, int64_t rank, int splits) {
    if (splits <= 1) return 0;
    (void)rank;
    return align256(static_cast<size_t>(splits) * M * N * 4) +
           static_cast<size_t>(splits) * M * kRankSlots * 4;
}

cf_status launch_lora_f32(const float* x, const float* w, const float* a, const float* b, float* y,
                          float* xa_out, int64_t M, int64_t N, int64_t K, int64_t rank, float scale,
                          int splits, void* workspace, hipStream_t stream) {
    const int64_t steps_total = ceil_div<int64_t>(K, kTK);
    if (splits < 1) splits = 1;
    // Whole K-steps per slice; the last slices may be short (or empty, then
    // they contribute zeros).
    const int64_t steps = ceil_div<int64_t>(steps_total, splits);
    F32Args args{};
    args.x = x;
    args.w = w;
    args.a = rank > 0 ? a : nullptr;
    args.b = rank > 0 ? b : nullptr;
    args.M = M;
    args.N = N;
    args.K = K;
    args.rank = rank;
    args.scale = scale;
    args.steps = static_cast<int>(steps);
    args.n_tiles = static_cast<int>(ceil_div<int64_t>(N, kTN));
    args.want_xa = xa_out != nullptr && rank > 0;
    float* part = nullptr;
    float* xa_part = nullptr;
    if (splits > 1) {
        part = static_cast<float*>(workspace);
        xa_part = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                           align256(static_cast<size_t>(splits) * M * N * 4));
        args.part = part;
        args.xa_part = xa_part;
    } else {
        args.y = y;
        args.xa_out = xa_out;
    }
    const int64_t tiles = ceil_div<int64_t>(M, kTM) * args.n_tiles;
    launch(lora_f32_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(splits)), dim3(kThreads), 0,
           stream, args);
    if (splits > 1) {
        const int64_t quads = M * N / 4;
        const int64_t extra = args.want_xa ? M * rank : 0;
        const unsigned grid = static_cast<unsigned>(ceil_div<int64_t>(quads + extra, kThreads));
        launch(lora_f32_sum_kernel, dim3(grid), dim3(kThreads), 0, stream,
               reinterpret_cast<const float4*>(part), reinterpret_cast<float4*>(y), xa_part,
               args.want_xa ? xa_out : nullptr, quads, M, rank, splits);
    }
    return check_launch("launching the fp32 MFMA LoRA linear", stream);
}

}  // namespace cf

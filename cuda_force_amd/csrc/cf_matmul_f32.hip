// fp32 GEMM on the bf16 MFMA units of gfx950: c[M, N] = a[M, K] @ b[K, N],
// row-major, the fp32 matrix product the reference's tensor-core matmul
// computes (cuda/include/cudaforge/tensor_core_matmul.cuh:40-51) and the
// base product of its LoRA linear.
//
// Every fp32 operand element v is split on its way into LDS into two bf16
// parts, hi = bf16(v) and lo = bf16(v - hi); each product takes three MFMAs,
// a_hi b_hi + a_hi b_lo + a_lo b_hi, accumulated in fp32 (about 2^-16 of
// each product dropped; TF32 keeps 2^-11). Splitting while staging makes the
// product one launch: the earlier form wrote both operands' bf16 parts to a
// workspace first (a memory-bound pass of ~10 bytes per element).
//
// Shape of the kernel:
//   * 128 x 128 output tile per workgroup of 4 waves; wave (wm, wn) owns rows
//     64 wm .. +63 and columns 64 wn .. +63 as 4 x 4 blocks of 16 x 16,
//     computed transposed (C^T = b^T a^T) so each lane holds 4 consecutive
//     output columns of one row (16-byte stores).
//   * K-step 32: each thread loads four 16-byte pieces of a and four of b
//     (fp32) into registers one step ahead, splits them and writes the bf16
//     planes to one of two LDS stages (64 KiB: two workgroups per CU); one
//     barrier per step. A second register set for two steps ahead took the
//     kernel to 272 registers (one wave per SIMD) and ran slower at every
//     size tried (1024^3: 26.7 -> 35.3 us). Rows past M, columns past N and k past K read as zero
//     through the buffer range check.
//   * a planes: [128 m][32 k], 64-byte rows, 16-byte chunk c of row r at
//     c ^ ((r >> 2) & 3) (ds_read_b128 of 16 rows spreads over the banks);
//     b planes: [32 k][128 n], 256-byte rows, chunk c of row r at
//     c ^ (2 (r & 3) + 8 ((r >> 3) & 1)), so the 16-lane groups of a
//     transposed read (ds_read_b64_tr_b16) touch distinct 32-byte bank
//     groups and rows 8 apart use the other 128-byte half.
//   * Small grids split the reduction: slice s covers K-steps [s steps,
//     (s + 1) steps); slices write fp32 partial outputs to a workspace that a
//     second launch sums in slice order (deterministic).
#include "cf_matmul_f32.hpp"

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kTM = 128;
constexpr int kTN = 128;
constexpr int kTK = 32;
constexpr int kThreads = 256;
constexpr int kAPlane = kTM * kTK * 2;  // 8 KiB
constexpr int kBPlane = kTK * kTN * 2;  // 8 KiB
constexpr int kOffAHi = 0;
constexpr int kOffALo = kOffAHi + kAPlane;
constexpr int kOffBHi = kOffALo + kAPlane;
constexpr int kOffBLo = kOffBHi + kBPlane;
constexpr int kStageBytes = kOffBLo + kBPlane;  // 32 KiB
constexpr int kLdsBytes = 2 * kStageBytes;      // 64 KiB
constexpr int kMaxSplits = 4;

struct Args {
    const float* a;
    const float* b;
    float* c;      // output (one slice) or nullptr
    float* part;   // [splits][M][N] partial outputs (several slices)
    int64_t M;
    int64_t N;
    int64_t K;
    int steps;     // K-steps per slice
    int n_tiles;
};

__device__ __forceinline__ int a_offset(int row, int k) {
    return row * (kTK * 2) + ((((k >> 3) ^ (row >> 2)) & 3) << 4) + (k & 7) * 2;
}

__device__ __forceinline__ int b_swizzle(int row) { return 2 * (row & 3) + 8 * ((row >> 3) & 1); }

/// Byte offset of the 8-byte piece holding columns 4 q .. 4 q + 3 of b-plane
/// row `row` (q = col / 4).
__device__ __forceinline__ int b_offset(int row, int q) {
    return row * (kTN * 2) + (((q >> 1) ^ b_swizzle(row)) << 4) + (q & 1) * 8;
}

__device__ __forceinline__ s16x4_t lds_read_tr(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

__device__ __forceinline__ bf16x8_t concat(s16x4_t lo, s16x4_t hi) {
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

/// The four values' bf16 high parts (returned) and low parts (lo_out),
/// packed two per word: the plain split, exact for values within bf16's
/// range (the kernel recomputes a tile that holds others).
__device__ __forceinline__ uint2 pack_hi_lo(const float4& v, uint2& lo_out) {
    uint2 hi;
    split_pk_as<false>(v.x, v.y, hi.x, lo_out.x);
    split_pk_as<false>(v.z, v.w, hi.y, lo_out.y);
    return hi;
}

__device__ __forceinline__ float4 as_float4(const uint4& v) {
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}

__global__ __launch_bounds__(kThreads) void matmul_f32_kernel(Args args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1;
    const int wn = wave & 1;
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
    const int64_t k_begin = static_cast<int64_t>(slice) * args.steps * kTK;

    const __amdgpu_buffer_rsrc_t abuf = make_buffer(args.a, static_cast<uint32_t>(M * K * 4));
    const __amdgpu_buffer_rsrc_t bbuf = make_buffer(args.b, static_cast<uint32_t>(K * N * 4));

    // Load roles: a piece i is row (tid + 256 i) / 8 of the tile, k 4 ((tid +
    // 256 i) % 8); b piece i is k row (tid + 256 i) / 32, columns 4 ((tid +
    // 256 i) % 32). Out-of-range pieces read zero (offset 2^31 is past every
    // buffer's range).
    uint4 sa[4];
    uint4 sb[4];
    auto load = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kThreads * i;
            const int64_t row = m0 + (idx >> 3);
            const int64_t k = k0 + 4 * (idx & 7);
            const bool ok = row < M && k < K;
            sa[i] = buffer_load16(abuf, ok ? static_cast<uint32_t>((row * K + k) * 4) : 0x80000000u, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kThreads * i;
            const int64_t k = k0 + (idx >> 5);
            const int64_t col = n0 + 4 * (idx & 31);
            const bool ok = k < K && col < N;
            sb[i] = buffer_load16(bbuf, ok ? static_cast<uint32_t>((k * N + col) * 4) : 0x80000000u, 0);
        }
    };
    auto store = [&](int stage) {
        uint8_t* base = lds + stage * kStageBytes;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kThreads * i;
            uint2 lo;
            const uint2 hi = pack_hi_lo(as_float4(sa[i]), lo);
            const int off = a_offset(idx >> 3, 4 * (idx & 7));
            *reinterpret_cast<uint2*>(base + kOffAHi + off) = hi;
            *reinterpret_cast<uint2*>(base + kOffALo + off) = lo;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + kThreads * i;
            uint2 lo;
            const uint2 hi = pack_hi_lo(as_float4(sb[i]), lo);
            const int off = b_offset(idx >> 5, idx & 31);
            *reinterpret_cast<uint2*>(base + kOffBHi + off) = hi;
            *reinterpret_cast<uint2*>(base + kOffBLo + off) = lo;
        }
    };


    // Fragment roles (16x16x32 MFMA, C^T = b^T a^T):
    //   B (a^T) of row block rb: lane holds a[64 wm + 16 rb + jl][k 8 g .. +7]
    //     (one ds_read_b128);
    //   A (b^T) of column block cb: lane holds b[k 8 g .. +7][64 wn + 16 cb + jl]
    //     (two transposed reads of k rows 8 g + jl / 4 and 8 g + 4 + jl / 4 at
    //     columns 64 wn + 16 cb + 4 (jl % 4) .. +3).
    int a_rd[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) a_rd[rb] = a_offset(64 * wm + 16 * rb + jl, 8 * g);
    int b_rd[4][2];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int q = (64 * wn + 16 * cb) / 4 + (jl & 3);
        b_rd[cb][0] = b_offset(8 * g + (jl >> 2), q);
        b_rd[cb][1] = b_offset(8 * g + 4 + (jl >> 2), q);
    }

    f32x4_t acc[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    auto compute = [&](int stage) {
        const uint8_t* base = lds + stage * kStageBytes;
        bf16x8_t bh[4];
        bf16x8_t bl[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            bh[cb] = concat(lds_read_tr(base + kOffBHi, b_rd[cb][0]), lds_read_tr(base + kOffBHi, b_rd[cb][1]));
            bl[cb] = concat(lds_read_tr(base + kOffBLo, b_rd[cb][0]), lds_read_tr(base + kOffBLo, b_rd[cb][1]));
        }
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const bf16x8_t ah = *reinterpret_cast<const bf16x8_t*>(base + kOffAHi + a_rd[rb]);
            const bf16x8_t al = *reinterpret_cast<const bf16x8_t*>(base + kOffALo + a_rd[rb]);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[cb], ah, acc[rb][cb], 0, 0, 0);
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh[cb], al, acc[rb][cb], 0, 0, 0);
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl[cb], ah, acc[rb][cb], 0, 0, 0);
            }
        }
    };

    // Stage j % 2 is written at the top of step j: every wave finished
    // reading it in step j - 2, before the barrier of step j - 1.
    load(k_begin);
    for (int j = 0; j < args.steps; ++j) {
        store(j & 1);
        __syncthreads();
        if (j + 1 < args.steps) load(k_begin + static_cast<int64_t>(j + 1) * kTK);
        compute(j & 1);
    }

    // The split above is exact for values within bf16's range. A value
    // outside it (inf, NaN, |v| > 0x7F7F) in this tile's operands always
    // leaves some accumulator non-finite under that split, and so does an
    // fp32 overflow. Such a tile (a rare one; the vote costs two barriers and
    // uses stage steps % 2, which no wave reads after the barrier of the last
    // step) is summed again in plain fp32 arithmetic from global memory:
    // slow, and exact in its inf / NaN / overflow behaviour.
    {
        float probe = 0.0f;
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                probe += (acc[rb][cb][0] + acc[rb][cb][1]) + (acc[rb][cb][2] + acc[rb][cb][3]);
            }
        }
        int* slots = reinterpret_cast<int*>(lds + (args.steps & 1) * kStageBytes);
        if (workgroup_any<kThreads / 64>(!__builtin_isfinite(probe), slots)) {
            const int64_t k_end = k_begin + static_cast<int64_t>(args.steps) * kTK < K
                                      ? k_begin + static_cast<int64_t>(args.steps) * kTK
                                      : K;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
                for (int cb = 0; cb < 4; ++cb) acc[rb][cb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
            for (int64_t k = k_begin; k < k_end; ++k) {
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    const int64_t row = m0 + 64 * wm + 16 * rb + jl;
                    if (row >= M) continue;
                    const float av = args.a[row * K + k];
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int64_t col = n0 + 64 * wn + 16 * cb + 4 * g + e;
                            if (col < N) acc[rb][cb][e] = __builtin_fmaf(av, args.b[k * N + col], acc[rb][cb][e]);
                        }
                    }
                }
            }
        }
    }

    // acc[rb][cb] lane holds c[m0 + 64 wm + 16 rb + jl][n0 + 64 wn + 16 cb + 4 g .. +3];
    // N is a multiple of 4, so the four columns are all inside or all outside.
    float* dst = args.c != nullptr ? args.c : args.part + static_cast<int64_t>(slice) * M * N;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        const int64_t row = m0 + 64 * wm + 16 * rb + jl;
        if (row >= M) continue;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const int64_t col = n0 + 64 * wn + 16 * cb + 4 * g;
            if (col < N) *reinterpret_cast<f32x4_t*>(dst + row * N + col) = acc[rb][cb];
        }
    }
}

/// c = sum over slices of part (slice order), four outputs per thread.
__global__ __launch_bounds__(kThreads) void matmul_f32_sum_kernel(const float4* __restrict__ part,
                                                                  float4* __restrict__ c, int64_t quads,
                                                                  int splits) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= quads) return;
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

size_t align256(size_t bytes) { return (bytes + 255) / 256 * 256; }

}  // namespace

bool matmul_f32_eligible(const void* a, const void* b, const void* c, int64_t M, int64_t N, int64_t K) {
    const bool fits = M * K * 4 < (1LL << 31) && K * N * 4 < (1LL << 31);
    return M > 0 && N > 0 && K > 0 && N % 4 == 0 && K % 4 == 0 && fits && host_aligned(a, 16) &&
           host_aligned(b, 16) && host_aligned(c, 16) &&
           ceil_div<int64_t>(M, kTM) * ceil_div<int64_t>(N, kTN) < (1LL << 31);
}

int matmul_f32_splits(int64_t M, int64_t N, int64_t K) {
    // Two workgroups per CU, at least four K-steps per slice (eight was
    // slower at 512^3: 20.5 against 14.8 us), at most
    // kMaxSplits slices (each slice writes and the sum reads M x N x 4 bytes):
    // at 1024^3, 4 slices took 19.9 us against 22.7 with 8 and 23.2 with 6.
    const int64_t tiles = ceil_div<int64_t>(M, kTM) * ceil_div<int64_t>(N, kTN);
    const int64_t steps = ceil_div<int64_t>(K, kTK);
    const int64_t target = 2 * static_cast<int64_t>(cu_count());
    int64_t splits = ceil_div<int64_t>(target, tiles);
    const int64_t most = steps / 4 > 1 ? steps / 4 : 1;
    if (splits > most) splits = most;
    if (splits > kMaxSplits) splits = kMaxSplits;
    return static_cast<int>(splits < 1 ? 1 : splits);
}

size_t matmul_f32_workspace_bytes(int64_t M, int64_t N, int splits) {
    return splits <= 1 ? 0 : align256(static_cast<size_t>(splits) * M * N * 4);
}

cf_status launch_matmul_f32(const float* a, const float* b, float* c, int64_t M, int64_t N, int64_t K,
                            int splits, void* workspace, hipStream_t stream) {
    const int64_t steps_total = ceil_div<int64_t>(K, kTK);
    if (splits < 1 || workspace == nullptr) splits = 1;
    const int64_t steps = ceil_div<int64_t>(steps_total, splits);
    Args args{};
    args.a = a;
    args.b = b;
    args.M = M;
    args.N = N;
    args.K = K;
    args.steps = static_cast<int>(steps);
    args.n_tiles = static_cast<int>(ceil_div<int64_t>(N, kTN));
    if (splits > 1) {
        args.part = static_cast<float*>(workspace);
    } else {
        args.c = c;
    }
    const int64_t tiles = ceil_div<int64_t>(M, kTM) * args.n_tiles;
    launch(matmul_f32_kernel, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(splits)), dim3(kThreads), 0,
           stream, args);
    if (splits > 1) {
        const int64_t quads = M * N / 4;
        launch(matmul_f32_sum_kernel, dim3(static_cast<unsigned>(ceil_div<int64_t>(quads, kThreads))),
               dim3(kThreads), 0, stream, reinterpret_cast<const float4*>(args.part), reinterpret_cast<float4*>(c),
               quads, splits);
    }
    return check_launch("launching the fp32 MFMA matmul", stream);
}

}  // namespace cf

// Fused LoRA linear on the bf16 MFMA units of gfx950:
//
//   y[M, N] = x[M, K] @ w[K, N] + scale * bf16(x @ a)[M, r] @ b[r, N]
//
// operator layout of the reference (cuda/include/cudaforge/lora_linear.cuh:26-31),
// r <= 16, bf16 operands, fp32 accumulation, bf16 output.
//
// Shape of the kernel:
//   * 256x256 output tile per workgroup, K-step 64, 8 waves (2 per SIMD) each
//     owning a 128x64 sub-tile: 4x2 v_mfma_f32_32x32x16_bf16 tiles, 128 fp32
//     accumulators per lane. Two waves per SIMD let one wave's LDS reads,
//     transposes and address work issue while the other's MFMAs execute.
//   * Operands pass through LDS in a K-major layout: each row holds 64 k as
//     eight 16-byte chunks, XOR-swizzled by the row's low and next three bits
//     so that fragment reads (8 consecutive rows) and transposed stores (rows
//     8 apart) both spread over the banks. Two stages: the next K-step's
//     global loads are in flight in registers while the current stage feeds
//     the MFMAs; one barrier per K-step.
//   * Global loads are buffer loads (32-bit lane offsets, uniform K offset,
//     hardware range check: x rows past M read as zero); nothing in the
//     K-loop is predicated.
//   * w is N-major, so each thread loads a 4(k) x 8(n) bf16 block as four
//     16-byte row segments and transposes it in registers with v_perm_b32
//     into four-k column pieces before its LDS store.
//   * The adapter down-projection x @ a rides in the same K-loop on the x tile
//     already in LDS (v_mfma_f32_16x16x32_bf16, 32 rows x 16 columns per wave,
//     ~6% extra MFMA work); x is read from HBM once.
//   * Epilogue: x @ a is rounded to bf16 (the reference materialises it as a
//     bf16 tensor), exchanged through LDS into the A-operand layout and
//     multiplied by bf16(scale * b) with one K=16 MFMA per 32x32 tile that
//     accumulates straight into the base accumulators; then the tile is
//     rounded to bf16 and stored. No second launch, no [M, r] HBM round trip.
//   * Workgroup ids are remapped so the tiles dispatched to one XCD (ids are
//     dealt round-robin over the 8 XCDs) form a band of 4 row-tiles sharing x
//     row-panels in that XCD's L2.
// The reference's fused kernel recomputes x @ a untiled in every block
// (cuda/src/lora_linear.cu:138-203).
#include "cf_lora_fused.hpp"

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;
constexpr int kThreads = 512;
constexpr int kLdsRow = kBK * 2;                    // bytes per K-major LDS row
constexpr int kTileA = kBM * kLdsRow;               // 32 KiB
constexpr int kTileB = kBN * kLdsRow;               // 32 KiB
constexpr int kTileAdapter = 16 * kLdsRow;          // 2 KiB: a^T [16][64]
constexpr int kStage = kTileA + kTileB + kTileAdapter;
constexpr int kLdsBytes = 2 * kStage;               // 132 KiB

/// Byte offset of 16-byte chunk `chunk` (0..7) of K-major LDS row `row`.
__device__ __forceinline__ int lds_offset(int row, int chunk) {
    return row * kLdsRow + ((chunk ^ (row & 7) ^ ((row >> 3) & 7)) << 4);
}

/// Transpose a 4(k) x 8(n) block of bf16: in[r] holds k-row r (8 n values);
/// out[j] receives the 4 k values of column j (low half first).
__device__ __forceinline__ void transpose4x8(const uint4 (&in)[4], uint2 (&out)[8]) {
    const uint32_t r0[4] = {in[0].x, in[0].y, in[0].z, in[0].w};
    const uint32_t r1[4] = {in[1].x, in[1].y, in[1].z, in[1].w};
    const uint32_t r2[4] = {in[2].x, in[2].y, in[2].z, in[2].w};
    const uint32_t r3[4] = {in[3].x, in[3].y, in[3].z, in[3].w};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        // Column 2d takes the low halves, column 2d + 1 the high halves.
        out[2 * d].x = __builtin_amdgcn_perm(r1[d], r0[d], 0x05040100u);
        out[2 * d].y = __builtin_amdgcn_perm(r3[d], r2[d], 0x05040100u);
        out[2 * d + 1].x = __builtin_amdgcn_perm(r1[d], r0[d], 0x07060302u);
        out[2 * d + 1].y = __builtin_amdgcn_perm(r3[d], r2[d], 0x07060302u);
    }
}

/// Tile coordinates for workgroup `pid`: undo the round-robin XCD dealing so
/// consecutive logical ids share an XCD, then walk 4-row bands of tiles.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcds = 8;
    constexpr int kGroupM = 4;
    const int total = tiles_m * tiles_n;
    int logical = pid;
    if (total % kXcds == 0) {
        const int per_xcd = total / kXcds;
        logical = (pid % kXcds) * per_xcd + pid / kXcds;
    }
    const int band = kGroupM * tiles_n;
    const int group = logical / band;
    const int first_m = group * kGroupM;
    const int rows_in_group = (tiles_m - first_m) < kGroupM ? (tiles_m - first_m) : kGroupM;
    const int in_group = logical % band;
    tm = first_m + in_group % rows_in_group;
    tn = in_group / rows_in_group;
}

struct FusedArgs {
    const uint16_t* x;
    const uint16_t* w;
    const uint16_t* a;
    const uint16_t* b;
    uint16_t* y;
    float* xa_out;
    int64_t M;
    int64_t N;
    int64_t K;
    int64_t rank;
    float scale;
    int tiles_m;
    int tiles_n;
};

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lora_fused_bf16_kernel(FusedArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 2;  // 0..1: 128-row half of the tile
    const int wn = wave & 3;   // 0..3: 64-column quarter of the tile
    int tm;
    int tn;
    tile_of(static_cast<int>(blockIdx.x), args.tiles_m, args.tiles_n, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * kBM;
    const int64_t n0 = static_cast<int64_t>(tn) * kBN;
    const int64_t M = args.M;
    const int64_t N = args.N;
    const int64_t K = args.K;
    const int64_t rank = args.rank;

    // ---- global load roles ----
    // x tile [256 rows][8 chunks]: chunk id i*512 + tid, row id>>3, chunk id&7.
    const int64_t rows_here = M - m0 < kBM ? M - m0 : kBM;
    const __amdgpu_buffer_rsrc_t xbuf =
        make_buffer(args.x + m0 * K, static_cast<uint32_t>(rows_here * K * 2));
    uint32_t xoff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int id = i * kThreads + tid;
        xoff[i] = static_cast<uint32_t>(((id >> 3) * K + (id & 7) * 8) * 2);
    }
    // w tile [64 k][256 n] as 4x8 blocks: k-quad tid>>5 (0..15), n-block tid&31.
    // A clamped column only feeds an output column >= N, which is never stored.
    const int wkq = tid >> 5;
    const int wnb = tid & 31;
    const int64_t wcol = n0 + wnb * 8 < N ? n0 + wnb * 8 : N - 8;
    const __amdgpu_buffer_rsrc_t wbuf = make_buffer(args.w, static_cast<uint32_t>(K * N * 2));
    const uint32_t woff = static_cast<uint32_t>((static_cast<int64_t>(wkq) * 4 * N + wcol) * 2);
    // a tile [64 k][16 j]: two elements per thread, k = tid>>3, j = (tid&7)*2 + e.
    // The resource spans exactly a (empty for the rank-0 matmul, so every lane
    // reads zero); columns past the rank are clamped onto the last one, which
    // is harmless: they only meet rows of b past the rank, read as zero below.
    const int ak = tid >> 3;
    const int aj = (tid & 7) * 2;
    const __amdgpu_buffer_rsrc_t abuf = make_buffer(args.a, static_cast<uint32_t>(K * rank * 2));
    uint32_t aoff[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int64_t j = aj + e < rank ? aj + e : (rank > 0 ? rank - 1 : 0);
        aoff[e] = static_cast<uint32_t>((ak * rank + j) * 2);
    }

    uint4 xr[4];
    uint4 wr[4];
    uint16_t ar[2];

    auto load_global = [&](int64_t k0) {
        const uint32_t xk = static_cast<uint32_t>(k0 * 2);
#pragma unroll
        for (int i = 0; i < 4; ++i) xr[i] = buffer_load16(xbuf, xoff[i], xk);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            wr[r] = buffer_load16(wbuf, woff, static_cast<uint32_t>((k0 + r) * N * 2));
        }
        const uint32_t ak0 = static_cast<uint32_t>(k0 * rank * 2);
#pragma unroll
        for (int e = 0; e < 2; ++e) ar[e] = buffer_load2(abuf, aoff[e], ak0);
    };

    auto store_lds = [&](int stage) {
        uint8_t* base = lds + stage * kStage;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int id = i * kThreads + tid;
            *reinterpret_cast<uint4*>(base + lds_offset(id >> 3, id & 7)) = xr[i];
        }
        uint2 cols[8];
        transpose4x8(wr, cols);
        uint8_t* bt = base + kTileA;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            *reinterpret_cast<uint2*>(bt + lds_offset(wnb * 8 + j, wkq >> 1) + (wkq & 1) * 8) =
                cols[j];
        }
        uint8_t* at = base + kTileA + kTileB;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            *reinterpret_cast<uint16_t*>(at + lds_offset(aj + e, ak >> 3) + (ak & 7) * 2) = ar[e];
        }
    };

    f32x16_t acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
        }
    }
    f32x4_t xacc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) xacc[t][r] = 0.0f;
    }

    // One K-step of MFMAs from LDS stage `stage`.
    auto compute = [&](int stage) {
        const uint8_t* ta = lds + stage * kStage;
        const uint8_t* tb = ta + kTileA;
        const uint8_t* tat = tb + kTileB;
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int chunk = kk * 2 + (lane >> 5);
            bf16x8_t af[4];
            bf16x8_t bfr[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const bf16x8_t*>(
                    ta + lds_offset(wm * 128 + i * 32 + (lane & 31), chunk));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(
                    tb + lds_offset(wn * 64 + j * 32 + (lane & 31), chunk));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        // Adapter down-projection: rows wave*32 .. wave*32+31, 16 columns.
#pragma unroll
        for (int kk = 0; kk < kBK / 32; ++kk) {
            const int chunk = kk * 4 + (lane >> 4);
            const bf16x8_t bv =
                *reinterpret_cast<const bf16x8_t*>(tat + lds_offset(lane & 15, chunk));
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf16x8_t av = *reinterpret_cast<const bf16x8_t*>(
                    ta + lds_offset(wave * 32 + t * 16 + (lane & 15), chunk));
                xacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, xacc[t], 0, 0, 0);
            }
        }
    };

    const int64_t k_tiles = K / kBK;
    load_global(0);
    store_lds(0);
    __syncthreads();
    // Steady state: prefetch K-step kt + 1 into registers, compute step kt,
    // park the prefetched step in the other stage. The last step is peeled so
    // the loop body has a single path.
    for (int64_t kt = 0; kt + 1 < k_tiles; ++kt) {
        const int stage = static_cast<int>(kt & 1);
        load_global((kt + 1) * kBK);
        compute(stage);
        store_lds(stage ^ 1);
        __syncthreads();
    }
    compute(static_cast<int>((k_tiles - 1) & 1));
    __syncthreads();

    // ---- epilogue ----
    // xa (bf16) exchange tile [256][16] in the idle stage-0 buffer.
    uint16_t* xa_lds = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = wave * 32 + t * 16 + 4 * (lane >> 4) + r;
            const int col = lane & 15;
            const float v = xacc[t][r];
            xa_lds[row * 16 + col] = static_cast<uint16_t>(f32_to_bf16_bits(v));
            if (args.xa_out != nullptr && tn == 0 && col < rank && m0 + row < M) {
                args.xa_out[(m0 + row) * rank + col] = v;
            }
        }
    }
    __syncthreads();

    // Up-projection: acc += xa_bf16 @ bf16(scale * b), one K=16 MFMA per 32x32
    // tile straight into the base accumulators. Rounding scale * b to bf16 is
    // exact for power-of-two scales (alpha / r = 2 in the usual configurations)
    // and otherwise adds one bf16 rounding to the adapter term, which the
    // reference already rounds to bf16 three times.
    const float scale = args.scale;
    bf16x8_t xa_frag[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = wm * 128 + i * 32 + (lane & 31);
        xa_frag[i] = *reinterpret_cast<const bf16x8_t*>(xa_lds + row * 16 + (lane >> 5) * 8);
    }
    // b through a resource spanning exactly [rank, N]: rows q >= rank read as
    // zero (they meet the clamped adapter columns); a column past N reads
    // some other element of b but only feeds an output column that is never
    // stored.
    const __amdgpu_buffer_rsrc_t bbuf = make_buffer(args.b, static_cast<uint32_t>(rank * N * 2));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
        uint16_t vals[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t q = (lane >> 5) * 8 + e;
            const float bv =
                bf16_bits_to_f32(buffer_load2(bbuf, static_cast<uint32_t>((q * N + col) * 2), 0));
            vals[e] = static_cast<uint16_t>(f32_to_bf16_bits(scale * bv));
        }
        const bf16x8_t b_frag = __builtin_bit_cast(bf16x8_t, vals);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa_frag[i], b_frag, acc[i][j], 0, 0, 0);
        }
    }

    // Store: accumulator (row 8*(r/4) + 4*(lane/32) + r%4, column lane%32)
    // rounded to bf16.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int64_t col = n0 + wn * 64 + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M && col < N) {
                    args.y[row * N + col] = static_cast<uint16_t>(f32_to_bf16_bits(acc[i][j][r]));
                }
            }
        }
    }
}

}  // namespace

bool lora_fused_eligible(const void* x, const void* w, int64_t M, int64_t N, int64_t K,
                         int64_t rank) {
    // Buffer offsets are 32-bit: w must span < 4 GiB and a 256-row x tile too.
    const bool offsets_fit = K * N * 2 < (1LL << 32) &&
                             static_cast<int64_t>(kBM) * K * 2 < (1LL << 32) &&
                             K * rank * 2 < (1LL << 32) && rank * N * 2 + N * 2 < (1LL << 32);
    return K % kBK == 0 && K > 0 && N % 8 == 0 && rank <= 16 && host_aligned(x, 16) &&
           host_aligned(w, 16) && offsets_fit &&
           ceil_div<int64_t>(M, kBM) * ceil_div<int64_t>(N, kBN) < (1LL << 31);
}

cf_status launch_lora_fused(const void* x, const void* w, const void* a, const void* b, void* y,
                            float* xa_out, int64_t M, int64_t N, int64_t K, int64_t rank,
                            float scale, hipStream_t stream) {
    FusedArgs args;
    args.x = static_cast<const uint16_t*>(x);
    args.w = static_cast<const uint16_t*>(w);
    args.a = static_cast<const uint16_t*>(a);
    args.b = static_cast<const uint16_t*>(b);
    args.y = static_cast<uint16_t*>(y);
    args.xa_out = xa_out;
    args.M = M;
    args.N = N;
    args.K = K;
    args.rank = rank;
    args.scale = scale;
    args.tiles_m = static_cast<int>(ceil_div<int64_t>(M, kBM));
    args.tiles_n = static_cast<int>(ceil_div<int64_t>(N, kBN));
    const int grid = args.tiles_m * args.tiles_n;
    lora_fused_bf16_kernel<<<grid, kThreads, 0, stream>>>(args);
    return check_launch("launching the fused bf16 LoRA kernel", stream);
}

}  // namespace cf

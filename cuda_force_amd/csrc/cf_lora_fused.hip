// Fused LoRA linear on the bf16 MFMA units of gfx950:
//
//   y[M, N] = x[M, K] @ w[K, N] + scale * bf16(x @ a)[M, r] @ b[r, N]
//
// operator layout of the reference (cuda/include/cudaforge/lora_linear.cuh:26-31),
// even r <= 16, bf16 operands, fp32 accumulation, bf16 output.
//
// Shape of the kernel:
//   * 256x256 output tile per workgroup, 8 waves (two per SIMD), each owning a
//     64x128 sub-tile held as 8x4 v_mfma_f32_16x16x32_bf16 accumulators (128
//     fp32 per lane, accumulated in place in VGPRs; the file is compiled with
//     -amdgpu-mfma-vgpr-form). The whole product is computed transposed,
//     C^T = w^T x^T: w supplies the A operand, x the B operand, so each lane
//     ends up holding 4 consecutive output columns of one row.
//   * Operands travel HBM -> LDS by buffer loads with the LDS destination
//     (`buffer_load_dwordx4 ... lds`), issued by waves 0-3 only (one per
//     SIMD): no registers are spent on prefetch,
//     rows past M and columns past N arrive as zeros through the buffer range
//     check. K-step 32, four LDS stages, prefetch distance three: the loads for
//     step j + 3 are issued while step j + 1 is read into fragment registers
//     and step j is multiplied.
//   * x keeps its K-major layout in LDS and travels two K-steps per load
//     (whole 128-byte lines of each row, 16-byte chunks swizzled by the
//     row's low three bits) into a ring of two slots. w keeps its N-major layout
//     (512-byte rows, chunks swizzled by k bits 0, 1 and 3) and is
//     transposed on the way out of LDS by ds_read_b64_tr_b16, which hands
//     each lane four k values of one column. All operand reads are free of
//     bank conflicts.
//   * The adapter down-projection rides in the same loop: x^T fragments
//     already in registers meet a^T fragments (also transposed out of LDS) in
//     one extra MFMA per 16 rows; each wave covers 32 of its 64 rows, ~6%
//     extra MFMA work, and x is read from HBM once.
//   * Epilogue: x @ a (rounded to bf16, as the reference materialises it) is
//     exchanged through LDS, b is read transposed from an LDS copy loaded at
//     kernel start, scale * b is split into bf16 high and low parts, and two
//     v_mfma_f32_16x16x16_bf16 per 16x16 block accumulate the adapter term
//     into the base accumulators.
//     The tile is rounded to bf16, staged per wave in LDS and written as
//     whole 256-byte row pieces with non-temporal 16-byte stores (or kept in
//     fp32 and stored from registers, 16 bytes per lane, for the fp32-output
//     matmul).
//   * Workgroup ids are remapped so the tiles dispatched to one XCD (ids are
//     dealt round-robin over the 8 XCDs) form a band of 4 row-tiles sharing x
//     row-panels in that XCD's L2.
//   * With a workspace, column tile 0 of each row tile publishes its bf16
//     x @ a fragments (device-scope stores, then a flag set to a token of
//     the dispatch), and workgroups that start after the first round find
//     the flag set and skip the adapter MFMAs of their K-loop, copying the
//     fragments instead. The flag is read once; nothing waits on it, so a
//     tile that finds it unset forms x @ a itself, with the same result.
// The reference's fused kernel recomputes x @ a untiled in every block
// (cuda/src/lora_linear.cu:138-203).
#include "cf_lora_fused.hpp"
#include "cf_lds_dma.hpp"

#include <cmath>

#include <type_traits>

// Index of the current dispatch packet in its hardware queue: it grows with
// every packet on that queue (graph replays included).
extern "C" __device__ uint64_t cf_queue_dispatch_index() __asm("llvm.amdgcn.dispatch.id");

namespace cf {
namespace {

/// A value no other dispatch of this process writes: the queue's packet
/// index mixed with the queue's address (two queues repeat indices). Flags
/// set to it are never cleared; whatever an earlier call (or the
/// workspace's previous owner) left there reads as unset.
__device__ __forceinline__ uint64_t dispatch_token() {
    const uint64_t queue = reinterpret_cast<uint64_t>(__builtin_amdgcn_queue_ptr());
    return cf_queue_dispatch_index() ^ (queue * 0x9E3779B97F4A7C15ull);
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 32;
constexpr int kStages = 4;
constexpr int kThreads = 512;
constexpr int kMaxFusedRank = 16;
constexpr int kXPair = kBM * 2 * kBK * 2;               // 32 KiB: [256 m][64 k], two K-steps
constexpr int kXSlots = 2;
constexpr int kTileW = kBK * kBN * 2;                    // 16 KiB: [32 k][256 n]
constexpr int kTileA = kBK * kMaxFusedRank * 2;          // 1 KiB:  [32 k][16 j]
constexpr int kStage = kTileW + kTileA;
constexpr int kTileB = kMaxFusedRank * kBN * 2;          // 8 KiB:  [16 j][256 n]
constexpr int kXaBytes = (kBM / 16) * 64 * 8;            // 8 KiB: bf16 x @ a fragments
constexpr int kOffW = kXSlots * kXPair;
constexpr int kOffB = kOffW + kStages * kStage;
constexpr int kOffXa = kOffB + kTileB;
constexpr int kOffReuse = kOffXa + kXaBytes;             // one word: take the published x @ a
constexpr int kLdsBytes = kOffReuse + 16;                // 148 KiB + 16 B
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(kThreads / 64 * 64 * 256 <= kOffB, "bf16 output staging stays clear of b and x @ a");

// LDS bank behaviour these layouts are built for (measured on gfx950 with
// SQ_LDS_BANK_CONFLICT): a ds_read_b64_tr_b16 serves lanes 0-31 and 32-63
// in separate cycles of 256 bytes, so the 16-lane groups 0 and 1 (2 and 3)
// must hit different 128-byte halves of the banks. A ds_read_b128 serves
// two 8-lane octets per cycle, octet o together with o ^ 3 or with 7 - o
// (the measurements allow both); the x swizzle is conflict-free either way.

/// Chunk swizzle of the x tile (128-byte rows of 8 chunks, two K-steps):
/// row r keeps logical chunk c in physical chunk c ^ (r & 7).
__device__ __forceinline__ int x_swizzle(int row) { return row & 7; }

/// Chunk swizzle of the w tile (512-byte rows of 32 chunks): k rows 0-3 of
/// a transposed read land in four different 32-byte bank groups, and rows
/// 8 apart (the other 16-lane group of the same cycle) in the other half.
__device__ __forceinline__ int w_swizzle(int row) { return 2 * (row & 3) + 8 * ((row >> 3) & 1); }

/// Same for the b tile, whose transposed reads take rows 4 apart per group.
__device__ __forceinline__ int b_swizzle(int row) { return 2 * (row & 3) + 8 * ((row >> 2) & 1); }

/// Byte offset in the a tile ([32 k][16 j], 32-byte rows) of row `row`,
/// byte `byte`: rows 8-15 and 24-31 swap 128-byte halves so the two
/// 16-lane groups of a transposed read use different banks.
__device__ __forceinline__ int a_offset(int row, int byte) {
    return (row * 32 + byte) ^ (((row >> 3) & 1) << 7);
}

__device__ __forceinline__ s16x4_t lds_read_tr(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

__device__ __forceinline__ bf16x8_t concat(s16x4_t lo, s16x4_t hi) {
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

struct FusedArgs {
    const uint16_t* x;
    const uint16_t* w;
    const uint16_t* a;
    const uint16_t* b;
    uint16_t* y;
    float* y32;  // fp32 output (kOutF32) instead of y
    float* xa_out;
    int64_t M;
    int64_t N;
    int64_t K;        // row length of x (row stride) and rows of w
    int64_t k_steps;  // K-steps (kBK each) per workgroup: even, >= 2; split K
                      // (fp32 output only): slice blockIdx.y covers K-steps
                      // [blockIdx.y * k_steps, +k_steps)
    int64_t rank;
    float scale;
    int tiles_m;
    int tiles_n;
    // Sharing x @ a within a row tile (adapter kernel with a workspace;
    // null otherwise): column tile 0 of row tile tm publishes its bf16 x @ a
    // fragments (the kXaBytes the epilogue exchanges through LDS) at
    // xa_pub + tm * kXaBytes, then sets xa_flags[tm] to the dispatch token.
    // Workgroups with ids from reuse_from on (they start once a first
    // round of workgroups has left its CUs) look at their row tile's flag
    // once, at the start: if it is set they skip the adapter MFMAs of the
    // K-loop and copy the fragments instead, else they compute x @ a as
    // every tile does. Nothing ever waits for a flag.
    uint8_t* xa_pub;
    uint64_t* xa_flags;
    int reuse_from;
};

/// Operand fragments of one K-step: x (B operand) row block rb(i), k
/// 8 (lane/16) .. +7 for lane%16's row; a (A operand of x @ a) column
/// lane%16, same k.
struct XFrags {
    bf16x8_t x[4];
    bf16x8_t a;
};

/// Epilogue of a 256 x 256 tile, shared by both K-loop schedules: the
/// adapter up-projection (x @ a exchanged through LDS, then
/// scale * b @ bf16(x @ a) on the MFMA units into the base accumulators),
/// then the stores. acc[jb][i] of wave `wave` holds output rows
/// wm*64 + 16 ((i + 2 wn) & 3) + lane%16, columns wn*128 + 16 jb + 4 (lane/16) .. +3;
/// xacc[t] holds (x @ a) for row block 2 wn + t of the wave's 64 rows. Every
/// wave must have finished reading operands from LDS (the first barrier
/// below, or the one before the staged stores, orders the reuse of the
/// operand area). kSplitB false: scale * b is exact in bf16 (the host
/// passes it for a scale of 0 or +-2^k, k >= 0), so its low part is zero and
/// only the high pass runs.
template <bool kAdapter, bool kOutF32, bool kSplitB = true>
__device__ __forceinline__ void finish_tile(const FusedArgs& args, uint8_t* lds, f32x4_t (&acc)[8][4],
                                            const f32x4_t (&xacc)[2], int wave, int lane, int tm,
                                            int tn, int64_t m0, int64_t n0, bool reused,
                                            uint64_t token) {
    const int wm = wave >> 1;
    const int wn = wave & 1;
    const int g = lane >> 4;
    const int jl = lane & 15;
    const int64_t M = args.M;
    const int64_t N = args.N;
    const int64_t rank = args.rank;
    if (kAdapter) {
        // x @ a: lane holds (x @ a)[row wm*64 + 16 (2 wn + t) + lane%16][4 g .. 4 g + 3].
        uint2* xa_lds = reinterpret_cast<uint2*>(lds + kOffXa);
        const bool write_xa = args.xa_out != nullptr && tn == 0;
        // A tile that took the published fragments has them in place already.
        if (!reused) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int rb = wm * 4 + wn * 2 + t;
                // Columns past the rank are padding (a reads zero there); an
                // infinite x makes them inf * 0 = NaN, kept out of the product
                // with b's zero rows.
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = 4 * g + e < rank ? xacc[t][e] : 0.0f;
                uint2 packed;
                packed.x = f32x2_to_bf16x2_canon(v[0], v[1]);
                packed.y = f32x2_to_bf16x2_canon(v[2], v[3]);
                xa_lds[rb * 64 + lane] = packed;
                const int64_t row = m0 + rb * 16 + jl;
                if (write_xa && row < M) {
                    float* dst = args.xa_out + row * rank;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (4 * g + e < rank) dst[4 * g + e] = xacc[t][e];
                    }
                }
            }
        }
        __syncthreads();
        if (args.xa_flags != nullptr && tn == 0) {
            // Publish the fragments for the row tile's other column tiles:
            // one 16-byte device-scope store per thread, every wave waits
            // until its stores are acknowledged (visible to all CUs), then
            // thread 0 sets the flag to this dispatch's token.
            const int tid = wave * 64 + lane;
            const uint4 v = *reinterpret_cast<const uint4*>(lds + kOffXa + 16 * tid);
            const u32x4_t bits = {v.x, v.y, v.z, v.w};
            __builtin_amdgcn_raw_buffer_store_b128(
                bits, make_buffer(args.xa_pub + static_cast<int64_t>(tm) * kXaBytes, kXaBytes),
                static_cast<uint32_t>(16 * tid), 0, kCacheDeviceScope);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0) {
                __hip_atomic_store(args.xa_flags + tm, token, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }

        // acc += scale * (b^T-block @ bf16(x @ a)^T-block), K = 16. scale * b
        // is formed in fp32 and split into two bf16 parts, hi + lo, each
        // multiplied by the bf16 x @ a on the MFMA units into the base
        // accumulators: the adapter term carries about 2^-17 relative error
        // for any scale (a single bf16(scale * b) would carry 2^-9 whenever
        // the scale is not a power of two), and no extra registers are live.
        // b is read transposed: lane j of group g reads b row 4g + j/4,
        // columns 4(j%4) .. +3 of the block and receives column j's four
        // adapter rows 4g .. 4g + 3.
        const float scale = args.scale;
        s16x4_t xa_frag[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xa_frag[i] =
                __builtin_bit_cast(s16x4_t, xa_lds[(wm * 4 + ((i + 2 * wn) & 3)) * 64 + lane]);
        }
        const uint8_t* tb = lds + kOffB;
        // Two passes (high parts, then low parts) keep one b fragment live.
#pragma unroll
        for (int part = 0; part < (kSplitB ? 2 : 1); ++part) {
            if (part == 1) {
                // An infinite x @ a meets only the high part of scale * b:
                // inf * lo would add NaN (lo = 0) or an infinity of the
                // other sign, where the fp32 product inf * b is +-inf.
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if ((xa_frag[i][e] & 0x7FFF) == 0x7F80) xa_frag[i][e] = 0;
                    }
                }
            }
#pragma unroll
            for (int jb = 0; jb < 8; ++jb) {
                const int row = 4 * g + (jl >> 2);
                const int chunk = 2 * (wn * 8 + jb) + ((jl & 3) >> 1);
                const s16x4_t raw = lds_read_tr(
                    tb, row * (kBN * 2) + ((chunk ^ b_swizzle(row)) << 4) + (jl & 1) * 8);
                s16x4_t bfrag;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = scale * bf16_bits_to_f32(static_cast<uint16_t>(raw[e]));
                    const uint32_t hi = f32_to_bf16_bits(v);
                    bfrag[e] = static_cast<short>(
                        part == 0 ? hi
                                  : f32_to_bf16_bits(v - bf16_bits_to_f32(static_cast<uint16_t>(hi))));
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[jb][i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(bfrag, xa_frag[i],
                                                                           acc[jb][i], 0, 0, 0);
                }
            }
        }
    }

    // Store: acc[jb][i] lane holds y[row wm*64 + 16 rb(i) + lane%16]
    // [columns wn*128 + 16 jb + 4 g .. +3]; N is a multiple of 8, so a
    // four- or eight-column group is entirely inside or outside the matrix.
    if constexpr (!kOutF32) {
        // bf16 output goes through LDS, so that each store instruction
        // writes whole rows (16 lanes x 16 bytes = 256 contiguous bytes of a
        // row, 4 rows per instruction) instead of 32-byte pieces of 16 rows.
        // Each wave stages its own 64x128 sub-tile (16 KiB, rows of 256
        // bytes) in the operand area, which every wave has left: the
        // barrier after the x @ a exchange, or the one below, orders that.
        // Chunk c (16 bytes) of row r sits at chunk c ^ (r & 15): the 8-byte
        // writes of a half-wave (16 rows, one chunk each) and the 16-byte
        // reads (whole rows) both spread over all banks.
        if constexpr (!kAdapter) __syncthreads();
        uint8_t* stage = lds + wave * (64 * 256);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = 16 * ((i + 2 * wn) & 3) + jl;
#pragma unroll
            for (int jb = 0; jb < 8; ++jb) {
                const int chunk = 2 * jb + (g >> 1);
                uint2 packed;
                packed.x = f32x2_to_bf16x2_canon(acc[jb][i][0], acc[jb][i][1]);
                packed.y = f32x2_to_bf16x2_canon(acc[jb][i][2], acc[jb][i][3]);
                *reinterpret_cast<uint2*>(stage + row * 256 + ((chunk ^ (row & 15)) << 4) +
                                          (g & 1) * 8) = packed;
            }
        }
        // Only this wave reads what it wrote: LDS operations of a wave
        // complete in order; the fence keeps the compiler from moving the
        // reads above the writes.
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const int c = lane & 15;
        const int64_t col = n0 + wn * 128 + 8 * c;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int row = 4 * s + (lane >> 4);
            const uint4 v =
                *reinterpret_cast<const uint4*>(stage + row * 256 + ((c ^ (row & 15)) << 4));
            const int64_t grow = m0 + wm * 64 + row;
            if (grow < M && col < N) store_stream16(args.y + grow * N + col, v);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t row = m0 + wm * 64 + 16 * ((i + 2 * wn) & 3) + jl;
        if (row >= M) continue;
        uint16_t* yrow = args.y + row * N;
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
            const int64_t col = n0 + wn * 128 + 16 * jb + 4 * g;
            if (kOutF32 && col < N) {
                // Split K: slice blockIdx.y of the K range writes its own
                // partial product.
                *reinterpret_cast<f32x4_t*>(args.y32 + static_cast<int64_t>(blockIdx.y) * M * N +
                                            row * N + col) = acc[jb][i];
            } else if (col < N) {
                uint2 packed;
                packed.x = f32x2_to_bf16x2_canon(acc[jb][i][0], acc[jb][i][1]);
                packed.y = f32x2_to_bf16x2_canon(acc[jb][i][2], acc[jb][i][3]);
                *reinterpret_cast<uint2*>(yrow + col) = packed;
            }
        }
    }
}

template <bool kAdapter, bool kOutF32, bool kSplitB = true>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void lora_fused_bf16_kernel(FusedArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    // Wave-uniform by construction; readfirstlane tells the compiler so that
    // everything derived from it (LDS destinations of the DMA) stays scalar.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1;  // 0..3: 64-row quarter of the tile
    const int wn = wave & 1;   // 0..1: 128-column half of the tile
    int tm;
    int tn;
    tile_of(static_cast<int>(blockIdx.x), args.tiles_m, args.tiles_n, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * kBM;
    const int64_t n0 = static_cast<int64_t>(tn) * kBN;
    const int64_t M = args.M;
    const int64_t N = args.N;
    const int64_t K = args.K;
    const int64_t k_first = static_cast<int64_t>(blockIdx.y) * args.k_steps * kBK;
    const int64_t rank = args.rank;

    // ---- HBM -> LDS roles (each load instruction fills 1 KiB of LDS, lane l
    // at byte 16 l; the global side is permuted to realise the swizzles) ----
    // Only waves 0-3 (one per SIMD) issue DMA, each for its own share and for
    // wave + 4's: a wave that stalls on a full address queue then always has
    // a SIMD-mate that keeps issuing MFMAs. `vw` below is the wave whose
    // share a piece fills.
    // x travels two K-steps at a time, as whole 128-byte lines of each row
    // (a 64-byte piece per K-step would make every line two L1 requests):
    // share vw covers rows 32 vw .. +31, 8 rows per load; lane -> row
    // 32 vw + 8 i + l/8, physical chunk l%8.
    const int64_t rows_here = M - m0 < kBM ? M - m0 : kBM;
    const i32x4_t xbuf = raw_buffer_words(args.x + m0 * K, static_cast<uint32_t>(rows_here * K * 2));
    uint32_t x_dma[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int vw = (wave & 3) + 4 * (i >> 2);
        const int row = 32 * vw + 8 * (i & 3) + (lane >> 3);
        const int chunk = (lane & 7) ^ x_swizzle(row);
        x_dma[i] = static_cast<uint32_t>((row * K + chunk * 8) * 2);
    }
    // w: share vw covers k-row pairs q = 2 vw + i; lane -> row 2q + l/32,
    // physical chunk l%32. Columns past N read as zero.
    const i32x4_t wbuf = raw_buffer_words(args.w, static_cast<uint32_t>(K * N * 2));
    uint32_t w_dma[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int vw = (wave & 3) + 4 * (i >> 1);
        const int row = 2 * (vw * 2 + (i & 1)) + (lane >> 5);
        const int64_t col = n0 + 8 * ((lane & 31) ^ w_swizzle(row));
        w_dma[i] = col < N ? static_cast<uint32_t>((row * N + col) * 2) : kOutOfRange;
    }
    // a: 4-byte pieces (two adapter columns; the rank is even); issuing wave
    // w fills bytes 256 w + 4 l, i.e. rows 8 w .. +7 in the a_offset layout
    // (an involution within the 256 bytes). Columns past the rank read as
    // zero.
    const i32x4_t abuf = raw_buffer_words(args.a, static_cast<uint32_t>(kAdapter ? K * rank * 2 : 0));
    uint32_t a_dma = kOutOfRange;
    if (kAdapter) {
        const int phys = 256 * (wave & 3) + 4 * lane;
        const int logical = phys ^ (((phys >> 8) & 1) << 7);  // rows 8-15, 24-31: bit 3 of row
        const int row = logical >> 5;
        const int col = (logical & 31) >> 1;
        a_dma = col < rank ? static_cast<uint32_t>((row * rank + col) * 2) : kOutOfRange;
    }

    // LDS byte address of the tile storage (the DMA takes it in M0).
    const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8_t*)lds));
    // DMA instructions of an issuing wave: pieces 0-3 of K-step kt are w
    // (shares wave and wave + 4), piece 4 is a (adapter only), into the stage
    // ring; pieces 0-7 of x pair p (K-steps 2p, 2p + 1) go into x slot p % 2.
    // The K-loop spreads them over a step's MFMAs rather than issuing them in
    // one burst after the barrier.
    auto issue_w = [&](int64_t kt, int piece) {
        const uint32_t stage = lds_addr + kOffW + static_cast<uint32_t>(kt % kStages) * kStage;
        const int64_t k0 = k_first + kt * kBK;
        if (piece < 4) {
            const int vw = (wave & 3) + 4 * (piece >> 1);
            dma16_m0(wbuf, stage + (vw * 2 + (piece & 1)) * 1024, w_dma[piece],
                  static_cast<uint32_t>(k0 * N * 2));
        } else if (kAdapter) {
            dma4_m0(abuf, stage + kTileW + (wave & 3) * 256, a_dma,
                 static_cast<uint32_t>(k0 * rank * 2));
        }
    };
    auto issue_x = [&](int64_t pair, int piece) {
        const uint32_t slot = lds_addr + static_cast<uint32_t>(pair % kXSlots) * kXPair;
        const int vw = (wave & 3) + 4 * (piece >> 2);
        dma16_m0(xbuf, slot + vw * 4096 + (piece & 3) * 1024, x_dma[piece],
              static_cast<uint32_t>(k_first * 2 + pair * 4 * kBK));
    };
    constexpr int kWLoads = kAdapter ? 5 : 4;  // w (+ a) DMA per K-step per issuing wave
    constexpr int kXLoads = 8;                 // x DMA per pair of K-steps per issuing wave

    // ---- LDS -> register fragment roles ----
    // x (B operand): fragment i holds row block rb(i) = (i + 2 wn) % 4 of the
    // wave's 64 rows (row wm*64 + 16 rb + lane%16, chunk lane/16), so that
    // the x @ a share of either wave is always fragments 0 and 1. The
    // swizzle only depends on row bit 2, which is lane bit 2.
    // Row wm*64 + 16 rb + lane%16 has row & 7 == lane & 7; the odd K-step of
    // a pair is the upper four chunks (byte offset ^ 64).
    const int x_rd = (wm * 64 + (lane & 15)) * (4 * kBK) + (((lane >> 4) ^ x_swizzle(lane)) << 4);
    // w (A operand, transposed read): group g = lane/16 takes k rows 8g .. 8g+3
    // (then +4); lane j of the group reads row 8g + j/4, columns 4(j%4) .. +3
    // of the 16-column block; the read returns column j's four k values.
    const int g = lane >> 4;
    const int jl = lane & 15;
    int w_rd[8];
#pragma unroll
    for (int jb = 0; jb < 8; ++jb) {
        const int row = 8 * g + (jl >> 2);
        const int chunk = 2 * (wn * 8 + jb) + ((jl & 3) >> 1);
        w_rd[jb] = row * (kBN * 2) + ((chunk ^ w_swizzle(row)) << 4) + (jl & 1) * 8;
    }
    const int a_rd0 = a_offset(8 * g + (jl >> 2), (jl & 3) * 8);
    const int a_rd1 = a_offset(8 * g + 4 + (jl >> 2), (jl & 3) * 8);

    // `xa` (true/false type): this K-loop forms x @ a (the a fragments are
    // read, the adapter MFMAs issued, a is copied into LDS).
    auto read_x = [&](XFrags& f, int64_t kt, auto xa) {
        const uint8_t* sx = lds + static_cast<int>((kt >> 1) % kXSlots) * kXPair;
        const int x_off = x_rd ^ (static_cast<int>(kt & 1) << 6);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rb = (i + 2 * wn) & 3;
            f.x[i] = *reinterpret_cast<const bf16x8_t*>(sx + x_off + rb * 2048);
        }
        if constexpr (kAdapter && decltype(xa)::value) {
            const uint8_t* sa = lds + kOffW + static_cast<int>(kt % kStages) * kStage + kTileW;
            f.a = concat(lds_read_tr(sa, a_rd0), lds_read_tr(sa, a_rd1));
        }
    };
    // w fragment jb (A operand): column wn*128 + 16 jb + lane%16, same k.
    auto read_w = [&](int64_t kt, int jb) {
        const uint8_t* sw = lds + kOffW + static_cast<int>(kt % kStages) * kStage;
        return concat(lds_read_tr(sw, w_rd[jb]), lds_read_tr(sw, w_rd[jb] + 4 * kBN * 2));
    };

    f32x4_t acc[8][4];  // [w column block jb][x fragment i]
#pragma unroll
    for (int jb = 0; jb < 8; ++jb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[jb][i] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    f32x4_t xacc[2];  // (x @ a)^T for row blocks 2 wn + t of this wave's 4
#pragma unroll
    for (int t = 0; t < 2; ++t) xacc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // The w fragments live in one register set: fragment jb of the next
    // K-step is read into it as soon as the 4 MFMAs of this step that use it
    // have issued. x is double-buffered (its fragments are used until the
    // end of the step).
    bf16x8_t wf[8];
    // On step kt the DMA goes out for K-step kt + 3 (w, a) and, on odd steps,
    // for x pair (kt + 3) / 2, whose slot the barrier of step kt has freed.
    auto multiply = [&](const XFrags& f, int64_t next_kt, auto read_next, auto issue, auto odd,
                        auto issuer, auto xa) {
        constexpr int kW = kAdapter && decltype(xa)::value ? kWLoads : 4;
        if constexpr (kAdapter && decltype(xa)::value) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                xacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a, f.x[t], xacc[t], 0, 0, 0);
            }
        }
#pragma unroll
        for (int jb = 0; jb < 8; ++jb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc[jb][i] =
                    __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[jb], f.x[i], acc[jb][i], 0, 0, 0);
            }
            if constexpr (decltype(read_next)::value) wf[jb] = read_w(next_kt, jb);
            if constexpr (decltype(issue)::value && decltype(issuer)::value) {
                if constexpr (decltype(odd)::value) issue_x((next_kt + 2) >> 1, jb);
                if (jb < kW) issue_w(next_kt + 2, jb);
            }
            // Left alone, the scheduler sinks each next-step w read to a few
            // MFMAs before its use; a scheduling barrier after every second
            // fragment group keeps the reads a group ahead. Only the adapter
            // kernel: the plain one would need more than 256 VGPRs.
            if (kAdapter && (jb & 1) == 1) __builtin_amdgcn_sched_barrier(0);
        }
    };

    // ---- prologue: b for the epilogue, then K-steps 0..2 in flight ----
    if (kAdapter) {
        const i32x4_t bbuf = raw_buffer_words(args.b, static_cast<uint32_t>(rank * N * 2));
        const int row = 2 * wave + (lane >> 5);
        const int64_t col = n0 + 8 * ((lane & 31) ^ b_swizzle(row));
        const uint32_t off =
            row < rank && col < N ? static_cast<uint32_t>((row * N + col) * 2) : kOutOfRange;
        dma16_m0(bbuf, lds_addr + kOffB + wave * 1024, off, 0);
    }
    // Sharing x @ a: whether this tile may take its row tile's published
    // fragments (decided once, by wave 4, before the first barrier).
    const bool may_reuse = kAdapter && args.xa_flags != nullptr && tn != 0 &&
                           static_cast<int>(blockIdx.x) >= args.reuse_from;
    const uint64_t token = kAdapter && args.xa_flags != nullptr ? dispatch_token() : 0;

    // The K-loop, instantiated for issuing (waves 0-3) and non-issuing waves;
    // the latter wait for nothing but the barriers (their vmcnt waits find
    // no DMA of their own in flight, or only the published fragments below).
    // Returns whether the tile took the published x @ a.
    auto run = [&](auto issuer) -> bool {
    const int64_t k_tiles = args.k_steps;  // even, >= 2
    auto issue_w_all = [&](int64_t kt) {
#pragma unroll
        for (int piece = 0; piece < kWLoads; ++piece) issue_w(kt, piece);
    };
    auto issue_x_all = [&](int64_t pair) {
#pragma unroll
        for (int piece = 0; piece < kXLoads; ++piece) issue_x(pair, piece);
    };
    // Issue order as if steps -2 and -1 had run: x pair 0, w 0, w 1 | x pair 1, w 2.
    if constexpr (decltype(issuer)::value) {
        issue_x_all(0);
        issue_w_all(0);
        issue_w_all(1);
        if (k_tiles > 2) {
            issue_x_all(1);
            issue_w_all(2);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kWLoads + kXLoads));
        } else {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWLoads));
        }
    } else {
        // One device-scope read of the flag, while waves 0-3 wait for the
        // first K-step; the answer goes to LDS before the barrier.
        if (may_reuse && wave == 4) {
            const uint64_t seen =
                __hip_atomic_load(args.xa_flags + tm, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0) *reinterpret_cast<uint32_t*>(lds + kOffReuse) = seen == token ? 1u : 0u;
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(63) & ~(15 << 8));  // lgkmcnt(0)
        }
    }
    bare_barrier();  // step 0 in LDS
    const bool reuse =
        may_reuse && __builtin_amdgcn_readfirstlane(*reinterpret_cast<const uint32_t*>(lds + kOffReuse)) != 0;

    using yes = std::true_type;
    using no = std::false_type;
    auto loop = [&](auto xa) {
    // w (+ a) DMA per K-step of this loop (the prologue above sent a for
    // K-steps 0-2 either way; without x @ a they are not read, and the
    // waits below only become more conservative for the first steps).
    constexpr int kW = kAdapter && decltype(xa)::value ? kWLoads : 4;
    XFrags f0;
    XFrags f1;
    read_x(f0, 0, xa);
#pragma unroll
    for (int jb = 0; jb < 8; ++jb) wf[jb] = read_w(0, jb);

    // Step kt: K-step kt + 1 must be in LDS (wait for this wave's loads,
    // then the barrier for everyone's), the loads for kt + 3 reuse the stage
    // of kt - 1 (read during step kt - 2, consumed in step kt - 1, so every
    // wave is past it once it is at this barrier), step kt + 1 is read into
    // registers while step kt is multiplied. x pair p goes out on step
    // 2p - 3 into the slot pair p - 2 left (its last K-step, 2p - 3, was read
    // during step 2p - 4) and is first read on step 2p - 1. Those reads of
    // K-step 2p - 3 are only consumed in step 2p - 3 itself, after the
    // barrier the overwriting DMA follows, so before the barrier of an odd
    // step every wave also drains its LDS reads (lgkmcnt 0): the slot is
    // then free by construction rather than by where the compiler happens
    // to place its own waits. DMA completes in issue order, so the wait
    // lets exactly the previous step's loads stay in flight: w (+ a) after
    // an even step, w (+ a) and an x pair after an odd one. The last four
    // steps are peeled so the loop body has no branches.
    // Steps with f0 as the current fragments are even, with f1 odd.
    auto step = [&](int64_t kt, XFrags& cur, XFrags& nxt, auto issue, auto wait_all, auto read,
                    auto odd) {
        if constexpr (decltype(read)::value) {
            if constexpr (decltype(wait_all)::value) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            } else if constexpr (decltype(odd)::value) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(kW) & ~(15 << 8));  // and lgkmcnt(0)
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(kW + kXLoads));
            }
            bare_barrier();
            read_x(nxt, kt + 1, xa);
        }
        multiply(cur, kt + 1, read, issue, odd, issuer, xa);
    };
    int64_t kt = 0;
    for (; kt + 4 < k_tiles; kt += 2) {
        step(kt, f0, f1, yes{}, no{}, yes{}, no{});
        step(kt + 1, f1, f0, yes{}, no{}, yes{}, yes{});
    }
    if (k_tiles >= 4) {
        step(kt, f0, f1, yes{}, no{}, yes{}, no{});
        step(kt + 1, f1, f0, no{}, no{}, yes{}, yes{});
        kt += 2;
    }
    step(kt, f0, f1, no{}, yes{}, yes{}, no{});
    step(kt + 1, f1, f0, no{}, no{}, no{}, yes{});
    };
    if (kAdapter && reuse) {
        // Waves 4-7 copy the published fragments (8 KiB) into the x @ a
        // area, at device scope: they were written by another workgroup,
        // possibly behind another XCD's L2, and were complete before the
        // flag was set. Nothing reads the area before the epilogue; the
        // last K-steps' vmcnt(0) and barrier order the copy before it.
        if constexpr (!decltype(issuer)::value) {
            const i32x4_t pbuf = raw_buffer_words(args.xa_pub + static_cast<int64_t>(tm) * kXaBytes,
                                                  static_cast<uint32_t>(kXaBytes));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int piece = 2 * (wave - 4) + i;
                dma16_device_m0(pbuf, lds_addr + kOffXa + piece * 1024, static_cast<uint32_t>(16 * lane),
                                static_cast<uint32_t>(piece * 1024));
            }
        }
        loop(no{});
    } else {
        loop(yes{});
    }
    return reuse;
    };
    const bool reused = wave < 4 ? run(std::true_type{}) : run(std::false_type{});

    finish_tile<kAdapter, kOutF32, kSplitB>(args, lds, acc, xacc, wave, lane, tm, tn, m0, n0, reused,
                                            token);
}

}  // namespace

bool lora_fused_eligible(const void* x, const void* w, const void* a, const void* b, int64_t M,
                         int64_t N, int64_t K, int64_t rank) {
    // Buffer offsets are 32-bit: w must span < 4 GiB, a 256-row x tile too.
    const bool offsets_fit = K * N * 2 < (1LL << 31) && static_cast<int64_t>(kBM) * K * 2 < (1LL << 31) &&
                             K * rank * 2 < (1LL << 31) && rank * N * 2 < (1LL << 31);
    const bool adapter_ok =
        rank == 0 || (rank <= kMaxFusedRank && rank % 2 == 0 && host_aligned(a, 4) &&
                      host_aligned(b, 16));
    return K % (2 * kBK) == 0 && K > 0 && N % 8 == 0 && adapter_ok && host_aligned(x, 16) &&
           host_aligned(w, 16) && offsets_fit &&
           ceil_div<int64_t>(M, kBM) * ceil_div<int64_t>(N, kBN) < (1LL << 31);
}

size_t lora_fused_workspace_bytes(int64_t M, int64_t rank) {
    if (M <= 0 || rank <= 0) return 0;
    const int64_t tiles_m = ceil_div<int64_t>(M, kBM);
    return static_cast<size_t>(ceil_div<int64_t>(tiles_m * 8, 256) * 256 + tiles_m * kXaBytes);
}

cf_status launch_lora_fused(const void* x, const void* w, const void* a, const void* b, void* y,
                            float* xa_out, int64_t M, int64_t N, int64_t K, int64_t rank,
                            float scale, void* workspace, hipStream_t stream) {
    FusedArgs args;
    args.x = static_cast<const uint16_t*>(x);
    args.w = static_cast<const uint16_t*>(w);
    args.a = static_cast<const uint16_t*>(a);
    args.b = static_cast<const uint16_t*>(b);
    args.y = static_cast<uint16_t*>(y);
    args.y32 = nullptr;
    args.xa_out = xa_out;
    args.M = M;
    args.N = N;
    args.K = K;
    args.k_steps = K / kBK;
    args.rank = rank;
    args.scale = scale;
    args.tiles_m = static_cast<int>(ceil_div<int64_t>(M, kBM));
    args.tiles_n = static_cast<int>(ceil_div<int64_t>(N, kBN));
    const int grid = args.tiles_m * args.tiles_n;
    // One workgroup fits a CU (148 KiB of LDS), so workgroups from id
    // cu_count() on start as the first ones leave; by then the first column
    // tile of their row tile (dealt to its XCD ahead of the row tile's other
    // column tiles) has usually published x @ a.
    args.xa_pub = nullptr;
    args.xa_flags = nullptr;
    args.reuse_from = grid;
    if (workspace != nullptr && rank > 0) {
        args.xa_flags = static_cast<uint64_t*>(workspace);
        args.xa_pub = static_cast<uint8_t*>(workspace) + ceil_div<int64_t>(args.tiles_m * 8, 256) * 256;
        args.reuse_from = cu_count();
    }
    // scale * b is exact in bf16 for every bf16 b when the scale is 0 or
    // +-2^k with k >= 0 (the exponent only moves up; an overflow gives the
    // infinity the fp32 product has): the epilogue then skips the pass over
    // the low parts, which would add zeros (config 3's scale of 2: 213.4 ->
    // 211.7 and 219.3 -> 218.7 us in two same-process A/Bs, within their
    // noise).
    int exponent = 0;
    const float mantissa = std::frexp(std::fabs(scale), &exponent);
    const bool exact_b = scale == 0.0f || (mantissa == 0.5f && exponent >= 1);
    if (rank > 0 && exact_b) {
        launch(lora_fused_bf16_kernel<true, false, false>, dim3(grid), dim3(kThreads), 0, stream, args);
    } else if (rank > 0) {
        launch(lora_fused_bf16_kernel<true, false>, dim3(grid), dim3(kThreads), 0, stream, args);
    } else {
        launch(lora_fused_bf16_kernel<false, false>, dim3(grid), dim3(kThreads), 0, stream, args);
    }
    return check_launch("launching the fused bf16 LoRA kernel", stream);
}

cf_status launch_matmul_bf16_f32out(const void* x, const void* w, float* y, int64_t M, int64_t N,
                                    int64_t K, int splits, hipStream_t stream) {
    CF_REQUIRE(splits >= 1 && K % (splits * 2 * kBK) == 0,
               "bf16 MFMA matmul: K = %lld does not split %d ways", static_cast<long long>(K), splits);
    FusedArgs args{};
    args.x = static_cast<const uint16_t*>(x);
    args.w = static_cast<const uint16_t*>(w);
    args.y32 = y;
    args.M = M;
    args.N = N;
    args.K = K;
    args.k_steps = K / kBK / splits;
    args.tiles_m = static_cast<int>(ceil_div<int64_t>(M, kBM));
    args.tiles_n = static_cast<int>(ceil_div<int64_t>(N, kBN));
    const int grid = args.tiles_m * args.tiles_n;
    launch(lora_fused_bf16_kernel<false, true>, dim3(grid, splits), dim3(kThreads), 0, stream, args);
    return check_launch("launching the bf16 MFMA matmul (fp32 output)", stream);
}

}  // namespace cf

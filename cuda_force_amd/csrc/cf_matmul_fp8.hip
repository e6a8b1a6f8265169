// fp8 (OCP e4m3fn) matmul on the fp8 MFMA units of gfx950:
//
//   y[M, N] = bf16(scale * (x[M, K] @ w[K, N]))
//
// x and w row-major fp8 codes (the operator layout of the LoRA linear and of
// the matmul the reference demonstrates tensor cores with,
// cuda/include/cudaforge/tensor_core_matmul.cuh:40-41), or w given K-major as
// w_t[N, K] (row-major; the weight layout of a torch Linear, y = x w_t^T, and
// the one fp8 GEMM libraries take), fp32 accumulation,
// one per-tensor scale (the product of the two operands' dequantisation
// scales) applied in the epilogue, bf16 output. The reference has no fp8
// path; this is the fp8 half of a bf16/fp8 MFMA matmul replacing its TF32
// demonstration.
//
// Shape of the kernel (the pipeline of the bf16 kernel in cf_lora_fused.hip,
// with operands of one byte):
//   * 256x256 output tile per workgroup, 8 waves (two per SIMD), each owning a
//     64x128 sub-tile held as 2x4 v_mfma_scale_f32_32x32x64_f8f6f4
//     accumulators (128 fp32 per lane). The MFMA's block scales are fixed at
//     the E8M0 code 127 (2^0), so it is a plain fp8 product. The product is
//     computed transposed, y^T = w^T x^T: w supplies the A operand, x the B
//     operand, so each lane holds runs of 4 consecutive output columns of
//     one row.
//   * K-step 64 (one MFMA deep). x travels two K-steps per buffer load with
//     the LDS destination, as whole 128-byte lines of each row, into a ring
//     of two slots; w ([64 k][256 n], 256-byte rows) into a ring of four
//     stages, prefetch distance three. Only waves 0-3 issue the DMA.
//   * B fragments (x): lane l reads 32 consecutive k bytes of row l % 32 as
//     two ds_read_b128. A fragments (w): 32 consecutive k values of column
//     l % 32 from an N-major tile, transposed on the way out of LDS by four
//     ds_read_b64_tr_b8 (each hands a lane 8 k values of one column). Both
//     tiles are swizzled so every read is free of bank conflicts.
//   * K-major w (kWT): w_t rows are K-contiguous like x rows, so w travels
//     and is read exactly as x is (128-byte row lines in a ring of two
//     two-K-step slots, two ds_read_b128 per fragment): half the LDS read
//     instructions of the transposed form, the same LDS footprint.
//   * Epilogue: scale, round to bf16, staged per wave in LDS and stored as
//     whole 256-byte row pieces.
//   * Workgroup ids are remapped so that the tiles of one XCD share x
//     row-panels in its L2 (tile_of).
//
// Shapes: any M; K a positive multiple of 128; N a positive multiple of 16;
// x, w and y 16-byte aligned; 32-bit buffer offsets over all of w (w[K, N])
// or over one 256-row panel of x and of w_t.
#include "cf_common.hpp"
#include "cf_lds_dma.hpp"

#include <type_traits>

namespace cf {
namespace {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x4v_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kBM = 256;
constexpr int kBN = 256;
constexpr int kBK = 64;                       // k values (bytes) per K-step
constexpr int kStages = 4;
constexpr int kThreads = 512;
constexpr int kXPair = kBM * 2 * kBK;         // 32 KiB: [256 m][128 k], two K-steps
constexpr int kXSlots = 2;
constexpr int kTileW = kBK * kBN;             // 16 KiB: [64 k][256 n]
constexpr int kOffW = kXSlots * kXPair;
constexpr int kLdsBytes = kOffW + kStages * kTileW;  // 128 KiB
static_assert(kLdsBytes <= 160 * 1024, "LDS budget of one gfx950 workgroup");
static_assert(kStages * kTileW == kXSlots * kXPair, "w_t slots take the place of the w stages");
static_assert(kThreads / 64 * 64 * 256 <= kLdsBytes, "output staging fits the operand area");

constexpr int kUnitScale = 127;  // E8M0 code of 2^0

// Bank behaviour (gfx950, 64 banks of 4 bytes): a 64-bit LDS read serves
// lanes 0-31 and 32-63 in separate 256-byte cycles; a ds_read_b128 serves
// two 8-lane octets per cycle, octet o together with o ^ 3 or with 7 - o.

/// Chunk swizzle of the x tile (128-byte rows of eight 16-byte chunks, two
/// K-steps). A B-fragment read has octet o on rows 8 (o % 4) .. +7, so the
/// octets served together (rows 0-7 with 24-31, 8-15 with 16-23) must hit
/// different 128-byte halves: bit 3 of the row flips the chunk's low bit.
__device__ __forceinline__ int x_swizzle(int row) { return (row & 7) ^ ((row >> 3) & 1); }

/// Chunk swizzle of the w tile (256-byte rows of sixteen chunks). A
/// transposed read takes eight consecutive k rows of one 32-byte column pair
/// in each cycle; moving the pair by k mod 8 puts them in eight different
/// 32-byte bank groups.
__device__ __forceinline__ int w_swizzle(int row) { return 2 * (row & 7); }

__device__ __forceinline__ i32x2_t lds_read_tr8(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        (lds_i32x2_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

struct Fp8Args {
    const uint8_t* x;
    const uint8_t* w;
    uint16_t* y;
    int64_t M;
    int64_t N;
    int64_t K;
    float scale;
    int tiles_m;
    int tiles_n;
};

template <bool kWT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void matmul_fp8_kernel(Fp8Args args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
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

    // ---- HBM -> LDS roles (each load fills 1 KiB of LDS, lane l at byte
    // 16 l; the global side is permuted to realise the swizzles). Waves 0-3
    // issue their own share and that of wave + 4 (`vw`). ----
    // x: share vw = rows 32 vw .. +31, 8 rows per load; lane -> row
    // 32 vw + 8 i + l/8, physical chunk l % 8. Rows past M read as zero.
    const int64_t rows_here = M - m0 < kBM ? M - m0 : kBM;
    const i32x4_t xbuf = uniform(raw_buffer_words(args.x + m0 * K, static_cast<uint32_t>(rows_here * K)));
    uint32_t x_dma[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int vw = (wave & 3) + 4 * (i >> 2);
        const int row = 32 * vw + 8 * (i & 3) + (lane >> 3);
        const int chunk = (lane & 7) ^ x_swizzle(row);
        x_dma[i] = static_cast<uint32_t>(row * K + chunk * 16);
    }
    // w[K, N]: share vw = k-row quads q = 2 vw + i % 2; lane -> row 4 q + l/16,
    // physical chunk l % 16. Columns past N read as zero.
    // w_t[N, K]: the 256 rows n0 .. +255 of the tile, mapped exactly as x's
    // rows (the same offsets, x_dma, in its own buffer). Rows past N read as
    // zero.
    const int64_t cols_here = N - n0 < kBN ? N - n0 : kBN;
    const i32x4_t wbuf = kWT ? uniform(raw_buffer_words(args.w + n0 * K, static_cast<uint32_t>(cols_here * K)))
                             : uniform(raw_buffer_words(args.w, static_cast<uint32_t>(K * N)));
    uint32_t w_dma[4];
    if constexpr (!kWT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vw = (wave & 3) + 4 * (i >> 1);
            const int row = 4 * (vw * 2 + (i & 1)) + (lane >> 4);
            const int64_t col = n0 + 16 * ((lane & 15) ^ w_swizzle(row));
            w_dma[i] = col < N ? static_cast<uint32_t>(row * N + col) : kOutOfRange;
        }
    }

    const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8_t*)lds));
    // issue_w takes a K-step for w[K, N], a pair of K-steps for w_t.
    auto issue_w = [&](int64_t t, int piece) {
        if constexpr (kWT) {
            const uint32_t slot = lds_addr + kOffW + static_cast<uint32_t>(t % kXSlots) * kXPair;
            const int vw = (wave & 3) + 4 * (piece >> 2);
            dma16_m0(wbuf, slot + vw * 4096 + (piece & 3) * 1024, x_dma[piece],
                  static_cast<uint32_t>(t * 2 * kBK));
        } else {
            const uint32_t stage = lds_addr + kOffW + static_cast<uint32_t>(t % kStages) * kTileW;
            const int vw = (wave & 3) + 4 * (piece >> 1);
            dma16_m0(wbuf, stage + (vw * 2 + (piece & 1)) * 1024, w_dma[piece],
                  static_cast<uint32_t>(t * kBK * N));
        }
    };
    auto issue_x = [&](int64_t pair, int piece) {
        const uint32_t slot = lds_addr + static_cast<uint32_t>(pair % kXSlots) * kXPair;
        const int vw = (wave & 3) + 4 * (piece >> 2);
        dma16_m0(xbuf, slot + vw * 4096 + (piece & 3) * 1024, x_dma[piece],
              static_cast<uint32_t>(pair * 2 * kBK));
    };
    constexpr int kWLoads = kWT ? 8 : 4;  // w DMA per pair of K-steps (w_t) or per K-step, per issuing wave
    constexpr int kXLoads = 8;            // x DMA per pair of K-steps per issuing wave

    // ---- LDS -> register fragment roles ----
    // x (B operand), row block i of the wave: row wm*64 + 32 i + l % 32,
    // logical chunks 2 (l / 32) and 2 (l / 32) + 1 of the K-step (the odd
    // K-step of a pair is logical chunks 4-7). The swizzle only depends on
    // row bits 0-3, which are lane bits 0-3.
    const int h = lane >> 5;
    const int x_row = wm * 64 + (lane & 31);
    const int x_rd0 = x_row * (2 * kBK) + (((2 * h) ^ x_swizzle(lane)) << 4);
    const int x_rd1 = x_row * (2 * kBK) + (((2 * h + 1) ^ x_swizzle(lane)) << 4);
    // w (A operand, transposed read), column block jb of the wave: lane l
    // receives column wn*128 + 32 jb + l % 32, k = 32 (l / 32) + 8 r + e
    // (byte e of read r). In 16-lane group g, lane j supplies the address of
    // k row 32 (g / 2) + 8 r + j / 2, columns 16 (g % 2) + 8 (j % 2) .. +7 of
    // the block.
    const int g = lane >> 4;
    const int jl = lane & 15;
    int w_rd[4];  // read r = 0 of each column block; read r adds 8 rows
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int row = 32 * (g >> 1) + (jl >> 1);
        const int chunk = wn * 8 + 2 * jb + (g & 1);
        w_rd[jb] = row * kBN + ((chunk ^ w_swizzle(row)) << 4) + (jl & 1) * 8;
    }
    // Rows r * 8 further keep row & 7, hence the same swizzle.
    // w_t (A operand, K-major), column block jb of the wave: lane l reads 32
    // consecutive k bytes of tile row wn*128 + 32 jb + l % 32, as x is read
    // (the swizzle again depends on lane bits 0-3 only).
    const int wt_rd0 = (wn * 128 + (lane & 31)) * (2 * kBK) + (((2 * h) ^ x_swizzle(lane)) << 4);
    const int wt_rd1 = (wn * 128 + (lane & 31)) * (2 * kBK) + (((2 * h + 1) ^ x_swizzle(lane)) << 4);

    struct XFrags {
        i32x8_t x[2];
    };
    auto read_x = [&](XFrags& f, int64_t kt) {
        const uint8_t* sx = lds + static_cast<int>((kt >> 1) % kXSlots) * kXPair;
        const int odd = static_cast<int>(kt & 1) << 6;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const i32x4v_t lo = *reinterpret_cast<const i32x4v_t*>(sx + ((x_rd0 ^ odd) + i * 32 * 2 * kBK));
            const i32x4v_t hi = *reinterpret_cast<const i32x4v_t*>(sx + ((x_rd1 ^ odd) + i * 32 * 2 * kBK));
            f.x[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    };
    auto read_w = [&](int64_t kt, int jb) {
        if constexpr (kWT) {
            const uint8_t* sw = lds + kOffW + static_cast<int>((kt >> 1) % kXSlots) * kXPair;
            const int odd = static_cast<int>(kt & 1) << 6;
            const i32x4v_t lo = *reinterpret_cast<const i32x4v_t*>(sw + ((wt_rd0 ^ odd) + jb * 32 * 2 * kBK));
            const i32x4v_t hi = *reinterpret_cast<const i32x4v_t*>(sw + ((wt_rd1 ^ odd) + jb * 32 * 2 * kBK));
            return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        }
        const uint8_t* sw = lds + kOffW + static_cast<int>(kt % kStages) * kTileW;
        const i32x2_t r0 = lds_read_tr8(sw, w_rd[jb]);
        const i32x2_t r1 = lds_read_tr8(sw, w_rd[jb] + 8 * kBN);
        const i32x2_t r2 = lds_read_tr8(sw, w_rd[jb] + 16 * kBN);
        const i32x2_t r3 = lds_read_tr8(sw, w_rd[jb] + 24 * kBN);
        const i32x4v_t lo = __builtin_shufflevector(r0, r1, 0, 1, 2, 3);
        const i32x4v_t hi = __builtin_shufflevector(r2, r3, 0, 1, 2, 3);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    f32x16_t acc[4][2];  // [w column block jb][x row block i]
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int t = 0; t < 16; ++t) acc[jb][i][t] = 0.0f;
        }
    }

    // w fragments live in one register set: fragment jb of the next K-step
    // is read into it once the two MFMAs of this step that use it have
    // issued. x is double-buffered. On step kt the issuing waves send out
    // the DMA for K-step kt + 3 (w) and, on odd steps, for x pair
    // (kt + 3) / 2, spread over the step's eight MFMAs. With w_t, odd steps
    // send out both operands' pair (kt + 3) / 2 and even steps send nothing.
    i32x8_t wf[4];
    auto multiply = [&](const XFrags& f, int64_t next_kt, auto read_next, auto issue, auto odd,
                        auto issuer) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                acc[jb][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                    wf[jb], f.x[i], acc[jb][i], 0, 0, 0, kUnitScale, 0, kUnitScale);
                if constexpr (decltype(issue)::value && decltype(issuer)::value) {
                    const int s = 2 * jb + i;
                    if constexpr (kWT) {
                        if constexpr (decltype(odd)::value) {
                            issue_x((next_kt + 2) >> 1, s);
                            issue_w((next_kt + 2) >> 1, s);
                        }
                    } else {
                        if constexpr (decltype(odd)::value) issue_x((next_kt + 2) >> 1, s);
                        if (s & 1) issue_w(next_kt + 2, s >> 1);
                    }
                }
            }
            if constexpr (decltype(read_next)::value) wf[jb] = read_w(next_kt, jb);
        }
    };

    auto run = [&](auto issuer) {
        const int64_t k_tiles = K / kBK;  // even, >= 2
        auto issue_w_all = [&](int64_t kt) {
#pragma unroll
            for (int piece = 0; piece < kWLoads; ++piece) issue_w(kt, piece);
        };
        auto issue_x_all = [&](int64_t pair) {
#pragma unroll
            for (int piece = 0; piece < kXLoads; ++piece) issue_x(pair, piece);
        };
        // Issue order as if steps -2 and -1 had run: x pair 0, w 0, w 1 | x pair 1, w 2.
        // With w_t: pair 0 of both | pair 1 of both.
        if constexpr (decltype(issuer)::value && kWT) {
            issue_x_all(0);
            issue_w_all(0);
            if (k_tiles > 2) {
                issue_x_all(1);
                issue_w_all(1);
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWLoads + kXLoads));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            }
        } else if constexpr (decltype(issuer)::value) {
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
        }
        bare_barrier();  // step 0 in LDS

        XFrags f0;
        XFrags f1;
        read_x(f0, 0);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) wf[jb] = read_w(0, jb);

        // Step kt: K-step kt + 1 must be in LDS (this wave's loads, then the
        // barrier for everyone's). The loads for kt + 3 reuse the stage of
        // kt - 1, which every wave has finished reading once it is at this
        // barrier; x pair p goes out on step 2p - 3 into the slot pair p - 2
        // left, once every wave has drained its reads of K-step 2p - 3. DMA completes in issue order, so the wait leaves exactly the
        // previous step's loads in flight: w after an even step, w and an x
        // pair after an odd one. With w_t both operands' pair p goes out on
        // step 2p - 3 and even steps issue nothing, so an even step leaves
        // one pair of both in flight and an odd step waits for everything.
        using yes = std::true_type;
        using no = std::false_type;
        auto step = [&](int64_t kt, XFrags& cur, XFrags& nxt, auto issue, auto wait_all, auto read,
                        auto odd) {
            if constexpr (decltype(read)::value) {
                // Odd steps also drain this wave's LDS reads (lgkmcnt 0):
                // the x (and w_t) pair sent out after this barrier overwrites
                // the slot whose last K-step was read in the step before and
                // is consumed only in this one.
                if constexpr (decltype(wait_all)::value) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
                } else if constexpr (kWT && decltype(odd)::value) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0) & ~(15 << 8));
                } else if constexpr (decltype(odd)::value) {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWLoads) & ~(15 << 8));
                } else {
                    __builtin_amdgcn_s_waitcnt(vmcnt_imm(kWLoads + kXLoads));
                }
                bare_barrier();
                read_x(nxt, kt + 1);
            }
            multiply(cur, kt + 1, read, issue, odd, issuer);
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
    if (wave < 4) {
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }

    // Store: acc[jb][i] element t of lane l is y[row wm*64 + 32 i + l % 32]
    // [column wn*128 + 32 jb + 8 (t / 4) + 4 (l / 32) + t % 4]; N is a
    // multiple of 16, so an eight-column run is entirely inside or outside.
    // The tile goes through LDS so that each store instruction writes whole
    // rows (16 lanes x 16 bytes = 256 contiguous bytes, 4 rows per
    // instruction) instead of 16 bytes of each of 32 rows: each wave stages
    // its 64 x 128 bf16 sub-tile (16 KiB, rows of 256 bytes) in the operand
    // area once every wave is past the K-loop. Chunk c (16 bytes) of row r
    // sits at chunk c ^ (r & 15), and rows with bit 4 set swap the two 8-byte
    // halves of their chunks: a half-wave's 8-byte writes (32 rows, one half
    // each) then cover all banks, and the 16-byte reads of whole rows too.
    __syncthreads();
    const float scale = args.scale;
    uint8_t* stage = lds + wave * (64 * 256);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = 32 * i + (lane & 31);
        const int flip = (r >> 4) & 1;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const f32x16_t& a = acc[jb][i];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = 4 * jb + q;
                uint2 packed;
                packed.x = f32x2_to_bf16x2_canon(scale * a[4 * q], scale * a[4 * q + 1]);
                packed.y = f32x2_to_bf16x2_canon(scale * a[4 * q + 2], scale * a[4 * q + 3]);
                *reinterpret_cast<uint2*>(stage + r * 256 + ((c ^ (r & 15)) << 4) + ((h ^ flip) << 3)) = packed;
            }
        }
    }
    // Only this wave reads what it wrote: LDS operations of a wave complete
    // in order; the fence keeps the compiler from moving the reads above.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const int c = lane & 15;
    const int64_t col = n0 + wn * 128 + 8 * c;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
        const int r = 4 * s + (lane >> 4);
        uint4 v = *reinterpret_cast<const uint4*>(stage + r * 256 + ((c ^ (r & 15)) << 4));
        if ((r >> 4) & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        const int64_t grow = m0 + wm * 64 + r;
        if (grow < M && col < N) store_stream16(args.y + grow * N + col, v);
    }
}

// ---- One wave per SIMD ------------------------------------------------------
// matmul_fp8_w4_kernel: the same 256x256 output tile with four waves, each
// owning a 128x128 sub-tile as 4x4 v_mfma_scale_f32_32x32x64_f8f6f4
// accumulators (256 fp32 per lane, in the accumulation registers; one wave
// per SIMD has 512 registers). Per MFMA this reads half the LDS bytes of a
// 64x128 sub-tile and issues half the scalar and barrier work per SIMD.
//   * K-tiles of 128 bytes, double-buffered in LDS for both operands
//     (32 KiB per operand and slot): x as whole 128-byte row lines (the x
//     swizzle); w_t (kWT) the same way, or w [K, N] as 128 k-rows of the
//     tile's 256 columns (the w swizzle), read transposed as in the
//     eight-wave kernel. Every wave copies a quarter of each (16 DMA per
//     K-tile).
//   * Fragments double-buffered in registers by K-half: the 16 MFMAs of one
//     half issue while the fragments of the next half are read.
//   * One barrier per K-tile, between its halves: by then every wave has
//     read all of K-tile t (so slot t % 2 takes K-tile t + 2, one DMA after
//     each MFMA of the second half) and K-tile t + 1 has landed (its DMA
//     went out one K-tile earlier).
constexpr int kW4Threads = 256;
constexpr int kW4Slot = kBM * 2 * kBK;  // 32 KiB: [256 rows][128 k]
constexpr int kW4OffW = 2 * kW4Slot;    // x slots 0 and 1, then w_t slots 0 and 1
constexpr int kW4Lds = 4 * kW4Slot;     // 128 KiB
static_assert(kW4Lds >= 4 * 128 * 256, "output staging (4 waves x 128 x 128 bf16) fits the operand area");

/// Reduction depths up to this take the eight-wave kernel: its shorter
/// prologue and epilogue outweigh this kernel's faster K-loop (equal at
/// 2048; at 8192 x 8192 x 1024 the eight-wave kernel is 4% faster, at
/// 8192^3 this one 8%).
constexpr int64_t kW4MinK = 2048;

/// s_waitcnt immediate that waits for every LDS operation of this wave.
constexpr int lgkmcnt0_imm() { return 15 | (3 << 14) | (7 << 4); }

template <bool kWT>
__global__ __launch_bounds__(kW4Threads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void matmul_fp8_w4_kernel(Fp8Args args) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[kW4Lds];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1;  // 128-row half of the tile
    const int wn = wave & 1;   // 128-column half of the tile
    int tm;
    int tn;
    tile_of(static_cast<int>(blockIdx.x), args.tiles_m, args.tiles_n, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * kBM;
    const int64_t n0 = static_cast<int64_t>(tn) * kBN;
    const int64_t M = args.M;
    const int64_t N = args.N;
    const int64_t K = args.K;

    // ---- HBM -> LDS: load i (0..7) of an operand copies tile rows
    // 64 wave + 8 i + l / 8, physical chunk l % 8 of the row's 128-byte line
    // (lane l lands at byte 16 l of the load's 1 KiB). With i = 2 a + b the
    // row's swizzle only depends on l / 8 and b, so two lane offsets serve
    // all eight loads; 16 a rows go into the scalar offset. Rows past M (x)
    // or N (w_t) read as zero.
    const int64_t rows_here = M - m0 < kBM ? M - m0 : kBM;
    const int64_t cols_here = N - n0 < kBN ? N - n0 : kBN;
    const i32x4_t xbuf = uniform(raw_buffer_words(args.x + m0 * K, static_cast<uint32_t>(rows_here * K)));
    const i32x4_t wbuf = kWT ? uniform(raw_buffer_words(args.w + n0 * K, static_cast<uint32_t>(cols_here * K)))
                             : uniform(raw_buffer_words(args.w, static_cast<uint32_t>(K * N)));
    uint32_t dma_off[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = 64 * wave + 8 * b + (lane >> 3);
        dma_off[b] = static_cast<uint32_t>(row * K + (((lane & 7) ^ x_swizzle(row)) << 4));
    }
    // w [K, N] (kWT false): load i (0..7) copies k rows 32 wave + 4 i + l / 16
    // of the K-tile, physical chunk l % 16 (16 columns). The swizzle takes row
    // bits 0-2, i.e. l / 16 and bit 0 of i, so two lane offsets serve the
    // eight loads; 8 (i / 2) rows go into the scalar offset. Columns past N
    // read as zero (the out-of-range marker plus a scalar offset below 2^31
    // stays out of range).
    uint32_t wkn_off[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int row = 32 * wave + 4 * b + (lane >> 4);
        const int64_t col = n0 + 16 * ((lane & 15) ^ w_swizzle(row));
        wkn_off[b] = col < N ? static_cast<uint32_t>(row * N + col) : kOutOfRange;
    }
    const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8_t*)lds));
    const uint32_t k16 = static_cast<uint32_t>(16 * K);
    // Load s (0..15) of K-tile t: x for even s, w for odd, load s / 2 of
    // the operand (both layouts fill 1 KiB at 8192 wave + 1024 i of the slot).
    auto issue_load = [&](int t, int slot, int s) {
        const int i = s >> 1;
        const uint32_t dst = lds_addr + static_cast<uint32_t>(slot * kW4Slot + wave * 8192 + i * 1024) +
                             ((s & 1) ? kW4OffW : 0);
        if (kWT || (s & 1) == 0) {
            const uint32_t sofs = static_cast<uint32_t>(t) * (2 * kBK) + static_cast<uint32_t>(i >> 1) * k16;
            dma16_m0((s & 1) ? wbuf : xbuf, dst, dma_off[i & 1], sofs);
        } else {
            const uint32_t sofs = static_cast<uint32_t>((static_cast<int64_t>(t) * (2 * kBK) + 8 * (i >> 1)) * N);
            dma16_m0(wbuf, dst, wkn_off[i & 1], sofs);
        }
    };

    // ---- LDS -> registers: block i of x (B operand) is tile row
    // wm*128 + 32 i + l % 32, block jb of w_t (A operand) tile row
    // wn*128 + 32 jb + l % 32; lane l takes k bytes 32 (l / 32) .. +31 of
    // the K-half as two ds_read_b128 (logical chunks 2 (l / 32) and
    // 2 (l / 32) + 1; the second K-half is chunks 4-7, byte offset ^ 64).
    const int h = lane >> 5;
    const int sw = x_swizzle(lane & 31);
    const int rd0 = (lane & 31) * (2 * kBK) + (((2 * h) ^ sw) << 4);
    const int rd1 = (lane & 31) * (2 * kBK) + (((2 * h + 1) ^ sw) << 4);
    const int x_base = wm * 128 * (2 * kBK);
    const int w_base = kW4OffW + wn * 128 * (2 * kBK);
    // w [K, N] (A operand, transposed read), column block jb of the wave:
    // lane l receives column wn*128 + 32 jb + l % 32, k = 32 (l / 32) + 8 r + e
    // of the K-half (byte e of read r), as in the eight-wave kernel; the
    // second K-half is 64 k-rows further (the swizzle takes row bits 0-2).
    const int g = lane >> 4;
    const int jl = lane & 15;
    int wkn_rd[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        const int row = 32 * (g >> 1) + (jl >> 1);
        const int chunk = wn * 8 + 2 * jb + (g & 1);
        wkn_rd[jb] = row * kBN + ((chunk ^ w_swizzle(row)) << 4) + (jl & 1) * 8;
    }
    auto read_a = [&](int slot, int half, int j) -> i32x8_t {
        const uint8_t* sw = lds + kW4OffW + slot * kW4Slot + half * 64 * kBN;
        const i32x2_t r0 = lds_read_tr8(sw, wkn_rd[j]);
        const i32x2_t r1 = lds_read_tr8(sw, wkn_rd[j] + 8 * kBN);
        const i32x2_t r2 = lds_read_tr8(sw, wkn_rd[j] + 16 * kBN);
        const i32x2_t r3 = lds_read_tr8(sw, wkn_rd[j] + 24 * kBN);
        const i32x4v_t lo = __builtin_shufflevector(r0, r1, 0, 1, 2, 3);
        const i32x4v_t hi = __builtin_shufflevector(r2, r3, 0, 1, 2, 3);
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };

    struct Frags {
        i32x8_t a[4];  // w_t blocks jb
        i32x8_t b[4];  // x blocks i
    };
    // `base` has bit 6 clear (slots, row blocks); the K-half flips bit 6 of
    // the lane's chunk offset.
    auto read_pair = [&](int base, int half) {
        const i32x4v_t lo = *reinterpret_cast<const i32x4v_t*>(lds + base + (rd0 ^ (half << 6)));
        const i32x4v_t hi = *reinterpret_cast<const i32x4v_t*>(lds + base + (rd1 ^ (half << 6)));
        return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    // Fragment r (0..7) of a K-half in the order the MFMAs below first use
    // them: a0, b0, b1, b2, b3, a1, a2, a3.
    auto read_frag = [&](Frags& f, int slot, int half, int r) {
        if (r >= 1 && r <= 4) {
            f.b[r - 1] = read_pair(x_base + slot * kW4Slot + (r - 1) * 32 * (2 * kBK), half);
        } else {
            const int j = r == 0 ? 0 : r - 4;
            if constexpr (kWT) {
                f.a[j] = read_pair(w_base + slot * kW4Slot + j * 32 * (2 * kBK), half);
            } else {
                f.a[j] = read_a(slot, half, j);
            }
        }
    };

    f32x16_t acc[4][4];  // [w_t block jb][x block i]
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int t = 0; t < 16; ++t) acc[jb][i][t] = 0.0f;
        }
    }
    // The 16 MFMAs of one K-half, each followed by its share of the other
    // work: on even MFMAs a fragment of the next K-half (read_next), on
    // every MFMA one of the 16 DMA of K-tile t + 2 (issue). The scheduling
    // barriers keep this order.
    auto multiply = [&](const Frags& f, Frags& next, int next_slot, int next_half, int issue_t, int issue_slot,
                        auto read_next, auto issue) {
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int jb = s >> 2;
            const int i = s & 3;
            acc[jb][i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                f.a[jb], f.b[i], acc[jb][i], 0, 0, 0, kUnitScale, 0, kUnitScale);
            if constexpr (decltype(read_next)::value) {
                if ((s & 1) == 0) read_frag(next, next_slot, next_half, s >> 1);
            }
            if constexpr (decltype(issue)::value) issue_load(issue_t, issue_slot, s);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int k_tiles = static_cast<int>(K / (2 * kBK));  // >= 1
#pragma unroll
    for (int s = 0; s < 16; ++s) issue_load(0, 0, s);
    if (k_tiles > 1) {
#pragma unroll
        for (int s = 0; s < 16; ++s) issue_load(1, 1, s);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
    } else {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    bare_barrier();  // K-tile 0 in LDS

    Frags f0;
    Frags f1;
#pragma unroll
    for (int r = 0; r < 8; ++r) read_frag(f0, 0, 0, r);
    // K-tile t (slot t % 2). The last two K-tiles are peeled so that the
    // loop body has no branch for the compiler to move the MFMAs across.
    using yes = std::true_type;
    using no = std::false_type;
    auto k_tile = [&](int t, auto issue, auto more) {
        const int slot = t & 1;
        // First half: multiply f0 while reading the second half into f1.
        multiply(f0, f1, slot, 1, 0, 0, yes{}, no{});
        // Every wave done reading slot `slot`; K-tile t + 1 landed.
        __builtin_amdgcn_s_waitcnt(lgkmcnt0_imm());
        if constexpr (decltype(more)::value) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        bare_barrier();
        // Second half: multiply f1 while reading K-tile t + 1's first half
        // and sending K-tile t + 2 into the slot just finished.
        multiply(f1, f0, slot ^ 1, 0, t + 2, slot, more, issue);
    };
    int t = 0;
    for (; t + 2 < k_tiles; ++t) k_tile(t, yes{}, yes{});
    if (k_tiles >= 2) k_tile(t++, no{}, yes{});
    k_tile(t, no{}, no{});

    // Store: acc[jb][i] element t of lane l is y[row wm*128 + 32 i + l % 32]
    // [column wn*128 + 32 jb + 8 (t / 4) + 4 (l / 32) + t % 4], staged per
    // wave as a 128 x 128 bf16 sub-tile (rows of 256 bytes, chunk c of row r
    // at c ^ (r & 15), rows with bit 4 set swapping the 8-byte halves of
    // their chunks) and stored as whole 256-byte row pieces.
    __syncthreads();
    const float scale = args.scale;
    uint8_t* stage = lds + wave * (128 * 256);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 32 * i + (lane & 31);
        const int flip = (r >> 4) & 1;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const f32x16_t& a = acc[jb][i];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int c = 4 * jb + q;
                uint2 packed;
                packed.x = f32x2_to_bf16x2_canon(scale * a[4 * q], scale * a[4 * q + 1]);
                packed.y = f32x2_to_bf16x2_canon(scale * a[4 * q + 2], scale * a[4 * q + 3]);
                *reinterpret_cast<uint2*>(stage + r * 256 + ((c ^ (r & 15)) << 4) + ((h ^ flip) << 3)) = packed;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const int c = lane & 15;
    const int64_t col = n0 + wn * 128 + 8 * c;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
        const int r = 4 * s + (lane >> 4);
        uint4 v = *reinterpret_cast<const uint4*>(stage + r * 256 + ((c ^ (r & 15)) << 4));
        if ((r >> 4) & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        const int64_t grow = m0 + wm * 128 + r;
        if (grow < M && col < N) store_stream16(args.y + grow * N + col, v);
    }
}

template <bool kWT>
cf_status launch_fp8_w4(const char* name, const void* x, const void* w, void* y, int64_t m, int64_t n,
                        int64_t k, float scale, void* stream) {
    Fp8Args args;
    args.x = static_cast<const uint8_t*>(x);
    args.w = static_cast<const uint8_t*>(w);
    args.y = static_cast<uint16_t*>(y);
    args.M = m;
    args.N = n;
    args.K = k;
    args.scale = scale;
    args.tiles_m = static_cast<int>(ceil_div<int64_t>(m, kBM));
    args.tiles_n = static_cast<int>(ceil_div<int64_t>(n, kBN));
    auto s = static_cast<hipStream_t>(stream);
    launch(matmul_fp8_w4_kernel<kWT>, dim3(args.tiles_m * args.tiles_n), dim3(kW4Threads), 0, s, args);
    return check_launch(name, s);
}

template <bool kWT>
cf_status launch_fp8(const char* name, const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k,
                     float scale, void* stream) {
    Fp8Args args;
    args.x = static_cast<const uint8_t*>(x);
    args.w = static_cast<const uint8_t*>(w);
    args.y = static_cast<uint16_t*>(y);
    args.M = m;
    args.N = n;
    args.K = k;
    args.scale = scale;
    args.tiles_m = static_cast<int>(ceil_div<int64_t>(m, kBM));
    args.tiles_n = static_cast<int>(ceil_div<int64_t>(n, kBN));
    auto s = static_cast<hipStream_t>(stream);
    launch(matmul_fp8_kernel<kWT>, dim3(args.tiles_m * args.tiles_n), dim3(kThreads), 0, s, args);
    return check_launch(name, s);
}

cf_status validate_fp8(const char* entry, int supported, const void* x, const void* w, void* y, int64_t m,
                       int64_t n, int64_t k) {
    if (!supported) {
        return fail(CF_ERR_UNSUPPORTED,
                    "%s: shape %lld x %lld x %lld is not tiled (k must be a positive multiple of 128, n of 16)",
                    entry, static_cast<long long>(m), static_cast<long long>(n), static_cast<long long>(k));
    }
    if (x == nullptr || w == nullptr || y == nullptr) {
        return fail(CF_ERR_INVALID_ARGUMENT, "%s: null pointer", entry);
    }
    if (!host_aligned(x, 16) || !host_aligned(w, 16) || !host_aligned(y, 16)) {
        return fail(CF_ERR_UNSUPPORTED, "%s: x, w and y must be 16-byte aligned", entry);
    }
    return CF_OK;
}

bool tiles_fit(int64_t m, int64_t n) {
    return ceil_div<int64_t>(m, kBM) * ceil_div<int64_t>(n, kBN) < (1LL << 31);
}

}  // namespace
}  // namespace cf

extern "C" {

int cf_matmul_fp8_shape_supported(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 16 != 0 || k % (2 * cf::kBK) != 0) return 0;
    // 32-bit buffer offsets: all of w, and one 256-row panel of x.
    if (k * n >= (1LL << 31) || static_cast<int64_t>(cf::kBM) * k >= (1LL << 31)) return 0;
    return cf::tiles_fit(m, n) ? 1 : 0;
}

int cf_matmul_fp8_wt_shape_supported(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || n % 16 != 0 || k % (2 * cf::kBK) != 0) return 0;
    // 32-bit buffer offsets: one 256-row panel of x and of w_t.
    if (static_cast<int64_t>(cf::kBM) * k >= (1LL << 31)) return 0;
    return cf::tiles_fit(m, n) ? 1 : 0;
}

cf_status cf_matmul_fp8(const void* x, const void* w, void* y, int64_t m, int64_t n, int64_t k, float scale,
                        void* stream) {
    CF_ENTRY();
    const cf_status st = cf::validate_fp8("cf_matmul_fp8", cf_matmul_fp8_shape_supported(m, n, k), x, w, y, m, n, k);
    if (st != CF_OK) return st;
    if (k <= cf::kW4MinK) {
        return cf::launch_fp8<false>("launching the fp8 MFMA matmul", x, w, y, m, n, k, scale, stream);
    }
    return cf::launch_fp8_w4<false>("launching the fp8 MFMA matmul (one wave per SIMD)", x, w, y, m, n, k, scale,
                                    stream);
}

cf_status cf_matmul_fp8_wt(const void* x, const void* w_t, void* y, int64_t m, int64_t n, int64_t k, float scale,
                           void* stream) {
    CF_ENTRY();
    const cf_status st =
        cf::validate_fp8("cf_matmul_fp8_wt", cf_matmul_fp8_wt_shape_supported(m, n, k), x, w_t, y, m, n, k);
    if (st != CF_OK) return st;
    if (k <= cf::kW4MinK) {
        return cf::launch_fp8<true>("launching the fp8 MFMA matmul (K-major w)", x, w_t, y, m, n, k, scale, stream);
    }
    return cf::launch_fp8_w4<true>("launching the fp8 MFMA matmul (K-major w, one wave per SIMD)", x, w_t, y, m, n,
                                   k, scale, stream);
}

}  // extern "C"

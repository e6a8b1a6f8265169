// Adapter backward of the LoRA linear on bf16 MFMA (gfx950), op layout:
//
//   G      = dy @ b^T                 [M, r]   rounded to bf16 (ATen autograd
//                                              sees a bf16 intermediate)
//   grad_b = scale * bf16(xa)^T @ dy  [r, N]
//   grad_a = scale * x^T @ bf16(G)    [K, r]
//
// derivatives of the reference's _lora_linear_reference
// (python/cudaforge/ops.py:178-185, tests/python/test_autograd.py:81-91).
//
// The work is two reductions over M of HBM-sized operands, so the design
// reads dy once and x once (the HBM floor) and keeps everything else small:
//   1. One pass over dy in 512-row x 256-column tiles (Mp = M rounded up to
//      512), two 64-row chunks in flight per workgroup, loaded with the
//      non-temporal hint (every byte is read once): each chunk goes
//      HBM -> registers -> LDS; G partial rows = chunk @
//      b^T (16x16x32 MFMA, row fragments by ds_read_b128, b fragments held in
//      registers) and grad_b partials += bf16(xa)^T-chunk @ chunk (16x16x32
//      MFMA; the chunk's fp32 xa arrives with one 16-byte load per thread
//      and is rounded and transposed into LDS, the m-contiguous operand is
//      read by ds_read_b64_tr_b16). Partials
//      go to fp32 workspaces, one slice per 256-column tile (G) and per
//      512-row tile (grad_b). 512-row tiles halve the grad_b/grad_a partials
//      of 256-row ones (37.8 against 39.5 us at 8192 x 4096 x 4096 r16,
//      operands cache-cold); three or four chunks in flight were slower.
//   2. One launch sums both in a fixed order: grad_b (times scale, cast) and
//      G -> GT (bf16 [16, Mp]).
//   3. The same column-reduction pass over x with GT: grad_a partials.
//   4. Their fixed-order sum, times scale, cast, stored transposed.
// Deterministic: every sum has a fixed order, no atomics.
#include "cf_lora_bwd.hpp"

#include <type_traits>

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kTileRows = 512;   // rows (M) per workgroup
constexpr int kTileCols = 256;   // columns per workgroup
constexpr int kChunkRows = 64;   // rows staged in LDS at a time
constexpr int kInFlight = 2;     // chunks loaded ahead per workgroup
constexpr int kThreads = 256;
constexpr int kRankPad = 16;     // adapter rank padded to one MFMA dimension
constexpr int kRowBytes = kTileCols * 2;
constexpr int kPiecesPerThread = kChunkRows * kTileCols * 2 / 16 / kThreads;  // 8
constexpr uint32_t kOutOfRange = 0x80000000u;
constexpr int kXatStride = kChunkRows + 8;  // bf16 per row of the transposed xa chunk

/// Chunk swizzle of the staged tile (512-byte rows of 32 16-byte chunks).
/// Even, so transposed reads keep their 32-byte column pairs; distinct over
/// rows 0-7 and over rows 8-15 (ds_read_b128 of 16 rows), and distinct in
/// its upper bits over rows {0-3, 8-11} and {4-7, 12-15} (the rows one
/// ds_read_b64_tr_b16 cycle touches).
__device__ __forceinline__ int tile_swizzle(int row) {
    return 2 * ((row & 3) + 4 * (((row >> 2) ^ (row >> 3)) & 1));
}

__device__ __forceinline__ int tile_offset(int row, int chunk) {
    return row * kRowBytes + ((chunk ^ tile_swizzle(row)) << 4);
}

__device__ __forceinline__ s16x4_t lds_read_tr(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

__device__ __forceinline__ bf16x8_t concat(s16x4_t lo, s16x4_t hi) {
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ uint32_t buffer_load4(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset,
                                                  uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b32(rsrc, voffset, soffset, 0);
}

struct ColumnArgs {
    const uint16_t* v;     // [M, C] bf16, the operand reduced over rows
    const uint16_t* pt;    // [16, Mp] bf16, the other factor, m-contiguous (x pass)
    const float* xa;       // [M, rank] fp32, the other factor of the dy pass
    const uint16_t* b;     // [rank, C] bf16 (row-dot pass only)
    float* colpart;        // [Mp / 256][16][C] fp32
    float* gpart;          // [ceil(C / 256)][Mp][16] fp32 (row-dot pass only)
    int64_t M;
    int64_t Mp;
    int64_t C;
    int64_t rank;
};

/// One kTileRows x 256-column tile of v: colpart[tile row][j][n] =
/// sum_m pt[j, m] * v[m, n] over the tile's rows; with kRowDot also
/// gpart[tile column][m][j] = sum_n v[m, n] * b[j, n] over its columns.
template <bool kRowDot>
__global__ __launch_bounds__(kThreads) void column_mfma_kernel(ColumnArgs args) {
    __shared__ __attribute__((aligned(16))) uint8_t tile[kChunkRows * kRowBytes];  // 32 KiB
    // dy pass: the chunk's xa, rounded to bf16 and transposed ([16 j][64 m],
    // rows padded by 16 bytes); rows j >= rank stay zero.
    __shared__ __attribute__((aligned(16))) uint16_t xat[kRowDot ? kRankPad : 1][kXatStride];

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int g = lane >> 4;
    const int jl = lane & 15;
    const int64_t C = args.C;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kTileCols;
    const int64_t mt = blockIdx.y;
    const int64_t m0 = mt * kTileRows;

    // Staging roles: piece i of thread tid is row 8 i + tid / 32, chunk
    // tid % 32 of the chunk; one wave reads two 512-byte row segments.
    // Rows past M and columns past C read as zero (buffer range check and an
    // out-of-range offset), so they add nothing to either reduction.
    const __amdgpu_buffer_rsrc_t vbuf =
        make_buffer(args.v, static_cast<uint32_t>(args.M * C * 2));
    const int piece_chunk = tid & 31;
    const int64_t piece_col = n0 + 8 * piece_chunk;
    const bool col_ok = piece_col < C;
    // kInFlight chunks in flight: slot s of each staging array holds chunk c
    // with c % kInFlight == s (the chunk loop below is unrolled, so slots are
    // registers).
    uint4 staged[kInFlight][kPiecesPerThread];
    // dy pass: thread t also loads bytes 16 t .. +15 of the chunk's xa rows
    // (64 x rank fp32, contiguous), i.e. flat elements 4 t .. 4 t + 3:
    // element q is xa[row0 + xa_row[q]][xa_col[q]].
    uint4 staged_xa[kInFlight];
#pragma unroll
    for (int s = 0; s < kInFlight; ++s) staged_xa[s] = make_uint4(0u, 0u, 0u, 0u);
    // x pass: the chunk's pt fragments, pt[j = lane % 16][row0 + 32 ms +
    // 8 (lane / 16) .. +7], loaded with the chunk so that waiting for them
    // never waits for a later chunk's loads.
    bf16x8_t staged_pt[kInFlight][2];
    int xa_row[4];
    int xa_col[4];
    if constexpr (kRowDot) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int idx = 4 * tid + q;
            xa_row[q] = idx / static_cast<int>(args.rank);
            xa_col[q] = idx % static_cast<int>(args.rank);
        }
        // Rows j >= rank of the transposed chunk are never written: zero
        // them once (the loop's first barrier orders this before any read).
        for (int i = tid; i < kRankPad * kXatStride; i += kThreads) (&xat[0][0])[i] = 0;
    }
    const __amdgpu_buffer_rsrc_t xabuf = make_buffer(
        args.xa, static_cast<uint32_t>(kRowDot ? args.M * args.rank * 4 : 0));
    const __amdgpu_buffer_rsrc_t ptbuf =
        make_buffer(args.pt, static_cast<uint32_t>(kRowDot ? 0 : kRankPad * args.Mp * 2));
    auto load_chunk = [&](int slot, int64_t row0) {
#pragma unroll
        for (int i = 0; i < kPiecesPerThread; ++i) {
            const int64_t row = row0 + 8 * i + (tid >> 5);
            const uint32_t off =
                col_ok ? static_cast<uint32_t>((row * C + piece_col) * 2) : kOutOfRange;
            staged[slot][i] = buffer_load16_stream(vbuf, off, 0);
        }
        if constexpr (kRowDot) {
            // Past the chunk's kChunkRows x rank elements (rank < 16), or past
            // M: zeros.
            const uint32_t off = 4 * tid < kChunkRows * args.rank
                                     ? static_cast<uint32_t>((row0 * args.rank + 4 * tid) * 4)
                                     : kOutOfRange;
            staged_xa[slot] = buffer_load16(xabuf, off, 0);
        } else {
#pragma unroll
            for (int ms = 0; ms < 2; ++ms) {
                const uint32_t off = static_cast<uint32_t>((jl * args.Mp + row0 + 32 * ms + 8 * g) * 2);
                staged_pt[slot][ms] = as_bf16x8(buffer_load16(ptbuf, off, 0));
            }
        }
    };
    auto store_chunk = [&](int slot) {
#pragma unroll
        for (int i = 0; i < kPiecesPerThread; ++i) {
            const int row = 8 * i + (tid >> 5);
            *reinterpret_cast<uint4*>(tile + tile_offset(row, piece_chunk)) = staged[slot][i];
        }
        if constexpr (kRowDot) {
            if (4 * tid < kChunkRows * args.rank) {
                const uint32_t v[4] = {staged_xa[slot].x, staged_xa[slot].y, staged_xa[slot].z,
                                       staged_xa[slot].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    xat[xa_col[q]][xa_row[q]] = static_cast<uint16_t>(f32_to_bf16_bits(__uint_as_float(v[q])));
                }
            }
        }
    };

    // Row-dot role: wave w owns chunk rows 16 w .. +15; b fragment s holds
    // b[j = lane % 16][n0 + 32 s + 8 (lane / 16) .. +7].
    bf16x8_t bfrag[8];
    if constexpr (kRowDot) {
        const __amdgpu_buffer_rsrc_t bbuf =
            make_buffer(args.b, static_cast<uint32_t>(args.rank * C * 2));
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int64_t col = n0 + 32 * s + 8 * g;
            const uint32_t off = (jl < args.rank && col < C)
                                     ? static_cast<uint32_t>((jl * C + col) * 2)
                                     : kOutOfRange;
            bfrag[s] = as_bf16x8(buffer_load16(bbuf, off, 0));
        }
    }

    // Column-reduction role: wave w owns column blocks 4 w .. 4 w + 3 (16
    // columns each); accumulator lane holds [j = 4 (lane / 16) + t][column
    // 16 cb + lane % 16].
    f32x4_t acc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int kChunks = kTileRows / kChunkRows;
#pragma unroll
    for (int c = 0; c < kInFlight && c < kChunks; ++c) load_chunk(c, m0 + c * kChunkRows);
#pragma unroll
    for (int chunk = 0; chunk < kChunks; ++chunk) {
        const int slot = chunk % kInFlight;
        const int64_t row0 = m0 + static_cast<int64_t>(chunk) * kChunkRows;
        __syncthreads();  // previous chunk's readers are done
        store_chunk(slot);
        __syncthreads();

        // pt fragments. The dy pass reads them from the transposed bf16 copy
        // of the chunk's xa in LDS (rounded as the transposed copy of the x
        // pass is); rows past M and columns past the rank are zero.
        bf16x8_t ptfrag[2];
#pragma unroll
        for (int ms = 0; ms < 2; ++ms) {
            if constexpr (kRowDot) {
                ptfrag[ms] = *reinterpret_cast<const bf16x8_t*>(&xat[jl][32 * ms + 8 * g]);
            } else {
                ptfrag[ms] = staged_pt[slot][ms];
            }
        }
        if (chunk + kInFlight < kChunks) load_chunk(slot, row0 + kInFlight * kChunkRows);

#pragma unroll
        for (int ms = 0; ms < 2; ++ms) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int cb = 4 * wave + c;
                const int row = 32 * ms + 8 * g + (jl >> 2);
                const int ch = 2 * cb + ((jl & 3) >> 1);
                const int off = tile_offset(row, ch) + (jl & 1) * 8;
                // Four rows further down: same swizzle parity pattern, so
                // recompute rather than add.
                const int off_hi = tile_offset(row + 4, ch) + (jl & 1) * 8;
                const bf16x8_t vfrag = concat(lds_read_tr(tile, off), lds_read_tr(tile, off_hi));
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ptfrag[ms], vfrag, acc[c], 0, 0, 0);
            }
        }

        if constexpr (kRowDot) {
            f32x4_t gacc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            const int row = 16 * wave + jl;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const bf16x8_t afrag =
                    *reinterpret_cast<const bf16x8_t*>(tile + tile_offset(row, 4 * s + g));
                gacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag[s], gacc, 0, 0, 0);
            }
            // gacc lane holds G[row 16 wave + 4 (lane / 16) + t][j = lane % 16].
            float* gp = args.gpart + (static_cast<int64_t>(blockIdx.x) * args.Mp + row0 +
                                      16 * wave + 4 * g) * kRankPad + jl;
#pragma unroll
            for (int t = 0; t < 4; ++t) gp[t * kRankPad] = gacc[t];
        }
    }

    // colpart[mt][j][n]: lane holds j = 4 (lane / 16) + t, n = n0 + 16 cb + lane % 16.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int64_t col = n0 + 16 * (4 * wave + c) + jl;
        if (col >= C) continue;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            args.colpart[(mt * kRankPad + 4 * g + t) * C + col] = acc[c][t];
        }
    }
}

/// total += at(t) for t = t .. tiles - 1 in that order, loads issued in
/// groups of 32, 16, 4, then 1 so a thread waits for memory a few times
/// rather than once per eight partials.
template <typename At>
__device__ __forceinline__ float ordered_sum(int64_t tiles, At at) {
    float total = 0.0f;
    int64_t t = 0;
    auto groups = [&](auto group) {
        constexpr int kGroup = decltype(group)::value;
        for (; t + kGroup <= tiles; t += kGroup) {
            float v[kGroup];
#pragma unroll
            for (int k = 0; k < kGroup; ++k) v[k] = at(t + k);
#pragma unroll
            for (int k = 0; k < kGroup; ++k) total += v[k];
        }
    };
    groups(std::integral_constant<int, 32>{});
    groups(std::integral_constant<int, 16>{});
    groups(std::integral_constant<int, 4>{});
    groups(std::integral_constant<int, 1>{});
    return total;
}

/// gt[j, m] = bf16(sum over column tiles of gpart[tile][m][j]), fixed order;
/// thread i of the launch handles element i.
__device__ __forceinline__ void sum_g(const float* __restrict__ gpart, uint16_t* __restrict__ gt,
                                      int64_t Mp, int64_t tiles, int64_t i) {
    if (i >= kRankPad * Mp) return;
    const int64_t m = i / kRankPad;
    const int64_t j = i % kRankPad;
    const float total =
        ordered_sum(tiles, [&](int64_t t) { return gpart[(t * Mp + m) * kRankPad + j]; });
    gt[j * Mp + m] = static_cast<uint16_t>(f32_to_bf16_bits(total));
}

/// out = scale * sum over row tiles of colpart[tile][j][n], j < rank, as
/// [rank, C] or (kTransposed) [C, rank]; fixed order; thread i handles
/// element i.
template <bool kTransposed>
__device__ __forceinline__ void finish(const float* __restrict__ colpart, uint16_t* __restrict__ out,
                                       int64_t tiles, int64_t rank, int64_t C, float scale, int64_t i) {
    if (i >= rank * C) return;
    const int64_t j = i / C;
    const int64_t n = i % C;
    const float total =
        ordered_sum(tiles, [&](int64_t t) { return colpart[(t * kRankPad + j) * C + n]; });
    const int64_t dst = kTransposed ? n * rank + j : j * C + n;
    out[dst] = static_cast<uint16_t>(f32_to_bf16_bits(scale * total));
}

/// After the dy pass: grad_b's fixed-order sum (first grad_b_blocks
/// workgroups) and G's (the rest) are independent, so one launch does both.
__global__ __launch_bounds__(kThreads) void after_dy_kernel(const float* __restrict__ colpart,
                                                            uint16_t* __restrict__ grad_b,
                                                            const float* __restrict__ gpart,
                                                            uint16_t* __restrict__ gt,
                                                            int64_t grad_b_blocks, int64_t row_tiles,
                                                            int64_t rank, int64_t N, float scale,
                                                            int64_t Mp, int64_t col_tiles) {
    const int64_t block = blockIdx.x;
    if (block < grad_b_blocks) {
        finish<false>(colpart, grad_b, row_tiles, rank, N, scale, block * kThreads + threadIdx.x);
    } else {
        sum_g(gpart, gt, Mp, col_tiles, (block - grad_b_blocks) * kThreads + threadIdx.x);
    }
}

/// grad_a's fixed-order sum after the x pass, stored transposed ([K, rank]).
__global__ __launch_bounds__(kThreads) void finish_grad_a_kernel(const float* __restrict__ colpart,
                                                                 uint16_t* __restrict__ grad_a,
                                                                 int64_t row_tiles, int64_t rank,
                                                                 int64_t K, float scale) {
    finish<true>(colpart, grad_a, row_tiles, rank, K, scale,
                 static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x);
}

struct Workspace {
    uint16_t* gt;
    float* gpart;
    float* colpart;
};

size_t align256(size_t bytes) { return (bytes + 255) / 256 * 256; }

Workspace carve(void* base, int64_t M, int64_t K, int64_t N) {
    const int64_t Mp = ceil_div<int64_t>(M, kTileRows) * kTileRows;
    uint8_t* p = static_cast<uint8_t*>(base);
    Workspace ws;
    ws.gt = reinterpret_cast<uint16_t*>(p);
    p += align256(static_cast<size_t>(kRankPad * Mp) * 2);
    ws.gpart = reinterpret_cast<float*>(p);
    p += align256(static_cast<size_t>(ceil_div<int64_t>(N, kTileCols) * Mp * kRankPad) * 4);
    ws.colpart = reinterpret_cast<float*>(p);
    (void)K;
    return ws;
}

}  // namespace

size_t lora_backward_fast_workspace_bytes(int64_t M, int64_t K, int64_t N) {
    if (M <= 0) return 0;
    const int64_t Mp = ceil_div<int64_t>(M, kTileRows) * kTileRows;
    const int64_t widest = K > N ? K : N;
    return align256(static_cast<size_t>(kRankPad * Mp) * 2) +
           align256(static_cast<size_t>(ceil_div<int64_t>(N, kTileCols) * Mp * kRankPad) * 4) +
           static_cast<size_t>(Mp / kTileRows * kRankPad * widest) * 4;
}

bool lora_backward_fast_eligible(const void* x, const void* dy, const void* b, int64_t M,
                                 int64_t K, int64_t N, int64_t rank) {
    // Buffer offsets are 32-bit with an out-of-range marker at 2^31.
    const int64_t Mp = ceil_div<int64_t>(M, kTileRows) * kTileRows;
    const bool fits = Mp * K * 2 < (1LL << 31) && Mp * N * 2 < (1LL << 31) &&
                      rank * N * 2 < (1LL << 31) && kRankPad * Mp * 2 < (1LL << 31) &&
                      Mp * rank * 4 < (1LL << 31);
    return M > 0 && K > 0 && N > 0 && rank > 0 && rank <= kRankPad && K % 8 == 0 && N % 8 == 0 &&
           fits && host_aligned(x, 16) && host_aligned(dy, 16) && host_aligned(b, 16);
}

cf_status launch_lora_backward_fast(const void* x, const void* dy, const void* b, const float* xa,
                                    void* grad_a, void* grad_b, int64_t M, int64_t K, int64_t N,
                                    int64_t rank, float scale, void* workspace,
                                    hipStream_t stream) {
    const int64_t Mp = ceil_div<int64_t>(M, kTileRows) * kTileRows;
    const int64_t row_tiles = Mp / kTileRows;
    const Workspace ws = carve(workspace, M, K, N);
    const unsigned small_grid = static_cast<unsigned>(ceil_div<int64_t>(kRankPad * Mp, kThreads));

    ColumnArgs dy_pass;
    dy_pass.v = static_cast<const uint16_t*>(dy);
    dy_pass.pt = nullptr;
    dy_pass.xa = xa;
    dy_pass.b = static_cast<const uint16_t*>(b);
    dy_pass.colpart = ws.colpart;
    dy_pass.gpart = ws.gpart;
    dy_pass.M = M;
    dy_pass.Mp = Mp;
    dy_pass.C = N;
    dy_pass.rank = rank;
    const int64_t n_tiles = ceil_div<int64_t>(N, kTileCols);
    launch(column_mfma_kernel<true>,
           dim3(dim3(static_cast<unsigned>(n_tiles), static_cast<unsigned>(row_tiles))),
           dim3(kThreads), 0, stream, dy_pass);
    const int64_t grad_b_blocks = ceil_div<int64_t>(rank * N, kThreads);
    launch(after_dy_kernel, dim3(static_cast<unsigned>(grad_b_blocks + small_grid)), dim3(kThreads),
           0, stream, ws.colpart, static_cast<uint16_t*>(grad_b), ws.gpart, ws.gt, grad_b_blocks,
           row_tiles, rank, N, scale, Mp, n_tiles);

    ColumnArgs x_pass;
    x_pass.v = static_cast<const uint16_t*>(x);
    x_pass.pt = ws.gt;
    x_pass.xa = nullptr;
    x_pass.b = nullptr;
    x_pass.colpart = ws.colpart;
    x_pass.gpart = nullptr;
    x_pass.M = M;
    x_pass.Mp = Mp;
    x_pass.C = K;
    x_pass.rank = rank;
    const int64_t k_tiles = ceil_div<int64_t>(K, kTileCols);
    launch(column_mfma_kernel<false>,
           dim3(dim3(static_cast<unsigned>(k_tiles), static_cast<unsigned>(row_tiles))),
           dim3(kThreads), 0, stream, x_pass);
    launch(finish_grad_a_kernel, dim3(static_cast<unsigned>(ceil_div<int64_t>(rank * K, kThreads))),
           dim3(kThreads), 0, stream, ws.colpart, static_cast<uint16_t*>(grad_a), row_tiles, rank,
           K, scale);
    return check_launch("launching the bf16 LoRA backward", stream);
}

}  // namespace cf

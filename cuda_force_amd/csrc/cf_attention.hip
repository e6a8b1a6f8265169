// Causal attention products of the transformer block on the bf16 MFMA units
// of gfx950:
//
//   scores[b, h, s, t] = sum_d q[b, s, h, d] * k[b, t, h, d]          (t <= s)
//   out[b, s, h, d]    = sum_{t <= s} probs[b, h, s, t] * v[b, t, h, d]
//
// the two batched products of examples/transformer_block.py:54 and :63
// (query @ key^T, then weights @ value, with the head transposes folded into
// the addressing). q, k, v and out keep the projections' [batch, seq,
// heads * head_dim] layout; scores and probs are [batch, heads, seq, seq],
// the layout the row softmax takes. fp32 accumulation, one rounding to bf16.
//
// Both products only touch the causal half:
//   * scores: one workgroup per 128 x 128 tile on or below the diagonal of a
//     head's [seq, seq] block, four waves of 64 x 64. A wave wholly above the
//     diagonal only helps copy the tile's rows, and tiles above it are never
//     written (the causal softmax does not read them). Entries above the diagonal inside a
//     written tile hold their dot products.
//   * out: keys past a query row's own position are skipped chunk by chunk
//     and masked inside the last chunk, so the probabilities above the
//     diagonal are never read as values.
//
// MFMA roles (v_mfma_f32_16x16x32_bf16; a lane holds A row l % 16 and B
// column l % 16, each over k = 8 (l / 16) .. +7, and D rows 4 (l / 16) + i of
// column l % 16):
//   * scores are computed transposed, S^T = K Q^T. The tile's q and k rows
//     are copied into LDS by buffer loads with the LDS destination (whole
//     256-byte rows, chunks swizzled for conflict-free reads); A and B
//     fragments are ds_read_b128 of k and q rows (head_dim is the contiguous
//     reduction index of both), and a lane ends with four consecutive keys
//     of one query row; each wave's 64 x 64 tile is then staged in LDS and
//     written as whole 128-byte row pieces.
//   * out is computed transposed too, O^T = V^T P^T. P^T fragments are
//     16-byte loads of probability rows; V^T fragments come out of an LDS copy
//     of each 64-key chunk of v (copied by buffer loads with the LDS
//     destination, shared by the workgroup's four waves) through
//     ds_read_b64_tr_b16, which hands each lane 4 consecutive keys of one
//     head dimension. A lane ends with four consecutive head dimensions of
//     one query row: one 8-byte store into the [batch, seq, hidden] output.
#include "cf_common.hpp"
#include "cf_lds_dma.hpp"

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

constexpr int kThreads = 256;
constexpr int kScoreTile = 128;  // queries and keys per scores workgroup
constexpr int kPvRows = 64;      // query rows per out workgroup (16 per wave)
constexpr int kPvChunk = 64;     // keys per step of the out product (two MFMA k-steps)
constexpr int kPvSub = kPvChunk / 32;
constexpr int kVPitch = 256;     // LDS bytes per staged q, k or v row (head_dim <= 128)
// A buffer offset past every range this file builds (all below 2^31): the
// load returns zeros. Rows past seq take it rather than their own offset,
// which for a large pitch could wrap around 2^32.
constexpr uint32_t kPastEnd = 0x80000000u;

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

/// 16-byte chunk swizzle of a staged v row (256-byte pitch): the four rows
/// of one 16-lane group of a transposed read land in four 32-byte bank
/// groups of one 128-byte half, and rows 8 further (the other group of the
/// same cycle) in the other half.
__device__ __forceinline__ int v_swizzle(int row) { return 2 * (row & 3) + 8 * ((row >> 3) & 1); }

__device__ __forceinline__ s16x4_t lds_read_tr(const uint8_t* base, int offset) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4_t*)((lds_u8_t*)(const_cast<uint8_t*>(base)) + offset));
}

/// Byte extent of one (batch, head) slice of a [batch, seq, heads * D]
/// tensor seen from its first element: rows past seq fall outside it.
__device__ __forceinline__ uint32_t head_extent(int64_t seq, int64_t heads, int d) {
    return static_cast<uint32_t>(((seq - 1) * heads * d + d) * 2);
}

/// Four fp32 values rounded to bf16 (c10::BFloat16's rounding) and stored
/// with one 8-byte store.
__device__ __forceinline__ void store4_bf16(uint16_t* p, const f32x4_t& v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(f32x2_to_bf16x2_canon(v[0], v[1]), f32x2_to_bf16x2_canon(v[2], v[3]));
}

/// Workgroup ids are dealt round-robin over the 8 XCDs; this renumbering
/// gives each XCD a contiguous range of logical ids (when the grid divides),
/// so the workgroups of one head share that XCD's L2.
__device__ __forceinline__ int64_t xcd_local(int64_t pid, int64_t total) {
    constexpr int kXcds = 8;
    return total % kXcds == 0 ? (pid % kXcds) * (total / kXcds) + pid / kXcds : pid;
}

/// scores for the causal tiles. Logical id = bh * tiles + tile, tile
/// enumerating the tiles (si, ti) with ti <= si row by row. The tile's 128
/// query rows and 128 key rows are copied HBM -> LDS by buffer loads with
/// the LDS destination (each load 4 whole rows), so every row is read once
/// per workgroup in whole 256-byte pieces.
template <int kD>
__global__ __launch_bounds__(kThreads) void attention_scores_kernel(const uint16_t* __restrict__ q,
                                                                    const uint16_t* __restrict__ k,
                                                                    uint16_t* __restrict__ scores, int64_t seq,
                                                                    int64_t heads, int tiles) {
    // q rows then k rows, 128 each at a 256-byte pitch, 16-byte chunk c of
    // row r at c ^ (r & 15); afterwards each wave's 8 KiB output staging.
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kScoreTile * kVPitch];  // 64 KiB
    const int64_t id = xcd_local(blockIdx.x, static_cast<int64_t>(gridDim.x));
    const int64_t bh = id / tiles;
    const int tile = static_cast<int>(id % tiles);
    int si = static_cast<int>((sqrtf(8.0f * static_cast<float>(tile) + 1.0f) - 1.0f) * 0.5f);
    while ((si + 1) * (si + 2) / 2 <= tile) ++si;
    while (si * (si + 1) / 2 > tile) --si;
    const int ti = tile - si * (si + 1) / 2;

    const int lane = static_cast<int>(threadIdx.x) & 63;
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int64_t q_row0 = static_cast<int64_t>(si) * kScoreTile;
    const int64_t k_row0 = static_cast<int64_t>(ti) * kScoreTile;
    const int64_t s0 = q_row0 + (wave >> 1) * 64;
    const int64_t t0 = k_row0 + (wave & 1) * 64;
    // Wave-uniform: a wave with nothing on or below the diagonal, or no
    // query row, still copies its share of the tiles and meets the barriers.
    const bool active = t0 <= s0 + 63 && s0 < seq;

    const int64_t b = bh / heads;
    const int64_t h = bh % heads;
    const int64_t head0 = (b * seq * heads + h) * kD;  // element of row 0, dim 0
    const int64_t pitch = heads * kD;                  // elements between consecutive rows
    const uint32_t extent = head_extent(seq, heads, kD);
    const i32x4_t qbuf = uniform(raw_buffer_words(q + head0, extent));
    const i32x4_t kbuf = uniform(raw_buffer_words(k + head0, extent));
    const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8_t*)lds));

    // Load n (0..31) of an operand fills rows 4 n .. 4 n + 3 of its tile:
    // lane l lands at byte 16 l, i.e. row 4 n + l / 16, physical chunk
    // l % 16, so it reads logical chunk (l % 16) ^ (row & 15). Rows past
    // seq and chunks past the head (head_dim < 128) read as zero.
    const int phys = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int n = 8 * wave + i;
        const int r = 4 * n + (lane >> 4);
        const int c = phys ^ (r & 15);
        const int64_t qr = q_row0 + r;
        const int64_t kr = k_row0 + r;
        const uint32_t qoff = qr < seq && c < kD / 8 ? static_cast<uint32_t>((qr * pitch + 8 * c) * 2) : kPastEnd;
        const uint32_t koff = kr < seq && c < kD / 8 ? static_cast<uint32_t>((kr * pitch + 8 * c) * 2) : kPastEnd;
        dma16_m0(qbuf, lds_addr + static_cast<uint32_t>(n * 1024), qoff, 0);
        dma16_m0(kbuf, lds_addr + static_cast<uint32_t>(kScoreTile * kVPitch + n * 1024), koff, 0);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();

    const int j = lane & 15;
    const int g = lane >> 4;
    f32x4_t acc[4][4];  // [key block][query block]
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) acc[tb][sb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    if (active) {
        // Fragment rows: key block tb is tile row (wave & 1) * 64 + 16 tb + j
        // (A), query block sb tile row (wave >> 1) * 64 + 16 sb + j (B); both
        // have row & 15 == j. K-step kk takes logical chunk 4 kk + g.
        const uint8_t* kt = lds + kScoreTile * kVPitch + ((wave & 1) * 64 + j) * kVPitch;
        const uint8_t* qt = lds + ((wave >> 1) * 64 + j) * kVPitch;
#pragma unroll
        for (int kk = 0; kk < kD / 32; ++kk) {
            const int off = ((4 * kk + g) ^ j) << 4;
            bf16x8_t a[4];
            bf16x8_t bq[4];
#pragma unroll
            for (int blk = 0; blk < 4; ++blk) {
                a[blk] = *reinterpret_cast<const bf16x8_t*>(kt + blk * 16 * kVPitch + off);
                bq[blk] = *reinterpret_cast<const bf16x8_t*>(qt + blk * 16 * kVPitch + off);
            }
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
                for (int sb = 0; sb < 4; ++sb) {
                    acc[tb][sb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tb], bq[sb], acc[tb][sb], 0, 0, 0);
                }
            }
        }
    }
    __syncthreads();  // every wave is done with the tiles before they are overwritten
    if (!active) return;

    // acc[tb][sb] lane holds S[s0 + 16 sb + j][t0 + 16 tb + 4 g .. +3]. The
    // wave's 64 x 64 tile goes through its own LDS area (rows of 128 bytes,
    // 16-byte chunk c of row r at c ^ (r & 7)) so that the stores write
    // whole 128-byte row pieces.
    uint8_t* stage = lds + wave * (64 * 128);
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        const int row = 16 * sb + j;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const int chunk = (2 * tb + (g >> 1)) ^ (row & 7);
            *reinterpret_cast<uint2*>(stage + row * 128 + chunk * 16 + (g & 1) * 8) =
                make_uint2(f32x2_to_bf16x2_canon(acc[tb][sb][0], acc[tb][sb][1]),
                           f32x2_to_bf16x2_canon(acc[tb][sb][2], acc[tb][sb][3]));
        }
    }
    // Only this wave reads what it wrote; the fence keeps the compiler from
    // moving the reads above the writes.
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // seq is a multiple of 8, so eight keys never straddle its end.
    uint16_t* out = scores + bh * seq * seq;
    const int c = lane & 7;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = 8 * i + (lane >> 3);
        const int64_t s = s0 + row;
        const int64_t t = t0 + 8 * c;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + row * 128 + ((c ^ (row & 7)) << 4));
        if (s < seq && t < seq) *reinterpret_cast<uint4*>(out + s * seq + t) = v;
    }
}

/// out rows s0 .. s0 + 63 of one (batch, head). blockIdx.x = rank * BH + bh
/// with rank 0 the last (longest) row tile, so the heaviest workgroups start
/// first.
template <int kD>
__global__ __launch_bounds__(kThreads) void attention_pv_kernel(const uint16_t* __restrict__ probs,
                                                                const uint16_t* __restrict__ v,
                                                                uint16_t* __restrict__ out, int64_t seq,
                                                                int64_t heads, int64_t bh_count, int tiles) {
    __shared__ __attribute__((aligned(16))) uint8_t vt[2][kPvChunk * kVPitch];  // 2 x 16 KiB

    const int64_t bh = blockIdx.x % bh_count;
    const int tile = tiles - 1 - static_cast<int>(blockIdx.x / bh_count);
    const int64_t s_first = static_cast<int64_t>(tile) * kPvRows;
    const int64_t s_end = s_first + kPvRows < seq ? s_first + kPvRows : seq;  // > s_first
    const int chunks = static_cast<int>(ceil_div<int64_t>(s_end, kPvChunk));

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int j = lane & 15;
    const int g = lane >> 4;
    const int64_t b = bh / heads;
    const int64_t h = bh % heads;
    const int64_t pitch = heads * kD;
    const int64_t head0 = (b * seq * heads + h) * kD;
    const i32x4_t vbuf = uniform(raw_buffer_words(v + head0, head_extent(seq, heads, kD)));
    const __amdgpu_buffer_rsrc_t pbuf =
        make_buffer(probs + bh * seq * seq, static_cast<uint32_t>(seq * seq * 2));
    const uint32_t lds_addr = static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u8_t*)&vt[0][0]));

    // v chunk c (64 keys) HBM -> LDS slot by buffer loads with the LDS
    // destination: load n (0..15, four per wave) fills rows 4 n .. 4 n + 3;
    // lane l lands at byte 16 l, i.e. row 4 n + l / 16, physical chunk
    // l % 16, so it reads logical chunk (l % 16) ^ v_swizzle(row). Keys past
    // seq and chunks past the head (head_dim < 128) read as zero.
    auto load_v = [&](int c, int slot) {
#pragma unroll
        for (int i = 0; i < kPvChunk / 16; ++i) {
            const int n = (kPvChunk / 16) * wave + i;
            const int row = 4 * n + (lane >> 4);
            const int chunk = (lane & 15) ^ v_swizzle(row);
            const int64_t t = static_cast<int64_t>(c) * kPvChunk + row;
            const uint32_t off =
                t < seq && chunk < kD / 8 ? static_cast<uint32_t>((t * pitch + 8 * chunk) * 2) : kPastEnd;
            dma16_m0(vbuf, lds_addr + static_cast<uint32_t>(slot * kPvChunk * kVPitch + n * 1024), off, 0);
        }
    };

    // This lane's query row (B column) and its probabilities for sub-step u
    // of chunk c: keys 64 c + 32 u + 8 g .. +7, those past the row's own
    // position zeroed.
    const int64_t s = s_first + 16 * wave + j;
    auto load_p = [&](int c, int u) {
        const int64_t t_first = static_cast<int64_t>(c) * kPvChunk + 32 * u + 8 * g;
        // Keys past seq lie past the row (and past s): masked below.
        const uint32_t off = s < seq ? static_cast<uint32_t>((s * seq + t_first) * 2) : kPastEnd;
        const uint4 raw = buffer_load16(pbuf, off, 0);
        const int64_t keep = s - t_first + 1;  // keys t_first .. s are kept
        uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t lo = 2 * e < keep ? 0x0000FFFFu : 0u;
            const uint32_t hi = 2 * e + 1 < keep ? 0xFFFF0000u : 0u;
            w[e] &= lo | hi;
        }
        return as_bf16x8(make_uint4(w[0], w[1], w[2], w[3]));
    };

    // V^T fragment of head dims 16 db .. +15 (A rows) over keys 32 u + 8 g
    // .. +7 of the chunk: lane j of group g reads key rows 32 u + 8 g + j / 4
    // (and 4 more), dims 16 db + 4 (j % 4) .. +3, and receives dim
    // 16 db + j's 4 keys. Rows 32 apart share the swizzle.
    const int vrow = 8 * g + (j >> 2);
    const int vsw = v_swizzle(vrow);  // the same for vrow + 4
    constexpr int kBlocks = kD / 16;
    f32x4_t acc[kBlocks];
#pragma unroll
    for (int db = 0; db < kBlocks; ++db) acc[db] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    load_v(0, 0);
    bf16x8_t pcur[kPvSub];
#pragma unroll
    for (int u = 0; u < kPvSub; ++u) pcur[u] = load_p(0, u);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    for (int c = 0; c < chunks; ++c) {
        const bool more = c + 1 < chunks;  // workgroup-uniform
        bf16x8_t pnext[kPvSub];
#pragma unroll
        for (int u = 0; u < kPvSub; ++u) pnext[u] = pcur[u];
        if (more) {
            // Slot (c + 1) % 2 was last read in step c - 1, before the
            // barrier that ended it.
            load_v(c + 1, (c + 1) & 1);
#pragma unroll
            for (int u = 0; u < kPvSub; ++u) pnext[u] = load_p(c + 1, u);
        }
        const uint8_t* tile_v = vt[c & 1];
#pragma unroll
        for (int u = 0; u < kPvSub; ++u) {
#pragma unroll
            for (int db = 0; db < kBlocks; ++db) {
                const int chunk = 2 * db + ((j & 3) >> 1);
                const int off = (32 * u + vrow) * kVPitch + ((chunk ^ vsw) << 4) + (j & 1) * 8;
                const s16x4_t lo = lds_read_tr(tile_v, off);
                const s16x4_t hi = lds_read_tr(tile_v, off + 4 * kVPitch);
                const bf16x8_t vfrag =
                    __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag, pcur[u], acc[db], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));  // the next chunk has landed
        __syncthreads();
#pragma unroll
        for (int u = 0; u < kPvSub; ++u) pcur[u] = pnext[u];
    }

    // acc[db] lane holds out[s][16 db + 4 g .. +3].
    if (s < seq) {
        uint16_t* row = out + head0 + s * pitch;
#pragma unroll
        for (int db = 0; db < kBlocks; ++db) store4_bf16(row + 16 * db + 4 * g, acc[db]);
    }
}

/// Shared argument checks; CF_OK when the kernels take the shape.
cf_status validate(const char* who, const void* a, const void* b, const void* out, cf_dtype dtype, int64_t batch,
                   int64_t seq, int64_t heads, int64_t head_dim) {
    CF_REQUIRE(a != nullptr && b != nullptr && out != nullptr, "%s: null pointer", who);
    CF_REQUIRE(batch > 0 && seq > 0 && heads > 0 && head_dim > 0, "%s: non-positive size", who);
    if (dtype != CF_BF16) {
        return fail(CF_ERR_UNSUPPORTED, "%s: dtype %s has no kernel (bfloat16 only)", who, dtype_name(dtype));
    }
    if (!(head_dim == 32 || head_dim == 64 || head_dim == 96 || head_dim == 128) || seq % 8 != 0) {
        return fail(CF_ERR_UNSUPPORTED, "%s: head_dim %lld (32, 64, 96 or 128) and seq %lld (a multiple of 8) "
                    "have no kernel", who, static_cast<long long>(head_dim), static_cast<long long>(seq));
    }
    CF_REQUIRE(host_aligned(a, 16) && host_aligned(b, 16) && host_aligned(out, 16),
               "%s: tensors must be 16-byte aligned", who);
    // Buffer offsets are 32-bit: one (batch, head) slice of either layout,
    // and the grids, must stay below 2^31.
    CF_REQUIRE(seq * heads * head_dim * 2 < (1LL << 31) && seq * seq * 2 < (1LL << 31) &&
                   batch * heads * ceil_div<int64_t>(seq, kPvRows) * ceil_div<int64_t>(seq, kPvRows) < (1LL << 31),
               "%s: batch %lld, seq %lld, heads %lld exceed the kernel's 32-bit offsets", who,
               static_cast<long long>(batch), static_cast<long long>(seq), static_cast<long long>(heads));
    return CF_OK;
}

}  // namespace
}  // namespace cf

extern "C" {

cf_status cf_attention_scores_causal(const void* q, const void* k, void* scores, cf_dtype dtype, int64_t batch,
                                     int64_t seq, int64_t heads, int64_t head_dim, void* stream) {
    CF_ENTRY();
    if (batch == 0 || seq == 0 || heads == 0) return CF_OK;
    const cf_status st = cf::validate("cf_attention_scores_causal", q, k, scores, dtype, batch, seq, heads, head_dim);
    if (st != CF_OK) return st;
    const int tiles_1d = static_cast<int>(cf::ceil_div<int64_t>(seq, cf::kScoreTile));
    const int tiles = tiles_1d * (tiles_1d + 1) / 2;
    const dim3 grid(static_cast<unsigned>(batch * heads * tiles));
    auto s = static_cast<hipStream_t>(stream);
    const auto* qp = static_cast<const uint16_t*>(q);
    const auto* kp = static_cast<const uint16_t*>(k);
    auto* sp = static_cast<uint16_t*>(scores);
    switch (head_dim) {
        case 32: cf::launch(cf::attention_scores_kernel<32>, grid, dim3(cf::kThreads), 0, s, qp, kp, sp, seq, heads, tiles); break;
        case 64: cf::launch(cf::attention_scores_kernel<64>, grid, dim3(cf::kThreads), 0, s, qp, kp, sp, seq, heads, tiles); break;
        case 96: cf::launch(cf::attention_scores_kernel<96>, grid, dim3(cf::kThreads), 0, s, qp, kp, sp, seq, heads, tiles); break;
        default: cf::launch(cf::attention_scores_kernel<128>, grid, dim3(cf::kThreads), 0, s, qp, kp, sp, seq, heads, tiles); break;
    }
    return cf::check_launch("launching the causal attention scores", s);
}

cf_status cf_attention_pv_causal(const void* probs, const void* v, void* out, cf_dtype dtype, int64_t batch,
                                 int64_t seq, int64_t heads, int64_t head_dim, void* stream) {
    CF_ENTRY();
    if (batch == 0 || seq == 0 || heads == 0) return CF_OK;
    const cf_status st = cf::validate("cf_attention_pv_causal", probs, v, out, dtype, batch, seq, heads, head_dim);
    if (st != CF_OK) return st;
    const int tiles = static_cast<int>(cf::ceil_div<int64_t>(seq, cf::kPvRows));
    const int64_t bh = batch * heads;
    const dim3 grid(static_cast<unsigned>(bh * tiles));
    auto s = static_cast<hipStream_t>(stream);
    const auto* pp = static_cast<const uint16_t*>(probs);
    const auto* vp = static_cast<const uint16_t*>(v);
    auto* op = static_cast<uint16_t*>(out);
    switch (head_dim) {
        case 32: cf::launch(cf::attention_pv_kernel<32>, grid, dim3(cf::kThreads), 0, s, pp, vp, op, seq, heads, bh, tiles); break;
        case 64: cf::launch(cf::attention_pv_kernel<64>, grid, dim3(cf::kThreads), 0, s, pp, vp, op, seq, heads, bh, tiles); break;
        case 96: cf::launch(cf::attention_pv_kernel<96>, grid, dim3(cf::kThreads), 0, s, pp, vp, op, seq, heads, bh, tiles); break;
        default: cf::launch(cf::attention_pv_kernel<128>, grid, dim3(cf::kThreads), 0, s, pp, vp, op, seq, heads, bh, tiles); break;
    }
    return cf::check_launch("launching the causal attention values", s);
}

}  // extern "C"

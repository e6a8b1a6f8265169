// LDS-staging helpers shared by the MFMA GEMM kernels (cf_lora_fused.hip,
// cf_matmul_fp8.hip): HBM -> LDS copies by buffer loads with the LDS
// destination, memory-counter waits, a bare barrier and the XCD-aware tile
// order.
#pragma once

#include "cf_common.hpp"

namespace cf {

// A buffer offset past every range: the load returns zeros.
constexpr uint32_t kOutOfRange = 0x80000000u;

/// s_waitcnt immediate that waits until at most n vector-memory operations
/// of this wave are outstanding (lgkm and exp counters not waited on).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

/// Buffer resource words for a raw (stride 0) buffer of `bytes` bytes.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4_t raw_buffer_words(const void* base, uint32_t bytes) {
    const uint64_t addr = reinterpret_cast<uint64_t>(base);
    return i32x4_t{static_cast<int>(addr & 0xffffffffu), static_cast<int>((addr >> 32) & 0xffffu),
                   static_cast<int>(bytes), kRawBufferFormat};
}

/// A buffer descriptor in scalar registers: the DMA takes it as an SGPR
/// operand; the value is wave-uniform, but the compiler cannot always prove
/// it (and an "s" operand it holds in VGPRs does not assemble).
__device__ __forceinline__ i32x4_t uniform(i32x4_t v) {
    return i32x4_t{__builtin_amdgcn_readfirstlane(v[0]), __builtin_amdgcn_readfirstlane(v[1]),
                   __builtin_amdgcn_readfirstlane(v[2]), __builtin_amdgcn_readfirstlane(v[3])};
}

/// HBM -> LDS copy of 16 (or 4) bytes per lane: lane l's bytes land at LDS
/// byte lds_dst + 16 l (4 l), read from buffer offset voffset + soffset
/// (zeros when out of range). On gfx950 the range check takes the sum: a lane
/// whose voffset is in range reads zeros once soffset carries it past the
/// buffer's size, for these copies and for plain buffer loads alike
/// (measured with in-bounds offsets), so a row offset may travel in soffset
/// and still be clipped at the buffer's end. Issued from inline assembly on purpose: the
/// compiler conservatively drains every LDS DMA in flight (vmcnt(0)) before
/// each transposed LDS read it emits, which would serialise the prefetch
/// pipeline; DMA it does not know about cannot trigger that. The caller
/// orders the copies itself (s_waitcnt vmcnt + barrier before the stage is
/// read); compiler-generated vmcnt waits only become more conservative.
/// The LDS base travels as an M0 operand: the compiler writes M0 itself (one
/// scalar instruction, often folded into the address add) and knows its
/// value afterwards, so nothing is saved or restored around the copy. The
/// s_nop 4 gives the five wait states a vector-memory instruction needs
/// after a VALU instruction writes an SGPR it reads (v_readlane of a spilled
/// SGPR, v_readfirstlane), and so also the one an M0 write needs: the
/// compiler's hazard recognizer does not look inside inline assembly, and a
/// kernel variant whose spill reloads fed the scalar offset one to four
/// instructions before the copy read stale offsets (wrong rows, no fault).
__device__ __forceinline__ void dma16_m0(i32x4_t rsrc, uint32_t lds_dst, uint32_t voffset,
                                         uint32_t soffset) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_dst)
                 : "memory");
}

/// dma16_m0 at device scope (sc1): reads what another workgroup published
/// with device-scope stores, past this XCD's L2.
__device__ __forceinline__ void dma16_device_m0(i32x4_t rsrc, uint32_t lds_dst, uint32_t voffset,
                                                uint32_t soffset) {
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen sc1 lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_dst)
                 : "memory");
}

__device__ __forceinline__ void dma4_m0(i32x4_t rsrc, uint32_t lds_dst, uint32_t voffset,
                                        uint32_t soffset) {
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :
                 : "v"(voffset), "s"(rsrc), "s"(soffset), "{m0}"(lds_dst)
                 : "memory");
}

/// Workgroup barrier that neither waits on memory counters nor lets the
/// compiler move memory accesses across it; the caller has already waited
/// for what the other waves must see.
__device__ __forceinline__ void bare_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
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

}  // namespace cf

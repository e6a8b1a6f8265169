// Shared device and host infrastructure for the gfx950 kernels.
//
// Device side: wave64 cross-lane reductions built on DPP (data-parallel
// primitives: a lane reads a neighbour's register inside the same VALU
// instruction, no LDS traffic, no barrier), 16-bit float conversions with
// explicit round-to-nearest-even, and 128-bit vector load/store types.
//
// Host side: the thread-local error slot behind cf_last_error(), the
// launch-check helper and cached per-device facts.
//
// The reference builds its reductions for 32-lane warps with
// __shfl_down_sync (cuda/include/cudaforge/cuda_utils.cuh:27-115) and a
// shared-memory exchange between warps. A CDNA4 wavefront has 64 lanes in
// four DPP "rows" of 16, so a 64-element quantisation block or a 16-lane
// group reduces with 4 DPP steps and no LDS at all, and a whole wave reduces
// with 4 more reads of one lane per row.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <tuple>
#include <type_traits>
#include <utility>

#include "../../include/cudaforge_hip.h"

namespace cf {

/// Lanes per wavefront on CDNA (gfx9 family, gfx950 included). The reference
/// hard-codes 32 (cpp/include/cudaforge/launch_config.hpp:22); every
/// reduction here is written for 64.
inline constexpr int kWaveSize = 64;

/// Elements per quantisation scale; kQuantBlockSize in the reference
/// (cuda/include/cudaforge/quantization.cuh:18).
inline constexpr int kQuantBlockSize = 64;

/// Default workgroup size for the streaming kernels: four waves, one per SIMD
/// of a CU.
inline constexpr int kDefaultBlockSize = 256;

/// Largest workgroup HIP permits on gfx950.
inline constexpr int kMaxBlockSize = 1024;

// ---------------------------------------------------------------------------
// Device: DPP cross-lane moves and reductions.
// ---------------------------------------------------------------------------

// DPP control words (GFX9 encoding).
inline constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1,0,3,2]
inline constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2,3,0,1]
inline constexpr int kDppRowRor4 = 0x124;       // rotate by 4 within a 16-lane row
inline constexpr int kDppRowRor8 = 0x128;       // rotate by 8 within a 16-lane row
inline constexpr int kDppRowHalfMirror = 0x141; // reverse each 8-lane half row

/// v from another lane of the same 16-lane row (the controls above never
/// address a lane outside it). bound_ctrl is set because that lets the
/// compiler fold the move into the reduction instruction that consumes it
/// (v_max_u32_dpp, v_add_f32_dpp: one VALU instruction per step instead of
/// two); with no out-of-row source it changes no value.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, 0xF, 0xF, true));
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<kCtrl>(__float_as_uint(v)));
}

struct MaxU32 {
    __device__ __forceinline__ static uint32_t apply(uint32_t a, uint32_t b) {
        return a > b ? a : b;
    }
};

struct AddF32 {
    __device__ __forceinline__ static float apply(float a, float b) { return a + b; }
};

struct MaxF32 {
    // fmaxf drops a NaN operand. Softmax inputs are never NaN in the configs;
    // where NaN must propagate (quantisation absmax) the kernels reduce the
    // integer bit pattern with MaxU32 instead.
    __device__ __forceinline__ static float apply(float a, float b) { return fmaxf(a, b); }
};

/// Reduce across groups of `kLanes` consecutive lanes (4, 8 or 16). Every
/// lane of the group ends with the group's result. All 64 lanes must be
/// active.
template <int kLanes, typename Op>
__device__ __forceinline__ uint32_t group_reduce_u32(uint32_t v) {
    static_assert(kLanes == 4 || kLanes == 8 || kLanes == 16, "group of 4, 8 or 16 lanes");
    v = Op::apply(v, dpp_u32<kDppQuadXor1>(v));
    v = Op::apply(v, dpp_u32<kDppQuadXor2>(v));
    if constexpr (kLanes == 8) {
        v = Op::apply(v, dpp_u32<kDppRowHalfMirror>(v));
    } else if constexpr (kLanes == 16) {
        v = Op::apply(v, dpp_u32<kDppRowRor4>(v));
        v = Op::apply(v, dpp_u32<kDppRowRor8>(v));
    }
    return v;
}

template <int kLanes, typename Op>
__device__ __forceinline__ float group_reduce_f32(float v) {
    static_assert(kLanes == 4 || kLanes == 8 || kLanes == 16, "group of 4, 8 or 16 lanes");
    v = Op::apply(v, dpp_f32<kDppQuadXor1>(v));
    v = Op::apply(v, dpp_f32<kDppQuadXor2>(v));
    if constexpr (kLanes == 8) {
        v = Op::apply(v, dpp_f32<kDppRowHalfMirror>(v));
    } else if constexpr (kLanes == 16) {
        v = Op::apply(v, dpp_f32<kDppRowRor4>(v));
        v = Op::apply(v, dpp_f32<kDppRowRor8>(v));
    }
    return v;
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

/// Whole-wave reduction; the result is uniform across the wave. The four row
/// results are combined in a fixed order, so the result is deterministic.
template <typename Op>
__device__ __forceinline__ float wave_reduce_f32(float v) {
    v = group_reduce_f32<16, Op>(v);
    const float r0 = readlane_f32(v, 0);
    const float r1 = readlane_f32(v, 16);
    const float r2 = readlane_f32(v, 32);
    const float r3 = readlane_f32(v, 48);
    return Op::apply(Op::apply(r0, r1), Op::apply(r2, r3));
}

/// Workgroup-wide reduction for kWaves waves through a kWaves-float LDS slot.
/// The result is returned to every thread. The trailing barrier lets the
/// caller reuse `slot` for a following reduction (the reference's second
/// barrier, cuda/include/cudaforge/cuda_utils.cuh:79-86, for the same reason).
template <int kWaves, typename Op>
__device__ __forceinline__ float block_reduce_f32(float v, float* slot) {
    v = wave_reduce_f32<Op>(v);
    if constexpr (kWaves == 1) {
        return v;
    } else {
        const int wave = static_cast<int>(threadIdx.x) / kWaveSize;
        if ((threadIdx.x & (kWaveSize - 1)) == 0) slot[wave] = v;
        __syncthreads();
        float total = slot[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) total = Op::apply(total, slot[w]);
        __syncthreads();
        return total;
    }
}

/// Workgroup-wide OR of a per-thread predicate, the same result on every
/// thread, through kWaves int slots of LDS that no other code reads or
/// writes between the call's two barriers (__syncthreads_or would add LDS of
/// its own, which costs kernels sized to the CU's 160 KiB a workgroup).
/// Every thread of the workgroup must call it.
template <int kWaves>
__device__ __forceinline__ bool workgroup_any(bool pred, int* slots) {
    const int wave = static_cast<int>(threadIdx.x) / kWaveSize;
    const bool any = __builtin_amdgcn_ballot_w64(pred) != 0;
    if ((threadIdx.x & (kWaveSize - 1)) == 0) slots[wave] = any ? 1 : 0;
    __syncthreads();
    int total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) total |= slots[w];
    __syncthreads();  // every wave has read the slots before they are reused
    return total != 0;
}

/// Workgroup barrier after LDS writes that does not wait for global loads:
/// s_waitcnt lgkmcnt(0) (this wave's LDS writes are done), then s_barrier.
/// __syncthreads() would also wait for every outstanding global load
/// (vmcnt(0)), which defeats loads meant to stay in flight across the
/// barrier. The empty asm statements keep the compiler from moving memory
/// accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    // vmcnt field at its maximum (no wait), expcnt 7 (no wait), lgkmcnt 0.
    __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Device: 16-bit float storage.
// ---------------------------------------------------------------------------

struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

/// fp32 -> bf16 with round-to-nearest-even; NaN becomes the canonical quiet
/// NaN 0x7FC0. Bit-identical to c10::BFloat16's conversion, which is what the
/// reference's `.to(torch.bfloat16)` uses.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

/// Two fp32 values -> two bf16 in one packed word (low half from `lo`) by
/// v_cvt_pk_bf16_f32. Bit-identical to f32_to_bf16_bits on every input
/// except NaN (checked on all 2^32 fp32 patterns on gfx950): the instruction
/// keeps a NaN's sign and payload where f32_to_bf16_bits returns 0x7FC0, so a
/// caller that can meet NaN must take f32_to_bf16_bits for it.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    typedef float f32x2_v __attribute__((ext_vector_type(2)));
    const f32x2_v f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_v));
}

/// f32_to_bf16_bits of two values, packed (first value in the low half):
/// bit-identical on every input, NaN -> 0x7FC0 included. NaNs are replaced by
/// the canonical quiet NaN before one v_cvt_pk_bf16_f32 (which would keep a
/// payload): about 2.5 VALU instructions per value against the software
/// rounding's 6, for epilogues that round whole output tiles.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_canon(float lo, float hi) {
    const float canon = __uint_as_float(0x7FC00000u);
    return f32x2_to_bf16x2_bits(lo != lo ? canon : lo, hi != hi ? canon : hi);
}

/// The bf16 high/low split of two fp32 values, hi = bf16(v) and
/// lo = bf16(v - hi), as packed words (first value in the low half), for the
/// kernels that run fp32 products as three bf16 MFMAs (hi*hi + hi*lo +
/// lo*hi). Two v_cvt_pk_bf16_f32 do the rounding: bit-identical to
/// f32_to_bf16_bits except that a NaN keeps its payload, which changes
/// nothing downstream (a NaN element gives NaN products either way). One
/// conversion per two values instead of the software rounding's several
/// instructions per value: these kernels spend their VALU time on the split.
///
/// Values outside bf16's finite range (|v| above 0x7F7F, +-inf) take another
/// split, so that the three products follow fp32 arithmetic (inf * w = +-inf
/// for w != 0, inf * 0 = NaN, a finite huge v times w finite):
///   * finite |v| > 0x7F7F: hi = +-0x7F7F, lo = bf16(v - hi), the finite
///     remainder (plain rounding would give hi = inf, lo = -inf);
///   * v = +-inf: hi = +-1, lo = +-inf (with hi = +-0x7F7F the other
///     operand's lo times it could overflow to an infinity of the wrong sign).
/// A NaN keeps the plain split (lo = NaN).
///
/// split_pk_as<false> is the plain split, exact for |v| within bf16's range;
/// split_pk_as<true> handles every value. Kernels pick one per wave: the
/// staging loops fold |v| of a whole K-step into abs_max3 and branch once on
/// wave_outside_bf16 (ordinary inputs pay half an instruction per value);
/// split_pk and split_pk4 make the same choice per call.
__device__ __forceinline__ float split_hi_special(float v) {
    const float big = __uint_as_float(0x7F7F0000u);
    return __builtin_isinf(v) ? __builtin_copysignf(1.0f, v) : __builtin_fminf(__builtin_fmaxf(v, -big), big);
}

/// max(m, |a|, |b|), one v_max3_f32; a NaN is ignored.
__device__ __forceinline__ float abs_max3(float m, float a, float b) {
    return __builtin_fmaxf(m, __builtin_fmaxf(__builtin_fabsf(a), __builtin_fabsf(b)));
}

/// True on every lane when some lane's m lies above bf16's finite range
/// (|v| > 0x7F7F or an infinity folded into m).
__device__ __forceinline__ bool wave_outside_bf16(float m) {
    return __builtin_amdgcn_ballot_w64(m > __uint_as_float(0x7F7F0000u)) != 0;
}

template <bool kWide>
__device__ __forceinline__ void split_pk_as(float v0, float v1, uint32_t& hi, uint32_t& lo) {
    if constexpr (kWide) {
        hi = f32x2_to_bf16x2_bits(split_hi_special(v0), split_hi_special(v1));
    } else {
        hi = f32x2_to_bf16x2_bits(v0, v1);
    }
    lo = f32x2_to_bf16x2_bits(v0 - __uint_as_float(hi << 16), v1 - __uint_as_float(hi & 0xFFFF0000u));
}

__device__ __forceinline__ void split_pk(float v0, float v1, uint32_t& hi, uint32_t& lo) {
    if (wave_outside_bf16(abs_max3(0.0f, v0, v1))) {
        split_pk_as<true>(v0, v1, hi, lo);
    } else {
        split_pk_as<false>(v0, v1, hi, lo);
    }
}

/// Four values (x, y into hi.x / lo.x; z, w into hi.y / lo.y), one choice.
__device__ __forceinline__ void split_pk4(float v0, float v1, float v2, float v3, uint2& hi, uint2& lo) {
    if (wave_outside_bf16(abs_max3(abs_max3(0.0f, v0, v1), v2, v3))) {
        split_pk_as<true>(v0, v1, hi.x, lo.x);
        split_pk_as<true>(v2, v3, hi.y, lo.y);
    } else {
        split_pk_as<false>(v0, v1, hi.x, lo.x);
        split_pk_as<false>(v2, v3, hi.y, lo.y);
    }
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
}

/// fp32 -> fp16, round-to-nearest-even (v_cvt_f16_f32 under the default
/// mode); a NaN becomes its sign over the quiet NaN 0x7E00, the rule of
/// c10::Half's conversion (what `.to(torch.float16)` gives), which the
/// hardware conversion does not follow for every NaN.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
    const uint32_t h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
    return f != f ? (((__float_as_uint(f) >> 16) & 0x8000u) | 0x7E00u) : h;
}

/// Storage traits: element type, how many fit a 16-byte vector, conversions.
template <typename T>
struct Storage;

template <>
struct Storage<float> {
    using elem = float;
    static constexpr int kPerVec = 4;
    __device__ __forceinline__ static float load(const float* p) { return *p; }
    __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};

template <>
struct Storage<bf16_t> {
    using elem = uint16_t;
    static constexpr int kPerVec = 8;
    __device__ __forceinline__ static float load(const bf16_t* p) {
        return bf16_bits_to_f32(p->bits);
    }
    __device__ __forceinline__ static void store(bf16_t* p, float v) {
        p->bits = static_cast<uint16_t>(f32_to_bf16_bits(v));
    }
    __device__ __forceinline__ static float from_bits(uint32_t h) { return bf16_bits_to_f32(h); }
    __device__ __forceinline__ static uint32_t to_bits(float v) { return f32_to_bf16_bits(v); }
    /// to_bits of two values packed (first in the low half), by one
    /// v_cvt_pk_bf16_f32: same bits, fewer VALU instructions.
    __device__ __forceinline__ static uint32_t to_bits2(float lo, float hi) {
        return f32x2_to_bf16x2_canon(lo, hi);
    }
};

template <>
struct Storage<f16_t> {
    using elem = uint16_t;
    static constexpr int kPerVec = 8;
    __device__ __forceinline__ static float load(const f16_t* p) { return f16_bits_to_f32(p->bits); }
    __device__ __forceinline__ static void store(f16_t* p, float v) {
        p->bits = static_cast<uint16_t>(f32_to_f16_bits(v));
    }
    __device__ __forceinline__ static float from_bits(uint32_t h) { return f16_bits_to_f32(h); }
    __device__ __forceinline__ static uint32_t to_bits(float v) { return f32_to_f16_bits(v); }
    __device__ __forceinline__ static uint32_t to_bits2(float lo, float hi) {
        return to_bits(lo) | (to_bits(hi) << 16);
    }
};

/// Unpack a 16-byte vector of T into 4 or 8 floats.
template <typename T>
__device__ __forceinline__ void unpack16(const uint4& v, float* out) {
    if constexpr (Storage<T>::kPerVec == 4) {
        out[0] = __uint_as_float(v.x);
        out[1] = __uint_as_float(v.y);
        out[2] = __uint_as_float(v.z);
        out[3] = __uint_as_float(v.w);
    } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = Storage<T>::from_bits(w[i] & 0xFFFFu);
            out[2 * i + 1] = Storage<T>::from_bits(w[i] >> 16);
        }
    }
}

/// Pack 4 or 8 floats into a 16-byte vector of T (rounding to T).
template <typename T>
__device__ __forceinline__ uint4 pack16(const float* in) {
    uint4 v;
    if constexpr (Storage<T>::kPerVec == 4) {
        v.x = __float_as_uint(in[0]);
        v.y = __float_as_uint(in[1]);
        v.z = __float_as_uint(in[2]);
        v.w = __float_as_uint(in[3]);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = Storage<T>::to_bits2(in[2 * i], in[2 * i + 1]);
        }
        v.x = w[0];
        v.y = w[1];
        v.z = w[2];
        v.w = w[3];
    }
    return v;
}

__device__ __forceinline__ bool aligned16(const void* p) {
    return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// ---------------------------------------------------------------------------
// Device: streaming (nontemporal) loads and stores.
//
// Data that is touched exactly once goes through global_load/store with the
// nontemporal hint, so it does not displace reused lines (weights, scales)
// in L2 and the Infinity Cache. Measured on MI355X with one-shot grids: a
// 256 MiB copy moves 5.97 TB/s with the hint on both sides against 5.54 TB/s
// without it.
// ---------------------------------------------------------------------------

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 load_stream16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(static_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void store_stream16(void* p, const uint4& v) {
    const u32x4_t w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, static_cast<u32x4_t*>(p));
}

__device__ __forceinline__ uint2 load_stream8(const void* p) {
    const u32x2_t v = __builtin_nontemporal_load(static_cast<const u32x2_t*>(p));
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ void store_stream8(void* p, const uint2& v) {
    const u32x2_t w = {v.x, v.y};
    __builtin_nontemporal_store(w, static_cast<u32x2_t*>(p));
}

// ---------------------------------------------------------------------------
// Device: buffer loads.
//
// A buffer resource (4 SGPRs: base, range in bytes, format word) lets a load
// address memory with a 32-bit per-lane VGPR offset plus a uniform SGPR
// offset, instead of a 64-bit VGPR address per load; loads whose lane offset
// falls outside the range return zero without faulting. The GEMM kernels use
// this to keep their prefetch addressing in a handful of registers.
// ---------------------------------------------------------------------------

/// Word 3 of a raw (untyped, unswizzled) buffer resource on gfx9-family parts.
inline constexpr int kRawBufferFormat = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(bytes), kRawBufferFormat);
}

__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset,
                                               uint32_t soffset) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

/// Cache-policy operand of the buffer intrinsics on gfx950: bit 1 is the
/// non-temporal (streaming) hint; bit 4 (sc1) gives the access device
/// scope: a store is acknowledged once it is visible to every CU of the GPU
/// (whichever XCD's L2 they sit behind), a load reads that level.
inline constexpr int kCacheNonTemporal = 2;
inline constexpr int kCacheDeviceScope = 16;

/// buffer_load16 with the non-temporal hint, for operands read exactly once
/// (the LoRA backward's passes over dy and x: 37.9 -> 34.7 us at 8192 x 4096
/// x 4096 against plain loads, bit-identical).
__device__ __forceinline__ uint4 buffer_load16_stream(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset,
                                                      uint32_t soffset) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, kCacheNonTemporal);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint16_t buffer_load2(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset,
                                                 uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b16(rsrc, voffset, soffset, 0);
}

__device__ __forceinline__ uint32_t load_stream4(const void* p) {
    return __builtin_nontemporal_load(static_cast<const uint32_t*>(p));
}

__device__ __forceinline__ void store_stream4(void* p, uint32_t v) {
    __builtin_nontemporal_store(v, static_cast<uint32_t*>(p));
}

// ---------------------------------------------------------------------------
// Host: errors, launch checks, device facts.
// ---------------------------------------------------------------------------

/// Record a failure for cf_last_error() and return its status.
cf_status fail(cf_status status, const char* format, ...) __attribute__((format(printf, 2, 3)));

/// Record a HIP failure (with its hipError_t) and return CF_ERR_HIP.
cf_status fail_hip(hipError_t error, const char* what);

/// After a launch: report launch-configuration errors, and with
/// CUDAFORGE_DEBUG_SYNC set also wait for the stream and report faults.
cf_status check_launch(const char* what, hipStream_t stream);

/// Compute units of the current device (cached per device, thread-safe).
int cu_count();

/// Events armed by cf_time_next_launch() for the calling thread's next
/// kernel launch; both null when none is armed.
struct LaunchEvents {
    hipEvent_t start;
    hipEvent_t stop;
};

/// Hand out and disarm the calling thread's armed events.
LaunchEvents take_launch_events();

/// Events for the kernel about to launch: the start event once (the entry
/// point's first kernel records its start), the stop event to every launch
/// until the entry point returns (the last kernel's completion stays
/// recorded), so an entry point of several kernels is timed whole.
LaunchEvents next_launch_events();

/// True when cf_time_next_launch() left events armed on the calling thread.
bool launch_events_armed();

/// Scope of one operator entry point: events armed by cf_time_next_launch()
/// belong to the entry point's first kernel launch, and an entry point that
/// returns without launching (empty input, invalid argument, unsupported
/// shape) disarms them on the way out, so they never time an unrelated
/// later launch.
struct EntryScope {
    EntryScope() = default;
    EntryScope(const EntryScope&) = delete;
    EntryScope& operator=(const EntryScope&) = delete;
    ~EntryScope() { take_launch_events(); }
};

/// Keep a launch error that did not go through hipGetLastError for the next
/// check_launch() on this thread.
void note_launch_error(hipError_t error);

/// Launch `kernel` on `stream`. When cf_time_next_launch() armed events on
/// this thread, the dispatch itself records them (hipExtLaunchKernel): the
/// entry point's first kernel its start, each kernel its completion, so their
/// elapsed time is the entry point's GPU time from its first kernel's start to
/// its last kernel's end, without the queue packets an event pair around the
/// call adds.
template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds_bytes,
                   hipStream_t stream, Args&&... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "argument count of the kernel");
    const LaunchEvents events = next_launch_events();
    if (events.start == nullptr && events.stop == nullptr) {
        kernel<<<grid, block, lds_bytes, stream>>>(std::forward<Args>(args)...);
        return;
    }
    std::tuple<KArgs...> values(std::forward<Args>(args)...);
    void* pointers[sizeof...(KArgs)];
    std::apply(
        [&](auto&... v) {
            int i = 0;
            ((pointers[i++] = static_cast<void*>(&v)), ...);
        },
        values);
    const hipError_t error =
        hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, pointers, lds_bytes,
                           stream, events.start, events.stop, 0);
    if (error != hipSuccess) note_launch_error(error);
}

/// True when `dtype` is one of the three storage types.
inline bool valid_dtype(cf_dtype dtype) {
    return dtype == CF_F32 || dtype == CF_F16 || dtype == CF_BF16;
}

inline const char* dtype_name(cf_dtype dtype) {
    switch (dtype) {
        case CF_F32:
            return "float32";
        case CF_F16:
            return "float16";
        case CF_BF16:
            return "bfloat16";
    }
    return "unknown";
}

inline size_t dtype_size(cf_dtype dtype) { return dtype == CF_F32 ? 4 : 2; }

inline bool host_aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

template <typename T>
constexpr T ceil_div(T a, T b) {
    return (a + b - 1) / b;
}

}  // namespace cf

/// First statement of every entry point that launches kernels.
#define CF_ENTRY() const ::cf::EntryScope cf_entry_scope_

/// Return early with CF_ERR_INVALID_ARGUMENT and a message when `cond` fails.
#define CF_REQUIRE(cond, ...)                                                   \
    do {                                                                        \
        if (!(cond)) return ::cf::fail(CF_ERR_INVALID_ARGUMENT, __VA_ARGS__);   \
    } while (false)

/// Run a host HIP call; on failure return CF_ERR_HIP naming the call.
#define CF_HIP_TRY(expr)                                                        \
    do {                                                                        \
        const hipError_t cf_hip_status_ = (expr);                               \
        if (cf_hip_status_ != hipSuccess) return ::cf::fail_hip(cf_hip_status_, #expr); \
    } while (false)

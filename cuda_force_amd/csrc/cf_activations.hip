// Elementwise activations for gfx950: silu, gelu (tanh form), swiglu.
//
// Semantics: _silu_reference, _gelu_reference and _swiglu_reference
// (python/cudaforge/ops.py:195-212): fp32 arithmetic for every storage type,
// one rounding to the storage type at the end. The reference's kernels are
// cuda/src/activations.cu:36-116.
//
// Design (HBM-bound: 2 bytes in and 2 out per bf16 element, 3 + 3 for
// swiglu): a one-shot grid in which every lane takes kUnroll 16-byte vectors
// 64 vectors apart (each wave instruction covers 1 KiB contiguous), issues
// all of its loads before the first use, and streams them with
// non-temporal hints; waves whose vectors are all in range load
// unconditionally (a guarded load makes the compiler wait for each load
// before issuing the next).
//
// Math: fp32 with the hardware exponential and reciprocal (v_exp_f32,
// v_rcp_f32; ~1e-6 relative against the float64 definitions here). The tanh
// GELU uses the identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)), the same cost
// as SiLU and free of tanh's cancellation near 0.
#include "cf_common.hpp"

namespace cf {
namespace {

constexpr int kUnroll = 4;

__device__ __forceinline__ float sigmoid_times(float x, float t) {
    // x / (1 + exp(-t)); exp overflow gives x * 0 = +-0, as the limit.
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-t));
}

struct Silu {
    __device__ __forceinline__ float operator()(float x, float) const { return sigmoid_times(x, x); }
};

struct GeluTanh {
    __device__ __forceinline__ float operator()(float x, float) const {
        const float k = 0.7978845608028654f;  // sqrt(2 / pi)
        const float u = k * fmaf(0.044715f * x, x * x, x);
        return sigmoid_times(x, 2.0f * u);
    }
};

struct SwiGlu {
    __device__ __forceinline__ float operator()(float g, float u) const { return sigmoid_times(g, g) * u; }
};

template <typename T, typename Op, bool kBinary, bool kFull>
__device__ __forceinline__ void elementwise_body(const T* __restrict__ a, const T* __restrict__ b,
                                                 T* __restrict__ y, int64_t count) {
    constexpr int kPer = Storage<T>::kPerVec;
    const Op op;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWaveSize) +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const int64_t first = wave * kWaveSize * kUnroll + lane;  // vector index
    const int64_t vectors = count / kPer;

    float va[kUnroll][kPer];
    float vb[kUnroll][kPer];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = first + static_cast<int64_t>(u) * kWaveSize;
        if (kFull || v < vectors) {
            unpack16<T>(load_stream16(a + v * kPer), va[u]);
            if (kBinary) unpack16<T>(load_stream16(b + v * kPer), vb[u]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t v = first + static_cast<int64_t>(u) * kWaveSize;
        if (!kFull && v >= vectors) continue;
        float out[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) out[i] = op(va[u][i], kBinary ? vb[u][i] : 0.0f);
        store_stream16(y + v * kPer, pack16<T>(out));
    }
    if (!kFull) {
        // Elements past the last whole vector (count % kPer), by the wave
        // holding the end.
        const int64_t tail = vectors * kPer + lane;
        if (tail < count && first - lane <= vectors && vectors < first - lane + kWaveSize * kUnroll) {
            const float vb1 = kBinary ? Storage<T>::load(b + tail) : 0.0f;
            Storage<T>::store(y + tail, op(Storage<T>::load(a + tail), vb1));
        }
    }
}

template <typename T, typename Op, bool kBinary>
__global__ __launch_bounds__(kDefaultBlockSize) void elementwise_kernel(const T* __restrict__ a,
                                                                        const T* __restrict__ b,
                                                                        T* __restrict__ y,
                                                                        int64_t count) {
    constexpr int kPer = Storage<T>::kPerVec;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWaveSize) +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const bool full = (wave + 1) * kWaveSize * kUnroll * kPer <= count;  // wave-uniform
    if (full) {
        elementwise_body<T, Op, kBinary, true>(a, b, y, count);
    } else {
        elementwise_body<T, Op, kBinary, false>(a, b, y, count);
    }
}

/// Unaligned tensors: one element per thread, grid-stride.
template <typename T, typename Op, bool kBinary>
__global__ __launch_bounds__(kDefaultBlockSize) void elementwise_scalar_kernel(const T* __restrict__ a,
                                                                               const T* __restrict__ b,
                                                                               T* __restrict__ y,
                                                                               int64_t count) {
    const Op op;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t threads = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t e = tid; e < count; e += threads) {
        const float vb = kBinary ? Storage<T>::load(b + e) : 0.0f;
        Storage<T>::store(y + e, op(Storage<T>::load(a + e), vb));
    }
}

template <typename T, typename Op, bool kBinary>
cf_status launch(const void* a, const void* b, void* y, int64_t count, hipStream_t stream,
                 const char* what) {
    constexpr int kPer = Storage<T>::kPerVec;
    const bool vec = host_aligned(a, 16) && host_aligned(y, 16) && (!kBinary || host_aligned(b, 16));
    if (vec) {
        // One wave per kUnroll * 64 vectors; the tail elements ride with the
        // wave holding the end (at least one wave).
        const int64_t per_wave = static_cast<int64_t>(kWaveSize) * kUnroll * kPer;
        const int64_t waves = ceil_div<int64_t>(count + 1, per_wave);
        const int64_t grid = ceil_div<int64_t>(waves, kDefaultBlockSize / kWaveSize);
        CF_REQUIRE(grid < (1LL << 31), "%s: %lld elements exceed the launch limit", what,
                   static_cast<long long>(count));
        cf::launch(elementwise_kernel<T, Op, kBinary>, dim3(static_cast<unsigned>(grid)),
                   dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(a),
                   static_cast<const T*>(b), static_cast<T*>(y), count);
    } else {
        const int64_t wanted = ceil_div<int64_t>(count, kDefaultBlockSize);
        const int64_t cap = static_cast<int64_t>(cu_count()) * 32;
        const int64_t grid = wanted < cap ? wanted : cap;
        cf::launch(elementwise_scalar_kernel<T, Op, kBinary>, dim3(static_cast<unsigned>(grid)),
                   dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(a),
                   static_cast<const T*>(b), static_cast<T*>(y), count);
    }
    return check_launch(what, stream);
}

template <typename Op, bool kBinary>
cf_status run(const void* a, const void* b, void* y, cf_dtype dtype, int64_t count, void* stream,
              const char* what) {
    auto s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case CF_F32:
            return launch<float, Op, kBinary>(a, b, y, count, s, what);
        case CF_BF16:
            return launch<bf16_t, Op, kBinary>(a, b, y, count, s, what);
        case CF_F16:
            return launch<f16_t, Op, kBinary>(a, b, y, count, s, what);
    }
    return fail(CF_ERR_UNSUPPORTED, "%s: unknown dtype %d", what, static_cast<int>(dtype));
}

}  // namespace
}  // namespace cf

extern "C" {

cf_status cf_silu(const void* x, void* y, cf_dtype dtype, int64_t count, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_silu: null pointer");
    return cf::run<cf::Silu, false>(x, nullptr, y, dtype, count, stream, "launching silu");
}

cf_status cf_gelu(const void* x, void* y, cf_dtype dtype, int64_t count, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_gelu: null pointer");
    return cf::run<cf::GeluTanh, false>(x, nullptr, y, dtype, count, stream, "launching gelu");
}

cf_status cf_swiglu(const void* gate, const void* up, void* y, cf_dtype dtype, int64_t count,
                    void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(gate != nullptr && up != nullptr && y != nullptr, "cf_swiglu: null pointer");
    return cf::run<cf::SwiGlu, true>(gate, up, y, dtype, count, stream, "launching swiglu");
}

}  // extern "C"

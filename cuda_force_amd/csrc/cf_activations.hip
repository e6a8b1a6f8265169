// Elementwise activations for gfx950: silu, gelu (tanh form), swiglu.
//
// Semantics: _silu_reference, _gelu_reference and _swiglu_reference
// (python/cudaforge/ops.py:195-212): fp32 arithmetic for every storage type,
// one rounding to the storage type at the end. The reference's kernels are
// cuda/src/activations.cu:36-116.
//
// Design: a grid-stride stream of 16-byte vectors, four in flight per lane;
// each element is read once and written once.
#include "cf_common.hpp"

namespace cf {
namespace {

struct Silu {
    __device__ __forceinline__ float operator()(float x, float) const {
        return x / (1.0f + expf(-x));
    }
};

struct GeluTanh {
    __device__ __forceinline__ float operator()(float x, float) const {
        const float k = 0.7978845608028654f;  // sqrt(2 / pi)
        const float inner = k * (x + 0.044715f * x * x * x);
        return 0.5f * x * (1.0f + tanhf(inner));
    }
};

struct SwiGlu {
    __device__ __forceinline__ float operator()(float g, float u) const {
        return (g / (1.0f + expf(-g))) * u;
    }
};

template <typename T, typename Op, bool kBinary, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void elementwise_kernel(const T* __restrict__ a,
                                                                        const T* __restrict__ b,
                                                                        T* __restrict__ y,
                                                                        int64_t count) {
    constexpr int kPer = Storage<T>::kPerVec;
    const Op op;
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t threads = static_cast<int64_t>(gridDim.x) * blockDim.x;
    if (kVec) {
        const int64_t vectors = count / kPer;
        for (int64_t v = tid; v < vectors; v += threads) {
            float va[kPer];
            float vb[kPer];
            unpack16<T>(reinterpret_cast<const uint4*>(a)[v], va);
            if (kBinary) unpack16<T>(reinterpret_cast<const uint4*>(b)[v], vb);
#pragma unroll
            for (int i = 0; i < kPer; ++i) va[i] = op(va[i], kBinary ? vb[i] : 0.0f);
            reinterpret_cast<uint4*>(y)[v] = pack16<T>(va);
        }
        for (int64_t e = vectors * kPer + tid; e < count; e += threads) {
            const float vb = kBinary ? Storage<T>::load(b + e) : 0.0f;
            Storage<T>::store(y + e, op(Storage<T>::load(a + e), vb));
        }
    } else {
        for (int64_t e = tid; e < count; e += threads) {
            const float vb = kBinary ? Storage<T>::load(b + e) : 0.0f;
            Storage<T>::store(y + e, op(Storage<T>::load(a + e), vb));
        }
    }
}

template <typename T, typename Op, bool kBinary>
cf_status launch(const void* a, const void* b, void* y, int64_t count, hipStream_t stream,
                 const char* what) {
    constexpr int kPer = Storage<T>::kPerVec;
    const bool vec = host_aligned(a, 16) && host_aligned(y, 16) && (!kBinary || host_aligned(b, 16));
    const int64_t work = vec ? ceil_div<int64_t>(count, kPer) : count;
    const int64_t wanted = ceil_div<int64_t>(work, kDefaultBlockSize);
    const int64_t cap = static_cast<int64_t>(cu_count()) * 32;
    const int64_t grid = wanted < cap ? (wanted < 1 ? 1 : wanted) : cap;
    if (vec) {
        elementwise_kernel<T, Op, kBinary, true>
            <<<static_cast<unsigned>(grid), kDefaultBlockSize, 0, stream>>>(
                static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(y), count);
    } else {
        elementwise_kernel<T, Op, kBinary, false>
            <<<static_cast<unsigned>(grid), kDefaultBlockSize, 0, stream>>>(
                static_cast<const T*>(a), static_cast<const T*>(b), static_cast<T*>(y), count);
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
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_silu: null pointer");
    return cf::run<cf::Silu, false>(x, nullptr, y, dtype, count, stream, "launching silu");
}

cf_status cf_gelu(const void* x, void* y, cf_dtype dtype, int64_t count, void* stream) {
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && y != nullptr, "cf_gelu: null pointer");
    return cf::run<cf::GeluTanh, false>(x, nullptr, y, dtype, count, stream, "launching gelu");
}

cf_status cf_swiglu(const void* gate, const void* up, void* y, cf_dtype dtype, int64_t count,
                    void* stream) {
    if (count <= 0) return CF_OK;
    CF_REQUIRE(gate != nullptr && up != nullptr && y != nullptr, "cf_swiglu: null pointer");
    return cf::run<cf::SwiGlu, true>(gate, up, y, dtype, count, stream, "launching swiglu");
}

}  // extern "C"

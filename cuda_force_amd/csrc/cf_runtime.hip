// Error plumbing, device facts and the byte-copy calibration kernel.
//
// The reference reports failures by throwing cudaforge::CudaError from
// CUDAFORGE_CHECK / CUDAFORGE_CHECK_LAUNCH
// (cuda/include/cudaforge/cuda_error.cuh:15-96). A C ABI cannot throw, so each
// entry point returns a cf_status and leaves its message in a thread-local
// slot; CUDAFORGE_DEBUG_SYNC keeps its meaning, but is read from the
// environment at run time rather than fixed at compile time.
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "cf_common.hpp"

namespace cf {
namespace {

thread_local char g_last_error[512] = "no error";
thread_local int g_last_hip_error = 0;
thread_local LaunchEvents g_launch_events = {nullptr, nullptr};
thread_local hipError_t g_pending_launch_error = hipSuccess;

bool debug_sync_enabled() {
    static const bool enabled = [] {
        const char* value = std::getenv("CUDAFORGE_DEBUG_SYNC");
        return value != nullptr && value[0] != '\0' && value[0] != '0';
    }();
    return enabled;
}

}  // namespace

cf_status fail(cf_status status, const char* format, ...) {
    va_list args;
    va_start(args, format);
    std::vsnprintf(g_last_error, sizeof(g_last_error), format, args);
    va_end(args);
    g_last_hip_error = 0;
    return status;
}

cf_status fail_hip(hipError_t error, const char* what) {
    std::snprintf(g_last_error, sizeof(g_last_error), "HIP error %d (%s): %s while %s",
                  static_cast<int>(error), hipGetErrorName(error), hipGetErrorString(error), what);
    g_last_hip_error = static_cast<int>(error);
    return CF_ERR_HIP;
}

LaunchEvents take_launch_events() {
    const LaunchEvents events = g_launch_events;
    g_launch_events = {nullptr, nullptr};
    return events;
}

LaunchEvents next_launch_events() {
    const LaunchEvents events = g_launch_events;
    g_launch_events.start = nullptr;
    return events;
}

bool launch_events_armed() {
    return g_launch_events.start != nullptr || g_launch_events.stop != nullptr;
}

void note_launch_error(hipError_t error) { g_pending_launch_error = error; }

cf_status check_launch(const char* what, hipStream_t stream) {
    const hipError_t pending = g_pending_launch_error;
    g_pending_launch_error = hipSuccess;
    const hipError_t launch = hipGetLastError();
    if (pending != hipSuccess) return fail_hip(pending, what);
    if (launch != hipSuccess) return fail_hip(launch, what);
    if (debug_sync_enabled()) {
        const hipError_t done = hipStreamSynchronize(stream);
        if (done != hipSuccess) return fail_hip(done, what);
    }
    return CF_OK;
}

int cu_count() {
    constexpr int kMaxDevices = 64;
    static std::mutex mutex;
    static int cached[kMaxDevices] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return 256;
    std::lock_guard<std::mutex> lock(mutex);
    if (cached[device] == 0) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) !=
                hipSuccess ||
            count <= 0) {
            count = 256;
        }
        cached[device] = count;
    }
    return cached[device];
}

namespace {

constexpr int kCopyUnroll = 4;

/// Streaming copy: every workgroup moves one contiguous chunk of
/// 256 x 4 16-byte vectors with nontemporal loads and stores (a one-shot grid
/// measured faster than a grid-stride loop on MI355X). Workgroups whose chunk
/// is entirely in range load unconditionally: a guarded load makes the
/// compiler wait for each load before issuing the next.
template <bool kFull>
__device__ __forceinline__ void copy16_body(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                            int64_t vectors, int64_t base) {
    uint4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + static_cast<int64_t>(u) * 256;
        if (kFull || i < vectors) v[u] = load_stream16(src + i);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + static_cast<int64_t>(u) * 256;
        if (kFull || i < vectors) store_stream16(dst + i, v[u]);
    }
}

__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, int64_t vectors) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * 256 * kCopyUnroll;
    const int64_t base = first + threadIdx.x;
    if (first + 256 * kCopyUnroll <= vectors) {  // workgroup-uniform
        copy16_body<true>(src, dst, vectors, base);
    } else {
        copy16_body<false>(src, dst, vectors, base);
    }
}

/// Read-mostly stream with the quantiser's access pattern: each lane loads
/// four 16-byte vectors (one 1 KiB piece per wave instruction, as the fp32
/// quantiser does) and writes 16 / kDivisor bytes derived from each, so
/// the kernel reads `vectors` x 16 bytes and writes a kDivisor-th of that.
/// Only whole workgroup chunks are processed.
template <int kDivisor>
__global__ __launch_bounds__(256) void stream_kernel(const uint4* __restrict__ src,
                                                     uint8_t* __restrict__ dst) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kCopyUnroll + threadIdx.x;
    uint4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) v[u] = load_stream16(src + base + u * 256);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kDivisor == 0) {
        // Read only: one 4-byte word per workgroup (1/4096 of the bytes
        // read) - thread 0's xor of its vectors - so the loads are not dead.
        // A plain store: L2 merges the words into whole lines, where 4096
        // scattered non-temporal 4-byte writes slowed a 64 MiB read by a
        // fifth.
        uint32_t folded = 0;
#pragma unroll
        for (int u = 0; u < kCopyUnroll; ++u) folded ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
        const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(folded)));
        if (threadIdx.x == 0) reinterpret_cast<uint32_t*>(dst)[blockIdx.x] = total;
        return;
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
        const int64_t i = base + u * 256;
        if constexpr (kDivisor == 1) {
            store_stream16(dst + 16 * i, v[u]);
        } else if constexpr (kDivisor == 2) {
            store_stream8(dst + 8 * i, make_uint2(v[u].x ^ v[u].y, v[u].z ^ v[u].w));
        } else {
            store_stream4(dst + 4 * i, v[u].x ^ v[u].y ^ v[u].z ^ v[u].w);
        }
    }
}

/// Write only: each lane stores four 16-byte vectors of its index (one
/// 1 KiB piece per wave instruction, the copy's store pattern); nothing is
/// read.
__global__ __launch_bounds__(256) void write_stream_kernel(uint4* __restrict__ dst) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kCopyUnroll + threadIdx.x;
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
        const uint32_t i = static_cast<uint32_t>(base + u * 256);
        store_stream16(dst + base + u * 256, make_uint4(i, ~i, i ^ 0x5bd1e995u, i + 1u));
    }
}

/// Write only, one 16-byte store per lane (the grid covers the bytes once),
/// with cache policy kPolicy on a buffer store: 2 non-temporal, 16
/// device-scope (sc1), 18 both, 0 none.
template <int kPolicy>
__global__ __launch_bounds__(256) void write_once_kernel(uint8_t* __restrict__ dst, uint32_t bytes) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const __amdgpu_buffer_rsrc_t out = make_buffer(dst, bytes);
    const u32x4_t v = {i, ~i, i ^ 0x5bd1e995u, i + 1u};
    __builtin_amdgcn_raw_buffer_store_b128(v, out, 16u * i, 0, kPolicy);
}

__global__ void copy_tail_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                 int64_t bytes) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes;
         i += stride) {
        dst[i] = src[i];
    }
}

}  // namespace
}  // namespace cf

extern "C" {

const char* cf_last_error(void) { return cf::g_last_error; }

int cf_last_hip_error(void) { return cf::g_last_hip_error; }

int cf_hip_error_is_sticky(int hip_error) {
    switch (static_cast<hipError_t>(hip_error)) {
        case hipErrorIllegalAddress:
        case hipErrorLaunchFailure:
        case hipErrorLaunchTimeOut:
        case hipErrorIllegalState:
        case hipErrorAssert:
        case hipErrorECCNotCorrectable:
            return 1;
        default:
            return 0;
    }
}

int cf_abi_version(void) { return 1; }

cf_status cf_time_next_launch(void* start_event, void* stop_event) {
    CF_REQUIRE((start_event == nullptr) == (stop_event == nullptr),
               "cf_time_next_launch: give both events or neither");
    cf::g_launch_events = {static_cast<hipEvent_t>(start_event), static_cast<hipEvent_t>(stop_event)};
    return CF_OK;
}

int cf_time_next_launch_armed(void) { return cf::launch_events_armed() ? 1 : 0; }

cf_status cf_stream_bytes(const void* src, void* dst, int64_t read_bytes, int divisor, void* stream) {
    CF_ENTRY();
    if (read_bytes <= 0) return CF_OK;
    CF_REQUIRE(dst != nullptr && (src != nullptr || divisor < 0), "cf_stream_bytes: null pointer");
    CF_REQUIRE(divisor == 1 || divisor == 2 || divisor == 4 || divisor == 0 ||
                   (divisor <= -1 && divisor >= -5),
               "cf_stream_bytes: divisor %d is not 1, 2, 4, 0 or -1 .. -5", divisor);
    CF_REQUIRE(divisor >= -1 || read_bytes < (1LL << 32),
               "cf_stream_bytes: the one-store-per-lane write streams take under 4 GiB");
    constexpr int64_t kChunk = 256 * cf::kCopyUnroll * 16;
    CF_REQUIRE(read_bytes % kChunk == 0, "cf_stream_bytes: %lld bytes are not a multiple of %lld",
               static_cast<long long>(read_bytes), static_cast<long long>(kChunk));
    CF_REQUIRE((divisor < 0 || cf::host_aligned(src, 16)) && cf::host_aligned(dst, 16),
               "cf_stream_bytes: src and dst must be 16-byte aligned");
    const int64_t grid = read_bytes / kChunk;
    CF_REQUIRE(grid < (1LL << 31), "cf_stream_bytes: %lld bytes exceed the launch limit",
               static_cast<long long>(read_bytes));
    auto s = static_cast<hipStream_t>(stream);
    const dim3 g(static_cast<unsigned>(grid));
    const auto* in = static_cast<const uint4*>(src);
    auto* out = static_cast<uint8_t*>(dst);
    const dim3 g_once(static_cast<unsigned>(grid * cf::kCopyUnroll));
    const auto bytes32 = static_cast<uint32_t>(read_bytes);
    if (divisor == -1) {
        cf::launch(cf::write_stream_kernel, g, dim3(256), 0, s, static_cast<uint4*>(dst));
    } else if (divisor == -2) {
        cf::launch(cf::write_once_kernel<2>, g_once, dim3(256), 0, s, out, bytes32);
    } else if (divisor == -3) {
        cf::launch(cf::write_once_kernel<16>, g_once, dim3(256), 0, s, out, bytes32);
    } else if (divisor == -4) {
        cf::launch(cf::write_once_kernel<18>, g_once, dim3(256), 0, s, out, bytes32);
    } else if (divisor == -5) {
        cf::launch(cf::write_once_kernel<0>, g_once, dim3(256), 0, s, out, bytes32);
    } else if (divisor == 0) {
        cf::launch(cf::stream_kernel<0>, g, dim3(256), 0, s, in, out);
    } else if (divisor == 1) {
        cf::launch(cf::stream_kernel<1>, g, dim3(256), 0, s, in, out);
    } else if (divisor == 2) {
        cf::launch(cf::stream_kernel<2>, g, dim3(256), 0, s, in, out);
    } else {
        cf::launch(cf::stream_kernel<4>, g, dim3(256), 0, s, in, out);
    }
    return cf::check_launch("launching the byte stream", s);
}

cf_status cf_copy_bytes(const void* src, void* dst, int64_t bytes, void* stream) {
    CF_ENTRY();
    if (bytes <= 0) return CF_OK;
    CF_REQUIRE(src != nullptr && dst != nullptr, "cf_copy_bytes: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    const bool vec = cf::host_aligned(src, 16) && cf::host_aligned(dst, 16);
    const int64_t vectors = vec ? bytes / 16 : 0;
    if (vectors > 0) {
        const int64_t grid = cf::ceil_div<int64_t>(vectors, 256 * cf::kCopyUnroll);
        CF_REQUIRE(grid < (1LL << 31), "cf_copy_bytes: %lld bytes exceed the launch limit",
                   static_cast<long long>(bytes));
        cf::launch(cf::copy16_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s,
                   static_cast<const uint4*>(src), static_cast<uint4*>(dst), vectors);
    }
    const int64_t done = vectors * 16;
    const int64_t rest = bytes - done;
    if (rest > 0) {
        const int64_t wanted = cf::ceil_div<int64_t>(rest, 256);
        const int grid = static_cast<int>(wanted < 65536 ? wanted : 65536);
        cf::launch(cf::copy_tail_kernel, dim3(grid), dim3(256), 0, s,
                   static_cast<const uint8_t*>(src) + done, static_cast<uint8_t*>(dst) + done,
                   rest);
    }
    return cf::check_launch("launching the byte copy", s);
}

}  // extern "C"

// Whole-array sum and per-row sums for gfx950.
//
// The reference's bound sum kernel (reduce_sum_warp, cuda/src/reduction.cu:60-89)
// ends with one global atomicAdd per block, so its result depends on block
// completion order. Here the sum is a fixed two-stage tree:
//
//   stage 1: G workgroups, each reducing one contiguous chunk with 16-byte
//            loads (four in flight and four independent accumulators per
//            lane; a grid-stride assignment measured 10-15% slower), a DPP wave
//            reduction and a 4-slot LDS exchange, into partial[G];
//   stage 2: one workgroup of 512 threads loads all of partial[0..G) at once
//            (eight loads in flight per lane; a strided loop of one load per
//            iteration cost 1.3 us at 16M elements), reduces it in a fixed
//            order and writes (or adds into) *out.
//
// Inputs of at most 256 KiB skip the tree: one workgroup of 1024 threads sums
// them (the same per-lane loop, sixteen loads in flight) and writes *out, one
// launch instead of two.
//
// G and the chunk size are functions of `count` only, so the same input gives
// the same bits on any device and on every run.
//
// cf_reduce_sum_noalloc runs the same two launches with the partials in a
// static device array instead of a caller workspace, for callers that cannot
// allocate (HIP graph capture, serving loops that forbid hipMalloc).
#include <mutex>

#include "cf_common.hpp"

namespace cf {
namespace {

constexpr int kWavesPerBlock = kDefaultBlockSize / kWaveSize;
constexpr int64_t kMaxPartials = 4096;  // 2048 and 8192 measured 2% and 0.5% slower at 256M
// One round of stage-1 loads (256 threads x 4 vectors x 16 bytes) per chunk
// at least, so mid-size inputs spread over more workgroups, each one round
// trip deep.
constexpr int kStage1Unroll = 4;
constexpr int64_t kMinChunk = 4096;
constexpr int kPartialsPerThread = 8;
constexpr int kStage2Threads = 512;
static_assert(kMaxPartials == kStage2Threads * kPartialsPerThread,
              "stage 2 loads every partial at once");

/// Number of stage-1 workgroups for `count` elements.
int64_t partial_count(int64_t count) {
    const int64_t wanted = ceil_div<int64_t>(count, kMinChunk);
    return wanted < kMaxPartials ? (wanted < 1 ? 1 : wanted) : kMaxPartials;
}

/// Sum of x[begin, end) over one workgroup of kThreads threads: 16-byte
/// loads, kUnroll in flight and four independent accumulators per lane, a
/// DPP wave reduction and an LDS exchange across the waves (every thread
/// receives the total). kVec: x 16-byte aligned, begin a multiple of
/// kPer * kThreads elements.
template <typename T, bool kVec, int kThreads, int kUnroll>
__device__ __forceinline__ float range_sum(const T* __restrict__ x, int64_t begin, int64_t end, float* slot) {
    constexpr int kPer = Storage<T>::kPerVec;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (kVec) {
        // Every vector is aligned and lies entirely before `end` unless it
        // straddles it (the scalar tail).
        constexpr int64_t step = static_cast<int64_t>(kThreads) * kPer;
        int64_t e = begin + static_cast<int64_t>(threadIdx.x) * kPer;
        // kUnroll loads in flight per lane: issued together, then accumulated
        // (one load per iteration left each lane waiting on its latency).
        for (; e + (kUnroll - 1) * step + kPer <= end; e += kUnroll * step) {
            uint4 raw[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) raw[u] = load_stream16(x + e + u * step);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                float v[kPer];
                unpack16<T>(raw[u], v);
#pragma unroll
                for (int i = 0; i < kPer; ++i) acc[i & 3] += v[i];
            }
        }
        for (; e + kPer <= end; e += step) {
            float v[kPer];
            unpack16<T>(load_stream16(x + e), v);
#pragma unroll
            for (int i = 0; i < kPer; ++i) acc[i & 3] += v[i];
        }
        for (int i = 0; i < kPer; ++i) {
            if (e + i < end) acc[0] += Storage<T>::load(x + e + i);
        }
    } else {
        for (int64_t e = begin + threadIdx.x; e < end; e += kThreads) {
            acc[0] += Storage<T>::load(x + e);
        }
    }
    return block_reduce_f32<kThreads / kWaveSize, AddF32>((acc[0] + acc[1]) + (acc[2] + acc[3]), slot);
}

template <typename T, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void sum_stage1_kernel(const T* __restrict__ x,
                                                                       float* __restrict__ partial,
                                                                       int64_t count,
                                                                       int64_t chunk) {
    __shared__ float slot[kWavesPerBlock];
    // chunk is a multiple of kPer * blockDim, so every chunk starts aligned.
    const int64_t begin = static_cast<int64_t>(blockIdx.x) * chunk;
    const int64_t end = begin + chunk < count ? begin + chunk : count;
    const float total = range_sum<T, kVec, kDefaultBlockSize, kStage1Unroll>(x, begin, end, slot);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

/// Inputs of at most kSingleLaunchBytes: one workgroup sums all of x and
/// writes (or adds into) *out - one launch instead of two. 16 loads in
/// flight per lane cover the largest such input in one round trip.
constexpr int kSingleThreads = 1024;
constexpr int kSingleUnroll = 16;
constexpr int64_t kSingleLaunchBytes = 256 * 1024;
static_assert(kSingleLaunchBytes == int64_t{kSingleThreads} * kSingleUnroll * 16,
              "one round of loads covers a single-launch input");

template <typename T, bool kVec>
__global__ __launch_bounds__(kSingleThreads) void sum_single_kernel(const T* __restrict__ x, int64_t count,
                                                                    float* __restrict__ out, int accumulate) {
    __shared__ float slot[kSingleThreads / kWaveSize];
    const float total = range_sum<T, kVec, kSingleThreads, kSingleUnroll>(x, 0, count, slot);
    if (threadIdx.x == 0) *out = accumulate ? *out + total : total;
}

__global__ __launch_bounds__(kStage2Threads) void sum_stage2_kernel(
    const float* __restrict__ partial, int64_t partials, float* __restrict__ out, int accumulate) {
    __shared__ float slot[kStage2Threads / kWaveSize];
    float v[kPartialsPerThread];
#pragma unroll
    for (int i = 0; i < kPartialsPerThread; ++i) {
        const int64_t p = static_cast<int64_t>(i) * kStage2Threads + threadIdx.x;
        v[i] = p < partials ? partial[p] : 0.0f;
    }
    const float acc = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    const float total = block_reduce_f32<kStage2Threads / kWaveSize, AddF32>(acc, slot);
    if (threadIdx.x == 0) *out = accumulate ? *out + total : total;
}

/// One wave per row; each lane strides the row with 16-byte vectors.
template <typename T, bool kVec>
__global__ __launch_bounds__(kDefaultBlockSize) void row_sum_kernel(const T* __restrict__ x,
                                                                    float* __restrict__ out,
                                                                    int64_t rows, int64_t cols) {
    constexpr int kPer = Storage<T>::kPerVec;
    const int lane = static_cast<int>(threadIdx.x) & (kWaveSize - 1);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock +
                         static_cast<int64_t>(threadIdx.x) / kWaveSize;
    const int64_t waves = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
    for (int64_t row = wave; row < rows; row += waves) {
        const T* xr = x + row * cols;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (kVec) {
            constexpr int64_t kStep = static_cast<int64_t>(kWaveSize) * kPer;
            int64_t e = static_cast<int64_t>(lane) * kPer;
            for (; e + 3 * kStep < cols; e += 4 * kStep) {  // four loads in flight per lane
                uint4 raw[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) raw[u] = load_stream16(xr + e + u * kStep);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    float v[kPer];
                    unpack16<T>(raw[u], v);
#pragma unroll
                    for (int i = 0; i < kPer; ++i) acc[i & 3] += v[i];
                }
            }
            for (; e < cols; e += kStep) {
                float v[kPer];
                unpack16<T>(load_stream16(xr + e), v);
#pragma unroll
                for (int i = 0; i < kPer; ++i) acc[i & 3] += v[i];
            }
        } else {
            for (int64_t e = lane; e < cols; e += kWaveSize) acc[0] += Storage<T>::load(xr + e);
        }
        const float total = wave_reduce_f32<AddF32>((acc[0] + acc[1]) + (acc[2] + acc[3]));
        if (lane == 0) out[row] = total;
    }
}

template <typename T>
cf_status launch_sum(const void* x, float* out, int64_t count, void* workspace,
                     int accumulate, hipStream_t stream) {
    constexpr int kPer = Storage<T>::kPerVec;
    if (count * static_cast<int64_t>(sizeof(T)) <= kSingleLaunchBytes) {
        if (host_aligned(x, 16)) {
            launch(sum_single_kernel<T, true>, dim3(1), dim3(kSingleThreads), 0, stream, static_cast<const T*>(x),
                   count, out, accumulate);
        } else {
            launch(sum_single_kernel<T, false>, dim3(1), dim3(kSingleThreads), 0, stream, static_cast<const T*>(x),
                   count, out, accumulate);
        }
        return check_launch("launching reduce_sum", stream);
    }
    const int64_t partials = partial_count(count);
    // Chunk rounded up to whole workgroup strides so every vector stays aligned.
    const int64_t stride = static_cast<int64_t>(kDefaultBlockSize) * kPer;
    const int64_t chunk = ceil_div<int64_t>(ceil_div<int64_t>(count, partials), stride) * stride;
    const int64_t grid = ceil_div<int64_t>(count, chunk);
    float* partial = static_cast<float*>(workspace);
    if (host_aligned(x, 16)) {
        launch(sum_stage1_kernel<T, true>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x), partial, count, chunk);
    } else {
        launch(sum_stage1_kernel<T, false>, dim3(static_cast<unsigned>(grid)),
               dim3(kDefaultBlockSize), 0, stream, static_cast<const T*>(x), partial, count, chunk);
    }
    launch(sum_stage2_kernel, dim3(1), dim3(kStage2Threads), 0, stream, partial, grid, out,
           accumulate);
    return check_launch("launching reduce_sum", stream);
}

template <typename T>
cf_status launch_row_sum(const void* x, float* out, int64_t rows, int64_t cols,
                         hipStream_t stream) {
    constexpr int kPer = Storage<T>::kPerVec;
    const int64_t max_waves = static_cast<int64_t>(cu_count()) * 16;
    const int64_t waves = rows < max_waves ? rows : max_waves;
    const int64_t grid = ceil_div<int64_t>(waves, kWavesPerBlock);
    if (cols % kPer == 0 && host_aligned(x, 16)) {
        launch(row_sum_kernel<T, true>, dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize),
               0, stream, static_cast<const T*>(x), out, rows, cols);
    } else {
        launch(row_sum_kernel<T, false>, dim3(static_cast<unsigned>(grid)), dim3(kDefaultBlockSize),
               0, stream, static_cast<const T*>(x), out, rows, cols);
    }
    return check_launch("launching row_sum", stream);
}

}  // namespace

/// Device address of `scratch` (below) on the current device, looked up
/// once per device with that device current and kept; never the host-side
/// name of the array, which is no device address.
cf_status noalloc_scratch(void** out);

}  // namespace cf

// Stage-1 partials of cf_reduce_sum_noalloc: every count needs at most
// kMaxPartials of them (16 KiB). Each device holds its own copy for the life
// of the process; all calls on one device share it.
static __device__ __align__(256) float scratch[cf::kMaxPartials];

namespace cf {

cf_status noalloc_scratch(void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mutex;
    static void* cached[kMaxDevices] = {};
    int device = 0;
    CF_HIP_TRY(hipGetDevice(&device));
    CF_REQUIRE(device >= 0 && device < kMaxDevices, "cf_reduce_sum_noalloc: device %d out of range", device);
    std::lock_guard<std::mutex> lock(mutex);
    if (cached[device] == nullptr) {
        void* ptr = nullptr;
        CF_HIP_TRY(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        CF_REQUIRE(ptr != nullptr, "cf_reduce_sum_noalloc: no device address for the scratch array");
        cached[device] = ptr;
    }
    *out = cached[device];
    return CF_OK;
}

}  // namespace cf

extern "C" {

size_t cf_reduce_sum_workspace_bytes(int64_t count) {
    if (count <= 0) return 0;
    return static_cast<size_t>(cf::partial_count(count)) * sizeof(float);
}

cf_status cf_reduce_sum(const void* x, cf_dtype x_dtype, float* out, int64_t count,
                        void* workspace, size_t workspace_bytes, int accumulate, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && out != nullptr, "cf_reduce_sum: null pointer");
    const size_t needed = cf_reduce_sum_workspace_bytes(count);
    CF_REQUIRE(workspace != nullptr && workspace_bytes >= needed,
               "cf_reduce_sum: workspace of %zu bytes given, %zu needed", workspace_bytes, needed);
    CF_REQUIRE(cf::host_aligned(workspace, 4), "cf_reduce_sum: workspace must be 4-byte aligned");
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::launch_sum<float>(x, out, count, workspace, accumulate, s);
        case CF_BF16:
            return cf::launch_sum<cf::bf16_t>(x, out, count, workspace, accumulate, s);
        case CF_F16:
            return cf::launch_sum<cf::f16_t>(x, out, count, workspace, accumulate, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_reduce_sum: unknown dtype %d",
                    static_cast<int>(x_dtype));
}

cf_status cf_reduce_sum_noalloc(const void* x, cf_dtype x_dtype, float* out, int64_t count,
                                int accumulate, void* stream) {
    CF_ENTRY();
    if (count <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && out != nullptr, "cf_reduce_sum_noalloc: null pointer");
    const size_t needed = cf_reduce_sum_workspace_bytes(count);
    CF_REQUIRE(needed <= sizeof(scratch),
               "cf_reduce_sum_noalloc: %lld elements need %zu bytes of partials, above the %zu-byte "
               "static scratch",
               static_cast<long long>(count), needed, sizeof(scratch));
    if (x_dtype != CF_F32 && x_dtype != CF_BF16 && x_dtype != CF_F16) {
        return cf::fail(CF_ERR_UNSUPPORTED, "cf_reduce_sum_noalloc: unknown dtype %d",
                        static_cast<int>(x_dtype));
    }
    void* partials = nullptr;
    const cf_status found = cf::noalloc_scratch(&partials);
    if (found != CF_OK) return found;
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::launch_sum<float>(x, out, count, partials, accumulate, s);
        case CF_BF16:
            return cf::launch_sum<cf::bf16_t>(x, out, count, partials, accumulate, s);
        case CF_F16:
            return cf::launch_sum<cf::f16_t>(x, out, count, partials, accumulate, s);
    }
    return CF_ERR_UNSUPPORTED;
}

cf_status cf_row_sum(const void* x, cf_dtype x_dtype, float* out, int64_t rows, int64_t cols,
                     void* stream) {
    CF_ENTRY();
    if (rows <= 0 || cols <= 0) return CF_OK;
    CF_REQUIRE(x != nullptr && out != nullptr, "cf_row_sum: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case CF_F32:
            return cf::launch_row_sum<float>(x, out, rows, cols, s);
        case CF_BF16:
            return cf::launch_row_sum<cf::bf16_t>(x, out, rows, cols, s);
        case CF_F16:
            return cf::launch_row_sum<cf::f16_t>(x, out, rows, cols, s);
    }
    return cf::fail(CF_ERR_UNSUPPORTED, "cf_row_sum: unknown dtype %d",
                    static_cast<int>(x_dtype));
}

}  // extern "C"

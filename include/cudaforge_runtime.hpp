// HIP runtime pieces the operators coexist with: owning streams, events and
// buffers, the stream scheduler, and the device / stream-ordered / pinned
// backends of the caching pool (cudaforge_pool.hpp).
//
// The C++ interface follows the reference's so code written against it
// compiles with the CUDA names swapped for these:
//   * `GpuScheduler`, `StreamLease`, `StreamStats`, `SchedulerStats`
//     (cuda/include/cudaforge/gpu_scheduler.cuh:16-142,
//     cuda/src/gpu_scheduler.cu:10-105): a fixed pool of streams handed out
//     round-robin from a relaxed atomic ticket, one ordering event per stream,
//     asynchronous copies with per-stream byte counts, cross-stream ordering
//     by event (`chain`), `synchronize_all` only at shutdown;
//   * `DeviceAllocatorBackend` (:150-168), `supports_stream_ordered_allocation`
//     (:175-186), `StreamOrderedAllocatorBackend` (:215-240),
//     `PinnedAllocatorBackend` (:243-258);
//   * the RAII wrappers `HipStream`, `HipEvent`, `DeviceBuffer`, `PinnedBuffer`
//     and the checked-call error `HipError` (cuda/include/cudaforge/
//     cuda_raii.cuh, cuda_error.cuh:15-96) in their HIP form.
//
// Differences on MI355X, by design:
//   * Every stream is created at the default priority. The reference asks for
//     the highest priority band; on MI355X systems work spread over streams of
//     different priorities has been seen to hang, and a pool whose streams all
//     share one priority gains nothing from raising it.
//   * Streams are non-blocking (`hipStreamNonBlocking`), as in the reference,
//     so nothing on the null stream serialises them.
//   * `DeviceBuffer::fill_zero` is a `hipMemsetAsync`: fine on a stream, not
//     meant for recording into a HIP graph.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "cudaforge_pool.hpp"

namespace cudaforge {

/// A failed HIP call: the status, and whether it poisoned the context.
class HipError : public std::runtime_error {
public:
    HipError(hipError_t status, const std::string& message)
        : std::runtime_error(message), status_(status) {}

    hipError_t status() const noexcept { return status_; }

    /// Sticky errors leave the context unusable (every later call fails);
    /// the others (an allocation failure, an invalid value) are recoverable.
    bool is_sticky() const noexcept { return is_sticky_status(status_); }

    static bool is_sticky_status(hipError_t status) noexcept {
        switch (status) {
            case hipErrorIllegalAddress:
            case hipErrorLaunchFailure:
            case hipErrorLaunchTimeOut:
            case hipErrorAssert:
            case hipErrorIllegalState:
            case hipErrorECCNotCorrectable:
                return true;
            default:
                return false;
        }
    }

private:
    hipError_t status_;
};

namespace runtime_detail {

[[noreturn]] inline void throw_hip_error(hipError_t status, const char* expression,
                                         const char* file, int line) {
    throw HipError(status, std::string("HIP error ") + hipGetErrorName(status) + " (" +
                               hipGetErrorString(status) + ") at " + file + ":" +
                               std::to_string(line) + ": " + expression);
}

}  // namespace runtime_detail

#define CUDAFORGE_HIP_CHECK(expression)                                                      \
    do {                                                                                      \
        const hipError_t cudaforge_status_ = (expression);                                    \
        if (cudaforge_status_ != hipSuccess) {                                                \
            ::cudaforge::runtime_detail::throw_hip_error(cudaforge_status_, #expression,      \
                                                         __FILE__, __LINE__);                 \
        }                                                                                     \
    } while (0)

/// Owning non-blocking stream at the default priority.
class HipStream {
public:
    HipStream() { CUDAFORGE_HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking)); }
    HipStream(const HipStream&) = delete;
    HipStream& operator=(const HipStream&) = delete;
    HipStream(HipStream&& other) noexcept : stream_(std::exchange(other.stream_, nullptr)) {}
    HipStream& operator=(HipStream&& other) noexcept {
        if (this != &other) {
            destroy();
            stream_ = std::exchange(other.stream_, nullptr);
        }
        return *this;
    }
    ~HipStream() { destroy(); }

    hipStream_t get() const noexcept { return stream_; }
    operator hipStream_t() const noexcept { return stream_; }  // NOLINT(google-explicit-constructor)

    /// Waits for this stream only; other streams keep running.
    void synchronize() const { CUDAFORGE_HIP_CHECK(hipStreamSynchronize(stream_)); }

    /// True once everything issued so far has finished.
    bool query() const {
        const hipError_t status = hipStreamQuery(stream_);
        if (status == hipSuccess) return true;
        if (status == hipErrorNotReady) return false;
        runtime_detail::throw_hip_error(status, "hipStreamQuery", __FILE__, __LINE__);
    }

private:
    void destroy() noexcept {
        if (stream_ != nullptr) static_cast<void>(hipStreamDestroy(stream_));
        stream_ = nullptr;
    }
    hipStream_t stream_ = nullptr;
};

/// Owning event; ordering events carry no timestamp.
class HipEvent {
public:
    enum class Purpose { Ordering, Timing };

    explicit HipEvent(Purpose purpose = Purpose::Ordering) : timing_(purpose == Purpose::Timing) {
        CUDAFORGE_HIP_CHECK(
            hipEventCreateWithFlags(&event_, timing_ ? hipEventDefault : hipEventDisableTiming));
    }
    HipEvent(const HipEvent&) = delete;
    HipEvent& operator=(const HipEvent&) = delete;
    HipEvent(HipEvent&& other) noexcept
        : event_(std::exchange(other.event_, nullptr)), timing_(other.timing_) {}
    HipEvent& operator=(HipEvent&& other) noexcept {
        if (this != &other) {
            destroy();
            event_ = std::exchange(other.event_, nullptr);
            timing_ = other.timing_;
        }
        return *this;
    }
    ~HipEvent() { destroy(); }

    hipEvent_t get() const noexcept { return event_; }
    bool timing_enabled() const noexcept { return timing_; }
    void record(hipStream_t stream) const { CUDAFORGE_HIP_CHECK(hipEventRecord(event_, stream)); }
    void synchronize() const { CUDAFORGE_HIP_CHECK(hipEventSynchronize(event_)); }
    bool query() const {
        const hipError_t status = hipEventQuery(event_);
        if (status == hipSuccess) return true;
        if (status == hipErrorNotReady) return false;
        runtime_detail::throw_hip_error(status, "hipEventQuery", __FILE__, __LINE__);
    }

    /// Milliseconds between two recorded timing events.
    static float elapsed_ms(const HipEvent& start, const HipEvent& stop) {
        float ms = 0.0f;
        CUDAFORGE_HIP_CHECK(hipEventElapsedTime(&ms, start.event_, stop.event_));
        return ms;
    }

private:
    void destroy() noexcept {
        if (event_ != nullptr) static_cast<void>(hipEventDestroy(event_));
        event_ = nullptr;
    }
    hipEvent_t event_ = nullptr;
    bool timing_ = false;
};

/// `waiter` waits on the device for `event`; the host is not blocked.
inline void stream_wait_event(hipStream_t waiter, const HipEvent& event) {
    CUDAFORGE_HIP_CHECK(hipStreamWaitEvent(waiter, event.get(), 0));
}

/// Owning device array of `count` elements of T.
template <typename T>
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(std::size_t count) : count_(count) {
        if (count_ > 0) CUDAFORGE_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&data_), bytes()));
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& other) noexcept
        : data_(std::exchange(other.data_, nullptr)), count_(std::exchange(other.count_, 0)) {}
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
        if (this != &other) {
            release();
            data_ = std::exchange(other.data_, nullptr);
            count_ = std::exchange(other.count_, 0);
        }
        return *this;
    }
    ~DeviceBuffer() { release(); }

    T* data() const noexcept { return data_; }
    std::size_t size() const noexcept { return count_; }
    std::size_t bytes() const noexcept { return count_ * sizeof(T); }
    bool empty() const noexcept { return count_ == 0; }

    void fill_zero(hipStream_t stream) const {
        if (count_ > 0) CUDAFORGE_HIP_CHECK(hipMemsetAsync(data_, 0, bytes(), stream));
    }
    /// Copies are bounds-checked on the host: a device-side overrun would
    /// corrupt a neighbouring allocation without faulting at the copy.
    void copy_from_host(const T* host, std::size_t count, hipStream_t stream) const {
        check_count(count);
        CUDAFORGE_HIP_CHECK(
            hipMemcpyAsync(data_, host, count * sizeof(T), hipMemcpyHostToDevice, stream));
    }
    void copy_to_host(T* host, std::size_t count, hipStream_t stream) const {
        check_count(count);
        CUDAFORGE_HIP_CHECK(
            hipMemcpyAsync(host, data_, count * sizeof(T), hipMemcpyDeviceToHost, stream));
    }

private:
    void check_count(std::size_t count) const {
        if (count > count_) {
            throw std::out_of_range("DeviceBuffer copy of " + std::to_string(count) +
                                    " elements into " + std::to_string(count_));
        }
    }
    void release() noexcept {
        if (data_ != nullptr) static_cast<void>(hipFree(data_));
        data_ = nullptr;
        count_ = 0;
    }
    T* data_ = nullptr;
    std::size_t count_ = 0;
};

/// Owning page-locked host array (the precondition for a copy to overlap).
template <typename T>
class PinnedBuffer {
public:
    explicit PinnedBuffer(std::size_t count) : count_(count) {
        if (count_ > 0) {
            CUDAFORGE_HIP_CHECK(
                hipHostMalloc(reinterpret_cast<void**>(&data_), bytes(), hipHostMallocDefault));
        }
    }
    PinnedBuffer(const PinnedBuffer&) = delete;
    PinnedBuffer& operator=(const PinnedBuffer&) = delete;
    PinnedBuffer(PinnedBuffer&& other) noexcept
        : data_(std::exchange(other.data_, nullptr)), count_(std::exchange(other.count_, 0)) {}
    ~PinnedBuffer() {
        if (data_ != nullptr) static_cast<void>(hipHostFree(data_));
    }

    T* data() const noexcept { return data_; }
    std::size_t size() const noexcept { return count_; }
    std::size_t bytes() const noexcept { return count_ * sizeof(T); }
    T& operator[](std::size_t i) noexcept { return data_[i]; }
    const T& operator[](std::size_t i) const noexcept { return data_[i]; }

private:
    T* data_ = nullptr;
    std::size_t count_ = 0;
};

struct StreamStats {
    std::uint64_t batches_dispatched = 0;
    std::uint64_t bytes_to_device = 0;
    std::uint64_t bytes_to_host = 0;
};

struct SchedulerStats {
    std::size_t stream_count = 0;
    std::uint64_t total_dispatches = 0;
    std::uint64_t total_bytes_to_device = 0;
    std::uint64_t total_bytes_to_host = 0;
    std::vector<StreamStats> per_stream;
};

/// Use of one pooled stream and its completion event. Work a holder issues to
/// the stream runs in issue order, so a copy-in -> kernels -> copy-out
/// sequence needs no locks; leases are not exclusive once the round-robin
/// wraps (stream i is handed out again after stream_count acquisitions).
class StreamLease {
public:
    StreamLease(const HipStream& stream, const HipEvent& done, std::size_t index)
        : stream_(&stream), done_(&done), index_(index) {}

    hipStream_t stream() const noexcept { return stream_->get(); }
    const HipEvent& completion_event() const noexcept { return *done_; }
    std::size_t index() const noexcept { return index_; }

    /// The event completes once everything issued to the stream so far has.
    void record_completion() const { done_->record(stream_->get()); }
    void synchronize() const { stream_->synchronize(); }
    bool complete() const { return stream_->query(); }

private:
    const HipStream* stream_;
    const HipEvent* done_;
    std::size_t index_;
};

/// A fixed pool of streams on one device, handed out round-robin.
class GpuScheduler {
public:
    explicit GpuScheduler(std::size_t stream_count, int device = 0) : device_(device) {
        if (stream_count == 0) throw std::invalid_argument("GpuScheduler requires at least one stream");
        CUDAFORGE_HIP_CHECK(hipSetDevice(device_));
        streams_.reserve(stream_count);
        events_.reserve(stream_count);
        for (std::size_t i = 0; i < stream_count; ++i) {
            streams_.emplace_back();
            events_.emplace_back(HipEvent::Purpose::Ordering);
        }
        stats_.resize(stream_count);
    }
    GpuScheduler(const GpuScheduler&) = delete;
    GpuScheduler& operator=(const GpuScheduler&) = delete;

    /// Streams with queued work must not be destroyed: drain first. A failure
    /// here cannot be reported from a destructor and the context is going away.
    ~GpuScheduler() {
        try {
            synchronize_all();
        } catch (const HipError&) {
        }
    }

    /// The next stream in round-robin order; never blocks and never queries
    /// the device.
    StreamLease acquire() {
        const std::uint64_t ticket = next_.fetch_add(1, std::memory_order_relaxed);
        const std::size_t index = static_cast<std::size_t>(ticket % streams_.size());
        return StreamLease(streams_[index], events_[index], index);
    }

    /// Asynchronous copy on the lease's stream; `host` must be pinned for it
    /// to overlap with anything.
    void copy_to_device(const StreamLease& lease, void* device, const void* host, std::size_t bytes) {
        if (bytes == 0) return;
        CUDAFORGE_HIP_CHECK(hipMemcpyAsync(device, host, bytes, hipMemcpyHostToDevice, lease.stream()));
        std::lock_guard<std::mutex> lock(stats_mutex_);
        stats_[lease.index()].bytes_to_device += bytes;
    }

    void copy_to_host(const StreamLease& lease, void* host, const void* device, std::size_t bytes) {
        if (bytes == 0) return;
        CUDAFORGE_HIP_CHECK(hipMemcpyAsync(host, device, bytes, hipMemcpyDeviceToHost, lease.stream()));
        std::lock_guard<std::mutex> lock(stats_mutex_);
        stats_[lease.index()].bytes_to_host += bytes;
    }

    /// `waiter`'s stream waits for `signaller`'s last recorded completion.
    static void chain(const StreamLease& waiter, const StreamLease& signaller) {
        stream_wait_event(waiter.stream(), signaller.completion_event());
    }

    void note_dispatch(const StreamLease& lease) {
        std::lock_guard<std::mutex> lock(stats_mutex_);
        ++stats_[lease.index()].batches_dispatched;
    }

    /// Waits for every stream (shutdown only: per batch it would drain the
    /// pipeline the pool exists to keep full).
    void synchronize_all() {
        for (const HipStream& stream : streams_) stream.synchronize();
    }

    SchedulerStats stats() const {
        std::lock_guard<std::mutex> lock(stats_mutex_);
        SchedulerStats out;
        out.stream_count = streams_.size();
        out.per_stream = stats_;
        for (const StreamStats& s : stats_) {
            out.total_dispatches += s.batches_dispatched;
            out.total_bytes_to_device += s.bytes_to_device;
            out.total_bytes_to_host += s.bytes_to_host;
        }
        return out;
    }

    std::size_t stream_count() const noexcept { return streams_.size(); }
    int device() const noexcept { return device_; }

    /// Lease for stream `index` (for callers that carry the index across an
    /// interface, such as the C ABI).
    StreamLease lease(std::size_t index) const {
        if (index >= streams_.size()) throw std::out_of_range("stream index out of range");
        return StreamLease(streams_[index], events_[index], index);
    }

private:
    int device_;
    std::vector<HipStream> streams_;
    std::vector<HipEvent> events_;
    std::atomic<std::uint64_t> next_{0};
    mutable std::mutex stats_mutex_;
    std::vector<StreamStats> stats_;
};

/// hipMalloc / hipFree. hipFree waits for the device, so freeing through the
/// pool (which caches instead) keeps that wait out of the steady state.
class DeviceAllocatorBackend {
public:
    void* allocate(std::size_t bytes) const {
        void* pointer = nullptr;
        // Null (not an exception) lets the pool report bad_alloc, after which a
        // caller can trim and retry.
        if (hipMalloc(&pointer, bytes) != hipSuccess) {
            static_cast<void>(hipGetLastError());
            return nullptr;
        }
        return pointer;
    }
    void deallocate(void* pointer, std::size_t) const noexcept { static_cast<void>(hipFree(pointer)); }
    static const char* name() { return "device"; }
};

/// True when the current device backs hipMallocAsync with a memory pool.
inline bool supports_stream_ordered_allocation() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) return false;
    int supported = 0;
    if (hipDeviceGetAttribute(&supported, hipDeviceAttributeMemoryPoolsSupported, device) != hipSuccess) {
        return false;
    }
    return supported != 0;
}

/// hipMallocAsync / hipFreeAsync on one stream: a free is ordered after the
/// work already queued on that stream, so returning a buffer a queued kernel
/// still reads is safe and costs no device-wide wait. Using the memory on
/// another stream needs an event, as any cross-stream dependency does.
class StreamOrderedAllocatorBackend {
public:
    StreamOrderedAllocatorBackend() = default;
    explicit StreamOrderedAllocatorBackend(hipStream_t stream) : stream_(stream) {}

    void* allocate(std::size_t bytes) const {
        void* pointer = nullptr;
        if (hipMallocAsync(&pointer, bytes, stream_) != hipSuccess) {
            static_cast<void>(hipGetLastError());
            return nullptr;
        }
        return pointer;
    }
    void deallocate(void* pointer, std::size_t) const noexcept {
        static_cast<void>(hipFreeAsync(pointer, stream_));
    }
    hipStream_t stream() const noexcept { return stream_; }
    static const char* name() { return "device-async"; }

private:
    hipStream_t stream_ = nullptr;
};

/// hipHostMalloc / hipHostFree: page-locked staging buffers for the copy path.
class PinnedAllocatorBackend {
public:
    void* allocate(std::size_t bytes) const {
        void* pointer = nullptr;
        if (hipHostMalloc(&pointer, bytes, hipHostMallocDefault) != hipSuccess) {
            static_cast<void>(hipGetLastError());
            return nullptr;
        }
        return pointer;
    }
    void deallocate(void* pointer, std::size_t) const noexcept { static_cast<void>(hipHostFree(pointer)); }
    static const char* name() { return "pinned"; }
};

}  // namespace cudaforge

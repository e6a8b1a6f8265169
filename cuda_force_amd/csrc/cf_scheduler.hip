// C ABI over the stream scheduler and the caching pools of
// include/cudaforge_runtime.hpp / include/cudaforge_pool.hpp.
//
// The reference exposes GpuScheduler and MemoryPool as C++ classes only
// (cuda/src/gpu_scheduler.cu, cpp/include/cudaforge/memory_pool.hpp); here the
// same classes back opaque handles so that any FFI can drive them. Exceptions
// become statuses: std::invalid_argument and std::out_of_range ->
// CF_ERR_INVALID_ARGUMENT, std::bad_alloc -> CF_ERR_OUT_OF_MEMORY, HipError ->
// CF_ERR_HIP with the HIP status kept for cf_last_hip_error().
#include <memory>
#include <new>
#include <stdexcept>

#include "cf_common.hpp"
#include "../../include/cudaforge_runtime.hpp"

struct cf_scheduler {
    explicit cf_scheduler(std::size_t count, int device) : impl(count, device) {}
    cudaforge::GpuScheduler impl;
};

struct cf_pool {
    virtual ~cf_pool() = default;
    virtual void* allocate(std::size_t bytes) = 0;
    virtual void deallocate(void* pointer) = 0;
    virtual void trim() = 0;
    virtual cudaforge::PoolStats stats() const = 0;
};

namespace cf {
namespace {

template <typename Backend>
struct PoolOf final : cf_pool {
    PoolOf(Backend backend, std::size_t min_block) : impl(std::move(backend), min_block) {}
    void* allocate(std::size_t bytes) override { return impl.allocate(bytes); }
    void deallocate(void* pointer) override { impl.deallocate(pointer); }
    void trim() override { impl.trim(); }
    cudaforge::PoolStats stats() const override { return impl.stats(); }
    cudaforge::MemoryPool<Backend> impl;
};

/// Runs `body`, turning the runtime's exceptions into statuses.
template <typename Body>
cf_status guarded(const char* what, Body&& body) {
    try {
        body();
        return CF_OK;
    } catch (const cudaforge::HipError& error) {
        return fail_hip(error.status(), what);
    } catch (const std::bad_alloc&) {
        return fail(CF_ERR_OUT_OF_MEMORY, "%s: the backend could not supply the block", what);
    } catch (const std::invalid_argument& error) {
        return fail(CF_ERR_INVALID_ARGUMENT, "%s: %s", what, error.what());
    } catch (const std::out_of_range& error) {
        return fail(CF_ERR_INVALID_ARGUMENT, "%s: %s", what, error.what());
    } catch (const std::exception& error) {
        return fail(CF_ERR_INVALID_ARGUMENT, "%s: %s", what, error.what());
    }
}

cf_status null_handle(const char* what) {
    return fail(CF_ERR_INVALID_ARGUMENT, "%s: null handle or output pointer", what);
}

cudaforge::StreamLease lease_of(const cf_scheduler* scheduler, int64_t index) {
    if (index < 0) throw std::out_of_range("stream index out of range");
    return scheduler->impl.lease(static_cast<std::size_t>(index));
}

}  // namespace
}  // namespace cf

using cf::guarded;
using cf::lease_of;
using cf::null_handle;

extern "C" {

cf_status cf_scheduler_create(int64_t stream_count, int device, cf_scheduler** out) {
    if (out == nullptr) return null_handle("cf_scheduler_create");
    *out = nullptr;
    if (stream_count <= 0) {
        return cf::fail(CF_ERR_INVALID_ARGUMENT, "GpuScheduler requires at least one stream");
    }
    return guarded("cf_scheduler_create", [&] {
        *out = new cf_scheduler(static_cast<std::size_t>(stream_count), device);
    });
}

cf_status cf_scheduler_destroy(cf_scheduler* scheduler) {
    if (scheduler == nullptr) return CF_OK;
    return guarded("cf_scheduler_destroy", [&] {
        try {
            scheduler->impl.synchronize_all();
        } catch (...) {
            delete scheduler;
            throw;
        }
        delete scheduler;
    });
}

cf_status cf_scheduler_acquire(cf_scheduler* scheduler, int64_t* index, void** stream) {
    if (scheduler == nullptr || index == nullptr) return null_handle("cf_scheduler_acquire");
    return guarded("cf_scheduler_acquire", [&] {
        const cudaforge::StreamLease lease = scheduler->impl.acquire();
        *index = static_cast<int64_t>(lease.index());
        if (stream != nullptr) *stream = lease.stream();
    });
}

cf_status cf_scheduler_stream(const cf_scheduler* scheduler, int64_t index, void** stream) {
    if (scheduler == nullptr || stream == nullptr) return null_handle("cf_scheduler_stream");
    return guarded("cf_scheduler_stream", [&] { *stream = lease_of(scheduler, index).stream(); });
}

int64_t cf_scheduler_stream_count(const cf_scheduler* scheduler) {
    return scheduler == nullptr ? 0 : static_cast<int64_t>(scheduler->impl.stream_count());
}

cf_status cf_scheduler_copy_to_device(cf_scheduler* scheduler, int64_t index, void* device,
                                      const void* host, size_t bytes) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_copy_to_device");
    return guarded("cf_scheduler_copy_to_device", [&] {
        scheduler->impl.copy_to_device(lease_of(scheduler, index), device, host, bytes);
    });
}

cf_status cf_scheduler_copy_to_host(cf_scheduler* scheduler, int64_t index, void* host,
                                    const void* device, size_t bytes) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_copy_to_host");
    return guarded("cf_scheduler_copy_to_host", [&] {
        scheduler->impl.copy_to_host(lease_of(scheduler, index), host, device, bytes);
    });
}

cf_status cf_scheduler_record_completion(cf_scheduler* scheduler, int64_t index) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_record_completion");
    return guarded("cf_scheduler_record_completion",
                   [&] { lease_of(scheduler, index).record_completion(); });
}

cf_status cf_scheduler_chain(cf_scheduler* scheduler, int64_t waiter, int64_t signaller) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_chain");
    return guarded("cf_scheduler_chain", [&] {
        cudaforge::GpuScheduler::chain(lease_of(scheduler, waiter), lease_of(scheduler, signaller));
    });
}

cf_status cf_scheduler_note_dispatch(cf_scheduler* scheduler, int64_t index) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_note_dispatch");
    return guarded("cf_scheduler_note_dispatch",
                   [&] { scheduler->impl.note_dispatch(lease_of(scheduler, index)); });
}

cf_status cf_scheduler_synchronize(cf_scheduler* scheduler, int64_t index) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_synchronize");
    return guarded("cf_scheduler_synchronize", [&] { lease_of(scheduler, index).synchronize(); });
}

cf_status cf_scheduler_query(cf_scheduler* scheduler, int64_t index, int* complete) {
    if (scheduler == nullptr || complete == nullptr) return null_handle("cf_scheduler_query");
    return guarded("cf_scheduler_query",
                   [&] { *complete = lease_of(scheduler, index).complete() ? 1 : 0; });
}

cf_status cf_scheduler_event_query(cf_scheduler* scheduler, int64_t index, int* complete) {
    if (scheduler == nullptr || complete == nullptr) return null_handle("cf_scheduler_event_query");
    return guarded("cf_scheduler_event_query", [&] {
        *complete = lease_of(scheduler, index).completion_event().query() ? 1 : 0;
    });
}

cf_status cf_scheduler_synchronize_all(cf_scheduler* scheduler) {
    if (scheduler == nullptr) return null_handle("cf_scheduler_synchronize_all");
    return guarded("cf_scheduler_synchronize_all", [&] { scheduler->impl.synchronize_all(); });
}

cf_status cf_scheduler_stats(const cf_scheduler* scheduler, cf_stream_stats* per_stream,
                             int64_t capacity, cf_stream_stats* totals) {
    if (scheduler == nullptr || (capacity > 0 && per_stream == nullptr)) {
        return null_handle("cf_scheduler_stats");
    }
    return guarded("cf_scheduler_stats", [&] {
        const cudaforge::SchedulerStats stats = scheduler->impl.stats();
        const std::size_t n = std::min<std::size_t>(stats.per_stream.size(),
                                                    capacity > 0 ? static_cast<std::size_t>(capacity) : 0);
        for (std::size_t i = 0; i < n; ++i) {
            per_stream[i].batches_dispatched = stats.per_stream[i].batches_dispatched;
            per_stream[i].bytes_to_device = stats.per_stream[i].bytes_to_device;
            per_stream[i].bytes_to_host = stats.per_stream[i].bytes_to_host;
        }
        if (totals != nullptr) {
            totals->batches_dispatched = stats.total_dispatches;
            totals->bytes_to_device = stats.total_bytes_to_device;
            totals->bytes_to_host = stats.total_bytes_to_host;
        }
    });
}

int cf_stream_ordered_allocation_supported(void) {
    return cudaforge::supports_stream_ordered_allocation() ? 1 : 0;
}

cf_status cf_pool_create(cf_pool_backend backend, void* stream, size_t min_block_bytes, cf_pool** out) {
    if (out == nullptr) return null_handle("cf_pool_create");
    *out = nullptr;
    return guarded("cf_pool_create", [&] {
        switch (backend) {
            case CF_POOL_HOST:
                *out = new cf::PoolOf<cudaforge::HostAllocatorBackend>({}, min_block_bytes);
                break;
            case CF_POOL_DEVICE:
                *out = new cf::PoolOf<cudaforge::DeviceAllocatorBackend>({}, min_block_bytes);
                break;
            case CF_POOL_DEVICE_ASYNC:
                *out = new cf::PoolOf<cudaforge::StreamOrderedAllocatorBackend>(
                    cudaforge::StreamOrderedAllocatorBackend(static_cast<hipStream_t>(stream)),
                    min_block_bytes);
                break;
            case CF_POOL_PINNED:
                *out = new cf::PoolOf<cudaforge::PinnedAllocatorBackend>({}, min_block_bytes);
                break;
            default:
                throw std::invalid_argument("unknown pool backend");
        }
    });
}

cf_status cf_pool_destroy(cf_pool* pool) {
    delete pool;
    return CF_OK;
}

cf_status cf_pool_allocate(cf_pool* pool, size_t bytes, void** out) {
    if (pool == nullptr || out == nullptr) return null_handle("cf_pool_allocate");
    *out = nullptr;
    return guarded("cf_pool_allocate", [&] { *out = pool->allocate(bytes); });
}

cf_status cf_pool_deallocate(cf_pool* pool, void* pointer) {
    if (pool == nullptr) return null_handle("cf_pool_deallocate");
    return guarded("cf_pool_deallocate", [&] { pool->deallocate(pointer); });
}

cf_status cf_pool_trim(cf_pool* pool) {
    if (pool == nullptr) return null_handle("cf_pool_trim");
    return guarded("cf_pool_trim", [&] { pool->trim(); });
}

cf_status cf_pool_get_stats(const cf_pool* pool, cf_pool_stats* out) {
    if (pool == nullptr || out == nullptr) return null_handle("cf_pool_get_stats");
    const cudaforge::PoolStats s = pool->stats();
    out->bytes_reserved = s.bytes_reserved;
    out->bytes_in_use = s.bytes_in_use;
    out->peak_bytes_in_use = s.peak_bytes_in_use;
    out->allocation_count = s.allocation_count;
    out->backend_allocations = s.backend_allocations;
    out->reuse_count = s.reuse_count;
    out->free_count = s.free_count;
    out->free_block_count = s.free_block_count;
    return CF_OK;
}

const char* cf_pool_backend_name(cf_pool_backend backend) {
    switch (backend) {
        case CF_POOL_HOST: return cudaforge::HostAllocatorBackend::name();
        case CF_POOL_DEVICE: return cudaforge::DeviceAllocatorBackend::name();
        case CF_POOL_DEVICE_ASYNC: return cudaforge::StreamOrderedAllocatorBackend::name();
        case CF_POOL_PINNED: return cudaforge::PinnedAllocatorBackend::name();
    }
    return nullptr;
}

}  // extern "C"

// Caching allocator with power-of-two size classes over a pluggable backend.
//
// The C++ interface of the reference's pool, kept alike so code written
// against it compiles unchanged (cpp/include/cudaforge/memory_pool.hpp):
//   * `MemoryPool<Backend>` (:76-205): allocate / deallocate / trim / stats /
//     backend_name, sizes rounded up to a power of two with a floor
//     (`min_block_bytes`, default 256), reuse from per-class free lists,
//     `std::bad_alloc` when the backend returns null, `std::invalid_argument`
//     for a pointer the pool did not hand out, every block (cached or still
//     checked out) returned to the backend by the destructor;
//   * `PoolStats` (:29-44) with `reuse_rate()`;
//   * the backend contract (:22-27): `void* allocate(size_t)` returning null on
//     failure, `void deallocate(void*, size_t) noexcept`, `static const char*
//     name()`; `HostAllocatorBackend` / `HostMemoryPool` (:209-216).
//
// Pure C++17 and free of HIP, so the pool logic is exercised on a host with no
// GPU; the device, stream-ordered and pinned backends live in
// cudaforge_runtime.hpp.
//
// Free lists are indexed by log2 of the block size (64 classes) instead of a
// hash map keyed by the size: a class lookup is a bit scan. One mutex guards
// the lists and the statistics; a pool serves per-batch allocations, not
// per-kernel ones, so it is uncontended in practice.
#pragma once

#include <algorithm>
#include <array>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <new>
#include <stdexcept>
#include <type_traits>
#include <unordered_map>
#include <utility>
#include <vector>

namespace cudaforge {

struct PoolStats {
    std::size_t bytes_reserved = 0;       ///< obtained from the backend and not yet returned
    std::size_t bytes_in_use = 0;         ///< checked out to callers
    std::size_t peak_bytes_in_use = 0;    ///< high-water mark of bytes_in_use
    std::uint64_t allocation_count = 0;   ///< calls to allocate() with a non-zero size
    std::uint64_t backend_allocations = 0;
    std::uint64_t reuse_count = 0;        ///< allocations served from a free list
    std::uint64_t free_count = 0;         ///< calls to deallocate() with a pool pointer
    std::size_t free_block_count = 0;     ///< blocks cached for reuse

    double reuse_rate() const {
        return allocation_count == 0 ? 0.0
                                      : static_cast<double>(reuse_count) /
                                            static_cast<double>(allocation_count);
    }
};

namespace pool_detail {

/// Smallest power of two >= value (value >= 1), or 0 if it does not fit.
inline std::size_t next_power_of_two(std::size_t value) {
    std::size_t p = 1;
    while (p < value) {
        if (p > (~static_cast<std::size_t>(0) >> 1)) return 0;
        p <<= 1;
    }
    return p;
}

inline int log2_of_power(std::size_t power) {
    int bit = 0;
    while ((static_cast<std::size_t>(1) << bit) != power) ++bit;
    return bit;
}

template <typename B, typename = void>
struct is_backend : std::false_type {};

template <typename B>
struct is_backend<
    B, std::void_t<decltype(std::declval<B&>().allocate(std::size_t{})),
                   decltype(std::declval<B&>().deallocate(static_cast<void*>(nullptr), std::size_t{})),
                   decltype(B::name())>>
    : std::integral_constant<
          bool, std::is_same<decltype(std::declval<B&>().allocate(std::size_t{})), void*>::value &&
                    noexcept(std::declval<B&>().deallocate(static_cast<void*>(nullptr), std::size_t{})) &&
                    std::is_convertible<decltype(B::name()), const char*>::value> {};

}  // namespace pool_detail

template <typename Backend>
class MemoryPool {
    static_assert(pool_detail::is_backend<Backend>::value,
                  "a pool backend needs void* allocate(size_t), a noexcept "
                  "deallocate(void*, size_t) and a static name()");

public:
    explicit MemoryPool(Backend backend = Backend{}, std::size_t min_block_bytes = 256)
        : backend_(std::move(backend)) {
        if (min_block_bytes == 0) throw std::invalid_argument("min_block_bytes must be non-zero");
        min_block_bytes_ = pool_detail::next_power_of_two(min_block_bytes);
        if (min_block_bytes_ == 0) throw std::invalid_argument("min_block_bytes is too large");
    }

    MemoryPool(const MemoryPool&) = delete;
    MemoryPool& operator=(const MemoryPool&) = delete;
    MemoryPool(MemoryPool&&) = delete;
    MemoryPool& operator=(MemoryPool&&) = delete;

    /// Every block goes back to the backend, including blocks a caller still
    /// holds: keeping them would leak the backing memory for good.
    ~MemoryPool() { release_everything(); }

    /// A block of at least `bytes` bytes, or nullptr for a zero-byte request.
    /// Throws std::bad_alloc when the backend cannot supply one.
    void* allocate(std::size_t bytes) {
        if (bytes == 0) return nullptr;
        const std::size_t block = class_bytes(bytes);
        std::lock_guard<std::mutex> lock(mutex_);
        ++stats_.allocation_count;
        std::vector<void*>& cached = free_lists_[pool_detail::log2_of_power(block)];
        void* pointer = nullptr;
        if (!cached.empty()) {
            pointer = cached.back();
            cached.pop_back();
            ++stats_.reuse_count;
            --stats_.free_block_count;
        } else {
            pointer = backend_.allocate(block);
            if (pointer == nullptr) throw std::bad_alloc();
            ++stats_.backend_allocations;
            stats_.bytes_reserved += block;
        }
        live_[pointer] = block;
        stats_.bytes_in_use += block;
        stats_.peak_bytes_in_use = std::max(stats_.peak_bytes_in_use, stats_.bytes_in_use);
        return pointer;
    }

    /// Returns a block to its class's free list; the size comes from the
    /// pool's own record. nullptr is a no-op; a pointer the pool did not hand
    /// out (or already took back) throws std::invalid_argument.
    void deallocate(void* pointer) {
        if (pointer == nullptr) return;
        std::lock_guard<std::mutex> lock(mutex_);
        const auto entry = live_.find(pointer);
        if (entry == live_.end()) {
            throw std::invalid_argument("MemoryPool::deallocate on a pointer it did not hand out");
        }
        const std::size_t block = entry->second;
        live_.erase(entry);
        stats_.bytes_in_use -= block;
        ++stats_.free_count;
        ++stats_.free_block_count;
        free_lists_[pool_detail::log2_of_power(block)].push_back(pointer);
    }

    /// Hands every cached block back to the backend; blocks still checked
    /// out are left alone.
    void trim() {
        std::lock_guard<std::mutex> lock(mutex_);
        for (std::size_t c = 0; c < free_lists_.size(); ++c) {
            const std::size_t block = static_cast<std::size_t>(1) << c;
            for (void* pointer : free_lists_[c]) {
                backend_.deallocate(pointer, block);
                stats_.bytes_reserved -= block;
            }
            free_lists_[c].clear();
        }
        stats_.free_block_count = 0;
    }

    PoolStats stats() const {
        std::lock_guard<std::mutex> lock(mutex_);
        return stats_;
    }

    /// The size class `bytes` is served from.
    std::size_t class_bytes(std::size_t bytes) const {
        const std::size_t rounded = pool_detail::next_power_of_two(bytes);
        if (rounded == 0) throw std::bad_alloc();
        return std::max(rounded, min_block_bytes_);
    }

    Backend& backend() { return backend_; }
    static const char* backend_name() { return Backend::name(); }

private:
    void release_everything() noexcept {
        std::lock_guard<std::mutex> lock(mutex_);
        for (std::size_t c = 0; c < free_lists_.size(); ++c) {
            for (void* pointer : free_lists_[c]) {
                backend_.deallocate(pointer, static_cast<std::size_t>(1) << c);
            }
            free_lists_[c].clear();
        }
        for (const auto& entry : live_) backend_.deallocate(entry.first, entry.second);
        live_.clear();
    }

    Backend backend_;
    std::size_t min_block_bytes_ = 256;
    mutable std::mutex mutex_;
    std::array<std::vector<void*>, 64> free_lists_;
    std::unordered_map<void*, std::size_t> live_;
    PoolStats stats_;
};

/// malloc / free. Lets the pool logic run without a GPU.
class HostAllocatorBackend {
public:
    void* allocate(std::size_t bytes) const { return std::malloc(bytes); }
    void deallocate(void* pointer, std::size_t) const noexcept { std::free(pointer); }
    static const char* name() { return "host"; }
};

using HostMemoryPool = MemoryPool<HostAllocatorBackend>;

}  // namespace cudaforge

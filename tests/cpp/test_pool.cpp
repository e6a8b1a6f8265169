// Host-side tests of include/cudaforge_pool.hpp, the cases of the reference's
// tests/cpp/test_memory_pool.cpp (:51-336) restated against this pool:
// zero-byte requests, reuse, size classes, the minimum block, statistics,
// trim, foreign pointers, the destructor, concurrency, and backend failure
// (bad_alloc, recovery by trim). Built with g++ by tests/test_runtime.py.
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "cudaforge_pool.hpp"

using cudaforge::MemoryPool;

static int g_failures = 0;
static int g_checks = 0;
#define CHECK(cond)                                                                  \
    do {                                                                             \
        ++g_checks;                                                                  \
        if (!(cond)) {                                                               \
            ++g_failures;                                                            \
            std::fprintf(stderr, "%s:%d: CHECK failed: %s\n", __FILE__, __LINE__, #cond); \
        }                                                                            \
    } while (0)
#define CHECK_THROWS(expr, type)                 \
    do {                                         \
        bool thrown = false;                     \
        try {                                    \
            expr;                                \
        } catch (const type&) {                  \
            thrown = true;                       \
        }                                        \
        CHECK(thrown && #expr " throws " #type); \
    } while (0)

struct Counters {
    std::atomic<long> allocations{0};
    std::atomic<long> deallocations{0};
    std::atomic<long> live_bytes{0};
};

/// malloc-backed backend that counts calls and can refuse once its byte
/// budget is spent.
struct CountingBackend {
    Counters* counters = nullptr;
    long budget = -1;  // < 0: unlimited
    void* allocate(std::size_t bytes) {
        if (budget >= 0 && counters->live_bytes.load() + static_cast<long>(bytes) > budget) return nullptr;
        ++counters->allocations;
        counters->live_bytes += static_cast<long>(bytes);
        return std::malloc(bytes);
    }
    void deallocate(void* pointer, std::size_t bytes) noexcept {
        ++counters->deallocations;
        counters->live_bytes -= static_cast<long>(bytes);
        std::free(pointer);
    }
    static const char* name() { return "counting"; }
};

struct FailingBackend {
    void* allocate(std::size_t) { return nullptr; }
    void deallocate(void*, std::size_t) noexcept {}
    static const char* name() { return "failing"; }
};

static void test_zero_and_null() {
    cudaforge::HostMemoryPool pool;
    CHECK(pool.allocate(0) == nullptr);
    pool.deallocate(nullptr);
    CHECK(pool.stats().allocation_count == 0);
}

static void test_writable() {
    cudaforge::HostMemoryPool pool;
    constexpr std::size_t kBytes = 3000;
    auto* p = static_cast<unsigned char*>(pool.allocate(kBytes));
    CHECK(p != nullptr);
    std::memset(p, 0xAB, kBytes);
    CHECK(p[0] == 0xAB && p[kBytes - 1] == 0xAB);
    pool.deallocate(p);
}

static void test_reuse_and_classes() {
    Counters c;
    MemoryPool<CountingBackend> pool(CountingBackend{&c});
    void* a = pool.allocate(4096);
    pool.deallocate(a);
    void* b = pool.allocate(4096);
    CHECK(b == a);
    CHECK(c.allocations == 1);
    CHECK(pool.stats().reuse_count == 1 && pool.stats().backend_allocations == 1);
    pool.deallocate(b);

    void* d = pool.allocate(3000);  // 4096 class
    CHECK(d == a);
    CHECK(c.allocations == 1);
    void* e = pool.allocate(5000);  // 8192 class: a new block
    CHECK(e != d);
    CHECK(c.allocations == 2);
    CHECK(pool.class_bytes(5000) == 8192 && pool.class_bytes(1) == 256);
    pool.deallocate(d);
    pool.deallocate(e);
}

static void test_minimum_block() {
    Counters c;
    MemoryPool<CountingBackend> pool(CountingBackend{&c}, 300);  // rounds to 512
    void* a = pool.allocate(8);
    pool.deallocate(a);
    void* b = pool.allocate(500);
    CHECK(b == a);
    CHECK(c.allocations == 1);
    pool.deallocate(b);
    CHECK_THROWS(MemoryPool<CountingBackend>(CountingBackend{&c}, 0), std::invalid_argument);
}

static void test_statistics() {
    cudaforge::HostMemoryPool pool;
    std::vector<void*> blocks;
    for (int i = 0; i < 4; ++i) blocks.push_back(pool.allocate(1024));
    auto peak = pool.stats();
    CHECK(peak.bytes_in_use == 4 * 1024);
    CHECK(peak.peak_bytes_in_use == 4 * 1024);
    CHECK(peak.allocation_count == 4);
    for (void* p : blocks) pool.deallocate(p);
    auto after = pool.stats();
    CHECK(after.bytes_in_use == 0);
    CHECK(after.peak_bytes_in_use == 4 * 1024);
    CHECK(after.free_block_count == 4);
    CHECK(after.bytes_reserved == 4 * 1024);
    CHECK(after.free_count == 4);

    cudaforge::HostMemoryPool warm;
    for (int i = 0; i < 100; ++i) warm.deallocate(warm.allocate(2048));
    CHECK(warm.stats().allocation_count == 100);
    CHECK(warm.stats().backend_allocations == 1);
    CHECK(warm.stats().reuse_rate() > 0.98);
}

static void test_trim() {
    Counters c;
    MemoryPool<CountingBackend> pool(CountingBackend{&c});
    void* cached = pool.allocate(1 << 16);
    void* held = pool.allocate(1 << 12);
    pool.deallocate(cached);
    CHECK(pool.stats().free_block_count == 1);
    pool.trim();
    CHECK(pool.stats().free_block_count == 0);
    CHECK(pool.stats().bytes_reserved == (1 << 12));
    CHECK(c.deallocations == 1);  // the checked-out block is untouched
    pool.deallocate(held);
    pool.trim();
    CHECK(pool.stats().bytes_reserved == 0);
    CHECK(c.deallocations == 2);
}

static void test_foreign_and_double_free() {
    cudaforge::HostMemoryPool pool;
    int on_stack = 0;
    CHECK_THROWS(pool.deallocate(&on_stack), std::invalid_argument);
    void* p = pool.allocate(64);
    pool.deallocate(p);
    CHECK_THROWS(pool.deallocate(p), std::invalid_argument);
}

static void test_destructor_releases_everything() {
    Counters c;
    {
        MemoryPool<CountingBackend> pool(CountingBackend{&c});
        void* a = pool.allocate(1000);
        void* b = pool.allocate(70000);
        pool.allocate(5);  // still checked out at destruction
        pool.deallocate(a);
        pool.deallocate(b);
    }
    CHECK(c.live_bytes == 0);
    CHECK(c.allocations == c.deallocations);
}

static void test_concurrency() {
    cudaforge::HostMemoryPool pool;
    constexpr int kThreads = 8;
    constexpr int kPerThread = 2000;
    std::atomic<int> errors{0};
    std::vector<std::thread> workers;
    for (int t = 0; t < kThreads; ++t) {
        workers.emplace_back([&, t] {
            for (int i = 0; i < kPerThread; ++i) {
                const std::size_t bytes = 64u << ((t + i) % 6);
                auto* p = static_cast<unsigned char*>(pool.allocate(bytes));
                p[0] = static_cast<unsigned char>(t);
                p[bytes - 1] = static_cast<unsigned char>(t);
                if (p[0] != t || p[bytes - 1] != t) ++errors;
                pool.deallocate(p);
            }
        });
    }
    for (auto& w : workers) w.join();
    const auto s = pool.stats();
    CHECK(errors == 0);
    CHECK(s.allocation_count == kThreads * kPerThread);
    CHECK(s.free_count == kThreads * kPerThread);
    CHECK(s.bytes_in_use == 0);
}

static void test_names() {
    CHECK(std::string(cudaforge::HostMemoryPool::backend_name()) == "host");
    CHECK(std::string(cudaforge::HostAllocatorBackend::name()) == "host");
    CHECK(std::string(MemoryPool<FailingBackend>::backend_name()) == "failing");
}

static void test_failures() {
    MemoryPool<FailingBackend> failing;
    CHECK_THROWS(failing.allocate(1024), std::bad_alloc);
    const auto s = failing.stats();
    CHECK(s.bytes_reserved == 0 && s.bytes_in_use == 0 && s.backend_allocations == 0);
    CHECK(s.allocation_count == 1);

    Counters c;
    MemoryPool<CountingBackend> pool(CountingBackend{&c, 1 << 20});
    void* first = pool.allocate(1 << 20);  // the whole budget
    CHECK(first != nullptr);
    pool.deallocate(first);
    // A different class does not fit while the cached block holds the budget.
    CHECK_THROWS(pool.allocate(1 << 19), std::bad_alloc);
    pool.trim();
    CHECK(c.deallocations == 1);
    CHECK(pool.stats().bytes_reserved == 0);
    void* retry = pool.allocate(1 << 19);
    CHECK(retry != nullptr);
    CHECK(pool.stats().bytes_in_use == (1 << 19));
    pool.deallocate(retry);
    CHECK(pool.stats().bytes_in_use == 0);
    CHECK_THROWS(pool.allocate(~static_cast<std::size_t>(0)), std::bad_alloc);
}

int main() {
    test_zero_and_null();
    test_writable();
    test_reuse_and_classes();
    test_minimum_block();
    test_statistics();
    test_trim();
    test_foreign_and_double_free();
    test_destructor_releases_everything();
    test_concurrency();
    test_names();
    test_failures();
    std::printf("%d checks, %d failures\n", g_checks, g_failures);
    return g_failures == 0 ? 0 : 1;
}

// bm_stress.cpp -- multithreaded stress of the C++ BlockManager through its
// C ABI, built with -fsanitize=thread from block_manager.cpp and status.cpp
// alone (tests/test_block_manager_tsan.py builds and runs it on the CPU).
//
// Each scenario restates one of the reference's loom models
// (src/block_manager.rs:304-548) as a randomized stress run with more threads
// and iterations than an exhaustive model can afford; ThreadSanitizer checks
// the interleavings for data races, the assertions check the invariants:
//   unique_ownership     no block is held by two allocators at once; all
//                        blocks return (concurrent_alloc_free_unique_ownership)
//   refcount_reclaim     a block with an extra reference never reaches the
//                        free list early (refcount_prevents_premature_reclaim)
//   stale_handle         a handle freed once is StaleHandle forever after,
//                        whatever reallocation happens meanwhile
//                        (stale_handle_rejected_after_reallocation)
//   generation           per block, generation == 1 + allocations, strictly
//                        increasing as any one thread sees it
//                        (generation_monotonic_per_block)
//   exhaustion           a full pool answers OutOfBlocks{1, 0}, nothing else
//                        (exhaustion_returns_out_of_blocks)
//   mixed                random allocate / reference / free / stale-probe mix
//                        with per-block live-reference accounting
#include <atomic>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <thread>
#include <vector>

#include "../../include/zealot_kv.h"

namespace {

int g_failures = 0;
std::atomic<int> g_thread_failures{0};

#define CHECK(cond, ...)                                              \
    do {                                                              \
        if (!(cond)) {                                                \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);                        \
            std::fprintf(stderr, "\n");                               \
            g_thread_failures.fetch_add(1);                           \
            return;                                                   \
        }                                                             \
    } while (0)

template <class F>
void run_threads(int n, F f) {
    std::vector<std::thread> ts;
    for (int t = 0; t < n; ++t) ts.emplace_back(f, t);
    for (auto &t : ts) t.join();
}

// Current generation of a block: a check with generation 0 is StaleHandle
// {id, 0, current} (every real generation is >= 1).
uint64_t generation_of(zk_block_manager *bm, uint64_t id) {
    uint64_t f[3] = {0, 0, 0};
    if (zk_bm_check(bm, zk_block_handle{id, 0}) != ZK_ERR_STALE_HANDLE) return 0;
    zk_last_error_detail(f);
    return f[2];
}

void unique_ownership(int threads, int blocks, int iters) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(blocks, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    std::vector<std::atomic<bool>> in_use(blocks);
    for (auto &x : in_use) x.store(false);
    run_threads(threads, [&](int) {
        for (int i = 0; i < iters; ++i) {
            zk_block_handle h;
            int rc = zk_bm_allocate(bm, &h);
            if (rc == ZK_ERR_OUT_OF_BLOCKS) continue;
            CHECK(rc == ZK_OK, "allocate rc %d", rc);
            CHECK(!in_use[h.block_id].exchange(true, std::memory_order_acq_rel), "block %llu held twice",
                  (unsigned long long)h.block_id);
            in_use[h.block_id].store(false, std::memory_order_release);
            CHECK(zk_bm_free(bm, h) == ZK_OK, "free failed");
        }
    });
    if (zk_bm_available(bm) != (size_t)blocks) {
        std::fprintf(stderr, "FAIL unique_ownership: %zu of %d blocks free\n", zk_bm_available(bm), blocks);
        ++g_failures;
    }
    zk_bm_destroy(bm);
}

void refcount_reclaim(int writers, int blocks, int iters) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(blocks, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    std::vector<std::atomic<bool>> in_use(blocks);
    for (auto &x : in_use) x.store(false);
    run_threads(writers + 1, [&](int t) {
        for (int i = 0; i < iters; ++i) {
            zk_block_handle h;
            int rc = zk_bm_allocate(bm, &h);
            if (rc == ZK_ERR_OUT_OF_BLOCKS) continue;
            CHECK(rc == ZK_OK, "allocate rc %d", rc);
            CHECK(!in_use[h.block_id].exchange(true, std::memory_order_acq_rel), "block %llu allocated twice",
                  (unsigned long long)h.block_id);
            if (t == 0) {  // the user: reference, then two frees; the first must not reclaim
                CHECK(zk_bm_reference(bm, h) == ZK_OK, "reference failed");
                CHECK(zk_bm_free(bm, h) == ZK_OK, "free 2->1 failed");
                CHECK(zk_bm_refcount(bm, h.block_id) == 1, "refcount after 2->1 is %zu",
                      zk_bm_refcount(bm, h.block_id));
                std::this_thread::yield();  // writers run while only the reference holds it
                in_use[h.block_id].store(false, std::memory_order_release);
                CHECK(zk_bm_free(bm, h) == ZK_OK, "free 1->0 failed");
            } else {
                in_use[h.block_id].store(false, std::memory_order_release);
                CHECK(zk_bm_free(bm, h) == ZK_OK, "free failed");
            }
        }
    });
    if (zk_bm_available(bm) != (size_t)blocks) {
        std::fprintf(stderr, "FAIL refcount_reclaim: %zu of %d blocks free\n", zk_bm_available(bm), blocks);
        ++g_failures;
    }
    zk_bm_destroy(bm);
}

void stale_handle(int threads, int iters) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(1, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    run_threads(threads, [&](int t) {
        for (int i = 0; i < iters; ++i) {
            zk_block_handle h;
            if (zk_bm_allocate(bm, &h) != ZK_OK) continue;
            CHECK(zk_bm_free(bm, h) == ZK_OK, "free failed");
            if (t % 2 == 0) {  // the freed handle stays stale, whoever reallocates meanwhile
                CHECK(zk_bm_free(bm, h) == ZK_ERR_STALE_HANDLE, "double free not stale");
                uint64_t f[3];
                CHECK(zk_last_error_detail(f) == ZK_ERR_STALE_HANDLE && f[0] == h.block_id &&
                          f[1] == h.generation && f[2] > h.generation,
                      "stale fields %llu %llu %llu", (unsigned long long)f[0], (unsigned long long)f[1],
                      (unsigned long long)f[2]);
                CHECK(zk_bm_reference(bm, h) == ZK_ERR_STALE_HANDLE, "stale reference accepted");
            }
        }
    });
    if (zk_bm_available(bm) != 1) {
        std::fprintf(stderr, "FAIL stale_handle: pool not whole\n");
        ++g_failures;
    }
    zk_bm_destroy(bm);
}

void generation(int threads, int blocks, int iters) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(blocks, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    std::vector<std::vector<std::pair<uint64_t, uint64_t>>> logs(threads);
    run_threads(threads, [&](int t) {
        for (int i = 0; i < iters; ++i) {
            zk_block_handle h;
            if (zk_bm_allocate(bm, &h) != ZK_OK) continue;
            logs[t].emplace_back(h.block_id, h.generation);
            CHECK(zk_bm_free(bm, h) == ZK_OK, "free failed");
        }
    });
    std::vector<uint64_t> allocs(blocks, 0);
    for (const auto &log : logs) {
        std::vector<uint64_t> prev(blocks, 0);
        for (const auto &e : log) {
            if (e.second <= prev[e.first]) {
                std::fprintf(stderr, "FAIL generation: block %llu gen %llu after %llu\n",
                             (unsigned long long)e.first, (unsigned long long)e.second,
                             (unsigned long long)prev[e.first]);
                ++g_failures;
            }
            prev[e.first] = e.second;
            ++allocs[e.first];
        }
    }
    for (int b = 0; b < blocks; ++b)
        if (generation_of(bm, b) != 1 + allocs[b]) {
            std::fprintf(stderr, "FAIL generation: block %d gen %llu, allocations %llu\n", b,
                         (unsigned long long)generation_of(bm, b), (unsigned long long)allocs[b]);
            ++g_failures;
        }
    if (zk_bm_available(bm) != (size_t)blocks) ++g_failures;
    zk_bm_destroy(bm);
}

void exhaustion(int threads, int iters) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(1, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    run_threads(threads, [&](int) {
        for (int i = 0; i < iters; ++i) {
            zk_block_handle h;
            int rc = zk_bm_allocate(bm, &h);
            if (rc == ZK_OK) {
                CHECK(zk_bm_free(bm, h) == ZK_OK, "free failed");
                continue;
            }
            uint64_t f[3];
            CHECK(rc == ZK_ERR_OUT_OF_BLOCKS, "unexpected rc %d", rc);
            CHECK(zk_last_error_detail(f) == ZK_ERR_OUT_OF_BLOCKS && f[0] == 1 && f[1] == 0, "fields");
        }
    });
    if (zk_bm_available(bm) != 1) ++g_failures;
    zk_bm_destroy(bm);
}

void mixed(int threads, int blocks, int iters, unsigned seed) {
    zk_block_manager *bm = nullptr;
    if (zk_bm_create(blocks, 16, &bm) != ZK_OK) return (void)g_thread_failures.fetch_add(1);
    std::vector<std::atomic<int>> live(blocks);  // live references over all threads
    for (auto &x : live) x.store(0);
    run_threads(threads, [&](int t) {
        std::mt19937 rng(seed + 7919u * (unsigned)t);
        std::vector<zk_block_handle> held, dead;  // one entry per reference this thread holds
        for (int i = 0; i < iters; ++i) {
            const unsigned op = rng() % 10;
            if (op < 4) {
                zk_block_handle h;
                int rc = zk_bm_allocate(bm, &h);
                if (rc == ZK_ERR_OUT_OF_BLOCKS) continue;
                CHECK(rc == ZK_OK, "allocate rc %d", rc);
                CHECK(live[h.block_id].fetch_add(1) == 0, "allocated a block with live references");
                held.push_back(h);
            } else if (op < 6 && !held.empty()) {
                const zk_block_handle h = held[rng() % held.size()];
                CHECK(zk_bm_reference(bm, h) == ZK_OK, "reference of a live handle failed");
                live[h.block_id].fetch_add(1);
                held.push_back(h);
            } else if (op < 9 && !held.empty()) {
                const size_t j = rng() % held.size();
                const zk_block_handle h = held[j];
                held[j] = held.back();
                held.pop_back();
                bool last = true;
                for (const auto &x : held) last = last && !(x.block_id == h.block_id && x.generation == h.generation);
                live[h.block_id].fetch_sub(1);
                CHECK(zk_bm_free(bm, h) == ZK_OK, "free of a live handle failed");
                if (last) dead.push_back(h);  // only this thread referenced it: may be gone now
            } else if (!dead.empty()) {
                // a handle whose references were all this thread's is stale
                // once freed, unless another thread referenced it first: it
                // cannot have (references come from holders only)
                const zk_block_handle h = dead[rng() % dead.size()];
                int rc = zk_bm_reference(bm, h);
                CHECK(rc == ZK_ERR_STALE_HANDLE, "reference of a freed handle: rc %d", rc);
            }
        }
        for (const auto &h : held) {
            live[h.block_id].fetch_sub(1);
            CHECK(zk_bm_free(bm, h) == ZK_OK, "final free failed");
        }
    });
    if (zk_bm_available(bm) != (size_t)blocks) {
        std::fprintf(stderr, "FAIL mixed: %zu of %d blocks free\n", zk_bm_available(bm), blocks);
        ++g_failures;
    }
    for (int b = 0; b < blocks; ++b)
        if (zk_bm_refcount(bm, b) != 0 || live[b].load() != 0) ++g_failures;
    zk_bm_destroy(bm);
}

}  // namespace

int main(int argc, char **argv) {
    const int threads = argc > 1 ? std::atoi(argv[1]) : 8;
    const int iters = argc > 2 ? std::atoi(argv[2]) : 2000;
    unique_ownership(threads, 4, iters);
    refcount_reclaim(threads - 1, 3, iters);
    stale_handle(threads, iters);
    generation(threads, 4, iters);
    exhaustion(threads, iters);
    mixed(threads, 16, iters, 12345u);
    const int fails = g_failures + g_thread_failures.load();
    std::printf("bm_stress: %d threads x %d iterations, %d failures\n", threads, iters, fails);
    return fails ? 1 : 0;
}

// block_manager.cpp -- generation-gated block allocator (host side).
//
// Semantics of src/block_manager.rs:86-164:
//  - create: InvalidBlockSize when block_size == 0; the free list is a stack
//    holding n-1 .. 0 so the first allocation returns block 0; every block
//    starts at generation 1, refcount 0 (block_manager.rs:88-104).
//  - allocate: pop, refcount := 1, handle carries the current generation; an
//    empty stack is OutOfBlocks{requested: 1, available: 0}
//    (block_manager.rs:108-122).
//  - free: check, refcount -= 1; when it drops from 1 to 0 the generation is
//    bumped and the block pushed back (block_manager.rs:125-135).
//  - reference: check, refcount += 1 (block_manager.rs:140-144).
//  - check: id >= n -> BlockNotAllocated, generation mismatch -> StaleHandle
//    (block_manager.rs:151-164).  One addition: a handle whose generation
//    matches a block that is free (refcount 0, only reachable with a handle
//    forged by hand) is BlockNotAllocated instead of wrapping the refcount.
// Thread-safe: the free stack is under a mutex, refcounts and generations are
// atomics, like the reference (Mutex + AtomicUsize/AtomicU64).
#include <atomic>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "zk_error.h"

struct zk_block_manager {
    size_t num_gpu_blocks = 0;
    size_t block_size = 0;
    std::mutex mu;
    std::vector<uint64_t> free_list;
    std::unique_ptr<std::atomic<uint64_t>[]> refcount;
    std::unique_ptr<std::atomic<uint64_t>[]> generation;
};

namespace {

int check(zk_block_manager *bm, zk_block_handle h) {
    if (h.block_id >= bm->num_gpu_blocks)
        return zk::set_error_typed(ZK_ERR_BLOCK_NOT_ALLOCATED, zk::ErrorKind::BlockNotAllocated, h.block_id);
    uint64_t cur = bm->generation[h.block_id].load(std::memory_order_acquire);
    if (h.generation != cur)
        return zk::set_error_typed(ZK_ERR_STALE_HANDLE, zk::ErrorKind::StaleHandle, h.block_id,
                                      h.generation, cur);
    return ZK_OK;
}

}  // namespace

extern "C" {

int zk_bm_create(size_t num_gpu_blocks, size_t block_size, zk_block_manager **out) {
    if (!out) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_bm_create: out is NULL");
    *out = nullptr;
    if (block_size == 0)
        return zk::set_error_typed(ZK_ERR_INVALID_BLOCK_SIZE, zk::ErrorKind::InvalidBlockSize, 0);
    auto *bm = new (std::nothrow) zk_block_manager();
    if (!bm) return zk::set_error(ZK_ERR_INTERNAL, "Internal error: BlockManager allocation failed");
    try {
        bm->num_gpu_blocks = num_gpu_blocks;
        bm->block_size = block_size;
        bm->free_list.resize(num_gpu_blocks);
        for (size_t i = 0; i < num_gpu_blocks; ++i) bm->free_list[i] = num_gpu_blocks - 1 - i;
        bm->refcount.reset(new std::atomic<uint64_t>[num_gpu_blocks]);
        bm->generation.reset(new std::atomic<uint64_t>[num_gpu_blocks]);
    } catch (const std::bad_alloc &) {
        delete bm;
        return zk::set_error(ZK_ERR_INTERNAL, "Internal error: BlockManager allocation failed");
    }
    for (size_t i = 0; i < num_gpu_blocks; ++i) {
        bm->refcount[i].store(0, std::memory_order_relaxed);
        bm->generation[i].store(1, std::memory_order_relaxed);
    }
    *out = bm;
    return ZK_OK;
}

void zk_bm_destroy(zk_block_manager *bm) { delete bm; }

int zk_bm_allocate(zk_block_manager *bm, zk_block_handle *out) {
    if (!bm || !out) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_bm_allocate: NULL argument");
    uint64_t id;
    {
        std::lock_guard<std::mutex> g(bm->mu);
        if (bm->free_list.empty())
            return zk::set_error_typed(ZK_ERR_OUT_OF_BLOCKS, zk::ErrorKind::OutOfBlocks, 1, 0);
        id = bm->free_list.back();
        bm->free_list.pop_back();
    }
    uint64_t gen = bm->generation[id].load(std::memory_order_acquire);
    bm->refcount[id].store(1, std::memory_order_release);
    out->block_id = id;
    out->generation = gen;
    return ZK_OK;
}

int zk_bm_free(zk_block_manager *bm, zk_block_handle h) {
    if (!bm) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_bm_free: NULL manager");
    if (int rc = check(bm, h)) return rc;
    uint64_t prev = bm->refcount[h.block_id].load(std::memory_order_acquire);
    do {
        if (prev == 0)
            return zk::set_error_typed(ZK_ERR_BLOCK_NOT_ALLOCATED, zk::ErrorKind::BlockNotAllocated,
                                          h.block_id);
    } while (!bm->refcount[h.block_id].compare_exchange_weak(prev, prev - 1,
                                                              std::memory_order_acq_rel));
    if (prev == 1) {
        bm->generation[h.block_id].fetch_add(1, std::memory_order_acq_rel);
        std::lock_guard<std::mutex> g(bm->mu);
        bm->free_list.push_back(h.block_id);
    }
    return ZK_OK;
}

int zk_bm_reference(zk_block_manager *bm, zk_block_handle h) {
    if (!bm) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_bm_reference: NULL manager");
    if (int rc = check(bm, h)) return rc;
    uint64_t prev = bm->refcount[h.block_id].load(std::memory_order_acquire);
    do {
        if (prev == 0)
            return zk::set_error_typed(ZK_ERR_BLOCK_NOT_ALLOCATED, zk::ErrorKind::BlockNotAllocated,
                                          h.block_id);
    } while (!bm->refcount[h.block_id].compare_exchange_weak(prev, prev + 1,
                                                              std::memory_order_acq_rel));
    return ZK_OK;
}

int zk_bm_check(zk_block_manager *bm, zk_block_handle h) {
    if (!bm) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_bm_check: NULL manager");
    if (int rc = check(bm, h)) return rc;
    if (bm->refcount[h.block_id].load(std::memory_order_acquire) == 0)
        return zk::set_error_typed(ZK_ERR_BLOCK_NOT_ALLOCATED, zk::ErrorKind::BlockNotAllocated, h.block_id);
    return ZK_OK;
}

size_t zk_bm_available(const zk_block_manager *bm) {
    if (!bm) return 0;
    auto *m = const_cast<zk_block_manager *>(bm);
    std::lock_guard<std::mutex> g(m->mu);
    return m->free_list.size();
}

size_t zk_bm_num_gpu_blocks(const zk_block_manager *bm) { return bm ? bm->num_gpu_blocks : 0; }
size_t zk_bm_block_size(const zk_block_manager *bm) { return bm ? bm->block_size : 0; }

size_t zk_bm_refcount(const zk_block_manager *bm, uint64_t block_id) {
    if (!bm || block_id >= bm->num_gpu_blocks) return 0;
    return (size_t)bm->refcount[block_id].load(std::memory_order_acquire);
}

}  // extern "C"

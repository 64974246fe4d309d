// kv_cache.cpp -- stateful paged KV cache (host side of src/kv_cache.rs).
//
// Owns the K and V pools of every layer in one HBM slab
//   [layer][K|V][num_blocks][Hkv][block_size][D]
// (per-pool layout of kv_cache.rs:41-50; one block id indexes every layer's
// pool, kv_cache.rs:241-253) and one slab of per-sequence device block tables
// [max_seqs][max_blocks_per_seq] (int32, -1 = unused, kv_cache.rs:107-124).
// The host keeps each sequence's BlockManager handles, so block tables,
// slot mappings and copy-on-write decisions are computed on the host and every
// data movement is one kernel launch (zk_append / zk_copy_blocks /
// zk_paged_decode) instead of per-(token, head) driver copies.
//
// Differences from the reference, all deliberate:
//  - store_kv / append_kv write through one slot-mapping launch; a position
//    without a block fails before anything is written.
//  - The write position advances once per token, when the last layer is
//    written (the reference advances on every append_kv call, i.e. once per
//    layer, and never on store_kv).
//  - release_seq returns the sequence's blocks to its BlockManager.
//  - fork_seq / copy-on-write and append_kv_batch have no reference
//    counterpart.
//  - Decode at layer l sees every token written at layer l, so a decode step
//    may interleave append_kv(l) and paged_decode(l) layer by layer.
// Not thread-safe: one thread drives a cache (as GpuContext, gpu_context.rs:23-26).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <functional>
#include <cstdint>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/zealot_dense.h"
#include "zk_common.h"

using zk::set_error;

namespace {

struct SeqState {
    std::vector<zk_block_handle> handles;
    zk_block_manager *bm = nullptr;
    bool borrowed = false;        // handles owned by the caller (zk_cache_bind_blocks)
    bool swapped = false;         // K/V held in host slots (zk_cache_swap_out)
    std::vector<int32_t> host_slots;  // host slot of block i while swapped
    size_t cached_tokens = 0;     // tokens written at the last layer
    size_t block_offset = 0;
    size_t max_blocks = 0;
    size_t slot = 0;
    std::vector<size_t> layer_len;  // tokens written per layer (decode length)
    std::vector<float> k_scales, v_scales;  // [layers * Hkv], fp8 pools
};

// Growable device buffer.
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    int ensure(size_t bytes, const char *what) {
        if (bytes <= cap) return ZK_OK;
        if (p) {
            // kernels queued earlier may still read the old buffer
            ZK_HIP_CHECK(hipDeviceSynchronize(), what);
            (void)hipFree(p);
        }
        p = nullptr;
        cap = 0;
        // a quarter more than asked: tables and batches grow a little at a
        // time, and each regrowth waits for the device
        size_t want = std::max<size_t>(bytes + bytes / 4, 4096);
        ZK_HIP_CHECK(hipMalloc(&p, want), what);
        cap = want;
        return ZK_OK;
    }
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

// Pinned staging buffer; reuse waits for the copy that last read it.  The
// cache cycles through a ring of them so the host only waits when the device
// is a whole ring of uploads behind.
struct Staging {
    void *p = nullptr;
    size_t cap = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
    int ensure(size_t bytes) {
        if (pending) {
            ZK_HIP_CHECK(hipEventSynchronize(done), "KVCache staging wait");
            pending = false;
        }
        if (!done) ZK_HIP_CHECK(hipEventCreateWithFlags(&done, hipEventDisableTiming), "KVCache event");
        if (bytes <= cap) return ZK_OK;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
        size_t want = std::max<size_t>(bytes + bytes / 4, 64 << 10);  // freeing pinned memory waits for the device
        ZK_HIP_CHECK(hipHostMalloc(&p, want, hipHostMallocDefault), "KVCache pinned staging");
        cap = want;
        return ZK_OK;
    }
    ~Staging() {
        if (pending && done) (void)hipEventSynchronize(done);
        if (p) (void)hipHostFree(p);
        if (done) (void)hipEventDestroy(done);
    }
};

// Device buffer whose last uploaded bytes are remembered: an upload of the
// same bytes is skipped (a decode step writes the same slot mapping and
// lengths for every layer).
struct CachedBuf {
    DevBuf dev;
    std::vector<char> last;
};

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
        else prev = -1;
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

}  // namespace

// Prefix subgroups of a decode batch (plan_sharing): each sequence's shared
// pages, the members of every subgroup ([nsg][32], -1 padded) and its pages.
struct SharePlan {
    std::vector<int32_t> seq_pb, sg_members, sg_pages;
    long total_pages = 0;
};

struct zk_kv_cache {
    size_t num_blocks = 0, block_size = 0, num_layers = 0, num_kv_heads = 0, head_dim = 0;
    int dtype = ZK_F32;
    size_t max_seqs = 0, max_blocks_per_seq = 0;
    int device = 0;
    int cus = 256;  // compute units of the device
    hipStream_t stream = nullptr;
    char *slab = nullptr;
    size_t pool_bytes = 0;
    int32_t *tables = nullptr;
    std::vector<size_t> free_slots;
    std::unordered_map<std::string, SeqState> seqs;
    CachedBuf d_meta;  // slot mappings, token rows, scales
    DevBuf d_cow;      // copy-on-write (src, dst) block ids
    DevBuf d_tblupd;   // block-table updates (offset, value)
    CachedBuf d_tbl;   // decode batch block tables [n][stride]
    CachedBuf d_batch; // decode batch lengths + scales
    // what the last decode plan was made from (shapes, lengths, prefix
    // groups, the uploaded tables and workspace); a call with the same bytes
    // reuses it
    std::vector<char> plan_sig;
    uint64_t tbl_version = 0;  // bumped whenever d_tbl receives different tables
    CachedBuf d_pre;   // prefill batch tables, row offsets, lengths, starts, scales
    DevBuf d_pws;      // prefill workspace
    DevBuf d_ws;     // decode workspace
    static constexpr int kStages = 16;
    Staging stage[kStages];
    int next_stage = 0;
    std::vector<int2> tbl_updates;  // pending writes into `tables`
    // Decode-table cache: the batch table is re-uploaded only when a block
    // table changed (epoch) or the batch is a different list of sequences.
    uint64_t epoch = 0;
    uint64_t dec_epoch = ~0ull;
    size_t dec_stride = 0;
    std::vector<const SeqState *> dec_ids;
    // Prefix-sharing cache: the last grouping and what it was made from
    // (epoch, batch, member cap, each sequence's fully written pages).
    SharePlan sh_plan;
    uint64_t sh_epoch = ~0ull;
    int sh_cap = 0;
    std::vector<const SeqState *> sh_ids;
    std::vector<size_t> sh_full;
    // Second stream for the chunk half of a mixed attention batch, so the
    // MFMA-bound prefill runs beside the HBM-bound decode (default priority).
    hipStream_t side = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    // Swap space: pinned host slots of one block of every pool (all layers,
    // K and V: 2 * L * block_bytes), lowest free slot first so a sequence's
    // blocks form long runs (one DMA each); device staging in chunks.
    char *host_pool = nullptr;
    size_t host_total = 0;
    std::vector<int32_t> host_free;  // sorted descending: back() is the lowest
    DevBuf d_stage, d_swap_ids;
    int dec_head_set = 0;     // queue-head set of the next decode launch that reuses its plan
    int last_sg = 0;          // prefix subgroups of the last paged_decode
    int64_t last_sg_pages = 0;  // and the pages they shared (summed over subgroups)

    size_t block_bytes() const { return block_size * num_kv_heads * head_dim * zk::elt_size(dtype); }
    char *k_pool(size_t layer) const { return slab + (2 * layer) * pool_bytes; }
    char *v_pool(size_t layer) const { return slab + (2 * layer + 1) * pool_bytes; }
    int32_t *table_row(size_t slot) const { return tables + slot * max_blocks_per_seq; }

    ~zk_kv_cache() {
        if (stream) (void)hipStreamSynchronize(stream);
        if (side) (void)hipStreamSynchronize(side);
        if (fork_ev) (void)hipEventDestroy(fork_ev);
        if (join_ev) (void)hipEventDestroy(join_ev);
        if (side) (void)hipStreamDestroy(side);
        if (host_pool) (void)hipHostFree(host_pool);
        if (slab) (void)hipFree(slab);
        if (tables) (void)hipFree(tables);
    }
};

namespace {

int find_seq(zk_kv_cache *c, const char *id, SeqState **out) {
    if (!c || !id) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache: NULL argument");
    auto it = c->seqs.find(id);
    if (it == c->seqs.end())
        return set_error(ZK_ERR_INTERNAL, std::string("Internal error: KVCache: unknown seq ") + id);
    *out = &it->second;
    return ZK_OK;
}

// Upload `bytes` from host memory to device memory on the cache stream.
int upload(zk_kv_cache *c, void *dst, const void *src, size_t bytes) {
    if (bytes == 0) return ZK_OK;
    Staging &st = c->stage[c->next_stage];
    c->next_stage = (c->next_stage + 1) % zk_kv_cache::kStages;
    if (int rc = st.ensure(bytes)) return rc;
    std::memcpy(st.p, src, bytes);
    ZK_HIP_CHECK(hipMemcpyAsync(dst, st.p, bytes, hipMemcpyHostToDevice, c->stream), "KVCache upload");
    ZK_HIP_CHECK(hipEventRecord(st.done, c->stream), "KVCache upload event");
    st.pending = true;
    return ZK_OK;
}

// Upload into a CachedBuf unless it already holds exactly these bytes.
int put(zk_kv_cache *c, CachedBuf &b, const void *host, size_t bytes, const char *what) {
    if (bytes && b.last.size() == bytes && std::memcmp(b.last.data(), host, bytes) == 0) return ZK_OK;
    b.last.clear();
    if (int rc = b.dev.ensure(bytes, what)) return rc;
    if (int rc = upload(c, b.dev.p, host, bytes)) return rc;
    b.last.assign((const char *)host, (const char *)host + bytes);
    return ZK_OK;
}

void queue_table_entry(zk_kv_cache *c, const SeqState &s, size_t idx, int32_t value) {
    c->tbl_updates.push_back(make_int2((int)(s.slot * c->max_blocks_per_seq + idx), value));
    ++c->epoch;
}

// Apply the queued block-table writes in one launch.  Writes may wait in the
// queue: the decode and prefill build their tables from the host handles, so
// only the device table rows (`zk_cache_block_table_ptr`, a fork's row copy,
// a row reset) need them, and those call this first.  Every write flushes
// too, so the queue stays short and a step's block allocations go to the
// device as one upload and one launch.
int flush_tables(zk_kv_cache *c) {
    if (c->tbl_updates.empty()) return ZK_OK;
    // The scatter writes its entries in parallel, so an entry queued twice
    // (an allocation, then a swap-out or a bind before any flush) would land
    // in either order: keep only the last write to each entry.  The queue is
    // in program order, and the stable sort keeps that order within an entry.
    std::vector<int2> &q = c->tbl_updates;
    std::stable_sort(q.begin(), q.end(), [](const int2 &a, const int2 &b) { return a.x < b.x; });
    size_t m = 0;
    for (size_t i = 0; i < q.size(); ++i)
        if (i + 1 == q.size() || q[i + 1].x != q[i].x) q[m++] = q[i];
    q.resize(m);
    const size_t n = q.size();
    int rc = c->d_tblupd.ensure(n * sizeof(int2), "KVCache table update");
    if (!rc) rc = upload(c, c->d_tblupd.p, c->tbl_updates.data(), n * sizeof(int2));
    if (!rc)
        rc = zk::scatter_i32(c->tables, (int64_t)(c->max_seqs * c->max_blocks_per_seq), (const int2 *)c->d_tblupd.p,
                             (int)n, c->stream);
    // on failure the writes stay queued (they are idempotent): the next flush
    // applies them, so the device rows never miss an entry the host recorded
    if (!rc) c->tbl_updates.clear();
    return rc;
}

// Copy-on-write of every (seq, block index) in `targets`: fresh blocks, one
// copy launch over every pool (all layers, K and V), drop the shared
// references, point the tables at the copies.  On an allocation failure
// nothing has been copied and the fresh blocks are returned.
int cow_blocks(zk_kv_cache *c, const std::vector<std::pair<SeqState *, size_t>> &targets) {
    if (targets.empty()) return ZK_OK;
    for (const auto &t : targets)
        if (t.first->borrowed)  // the caller owns these handles: it must not see them replaced
            return set_error(ZK_ERR_FAILED_PRECONDITION,
                             "Failed precondition: KVCache: copy-on-write of a block whose handle the caller "
                             "owns (bound sequence)");
    // pairs with the same source next to each other: the copy kernel then
    // reads each shared block once per run of forks copying it
    std::vector<std::pair<SeqState *, size_t>> sorted(targets);
    std::stable_sort(sorted.begin(), sorted.end(), [](const auto &x, const auto &y) {
        return x.first->handles[x.second].block_id < y.first->handles[y.second].block_id;
    });
    const auto &tg = sorted;
    const size_t n = tg.size();
    std::vector<zk_block_handle> fresh(n);
    std::vector<int32_t> pairs(2 * n);
    for (size_t i = 0; i < n; ++i) {
        SeqState &s = *tg[i].first;
        if (zk_bm_allocate(s.bm, &fresh[i]) != ZK_OK) {
            const zk::ErrorSnapshot saved = zk::save_error();
            for (size_t j = 0; j < i; ++j) (void)zk_bm_free(tg[j].first->bm, fresh[j]);
            return zk::restore_error(saved);
        }
        pairs[i] = (int32_t)s.handles[tg[i].second].block_id;
        pairs[n + i] = (int32_t)fresh[i].block_id;
    }
    int rc = c->d_cow.ensure(pairs.size() * sizeof(int32_t), "KVCache cow scratch");
    if (!rc) rc = upload(c, c->d_cow.p, pairs.data(), pairs.size() * sizeof(int32_t));
    if (!rc) {
        std::vector<void *> pools(2 * c->num_layers);
        for (size_t l = 0; l < c->num_layers; ++l) {
            pools[2 * l] = c->k_pool(l);
            pools[2 * l + 1] = c->v_pool(l);
        }
        const int32_t *d = (const int32_t *)c->d_cow.p;
        rc = zk_copy_blocks(pools.data(), (int)pools.size(), (int64_t)c->block_bytes(), (int64_t)c->num_blocks,
                            d, d + n, (int64_t)n, c->stream);
    }
    if (rc) {
        const zk::ErrorSnapshot saved = zk::save_error();
        for (size_t j = 0; j < n; ++j) (void)zk_bm_free(tg[j].first->bm, fresh[j]);
        return zk::restore_error(saved);
    }
    int first_rc = ZK_OK;
    zk::ErrorSnapshot first_err;
    for (size_t i = 0; i < n; ++i) {
        SeqState &s = *tg[i].first;
        size_t idx = tg[i].second;
        int frc = zk_bm_free(s.bm, s.handles[idx]);
        if (frc && !first_rc) {
            first_rc = frc;
            first_err = zk::save_error();
        }
        s.handles[idx] = fresh[i];
        queue_table_entry(c, s, idx, (int32_t)fresh[i].block_id);
    }
    rc = flush_tables(c);
    if (first_rc) return zk::restore_error(first_err);
    return rc;
}

void release_host_slots(zk_kv_cache *c, SeqState &s) {
    for (int32_t h : s.host_slots) c->host_free.push_back(h);
    std::sort(c->host_free.begin(), c->host_free.end(), std::greater<int32_t>());
    s.host_slots.clear();
    s.swapped = false;
}

size_t host_slot_bytes(const zk_kv_cache *c) { return 2 * c->num_layers * c->block_bytes(); }

// Moves blocks between the pools and host slots: pairs (slot, device block)
// sorted by slot, staged through device memory in chunks, one DMA per run of
// consecutive slots.  out: pools -> host, else host -> pools.
int swap_move(zk_kv_cache *c, std::vector<std::pair<int32_t, int32_t>> &pairs, bool out) {
    if (pairs.empty()) return ZK_OK;
    std::sort(pairs.begin(), pairs.end());
    const size_t sb = host_slot_bytes(c);
    constexpr size_t kStageBytes = 512ull << 20;
    const size_t chunk = std::max<size_t>(1, kStageBytes / sb);
    const size_t n = pairs.size();
    std::vector<int32_t> blocks(n);
    for (size_t i = 0; i < n; ++i) blocks[i] = pairs[i].second;
    if (int rc = c->d_swap_ids.ensure(n * sizeof(int32_t), "KVCache swap ids")) return rc;
    if (int rc = upload(c, c->d_swap_ids.p, blocks.data(), n * sizeof(int32_t))) return rc;
    if (int rc = c->d_stage.ensure(std::min(n, chunk) * sb, "KVCache swap staging")) return rc;
    char *stage = (char *)c->d_stage.p;
    for (size_t c0 = 0; c0 < n; c0 += chunk) {
        const size_t cn = std::min(chunk, n - c0);
        if (out && (int)cn > 0)
            if (int rc = zk::swap_stage(c->slab, c->pool_bytes, c->block_bytes(), (int)(2 * c->num_layers),
                                        (const int32_t *)c->d_swap_ids.p + c0, (int)cn, stage, (int64_t)c->num_blocks,
                                        true, c->stream))
                return rc;
        for (size_t r0 = 0; r0 < cn;) {  // runs of consecutive host slots
            size_t r1 = r0 + 1;
            while (r1 < cn && pairs[c0 + r1].first == pairs[c0 + r1 - 1].first + 1) ++r1;
            char *host = c->host_pool + (size_t)pairs[c0 + r0].first * sb;
            char *dev = stage + r0 * sb;
            ZK_HIP_CHECK(hipMemcpyAsync(out ? host : dev, out ? dev : host, (r1 - r0) * sb,
                                        out ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice, c->stream),
                         "KVCache swap copy");
            r0 = r1;
        }
        if (!out)
            if (int rc = zk::swap_stage(c->slab, c->pool_bytes, c->block_bytes(), (int)(2 * c->num_layers),
                                        (const int32_t *)c->d_swap_ids.p + c0, (int)cn, stage, (int64_t)c->num_blocks,
                                        false, c->stream))
                return rc;
    }
    return ZK_OK;
}

int write_tokens(zk_kv_cache *c, size_t layer, SeqState &s, const char *id, const void *k, const void *v,
                 zk_dtype src_dtype, size_t start, size_t n, const char *what) {
    if (layer >= c->num_layers)
        return set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: KVCache ") + what +
                                                      ": layer " + std::to_string(layer) + " out of range");
    if (src_dtype != ZK_F32 && src_dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: KVCache ") + what + ": bad src dtype");
    if (n == 0) return ZK_OK;
    if (!k || !v) return set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: KVCache ") + what + ": NULL k/v");
    if (int rc = flush_tables(c)) return rc;
    if (s.swapped)
        return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + id + " is swapped out");
    const size_t bs = c->block_size;
    size_t last_idx = (start + n - 1) / bs;
    if (last_idx >= s.handles.size())  // kv_cache.rs:234-239
        return set_error(ZK_ERR_INTERNAL, std::string("Internal error: KVCache ") + what + ": block_idx " +
                                              std::to_string(last_idx) + " OOB (have " +
                                              std::to_string(s.handles.size()) + " blocks)");
    if (c->dtype == ZK_FP8_E4M3 && s.k_scales.empty())
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         std::string("Failed precondition: fp8 scales not set for seq ") + id);
    // Copy-on-write every shared block this write touches.
    std::vector<std::pair<SeqState *, size_t>> shared;
    for (size_t idx = start / bs; idx <= last_idx; ++idx)
        if (zk_bm_refcount(s.bm, s.handles[idx].block_id) > 1) shared.emplace_back(&s, idx);
    if (int rc = cow_blocks(c, shared)) return rc;

    const size_t H = c->num_kv_heads;
    const bool fp8 = c->dtype == ZK_FP8_E4M3;
    size_t slots_bytes = n * sizeof(int64_t);
    size_t rows_bytes = fp8 ? n * sizeof(int32_t) : 0;
    size_t scale_bytes = fp8 ? 2 * H * sizeof(float) : 0;
    size_t total = slots_bytes + rows_bytes + scale_bytes;
    std::vector<char> host(total);
    int64_t *slots = (int64_t *)host.data();
    for (size_t t = 0; t < n; ++t) {
        size_t g = start + t;
        slots[t] = (int64_t)s.handles[g / bs].block_id * (int64_t)bs + (int64_t)(g % bs);
    }
    if (fp8) {
        std::memset(host.data() + slots_bytes, 0, rows_bytes);  // every token uses scale row 0
        float *sc = (float *)(host.data() + slots_bytes + rows_bytes);
        std::memcpy(sc, s.k_scales.data() + layer * H, H * sizeof(float));
        std::memcpy(sc + H, s.v_scales.data() + layer * H, H * sizeof(float));
    }
    if (int rc = put(c, c->d_meta, host.data(), total, "KVCache slot mapping")) return rc;
    char *d = (char *)c->d_meta.dev.p;
    const int32_t *d_rows = fp8 ? (const int32_t *)(d + slots_bytes) : nullptr;
    const float *d_ks = fp8 ? (const float *)(d + slots_bytes + rows_bytes) : nullptr;
    const float *d_vs = fp8 ? d_ks + H : nullptr;
    if (int rc = zk_append(c->k_pool(layer), c->v_pool(layer), (zk_dtype)c->dtype, k, v, src_dtype,
                           (const int64_t *)d, (int64_t)n, (int)H, (int)c->head_dim, (int)bs,
                           (int64_t)c->num_blocks, d_ks, d_vs, d_rows, c->stream))
        return rc;
    s.layer_len[layer] = std::max(s.layer_len[layer], start + n);
    if (layer + 1 == c->num_layers) {
        s.cached_tokens = std::max(s.cached_tokens, start + n);
        s.block_offset = s.cached_tokens % bs;
    }
    return ZK_OK;
}

// Shared prefixes of a decode batch: sequences whose tables start with the
// same blocks (fork_seq) read those pages once per subgroup.  A subgroup
// holds at most `cap` members (32 query rows / G) and shares the longest
// common run of leading blocks that every member has fully written at this
// layer; runs shorter than kMinSharedPages are not worth a subgroup.
constexpr size_t kMinSharedPages = 16;

constexpr int kSgStride = 32;  // member slots per subgroup (the kernel's layout)

// full[i]: the pages of sequence i fully written at the layer
void plan_sharing(const std::vector<const SeqState *> &seqs, const std::vector<size_t> &full, int cap,
                  SharePlan &out) {
    const int n = (int)seqs.size();
    out.seq_pb.assign(n, 0);
    out.sg_members.clear();
    out.sg_pages.clear();
    out.total_pages = 0;
    std::vector<std::pair<uint64_t, int>> keyed;
    for (int i = 0; i < n; ++i)
        if (full[i] >= kMinSharedPages) keyed.emplace_back(seqs[i]->handles[0].block_id, i);
    std::sort(keyed.begin(), keyed.end());
    for (size_t a = 0; a < keyed.size();) {
        size_t b = a;
        while (b < keyed.size() && keyed[b].first == keyed[a].first) ++b;
        for (size_t c0 = a; c0 + 1 < b; c0 += (size_t)cap) {  // chunks of <= cap members
            const size_t c1 = std::min(b, c0 + (size_t)cap);
            if (c1 - c0 < 2) break;
            const SeqState *first = seqs[keyed[c0].second];
            size_t S = SIZE_MAX;
            for (size_t m = c0; m < c1; ++m) S = std::min(S, full[keyed[m].second]);
            for (size_t m = c0 + 1; m < c1 && S > 0; ++m) {
                const auto &h = seqs[keyed[m].second]->handles;
                size_t j = 0;
                while (j < S && h[j].block_id == first->handles[j].block_id) ++j;
                S = j;
            }
            if (S < kMinSharedPages) continue;
            const size_t base = out.sg_members.size();
            out.sg_members.resize(base + kSgStride, -1);
            for (size_t m = c0; m < c1; ++m) {
                out.sg_members[base + (m - c0)] = keyed[m].second;
                out.seq_pb[keyed[m].second] = (int32_t)S;
            }
            out.sg_pages.push_back((int32_t)S);
            out.total_pages += (long)S;
        }
        a = b;
    }
}

// What a batched write does before and after its copy kernel: validation,
// copy-on-write of every shared target block and the slot mapping (uploaded
// with, for fp8 pools, each token's batch row and the sequences' scales at
// this layer); afterwards the per-layer lengths and, at the last layer, the
// sequences' token counts.
struct WritePrep {
    std::vector<SeqState *> seqs;
    size_t T = 0;
    const int64_t *d_slots = nullptr;
    const int32_t *d_rows = nullptr;
    const float *d_ks = nullptr, *d_vs = nullptr;
};

int prepare_write(zk_kv_cache *c, size_t layer, const char *const *ids, const int32_t *num_tokens, int n,
                  bool have_src, WritePrep &w, bool upload_slots = true) {
    if (!c || (n > 0 && (!ids || !num_tokens)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write batch: NULL argument");
    if (layer >= c->num_layers)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write batch: layer out of range");
    if (n <= 0) return ZK_OK;
    DeviceGuard g(c->device);
    if (int rc = flush_tables(c)) return rc;
    const size_t bs = c->block_size, H = c->num_kv_heads;
    const bool fp8 = c->dtype == ZK_FP8_E4M3;
    std::vector<SeqState *> &seqs = w.seqs;
    seqs.assign((size_t)n, nullptr);
    size_t T = 0;
    for (int i = 0; i < n; ++i) {
        if (int rc = find_seq(c, ids[i], &seqs[i])) return rc;
        if (seqs[i]->swapped)
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + ids[i] +
                                                             " is swapped out");
        for (int j = 0; j < i; ++j)
            if (seqs[j] == seqs[i])
                return set_error(ZK_ERR_INVALID_ARGUMENT,
                                 std::string("Internal error: KVCache write batch: seq ") + ids[i] + " twice");
        if (num_tokens[i] < 0)
            return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write batch: negative token count");
        const SeqState &s = *seqs[i];
        if (num_tokens[i] > 0) {
            const size_t last = (s.cached_tokens + (size_t)num_tokens[i] - 1) / bs;
            if (last >= s.handles.size())  // kv_cache.rs:234-239
                return set_error(ZK_ERR_INTERNAL, "Internal error: KVCache append_kv: block_idx " +
                                                      std::to_string(last) + " OOB (have " +
                                                      std::to_string(s.handles.size()) + " blocks)");
        }
        if (fp8 && s.k_scales.empty())
            return set_error(ZK_ERR_FAILED_PRECONDITION,
                             std::string("Failed precondition: fp8 scales not set for seq ") + ids[i]);
        T += (size_t)num_tokens[i];
    }
    if (T == 0) return ZK_OK;
    if (!have_src) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write batch: NULL k/v");
    std::vector<std::pair<SeqState *, size_t>> shared;  // copy-on-write of every shared target
    for (int i = 0; i < n; ++i) {
        SeqState &s = *seqs[i];
        if (num_tokens[i] == 0) continue;
        for (size_t idx = s.cached_tokens / bs; idx <= (s.cached_tokens + (size_t)num_tokens[i] - 1) / bs; ++idx)
            if (zk_bm_refcount(s.bm, s.handles[idx].block_id) > 1) shared.emplace_back(&s, idx);
    }
    if (int rc = cow_blocks(c, shared)) return rc;
    w.T = T;
    if (!upload_slots) return ZK_OK;  // the caller's kernel finds the slots itself
    const size_t slots_bytes = T * sizeof(int64_t);
    const size_t rows_bytes = fp8 ? T * sizeof(int32_t) : 0;
    const size_t scale_bytes = fp8 ? 2 * (size_t)n * H * sizeof(float) : 0;
    std::vector<char> host(slots_bytes + rows_bytes + scale_bytes);
    int64_t *slots = (int64_t *)host.data();
    int32_t *rows = fp8 ? (int32_t *)(host.data() + slots_bytes) : nullptr;
    size_t t = 0;
    for (int i = 0; i < n; ++i) {
        const SeqState &s = *seqs[i];
        for (int j = 0; j < num_tokens[i]; ++j, ++t) {
            const size_t pos = s.cached_tokens + (size_t)j;
            slots[t] = (int64_t)s.handles[pos / bs].block_id * (int64_t)bs + (int64_t)(pos % bs);
            if (fp8) rows[t] = i;
        }
    }
    if (fp8) {
        float *sc = (float *)(host.data() + slots_bytes + rows_bytes);
        for (int i = 0; i < n; ++i) {
            std::memcpy(sc + (size_t)i * H, seqs[i]->k_scales.data() + layer * H, H * sizeof(float));
            std::memcpy(sc + (size_t)n * H + (size_t)i * H, seqs[i]->v_scales.data() + layer * H, H * sizeof(float));
        }
    }
    if (int rc = put(c, c->d_meta, host.data(), host.size(), "KVCache slot mapping")) return rc;
    char *d = (char *)c->d_meta.dev.p;
    w.T = T;
    w.d_slots = (const int64_t *)d;
    w.d_rows = fp8 ? (const int32_t *)(d + slots_bytes) : nullptr;
    w.d_ks = fp8 ? (const float *)(d + slots_bytes + rows_bytes) : nullptr;
    w.d_vs = fp8 ? w.d_ks + (size_t)n * H : nullptr;
    return ZK_OK;
}

void finish_write(zk_kv_cache *c, size_t layer, const int32_t *num_tokens, int n, WritePrep &w) {
    for (int i = 0; i < n; ++i) {
        SeqState &s = *w.seqs[i];
        s.layer_len[layer] = std::max(s.layer_len[layer], s.cached_tokens + (size_t)num_tokens[i]);
    }
    if (layer + 1 == c->num_layers)
        for (int i = 0; i < n; ++i) {
            w.seqs[i]->cached_tokens += (size_t)num_tokens[i];
            w.seqs[i]->block_offset = w.seqs[i]->cached_tokens % c->block_size;
        }
}

}  // namespace

extern "C" {

int zk_cache_create(size_t num_blocks, size_t block_size, size_t num_layers, size_t num_kv_heads,
                    size_t head_dim, zk_dtype dtype, size_t max_seqs, size_t max_blocks_per_seq,
                    void *stream, zk_kv_cache **out) {
    if (!out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_cache_create: out is NULL");
    *out = nullptr;
    if (block_size == 0) return zk::set_error_typed(ZK_ERR_INVALID_BLOCK_SIZE, zk::ErrorKind::InvalidBlockSize, 0);
    if (!zk::valid_dtype(dtype) || num_blocks == 0 || num_layers == 0 || num_kv_heads == 0 ||
        head_dim == 0 || max_seqs == 0 || max_blocks_per_seq == 0 || num_blocks > 0x7fffffffu)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_cache_create: bad shape");
    auto *c = new (std::nothrow) zk_kv_cache();
    if (!c) return set_error(ZK_ERR_INTERNAL, "Internal error: KVCache allocation failed");
    c->num_blocks = num_blocks;
    c->block_size = block_size;
    c->num_layers = num_layers;
    c->num_kv_heads = num_kv_heads;
    c->head_dim = head_dim;
    c->dtype = dtype;
    c->max_seqs = max_seqs;
    c->max_blocks_per_seq = max_blocks_per_seq;
    c->stream = (hipStream_t)stream;
    if (hipGetDevice(&c->device) != hipSuccess) c->device = 0;
    if (hipDeviceGetAttribute(&c->cus, hipDeviceAttributeMultiprocessorCount, c->device) != hipSuccess || c->cus <= 0)
        c->cus = 256;
    c->pool_bytes = ((num_blocks * c->block_bytes()) + 255) & ~(size_t)255;
    size_t slab_bytes = 2 * num_layers * c->pool_bytes;
    hipError_t e = hipMalloc((void **)&c->slab, slab_bytes);
    if (e == hipSuccess) e = hipMemsetAsync(c->slab, 0, slab_bytes, c->stream);  // alloc_zeros, kv_cache.rs:79-88
    if (e == hipSuccess) e = hipMalloc((void **)&c->tables, max_seqs * max_blocks_per_seq * sizeof(int32_t));
    if (e == hipSuccess)
        e = hipMemsetAsync(c->tables, 0xff, max_seqs * max_blocks_per_seq * sizeof(int32_t), c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        delete c;
        return set_error(ZK_ERR_HIP, std::string("Internal error: KVCache pool alloc: ") + hipGetErrorString(e));
    }
    c->free_slots.reserve(max_seqs);
    for (size_t i = 0; i < max_seqs; ++i) c->free_slots.push_back(max_seqs - 1 - i);
    *out = c;
    return ZK_OK;
}

void zk_cache_destroy(zk_kv_cache *c) { delete c; }

int zk_cache_register_seq(zk_kv_cache *c, const char *id, size_t max_blocks) {
    if (!c || !id) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache: NULL argument");
    if (c->seqs.count(id)) return set_error(ZK_ERR_ALREADY_EXISTS, std::string("Already exists: seq ") + id);
    if (max_blocks == 0 || max_blocks > c->max_blocks_per_seq)
        return zk::set_error_typed(ZK_ERR_SEQUENCE_TOO_LONG, zk::ErrorKind::SequenceTooLong, max_blocks,
                                   c->max_blocks_per_seq);
    if (c->free_slots.empty())
        return set_error(ZK_ERR_FAILED_PRECONDITION, "Failed precondition: KVCache: all sequence slots in use");
    DeviceGuard g(c->device);
    SeqState s;
    s.max_blocks = max_blocks;
    s.layer_len.assign(c->num_layers, 0);
    s.slot = c->free_slots.back();
    if (int rc = flush_tables(c)) return rc;  // queued writes land before the row is reset
    std::vector<int32_t> row(c->max_blocks_per_seq, -1);
    if (int rc = upload(c, c->table_row(s.slot), row.data(), row.size() * sizeof(int32_t))) return rc;
    c->free_slots.pop_back();
    c->seqs.emplace(id, std::move(s));
    return ZK_OK;
}

int zk_cache_alloc_block(zk_kv_cache *c, const char *id, zk_block_manager *bm, size_t *block_id) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (!bm) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache alloc_block: NULL manager");
    if (s->bm && s->bm != bm)
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         "Failed precondition: KVCache alloc_block: sequence uses another BlockManager");
    if (s->borrowed)
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         "Failed precondition: KVCache alloc_block: the sequence's blocks are bound by the caller");
    if (s->swapped)
        return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + id +
                                                         " is swapped out");
    if (zk_bm_num_gpu_blocks(bm) > c->num_blocks)
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         "Failed precondition: KVCache alloc_block: BlockManager larger than the pool");
    if (s->handles.size() >= s->max_blocks)
        return set_error(ZK_ERR_INTERNAL, "Internal error: block_table slice oob");  // kv_cache.rs:148
    DeviceGuard g(c->device);
    zk_block_handle h;
    if (int rc = zk_bm_allocate(bm, &h)) return rc;
    queue_table_entry(c, *s, s->handles.size(), (int32_t)h.block_id);  // applied by the next flush_tables
    s->bm = bm;
    s->handles.push_back(h);
    if (block_id) *block_id = (size_t)h.block_id;
    return ZK_OK;
}

int zk_cache_release_seq(zk_kv_cache *c, const char *id) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    DeviceGuard g(c->device);
    int first_rc = ZK_OK;
    zk::ErrorSnapshot first_err;
    for (const auto &h : s->handles) {
        if (s->borrowed) break;  // the caller frees its own handles
        int rc = zk_bm_free(s->bm, h);
        if (rc && !first_rc) {
            first_rc = rc;
            first_err = zk::save_error();
        }
    }
    release_host_slots(c, *s);
    int rc = flush_tables(c);  // queued writes for this row land before the reset
    std::vector<int32_t> row(c->max_blocks_per_seq, -1);
    if (!rc) rc = upload(c, c->table_row(s->slot), row.data(), row.size() * sizeof(int32_t));
    c->free_slots.push_back(s->slot);
    c->seqs.erase(id);
    ++c->epoch;
    if (first_rc) return zk::restore_error(first_err);
    return rc;
}

int zk_cache_fork_seq(zk_kv_cache *c, const char *parent, const char *child) {
    SeqState *p;
    if (int rc = find_seq(c, parent, &p)) return rc;
    if (!child) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache fork: NULL child");
    if (c->seqs.count(child)) return set_error(ZK_ERR_ALREADY_EXISTS, std::string("Already exists: seq ") + child);
    if (p->borrowed)
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         "Failed precondition: KVCache fork: the parent's blocks are owned by the caller");
    if (p->swapped)
        return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + parent +
                                                         " is swapped out");
    if (c->free_slots.empty())
        return set_error(ZK_ERR_FAILED_PRECONDITION, "Failed precondition: KVCache: all sequence slots in use");
    DeviceGuard g(c->device);
    size_t done = 0;
    for (; done < p->handles.size(); ++done)
        if (zk_bm_reference(p->bm, p->handles[done])) break;
    if (done < p->handles.size()) {
        const zk::ErrorSnapshot saved = zk::save_error();
        for (size_t i = 0; i < done; ++i) (void)zk_bm_free(p->bm, p->handles[i]);
        return zk::restore_error(saved);
    }
    if (flush_tables(c) != ZK_OK) {  // the parent's row is copied below
        const zk::ErrorSnapshot saved = zk::save_error();
        for (const auto &h : p->handles) (void)zk_bm_free(p->bm, h);
        return zk::restore_error(saved);
    }
    SeqState s = *p;
    s.slot = c->free_slots.back();
    const hipError_t e = hipMemcpyAsync(c->table_row(s.slot), c->table_row(p->slot),
                                        c->max_blocks_per_seq * sizeof(int32_t), hipMemcpyDeviceToDevice, c->stream);
    if (e != hipSuccess) {  // no child: give back the references taken for it
        for (const auto &h : p->handles) (void)zk_bm_free(p->bm, h);
        return set_error(ZK_ERR_HIP, std::string("Internal error: KVCache fork table copy: ") + hipGetErrorString(e));
    }
    c->free_slots.pop_back();
    c->seqs.emplace(child, std::move(s));
    ++c->epoch;
    return ZK_OK;
}

int zk_cache_store_kv(zk_kv_cache *c, size_t layer, const char *id, const void *k, const void *v,
                      zk_dtype src_dtype, size_t start_token, size_t n_tokens) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    DeviceGuard g(c->device);
    return write_tokens(c, layer, *s, id, k, v, src_dtype, start_token, n_tokens, "store_kv");
}

int zk_cache_append_kv(zk_kv_cache *c, size_t layer, const char *id, const void *k, const void *v,
                       zk_dtype src_dtype) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    DeviceGuard g(c->device);
    return write_tokens(c, layer, *s, id, k, v, src_dtype, s->cached_tokens, 1, "append_kv");
}

int zk_cache_write_batch(zk_kv_cache *c, size_t layer, const char *const *ids, const int32_t *num_tokens, int n,
                         const void *k, const void *v, zk_dtype src_dtype, int64_t src_token_stride) {
    if (src_dtype != ZK_F32 && src_dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write batch: bad src dtype");
    WritePrep w;
    if (int rc = prepare_write(c, layer, ids, num_tokens, n, k && v, w)) return rc;
    if (w.T == 0) return ZK_OK;
    if (int rc = zk::append(c->k_pool(layer), c->v_pool(layer), (zk_dtype)c->dtype, k, v, src_dtype,
                            src_token_stride, w.d_slots, (int64_t)w.T, (int)c->num_kv_heads, (int)c->head_dim,
                            (int)c->block_size, (int64_t)c->num_blocks, w.d_ks, w.d_vs, w.d_rows, c->stream))
        return rc;
    finish_write(c, layer, num_tokens, n, w);
    return ZK_OK;
}

int zk_cache_write_batch_qkv(zk_kv_cache *c, size_t layer, const char *const *ids, const int32_t *num_tokens, int n,
                             const void *x, const void *w_qkv, int64_t hidden, int num_heads, void *qkv) {
    if (!c) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write qkv: NULL cache");
    const int64_t qcols = (int64_t)num_heads * (int64_t)c->head_dim,
                  cols = qcols + 2 * (int64_t)c->num_kv_heads * (int64_t)c->head_dim;
    if (num_heads <= 0 || hidden <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write qkv: bad shape");
    if (x && qkv && n > 0 && num_tokens) {  // the projection reads x while it writes qkv
        int64_t rows = 0;
        for (int i = 0; i < n; ++i) rows += num_tokens[i] > 0 ? num_tokens[i] : 0;
        const uintptr_t xa = (uintptr_t)x, xb = xa + (uintptr_t)(rows * hidden * 2), qa = (uintptr_t)qkv,
                        qb = qa + (uintptr_t)(rows * cols * 2);
        if (rows > 0 && xa < qb && qa < xb)
            return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache write qkv: qkv overlaps x");
    }
    WritePrep w;
    if (int rc = prepare_write(c, layer, ids, num_tokens, n, x && w_qkv && qkv, w)) return rc;
    if (w.T == 0) return ZK_OK;
    const int64_t T = (int64_t)w.T;
    bool fused = false;
    if (c->dtype == ZK_BF16) {  // the projection's split-k sums, if its plan keeps them, go straight to the pools
        struct ToPools : zk::SplitSumsConsumer {
            zk_kv_cache *c;
            size_t layer;
            int64_t T, cols, qcols;
            void *qkv;
            const int64_t *slots;
            int operator()(const float *partial, int splits) const override {
                return zk::append_split_sums(c->k_pool(layer), c->v_pool(layer), partial, splits, T, cols, qkv, cols,
                                             qcols, slots, (int)c->num_kv_heads, (int)c->head_dim, (int)c->block_size,
                                             (int64_t)c->num_blocks, c->stream);
            }
        } to_pools;
        to_pools.c = c;
        to_pools.layer = layer;
        to_pools.T = T;
        to_pools.cols = cols;
        to_pools.qcols = qcols;
        to_pools.qkv = qkv;
        to_pools.slots = w.d_slots;
        if (int rc = zk::linear_split_sums(x, w_qkv, qkv, T, cols, hidden, c->stream, to_pools, &fused)) return rc;
    } else if (int rc = zk_linear(x, w_qkv, qkv, T, cols, hidden, ZK_BF16, ZK_BF16, c->stream)) {
        return rc;
    }
    if (!fused) {
        const char *y = (const char *)qkv;
        if (int rc = zk::append(c->k_pool(layer), c->v_pool(layer), (zk_dtype)c->dtype, y + 2 * qcols,
                                y + 2 * (qcols + (int64_t)c->num_kv_heads * c->head_dim), ZK_BF16, cols, w.d_slots, T,
                                (int)c->num_kv_heads, (int)c->head_dim, (int)c->block_size, (int64_t)c->num_blocks,
                                w.d_ks, w.d_vs, w.d_rows, c->stream))
            return rc;
    }
    finish_write(c, layer, num_tokens, n, w);
    return ZK_OK;
}

int zk_cache_append_kv_batch(zk_kv_cache *c, size_t layer, const char *const *ids, int n, const void *k,
                             const void *v, zk_dtype src_dtype) {
    std::vector<int32_t> ones(n > 0 ? (size_t)n : 0, 1);
    return zk_cache_write_batch(c, layer, ids, ones.data(), n, k, v, src_dtype, 0);
}

int zk_cache_bind_blocks(zk_kv_cache *c, zk_block_manager *bm, const char *const *ids, int n,
                         const zk_block_handle *blocks, const size_t *num_blocks, const size_t *tokens_before) {
    if (!c || !bm || (n > 0 && (!ids || !num_blocks)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache bind_blocks: NULL argument");
    if (n <= 0) return ZK_OK;
    if (zk_bm_block_size(bm) != c->block_size || zk_bm_num_gpu_blocks(bm) > c->num_blocks)
        return set_error(ZK_ERR_FAILED_PRECONDITION,
                         "Failed precondition: KVCache bind_blocks: BlockManager does not match the pool");
    // validate everything before changing anything
    size_t total = 0, fresh = 0;
    for (int i = 0; i < n; ++i) {
        if (!ids[i]) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache bind_blocks: NULL id");
        for (int j = 0; j < i; ++j)
            if (std::strcmp(ids[j], ids[i]) == 0)
                return set_error(ZK_ERR_INVALID_ARGUMENT,
                                 std::string("Internal error: KVCache bind_blocks: seq ") + ids[i] + " twice");
        if (num_blocks[i] > c->max_blocks_per_seq)
            return zk::set_error_typed(ZK_ERR_SEQUENCE_TOO_LONG, zk::ErrorKind::SequenceTooLong, num_blocks[i],
                                       c->max_blocks_per_seq);
        auto it = c->seqs.find(ids[i]);
        const size_t have = it == c->seqs.end() ? 0 : it->second.cached_tokens;
        if (it == c->seqs.end()) {
            ++fresh;
        } else if (!it->second.borrowed) {
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: KVCache bind_blocks: seq ") +
                                                             ids[i] + " owns its blocks (alloc_block / fork_seq)");
        } else if (it->second.bm != bm) {
            return set_error(ZK_ERR_FAILED_PRECONDITION,
                             "Failed precondition: KVCache bind_blocks: sequence uses another BlockManager");
        }
        if (tokens_before && tokens_before[i] != have)
            return set_error(ZK_ERR_FAILED_PRECONDITION,
                             std::string("Failed precondition: KVCache bind_blocks: seq ") + ids[i] + " holds " +
                                 std::to_string(have) + " tokens, the caller expects " +
                                 std::to_string(tokens_before[i]));
        if (have > num_blocks[i] * c->block_size)
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: KVCache bind_blocks: seq ") +
                                                             ids[i] + " would lose written tokens");
        if (num_blocks[i] && !blocks)
            return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache bind_blocks: NULL blocks");
        for (size_t j = 0; j < num_blocks[i]; ++j)
            if (int rc = zk_bm_check(bm, blocks[total + j])) return rc;  // stale handles rejected
        total += num_blocks[i];
    }
    if (fresh > c->free_slots.size())
        return set_error(ZK_ERR_FAILED_PRECONDITION, "Failed precondition: KVCache: all sequence slots in use");
    DeviceGuard g(c->device);
    size_t off = 0;
    for (int i = 0; i < n; ++i) {
        auto it = c->seqs.find(ids[i]);
        if (it == c->seqs.end()) {
            SeqState st;
            st.max_blocks = c->max_blocks_per_seq;
            st.layer_len.assign(c->num_layers, 0);
            st.slot = c->free_slots.back();
            st.borrowed = true;
            st.bm = bm;
            c->free_slots.pop_back();
            it = c->seqs.emplace(ids[i], std::move(st)).first;  // free slots' rows hold -1
        }
        SeqState &st = it->second;
        const zk_block_handle *h = blocks + off;
        for (size_t j = 0; j < num_blocks[i]; ++j)
            if (j >= st.handles.size() || st.handles[j].block_id != h[j].block_id)
                queue_table_entry(c, st, j, (int32_t)h[j].block_id);
        for (size_t j = num_blocks[i]; j < st.handles.size(); ++j) queue_table_entry(c, st, j, -1);
        st.handles.assign(h, h + num_blocks[i]);
        for (size_t &l : st.layer_len) l = std::min(l, num_blocks[i] * c->block_size);
        off += num_blocks[i];
    }
    return flush_tables(c);
}

int zk_cache_enable_swap(zk_kv_cache *c, size_t num_host_blocks) {
    if (!c) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap: NULL cache");
    if (c->host_pool) return set_error(ZK_ERR_ALREADY_EXISTS, "Already exists: KVCache swap space");
    if (num_host_blocks == 0 || num_host_blocks > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap: bad host block count");
    DeviceGuard g(c->device);
    ZK_HIP_CHECK(hipHostMalloc((void **)&c->host_pool, num_host_blocks * host_slot_bytes(c), hipHostMallocDefault),
                 "KVCache swap space");
    c->host_total = num_host_blocks;
    c->host_free.resize(num_host_blocks);
    for (size_t i = 0; i < num_host_blocks; ++i) c->host_free[i] = (int32_t)(num_host_blocks - 1 - i);
    return ZK_OK;
}

int zk_cache_seq_swapped(zk_kv_cache *c, const char *id, int *swapped) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (swapped) *swapped = s->swapped ? 1 : 0;
    return ZK_OK;
}

int zk_cache_swap_space(zk_kv_cache *c, size_t *total, size_t *free_blocks) {
    if (!c) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap: NULL cache");
    if (total) *total = c->host_total;
    if (free_blocks) *free_blocks = c->host_free.size();
    return ZK_OK;
}

int zk_cache_swap_out(zk_kv_cache *c, const char *const *ids, int n) {
    if (!c || (n > 0 && !ids)) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap_out: NULL argument");
    if (n <= 0) return ZK_OK;
    if (!c->host_pool)
        return set_error(ZK_ERR_FAILED_PRECONDITION, "Failed precondition: KVCache swap_out: no swap space");
    std::vector<SeqState *> seqs((size_t)n);
    std::vector<size_t> nblk((size_t)n);
    size_t need = 0;
    for (int i = 0; i < n; ++i) {
        if (int rc = find_seq(c, ids[i], &seqs[i])) return rc;
        for (int j = 0; j < i; ++j)
            if (seqs[j] == seqs[i])
                return set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: KVCache swap_out: seq ") + ids[i] + " twice");
        if (seqs[i]->swapped)
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + ids[i] +
                                                             " is swapped out");
        size_t written = 0;
        for (size_t l : seqs[i]->layer_len) written = std::max(written, l);
        nblk[i] = (written + c->block_size - 1) / c->block_size;
        need += nblk[i];
    }
    if (need > c->host_free.size())
        return zk::set_error_typed(ZK_ERR_OUT_OF_BLOCKS, zk::ErrorKind::OutOfBlocks, need, c->host_free.size());
    DeviceGuard g(c->device);
    std::vector<std::pair<int32_t, int32_t>> pairs;
    pairs.reserve(need);
    for (int i = 0; i < n; ++i) {
        SeqState &s = *seqs[i];
        s.host_slots.resize(nblk[i]);
        for (size_t b = 0; b < nblk[i]; ++b) {
            s.host_slots[b] = c->host_free.back();
            c->host_free.pop_back();
            pairs.emplace_back(s.host_slots[b], (int32_t)s.handles[b].block_id);
        }
    }
    int rc = swap_move(c, pairs, true);
    if (rc) {  // nothing was given up: put the slots back
        for (int i = 0; i < n; ++i) release_host_slots(c, *seqs[i]);
        return rc;
    }
    // the device blocks are free from here on; later writes into them are
    // queued after the staging copy on the same stream
    int first_rc = ZK_OK;
    zk::ErrorSnapshot first_err;
    for (int i = 0; i < n; ++i) {
        SeqState &s = *seqs[i];
        for (size_t j = 0; j < s.handles.size(); ++j) {
            queue_table_entry(c, s, j, -1);
            if (!s.borrowed) {
                int r = zk_bm_free(s.bm, s.handles[j]);
                if (r && !first_rc) {
                    first_rc = r;
                    first_err = zk::save_error();
                }
            }
        }
        s.handles.clear();
        s.swapped = true;
    }
    rc = flush_tables(c);
    if (first_rc) return zk::restore_error(first_err);
    return rc;
}

int zk_cache_swap_in(zk_kv_cache *c, const char *const *ids, int n, zk_block_manager *bm) {
    if (!c || (n > 0 && !ids)) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap_in: NULL argument");
    if (n <= 0) return ZK_OK;
    std::vector<SeqState *> seqs((size_t)n);
    for (int i = 0; i < n; ++i) {
        if (int rc = find_seq(c, ids[i], &seqs[i])) return rc;
        for (int j = 0; j < i; ++j)
            if (seqs[j] == seqs[i])
                return set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: KVCache swap_in: seq ") + ids[i] + " twice");
        SeqState &s = *seqs[i];
        if (!s.swapped)
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + ids[i] +
                                                             " is not swapped out");
        if (s.borrowed) {
            if (s.handles.size() < s.host_slots.size())
                return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + ids[i] +
                                                                 ": bind its new blocks before swap_in");
        } else {
            if (!bm && !s.bm)
                return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap_in: NULL manager");
            if (bm && s.bm && bm != s.bm)
                return set_error(ZK_ERR_FAILED_PRECONDITION,
                                 "Failed precondition: KVCache swap_in: sequence uses another BlockManager");
        }
    }
    DeviceGuard g(c->device);
    // fresh device blocks for the sequences the cache owns: all or nothing
    std::vector<std::vector<zk_block_handle>> fresh((size_t)n);
    for (int i = 0; i < n; ++i) {
        SeqState &s = *seqs[i];
        if (s.borrowed) continue;
        zk_block_manager *m = s.bm ? s.bm : bm;
        for (size_t b = 0; b < s.host_slots.size(); ++b) {
            zk_block_handle h;
            if (zk_bm_allocate(m, &h) != ZK_OK) {
                const zk::ErrorSnapshot saved = zk::save_error();
                for (int j = 0; j <= i; ++j)
                    for (const auto &x : fresh[j]) (void)zk_bm_free(seqs[j]->bm ? seqs[j]->bm : bm, x);
                return zk::restore_error(saved);
            }
            fresh[i].push_back(h);
        }
    }
    std::vector<std::pair<int32_t, int32_t>> pairs;
    for (int i = 0; i < n; ++i) {
        SeqState &s = *seqs[i];
        if (!s.borrowed) {
            s.bm = s.bm ? s.bm : bm;
            s.handles = fresh[i];
            for (size_t j = 0; j < s.handles.size(); ++j) queue_table_entry(c, s, j, (int32_t)s.handles[j].block_id);
        }
        for (size_t b = 0; b < s.host_slots.size(); ++b)
            pairs.emplace_back(s.host_slots[b], (int32_t)s.handles[b].block_id);
    }
    if (int rc = flush_tables(c)) return rc;
    if (int rc = swap_move(c, pairs, false)) return rc;
    for (int i = 0; i < n; ++i) release_host_slots(c, *seqs[i]);
    return ZK_OK;
}

int zk_cache_set_fp8_scales(zk_kv_cache *c, const char *id, const float *k_scales, const float *v_scales) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (c->dtype != ZK_FP8_E4M3)
        return set_error(ZK_ERR_FAILED_PRECONDITION, "Failed precondition: KVCache pools are not fp8");
    if (!k_scales || !v_scales)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache set_fp8_scales: NULL scales");
    size_t n = c->num_layers * c->num_kv_heads;
    for (size_t i = 0; i < n; ++i)
        if (!(k_scales[i] > 0.0f) || !(v_scales[i] > 0.0f))
            return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache set_fp8_scales: scales must be > 0");
    s->k_scales.assign(k_scales, k_scales + n);
    s->v_scales.assign(v_scales, v_scales + n);
    return ZK_OK;
}

int zk_cache_block_table_ptr(zk_kv_cache *c, const char *id, const int32_t **out) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (!out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache: NULL out");
    DeviceGuard g(c->device);
    if (int rc = flush_tables(c)) return rc;
    *out = c->table_row(s->slot);
    return ZK_OK;
}

void *zk_cache_k_pool_ptr(zk_kv_cache *c, size_t layer) {
    return (c && layer < c->num_layers) ? c->k_pool(layer) : nullptr;
}
void *zk_cache_v_pool_ptr(zk_kv_cache *c, size_t layer) {
    return (c && layer < c->num_layers) ? c->v_pool(layer) : nullptr;
}

int zk_cache_max_blocks(zk_kv_cache *c, const char *id, size_t *out) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (out) *out = s->max_blocks;
    return ZK_OK;
}

int zk_cache_seq_state(zk_kv_cache *c, const char *id, size_t *cached_tokens, size_t *block_offset,
                       size_t *num_blocks) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (cached_tokens) *cached_tokens = s->cached_tokens;
    if (block_offset) *block_offset = s->block_offset;
    if (num_blocks) *num_blocks = s->handles.size();
    return ZK_OK;
}

int zk_cache_block_ids(zk_kv_cache *c, const char *id, int64_t *ids, size_t *n) {
    SeqState *s;
    if (int rc = find_seq(c, id, &s)) return rc;
    if (!n) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache block_ids: NULL n");
    size_t cnt = std::min(*n, s->handles.size());
    for (size_t i = 0; ids && i < cnt; ++i) ids[i] = (int64_t)s->handles[i].block_id;
    *n = s->handles.size();
    return ZK_OK;
}

}  // extern "C"

namespace {

// Decode at `layer` of entries seqs[i] (a sequence may appear more than once)
// with context lens[i] (default: the tokens written at the layer) and q / out
// row q_rows[i] (default: i); forked prefixes are shared when `share` holds
// and the lengths are the layer's.
int decode_batch(zk_kv_cache *c, size_t layer, const std::vector<const SeqState *> &seqs,
                 const std::vector<int32_t> *lens_in, const std::vector<int32_t> *q_rows, const void *q,
                 zk_dtype q_dtype, int64_t q_stride, void *out, int num_heads, float scale, zk_gqa_mapping mapping,
                 bool share, const zk::AppendRows *append = nullptr, int max_waves = 0) {
    const int n = (int)seqs.size();
    if (n <= 0) return ZK_OK;
    const size_t H = c->num_kv_heads;
    const bool fp8 = c->dtype == ZK_FP8_E4M3;
    size_t stride = 1;
    for (const SeqState *s : seqs) stride = std::max(stride, s->handles.size());
    // Block tables [n][stride]: re-uploaded only when some table changed or
    // the batch differs from the previous call's.
    if (c->dec_epoch != c->epoch || c->dec_ids != seqs || c->dec_stride != stride) {
        std::vector<int32_t> tbl((size_t)n * stride, -1);
        for (int i = 0; i < n; ++i)
            for (size_t j = 0; j < seqs[i]->handles.size(); ++j)
                tbl[(size_t)i * stride + j] = (int32_t)seqs[i]->handles[j].block_id;
        c->dec_epoch = ~0ull;
        const bool same = c->d_tbl.last.size() == tbl.size() * sizeof(int32_t) &&
                          std::memcmp(c->d_tbl.last.data(), tbl.data(), c->d_tbl.last.size()) == 0;
        if (!same) ++c->tbl_version;
        if (int rc = put(c, c->d_tbl, tbl.data(), tbl.size() * sizeof(int32_t), "KVCache decode tables")) return rc;
        c->dec_epoch = c->epoch;
        c->dec_ids = seqs;
        c->dec_stride = stride;
    }
    // Shared prefixes of forked sequences (bf16 MFMA shapes only).  The
    // grouping depends on the tables (epoch), the batch and the pages each
    // sequence has fully written at the layer; the layers of one step
    // usually agree on all three, so the last grouping is kept and reused.
    static const SharePlan no_sharing;
    const SharePlan *spp = &no_sharing;
    if (share && !lens_in && num_heads > 0 && num_heads % (int)H == 0 &&
        zk::paged_decode_shares_prefixes(c->dtype, (int)c->head_dim, (int)c->block_size, num_heads, (int)H)) {
        const int cap = 32 / (num_heads / (int)H);
        std::vector<size_t> full(n);
        for (int i = 0; i < n; ++i)
            full[i] = std::min(seqs[i]->handles.size(), seqs[i]->layer_len[layer] / c->block_size);
        if (c->sh_epoch != c->epoch || c->sh_cap != cap || c->sh_ids != seqs || c->sh_full != full) {
            c->sh_epoch = ~0ull;
            plan_sharing(seqs, full, cap, c->sh_plan);
            c->sh_epoch = c->epoch;
            c->sh_cap = cap;
            c->sh_ids = seqs;
            c->sh_full = std::move(full);
        }
        spp = &c->sh_plan;
    }
    const SharePlan &sp = *spp;
    const int nsg = (int)sp.sg_pages.size();
    if (append && nsg)  // the appended token's page is written by its sequence's own item, never a shared one
        for (int i = 0; i < n; ++i)
            if ((size_t)sp.seq_pb[i] * c->block_size >= seqs[i]->layer_len[layer])
                return set_error(ZK_ERR_INTERNAL, "Internal error: KVCache decode_append: token in a shared page");
    // Lengths at this layer, (fp8) this layer's scales [2][n][H], (shared
    // prefixes) seq_pb [n], sg_members [nsg][32], sg_pages [nsg].
    auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t len_bytes = a256((size_t)n * sizeof(int32_t));
    const size_t sc_bytes = a256(fp8 ? 2 * (size_t)n * H * sizeof(float) : 0);
    const size_t share_ints = nsg ? (size_t)n + sp.sg_members.size() + sp.sg_pages.size() : 0;
    const size_t share_bytes = a256(share_ints * sizeof(int32_t));
    const size_t rows_bytes = q_rows ? (size_t)n * sizeof(int32_t) : 0;
    const size_t total = len_bytes + sc_bytes + share_bytes + rows_bytes;
    std::vector<char> host(total, 0);
    int32_t *lens = (int32_t *)host.data();
    float *sc = (float *)(host.data() + len_bytes);
    for (int i = 0; i < n; ++i) {
        lens[i] = lens_in ? (*lens_in)[i] : (int32_t)seqs[i]->layer_len[layer];
        if (fp8) {
            std::memcpy(sc + (size_t)i * H, seqs[i]->k_scales.data() + layer * H, H * sizeof(float));
            std::memcpy(sc + (size_t)n * H + (size_t)i * H, seqs[i]->v_scales.data() + layer * H, H * sizeof(float));
        }
    }
    int32_t *sh = (int32_t *)(host.data() + len_bytes + sc_bytes);
    size_t o_pb = 0, o_mem = 0, o_pages = 0;
    if (nsg) {
        o_pb = 0;
        o_mem = o_pb + (size_t)n;
        o_pages = o_mem + sp.sg_members.size();
        std::memcpy(sh + o_pb, sp.seq_pb.data(), (size_t)n * sizeof(int32_t));
        std::memcpy(sh + o_mem, sp.sg_members.data(), sp.sg_members.size() * sizeof(int32_t));
        std::memcpy(sh + o_pages, sp.sg_pages.data(), sp.sg_pages.size() * sizeof(int32_t));
    }
    if (q_rows) std::memcpy(host.data() + len_bytes + sc_bytes + share_bytes, q_rows->data(), rows_bytes);
    if (int rc = put(c, c->d_batch, host.data(), total, "KVCache decode batch")) return rc;
    size_t ws = zk::paged_decode_workspace(n, num_heads, (int)c->head_dim, (int)stride, (int)c->block_size, nsg > 0);
    if (int rc = c->d_ws.ensure(ws, "KVCache decode workspace")) return rc;
    char *d = (char *)c->d_batch.dev.p;
    const float *dks = fp8 ? (const float *)(d + len_bytes) : nullptr;
    const float *dvs = fp8 ? dks + (size_t)n * H : nullptr;
    const int32_t *dsh = (const int32_t *)(d + len_bytes + sc_bytes);
    zk::PrefixGroups pg{dsh + o_pb, dsh + o_mem, dsh + o_pages, nsg, sp.total_pages};
    c->last_sg = nsg;
    c->last_sg_pages = sp.total_pages;
    const int32_t *drows = q_rows ? (const int32_t *)(d + len_bytes + sc_bytes + share_bytes) : nullptr;
    // The plan (work items over sequence indices and page ranges, each
    // carrying the block ids of its first pages, in the workspace) depends on
    // the shapes, the lengths, the prefix groups and the tables, not on the
    // layer's pools, q or scales: the layers of one step share it.
    const uintptr_t hdr[] = {(uintptr_t)n,          (uintptr_t)num_heads,     stride,
                             (uintptr_t)nsg,        (uintptr_t)sp.total_pages, (uintptr_t)c->d_ws.p,
                             (uintptr_t)c->d_ws.cap, (uintptr_t)c->tbl_version, (uintptr_t)max_waves};
    std::vector<char> sig((const char *)hdr, (const char *)hdr + sizeof(hdr));
    sig.insert(sig.end(), host.data(), host.data() + len_bytes);
    sig.insert(sig.end(), host.data() + len_bytes + sc_bytes, host.data() + len_bytes + sc_bytes + share_bytes);
    const bool reuse = sig == c->plan_sig;
    c->plan_sig.clear();
    int rc = zk::paged_decode(q, q_dtype, c->k_pool(layer), c->v_pool(layer), (zk_dtype)c->dtype, out,
                              (const int32_t *)c->d_tbl.dev.p, (const int32_t *)d, n, num_heads, (int)H,
                              (int)c->head_dim, (int)c->block_size, (int)stride, (int64_t)c->num_blocks, scale,
                              mapping, dks, dvs, c->d_ws.p, c->d_ws.cap, c->stream, nsg ? &pg : nullptr, drows,
                              q_stride, /*trusted_tables=*/true,  // built from the sequences' handles
                              reuse, append, &c->dec_head_set, max_waves);
    if (rc == ZK_OK) c->plan_sig = std::move(sig);
    return rc;
}

// Looks up ids[0..n) (each must be registered; fp8 caches need scales).
int find_seqs(zk_kv_cache *c, const char *const *ids, int n, std::vector<const SeqState *> &out) {
    out.resize(n > 0 ? (size_t)n : 0);
    for (int i = 0; i < n; ++i) {
        SeqState *s;
        if (int rc = find_seq(c, ids[i], &s)) return rc;
        if (c->dtype == ZK_FP8_E4M3 && s->k_scales.empty())
            return set_error(ZK_ERR_FAILED_PRECONDITION,
                             std::string("Failed precondition: fp8 scales not set for seq ") + ids[i]);
        if (s->swapped)
            return set_error(ZK_ERR_FAILED_PRECONDITION, std::string("Failed precondition: seq ") + ids[i] +
                                                             " is swapped out");
        out[i] = s;
    }
    return ZK_OK;
}

// Causal chunked-prefill attention of chunk rows through zk_paged_prefill:
// entry i is seqs[i]'s last len[i] tokens at the layer, at q / out rows
// off[i] .. off[i] + len[i].
int prefill_batch(zk_kv_cache *c, size_t layer, const std::vector<const SeqState *> &seqs,
                  const std::vector<int32_t> &len, const std::vector<int64_t> &off, int64_t total_rows, const void *q,
                  zk_dtype q_dtype, int64_t q_stride, void *out, int num_heads, float scale, zk_gqa_mapping mapping,
                  hipStream_t launch, int max_groups = 0) {
    const int n = (int)seqs.size();
    if (n <= 0) return ZK_OK;
    const size_t H = c->num_kv_heads;
    const bool fp8 = c->dtype == ZK_FP8_E4M3;
    size_t stride = 1;
    for (const SeqState *s : seqs) stride = std::max(stride, s->handles.size());
    auto a256 = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t tbl_bytes = a256((size_t)n * stride * sizeof(int32_t));
    const size_t off_bytes = a256((size_t)n * sizeof(int64_t));
    const size_t i32_bytes = a256((size_t)n * sizeof(int32_t));
    const size_t sc_bytes = fp8 ? 2 * (size_t)n * H * sizeof(float) : 0;
    std::vector<char> host(tbl_bytes + off_bytes + 2 * i32_bytes + sc_bytes, 0);
    int32_t *tbl = (int32_t *)host.data();
    int64_t *qo = (int64_t *)(host.data() + tbl_bytes);
    int32_t *ql = (int32_t *)(host.data() + tbl_bytes + off_bytes);
    int32_t *st = (int32_t *)(host.data() + tbl_bytes + off_bytes + i32_bytes);
    float *sc = (float *)(host.data() + tbl_bytes + off_bytes + 2 * i32_bytes);
    for (int i = 0; i < n; ++i) {
        for (size_t j = 0; j < stride; ++j)
            tbl[(size_t)i * stride + j] = j < seqs[i]->handles.size() ? (int32_t)seqs[i]->handles[j].block_id : -1;
        qo[i] = off[i];
        ql[i] = len[i];
        st[i] = (int32_t)seqs[i]->layer_len[layer] - len[i];
        if (fp8) {
            std::memcpy(sc + (size_t)i * H, seqs[i]->k_scales.data() + layer * H, H * sizeof(float));
            std::memcpy(sc + (size_t)n * H + (size_t)i * H, seqs[i]->v_scales.data() + layer * H, H * sizeof(float));
        }
    }
    if (int rc = put(c, c->d_pre, host.data(), host.size(), "KVCache prefill batch")) return rc;
    const size_t ws = zk_paged_prefill_workspace_size(n, total_rows, num_heads, (int)H);
    if (int rc = c->d_pws.ensure(ws, "KVCache prefill workspace")) return rc;
    char *d = (char *)c->d_pre.dev.p;
    const float *dks = fp8 ? (const float *)(d + tbl_bytes + off_bytes + 2 * i32_bytes) : nullptr;
    const float *dvs = fp8 ? dks + (size_t)n * H : nullptr;
    if (launch != c->stream) {  // the launch stream waits for everything queued so far
        ZK_HIP_CHECK(hipEventRecord(c->fork_ev, c->stream), "KVCache prefill fork");
        ZK_HIP_CHECK(hipStreamWaitEvent(launch, c->fork_ev, 0), "KVCache prefill fork");
    }
    return zk::paged_prefill_rows(q, q_dtype, c->k_pool(layer), c->v_pool(layer), (zk_dtype)c->dtype, out,
                                  (const int32_t *)d, (const int64_t *)(d + tbl_bytes),
                                  (const int32_t *)(d + tbl_bytes + off_bytes),
                                  (const int32_t *)(d + tbl_bytes + off_bytes + i32_bytes), n, total_rows, num_heads,
                                  (int)H, (int)c->head_dim, (int)c->block_size, (int)stride,
                                  (int64_t)c->num_blocks, scale, 1, mapping, dks, dvs, c->d_pws.p, c->d_pws.cap,
                                  launch, q_stride, max_groups);
}

int ensure_side_stream(zk_kv_cache *c) {
    if (c->side) return ZK_OK;
    ZK_HIP_CHECK(hipEventCreateWithFlags(&c->fork_ev, hipEventDisableTiming), "KVCache side stream");
    ZK_HIP_CHECK(hipEventCreateWithFlags(&c->join_ev, hipEventDisableTiming), "KVCache side stream");
    ZK_HIP_CHECK(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking), "KVCache side stream");
    return ZK_OK;
}

}  // namespace

extern "C" {

int zk_cache_paged_decode(zk_kv_cache *c, size_t layer, const char *const *ids, int n, const void *q,
                          zk_dtype q_dtype, void *out, int num_heads, float scale, zk_gqa_mapping mapping) {
    if (!c || (n > 0 && !ids)) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache decode: NULL argument");
    if (layer >= c->num_layers)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache decode: layer out of range");
    if (n <= 0) return ZK_OK;
    DeviceGuard g(c->device);
    std::vector<const SeqState *> seqs;
    if (int rc = find_seqs(c, ids, n, seqs)) return rc;
    return decode_batch(c, layer, seqs, nullptr, nullptr, q, q_dtype, 0, out, num_heads, scale, mapping, true);
}

int zk_cache_decode_append(zk_kv_cache *c, size_t layer, const char *const *ids, int n, const void *k, const void *v,
                           zk_dtype src_dtype, const void *q, zk_dtype q_dtype, void *out, int num_heads, float scale,
                           zk_gqa_mapping mapping) {
    if (!c || (n > 0 && !ids))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache decode_append: NULL argument");
    if (layer >= c->num_layers)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache decode_append: layer out of range");
    if (n <= 0) return ZK_OK;
    if (!q || !out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache decode_append: NULL q / out");
    DeviceGuard g(c->device);
    const std::vector<int32_t> ones((size_t)n, 1);
    const bool fuse = c->dtype == ZK_BF16 && src_dtype == ZK_BF16 && k && v &&
                      (((uintptr_t)k | (uintptr_t)v) & 15u) == 0 && (c->head_dim * 2) % 16 == 0 &&
                      zk::paged_decode_fuses_append(c->dtype, (int)c->head_dim, (int)c->block_size, num_heads,
                                                    (int)c->num_kv_heads);
    if (!fuse) {  // the two calls
        if (int rc = zk_cache_write_batch(c, layer, ids, ones.data(), n, k, v, src_dtype, 0)) return rc;
        return zk_cache_paged_decode(c, layer, ids, n, q, q_dtype, out, num_heads, scale, mapping);
    }
    WritePrep w;  // validation and copy-on-write; the decode kernel stores the rows
    if (int rc = prepare_write(c, layer, ids, ones.data(), n, true, w, /*upload_slots=*/false)) return rc;
    finish_write(c, layer, ones.data(), n, w);
    const std::vector<const SeqState *> seqs(w.seqs.begin(), w.seqs.end());
    const zk::AppendRows rows{k, v, (int64_t)(c->num_kv_heads * c->head_dim * 2)};
    return decode_batch(c, layer, seqs, nullptr, nullptr, q, q_dtype, 0, out, num_heads, scale, mapping, true, &rows);
}

int zk_cache_attention_batch(zk_kv_cache *c, size_t layer, const char *const *ids, const int32_t *num_tokens, int n,
                             const void *q, zk_dtype q_dtype, int64_t q_token_stride, void *out, int num_heads,
                             float scale, zk_gqa_mapping mapping) {
    if (!c || (n > 0 && (!ids || !num_tokens)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache attention batch: NULL argument");
    if (layer >= c->num_layers)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache attention batch: layer out of range");
    if (n <= 0) return ZK_OK;
    DeviceGuard g(c->device);
    std::vector<const SeqState *> seqs;
    if (int rc = find_seqs(c, ids, n, seqs)) return rc;
    // rows of entry i: off .. off + num_tokens[i], packed in batch order
    std::vector<const SeqState *> dec, pre;
    std::vector<int32_t> dec_rows, pre_len;
    std::vector<int64_t> pre_off;
    int64_t row = 0;
    for (int i = 0; i < n; ++i) {
        const int nt = num_tokens[i];
        if (nt < 0 || (size_t)nt > seqs[i]->layer_len[layer])
            return set_error(ZK_ERR_INVALID_ARGUMENT,
                             std::string("Internal error: KVCache attention batch: seq ") + ids[i] +
                                 " has fewer tokens at this layer than its rows (write the layer first)");
        if (nt == 1) {
            dec.push_back(seqs[i]);
            dec_rows.push_back((int32_t)row);
        } else if (nt > 1) {
            pre.push_back(seqs[i]);
            pre_len.push_back(nt);
            pre_off.push_back(row);
        }
        row += nt;
    }
    if (row > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache attention batch: too many rows");
    if (!q || !out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache attention batch: NULL q/out");
    const bool identity = dec.size() == (size_t)n;  // all decode rows, in batch order
    size_t pre_pages = 0;
    for (const SeqState *s : pre) pre_pages = std::max(pre_pages, s->handles.size());
    const bool mfma_prefill = !pre.empty() &&
                              zk::paged_prefill_supported(c->dtype, (int)c->head_dim, (int)c->block_size, num_heads,
                                                          (int)c->num_kv_heads) &&
                              pre_pages <= (size_t)zk::kPrefillMaxPages;
    if (mfma_prefill) {
        // chunks first, on the side stream when decodes share the step, so
        // the two kernels overlap; the cache stream waits for both at the end.
        // Each gets part of every CU: one four-wave prefill workgroup (a wave
        // on each SIMD) and two decode waves (the HBM-bound decode streams as
        // fast on two waves a CU as on four; four, one beside each prefill
        // wave, measured 0.78 against 0.73 ms a mixed step)
        hipStream_t ps = c->stream;
        int pre_groups = 0, dec_waves = 0;
        if (!dec.empty()) {
            if (int rc = ensure_side_stream(c)) return rc;
            ps = c->side;
            pre_groups = c->cus;
            dec_waves = 2 * c->cus;
        }
        int rc = prefill_batch(c, layer, pre, pre_len, pre_off, row, q, q_dtype, q_token_stride, out, num_heads,
                               scale, mapping, ps, pre_groups);
        if (!rc)
            rc = decode_batch(c, layer, dec, nullptr, identity ? nullptr : &dec_rows, q, q_dtype, q_token_stride, out,
                              num_heads, scale, mapping, true, nullptr, dec_waves);
        if (ps != c->stream) {
            hipError_t e = hipEventRecord(c->join_ev, ps);
            if (e == hipSuccess) e = hipStreamWaitEvent(c->stream, c->join_ev, 0);
            if (e != hipSuccess && !rc)
                rc = set_error(ZK_ERR_HIP, std::string("Internal error: KVCache prefill join: ") + hipGetErrorString(e));
        }
        return rc;
    }
    if (int rc = decode_batch(c, layer, dec, nullptr, identity ? nullptr : &dec_rows, q, q_dtype, q_token_stride, out,
                              num_heads, scale, mapping, true))
        return rc;
    if (pre.empty()) return ZK_OK;
    // shapes without the MFMA prefill: every chunk row is a decode of its
    // causal context (start + t + 1 tokens)
    std::vector<const SeqState *> ex;
    std::vector<int32_t> ex_len, ex_rows;
    for (size_t i = 0; i < pre.size(); ++i) {
        const int32_t start = (int32_t)pre[i]->layer_len[layer] - pre_len[i];
        for (int t = 0; t < pre_len[i]; ++t) {
            ex.push_back(pre[i]);
            ex_len.push_back(start + t + 1);
            ex_rows.push_back((int32_t)(pre_off[i] + t));
        }
    }
    return decode_batch(c, layer, ex, &ex_len, &ex_rows, q, q_dtype, q_token_stride, out, num_heads, scale, mapping,
                        false);
}

int zk_cache_decode_sharing(zk_kv_cache *c, int *subgroups, int64_t *shared_pages) {
    if (!c) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache: NULL argument");
    if (subgroups) *subgroups = c->last_sg;
    if (shared_pages) *shared_pages = c->last_sg_pages;
    return ZK_OK;
}

}  // extern "C"

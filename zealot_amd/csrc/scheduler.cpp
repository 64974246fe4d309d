// scheduler.cpp -- continuous-batching scheduler over a shared BlockManager
// (host side, no GPU calls).
//
// Semantics of src/scheduler.rs:156-478:
//  - admission control: a sequence whose worst case (prompt + max_tokens)
//    needs more blocks than the pool holds is SequenceTooLong
//    (scheduler.rs:225-253); arrivals are numbered in submission order.
//  - waiting queue ordered by (priority desc, arrival asc), stable insert
//    (scheduler.rs:259-265).
//  - schedule (scheduler.rs:267-344): (1) chunks for prefilling sequences
//    whose previous chunk finished, within max_prefill_tokens; (2) promote
//    waiting -> prefilling while max_num_seqs, the token budget (first
//    promotion always fits) and free blocks allow, allocating the blocks the
//    first chunk needs; (3) top up blocks of every prefilling, then decoding
//    sequence, preempting on OutOfBlocks the lowest-priority, latest-arrived
//    other sequence of the same queue (its blocks freed, back to waiting for
//    a full recompute; scheduler.rs:347-393); (4) batch = prefilling with a
//    chunk, then decoding.
//  - Sequence::len (scheduler.rs:115-121), is_final_chunk (:150-152),
//    finish / promote_to_decoding / advance_prefill / cancel / is_idle
//    (scheduler.rs:396-474).
//
// Differences, each deliberate:
//  - the BlockManager may be shared with the KV cache (the reference builds a
//    private one, scheduler.rs:215, which no KV code can see): block tables
//    are then derived from each sequence's handles;
//  - step_input of a prefill chunk holds the preserved output tokens (after a
//    preemption) on the final chunk only, after the whole prompt; the
//    reference appends them to every chunk (scheduler.rs:128-140), which for a
//    multi-chunk recompute puts them in the middle of the prompt.  A
//    single-chunk recompute is the same in both;
//  - a request id already queued or running is rejected (AlreadyExists): ids
//    key the KV cache's sequences;
//  - with swap space configured (swap_blocks > 0), a victim whose KV fits
//    the remaining host space is swapped instead of recomputed (the policy of
//    docs/architecture.md:452-469: swap first, recompute when the swap pool
//    is full): it keeps its prefill position and outputs, and is listed in
//    swapped_out; when re-admitted it is listed in swapped_in and resumes as
//    it stood (a decoding sequence goes straight back to decoding);
//  - a sequence whose blocks do not cover len() after the top-up (no victim
//    was left, scheduler.rs:386) stays out of the batch until a later step
//    finds its blocks, as the reference's comment there intends; the
//    reference batches it anyway, and its step would write past its blocks.
#include <algorithm>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "zk_common.h"
#include "../../include/zealot_sched.h"

namespace {

struct Seq {
    std::string id;
    std::vector<int64_t> prompt, output;
    size_t max_tokens = 0;
    int priority = ZK_PRIORITY_MEDIUM;
    uint64_t arrival = 0;
    bool running = false;
    std::vector<zk_block_handle> blocks;
    bool prefill_pending = true;
    size_t prefill_pos = 0, chunk_size = 0;
    bool swapped = false;  // preempted with its KV moved to host slots
    size_t swap_blocks = 0;

    size_t len() const {  // scheduler.rs:115-121
        return prefill_pending ? prefill_pos + output.size() + chunk_size : prompt.size() + output.size();
    }
    bool final_chunk() const { return prefill_pos + chunk_size >= prompt.size(); }  // scheduler.rs:150-152
    size_t remaining() const { return prompt.size() > prefill_pos ? prompt.size() - prefill_pos : 0; }
    // Tokens fed to the runner this step and KV positions before them.
    size_t step_tokens() const {
        if (!prefill_pending) return 1;
        const size_t chunk = std::min(chunk_size, remaining());
        return chunk + (final_chunk() ? output.size() : 0);
    }
    size_t tokens_before() const { return prefill_pending ? prefill_pos : len() - 1; }
    // KV tokens a preempted sequence holds (nothing of the chunk in flight).
    size_t kv_tokens() const { return prefill_pending ? prefill_pos : prompt.size() + output.size() - 1; }
    // Order of the waiting queue: priority desc, arrival asc.
    bool before_or_tie(const Seq &o) const {
        return std::make_tuple(-priority, arrival) <= std::make_tuple(-o.priority, o.arrival);
    }
};

size_t blocks_for(size_t tokens, size_t bs) { return (tokens + bs - 1) / bs; }

}  // namespace

struct zk_sequence {
    Seq s;
};

struct zk_scheduler {
    zk_sched_config cfg{};
    zk_block_manager *bm = nullptr;
    bool owns_bm = false;
    std::vector<Seq> waiting, prefilling, decoding;
    uint64_t next_arrival = 0;
    // snapshot of the last schedule() output
    std::vector<zk_sched_entry> out;
    std::vector<std::string> out_ids, pre_ids, swap_out_ids, swap_in_ids;
    std::vector<const char *> pre_ptrs, swap_out_ptrs, swap_in_ptrs;
    size_t swap_used = 0;  // host blocks held by swapped sequences
    std::vector<zk_block_handle> out_blocks;

    ~zk_scheduler() {
        if (owns_bm) zk_bm_destroy(bm);
    }

    void insert_waiting(Seq &&s) {
        auto pos = std::partition_point(waiting.begin(), waiting.end(),
                                        [&](const Seq &w) { return w.before_or_tie(s); });
        waiting.insert(pos, std::move(s));
    }

    void free_blocks(Seq &s) {
        for (const zk_block_handle &h : s.blocks) (void)zk_bm_free(bm, h);  // owned handles (scheduler.rs:369)
        s.blocks.clear();
    }

    // scheduler.rs:347-393: grow queue[idx]'s blocks to cover len(); returns
    // the requester's index after preemptions.
    size_t ensure_blocks(std::vector<Seq> &queue, size_t idx, std::vector<std::string> &preempted,
                         std::vector<std::string> &swapped_out) {
        const size_t need = blocks_for(queue[idx].len(), cfg.block_size);
        while (queue[idx].blocks.size() < need) {
            zk_block_handle h;
            if (zk_bm_allocate(bm, &h) == ZK_OK) {
                queue[idx].blocks.push_back(h);
                continue;
            }
            // victim: lowest priority, then latest arrival, other than the requester
            size_t vi = queue.size();
            for (size_t i = 0; i < queue.size(); ++i) {
                if (i == idx) continue;
                if (vi == queue.size() || queue[i].priority < queue[vi].priority ||
                    (queue[i].priority == queue[vi].priority && queue[i].arrival > queue[vi].arrival))
                    vi = i;
            }
            if (vi == queue.size()) break;  // only the requester is left: wait for the next step
            Seq victim = std::move(queue[vi]);
            queue.erase(queue.begin() + (ptrdiff_t)vi);
            free_blocks(victim);
            victim.chunk_size = 0;
            victim.running = false;
            const size_t kv = victim.kv_tokens(), kvb = blocks_for(kv, cfg.block_size);
            if (kv > 0 && swap_used + kvb <= cfg.swap_blocks) {
                // swap: the runner moves its KV to host slots before the
                // blocks are reused; it resumes where it stopped
                victim.swapped = true;
                victim.swap_blocks = kvb;
                swap_used += kvb;
                swapped_out.push_back(victim.id);
            } else {  // recompute (scheduler.rs:372-376)
                victim.prefill_pending = true;
                victim.prefill_pos = 0;
                preempted.push_back(victim.id);
            }
            insert_waiting(std::move(victim));
            if (vi < idx) --idx;
        }
        return idx;
    }

    Seq *find_running(const char *id, std::vector<Seq> **queue = nullptr, size_t *idx = nullptr) {
        for (auto *q : {&prefilling, &decoding})
            for (size_t i = 0; i < q->size(); ++i)
                if ((*q)[i].id == id) {
                    if (queue) *queue = q;
                    if (idx) *idx = i;
                    return &(*q)[i];
                }
        return nullptr;
    }

    bool known(const char *id) {
        if (find_running(id)) return true;
        for (const Seq &s : waiting)
            if (s.id == id) return true;
        return false;
    }
};

extern "C" {

int zk_sched_create(const zk_sched_config *cfg, zk_block_manager *bm, zk_scheduler **out) {
    if (!cfg || !out) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_create: NULL argument");
    *out = nullptr;
    zk_block_manager *use = bm;
    if (!use) {
        if (int rc = zk_bm_create(cfg->num_gpu_blocks, cfg->block_size, &use)) return rc;  // scheduler.rs:215
    } else if (zk_bm_block_size(bm) != cfg->block_size || zk_bm_num_gpu_blocks(bm) != cfg->num_gpu_blocks) {
        return zk::set_error(ZK_ERR_FAILED_PRECONDITION,
                             "Failed precondition: scheduler config and shared BlockManager disagree on "
                             "block_size / num_gpu_blocks");
    }
    auto *s = new (std::nothrow) zk_scheduler();
    if (!s) {
        if (!bm) zk_bm_destroy(use);
        return zk::set_error(ZK_ERR_INTERNAL, "Internal error: scheduler allocation failed");
    }
    s->cfg = *cfg;
    s->bm = use;
    s->owns_bm = bm == nullptr;
    *out = s;
    return ZK_OK;
}

void zk_sched_destroy(zk_scheduler *s) {
    if (!s) return;
    // running sequences still hold blocks of a shared manager: return them
    if (!s->owns_bm)
        for (auto *q : {&s->prefilling, &s->decoding})
            for (Seq &q_s : *q) s->free_blocks(q_s);
    delete s;
}

zk_block_manager *zk_sched_block_manager(zk_scheduler *s) { return s ? s->bm : nullptr; }

int zk_sched_make_sequence(zk_scheduler *s, const char *id, const int64_t *prompt, size_t prompt_len,
                           size_t max_tokens, int priority, zk_sequence **out) {
    if (!s || !id || !out || (prompt_len && !prompt))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_make_sequence: NULL argument");
    *out = nullptr;
    if (priority < ZK_PRIORITY_LOWEST || priority > ZK_PRIORITY_HIGHEST)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_make_sequence: bad priority");
    const size_t worst = blocks_for(prompt_len + max_tokens, s->cfg.block_size);  // scheduler.rs:234-240
    if (worst > s->cfg.num_gpu_blocks)
        return zk::set_error_typed(ZK_ERR_SEQUENCE_TOO_LONG, zk::ErrorKind::SequenceTooLong, worst,
                                   s->cfg.num_gpu_blocks);
    auto *q = new (std::nothrow) zk_sequence();
    if (!q) return zk::set_error(ZK_ERR_INTERNAL, "Internal error: sequence allocation failed");
    q->s.id = id;
    q->s.prompt.assign(prompt, prompt + prompt_len);
    q->s.max_tokens = max_tokens;
    q->s.priority = priority;
    q->s.arrival = s->next_arrival++;
    *out = q;
    return ZK_OK;
}

void zk_sequence_destroy(zk_sequence *q) { delete q; }

int zk_sched_add(zk_scheduler *s, zk_sequence *q) {
    if (!s || !q) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_add: NULL argument");
    if (s->known(q->s.id.c_str()))
        return zk::set_error(ZK_ERR_ALREADY_EXISTS, "Already exists: seq " + q->s.id);
    s->insert_waiting(std::move(q->s));
    delete q;
    return ZK_OK;
}

int zk_sched_schedule(zk_scheduler *s, zk_sched_output *out) {
    if (!s || !out) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_schedule: NULL argument");
    const zk_sched_config &cfg = s->cfg;
    std::vector<std::string> preempted, swapped_out, swapped_in;
    // 1. next chunks of prefilling sequences (scheduler.rs:270-282)
    size_t prefill_tokens = 0;
    for (Seq &q : s->prefilling) {
        if (q.prefill_pending && q.chunk_size == 0) {
            const size_t chunk = std::min(q.remaining(), cfg.prefill_chunk_size);
            if (prefill_tokens + chunk > cfg.max_prefill_tokens) break;
            q.chunk_size = chunk;
            prefill_tokens += chunk;
        }
    }
    // 2. waiting -> prefilling (scheduler.rs:284-309)
    while (!s->waiting.empty()) {
        if (s->prefilling.size() + s->decoding.size() >= cfg.max_num_seqs) break;
        const Seq &w = s->waiting.front();
        const bool resume_decode = w.swapped && !w.prefill_pending;  // back to decoding, no prompt tokens
        const size_t chunk = resume_decode ? 0 : std::min(w.remaining(), cfg.prefill_chunk_size);
        if (!resume_decode && prefill_tokens + chunk > cfg.max_prefill_tokens && prefill_tokens > 0) break;
        const size_t need = resume_decode ? blocks_for(w.len(), cfg.block_size)
                                          : blocks_for(w.prefill_pos + chunk + w.output.size(), cfg.block_size);
        if (zk_bm_available(s->bm) < need) break;
        Seq q = std::move(s->waiting.front());
        s->waiting.erase(s->waiting.begin());
        while (q.blocks.size() < need) {
            zk_block_handle h;
            if (int rc = zk_bm_allocate(s->bm, &h)) {  // another user of a shared manager took blocks
                s->free_blocks(q);
                s->insert_waiting(std::move(q));
                return rc;
            }
            q.blocks.push_back(h);
        }
        q.running = true;
        if (q.swapped) {
            s->swap_used -= q.swap_blocks;
            q.swapped = false;
            q.swap_blocks = 0;
            swapped_in.push_back(q.id);
        }
        if (resume_decode) {
            s->decoding.push_back(std::move(q));
            continue;
        }
        q.chunk_size = chunk;
        prefill_tokens += chunk;
        s->prefilling.push_back(std::move(q));
    }
    // 3. blocks for every running sequence (scheduler.rs:311-334)
    for (size_t i = 0; i < s->prefilling.size(); ++i) i = s->ensure_blocks(s->prefilling, i, preempted, swapped_out);
    for (size_t i = 0; i < s->decoding.size(); ++i) i = s->ensure_blocks(s->decoding, i, preempted, swapped_out);
    // 4. batch: prefilling with a chunk, then decoding (scheduler.rs:336-343);
    // a sequence left short of blocks waits for the next step
    auto covered = [&](const Seq &q) { return q.blocks.size() >= blocks_for(q.len(), cfg.block_size); };
    std::vector<const Seq *> batch;
    for (const Seq &q : s->prefilling)
        if (q.chunk_size > 0 && covered(q)) batch.push_back(&q);
    for (const Seq &q : s->decoding)
        if (covered(q)) batch.push_back(&q);
    size_t nblk = 0;
    for (const Seq *q : batch) nblk += q->blocks.size();
    s->out.assign(batch.size(), zk_sched_entry{});
    s->out_ids.resize(batch.size());
    s->out_blocks.resize(nblk);
    size_t off = 0;
    for (size_t i = 0; i < batch.size(); ++i) {
        const Seq &q = *batch[i];
        s->out_ids[i] = q.id;
        std::copy(q.blocks.begin(), q.blocks.end(), s->out_blocks.begin() + (ptrdiff_t)off);
        zk_sched_entry &e = s->out[i];
        e.is_prefill = q.prefill_pending;
        e.is_final_chunk = q.prefill_pending && q.final_chunk();
        e.num_tokens = q.step_tokens();
        e.tokens_before = q.tokens_before();
        e.len = q.len();
        e.num_blocks = q.blocks.size();
        e.block_offset = off;
        off += q.blocks.size();
    }
    for (size_t i = 0; i < batch.size(); ++i) {
        s->out[i].request_id = s->out_ids[i].c_str();
        s->out[i].blocks = s->out_blocks.data() + s->out[i].block_offset;
    }
    s->pre_ids = std::move(preempted);
    s->pre_ptrs.resize(s->pre_ids.size());
    for (size_t i = 0; i < s->pre_ids.size(); ++i) s->pre_ptrs[i] = s->pre_ids[i].c_str();
    out->batch = s->out.data();
    out->batch_len = s->out.size();
    out->preempted = s->pre_ptrs.data();
    out->num_preempted = s->pre_ptrs.size();
    out->blocks = s->out_blocks.data();
    // a sequence re-admitted from swap and preempted again within one step
    // never left host memory: swapped out again, report neither; preempted by
    // recompute, only the drop (which frees its host slots)
    for (auto it = swapped_in.begin(); it != swapped_in.end();) {
        auto o = std::find(swapped_out.begin(), swapped_out.end(), *it);
        if (o != swapped_out.end()) {
            swapped_out.erase(o);
            it = swapped_in.erase(it);
        } else if (std::find(s->pre_ids.begin(), s->pre_ids.end(), *it) != s->pre_ids.end()) {
            it = swapped_in.erase(it);
        } else {
            ++it;
        }
    }
    s->swap_out_ids = std::move(swapped_out);
    s->swap_in_ids = std::move(swapped_in);
    s->swap_out_ptrs.resize(s->swap_out_ids.size());
    s->swap_in_ptrs.resize(s->swap_in_ids.size());
    for (size_t i = 0; i < s->swap_out_ids.size(); ++i) s->swap_out_ptrs[i] = s->swap_out_ids[i].c_str();
    for (size_t i = 0; i < s->swap_in_ids.size(); ++i) s->swap_in_ptrs[i] = s->swap_in_ids[i].c_str();
    out->swapped_out = s->swap_out_ptrs.data();
    out->num_swapped_out = s->swap_out_ptrs.size();
    out->swapped_in = s->swap_in_ptrs.data();
    out->num_swapped_in = s->swap_in_ptrs.size();
    return ZK_OK;
}

int zk_sched_push_token(zk_scheduler *s, const char *id, int64_t token) {
    if (!s || !id) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_push_token: NULL argument");
    Seq *q = s->find_running(id);
    if (!q) return zk::set_error(ZK_ERR_INTERNAL, std::string("Internal error: scheduler: no running seq ") + id);
    q->output.push_back(token);
    return ZK_OK;
}

int zk_sched_mark_prefilled(zk_scheduler *s, const char *id) {  // scheduler.rs:146-148
    if (!s || !id) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_mark_prefilled: NULL argument");
    Seq *q = s->find_running(id);
    if (!q) return zk::set_error(ZK_ERR_INTERNAL, std::string("Internal error: scheduler: no running seq ") + id);
    q->prefill_pending = false;
    return ZK_OK;
}

void zk_sched_promote_to_decoding(zk_scheduler *s, const char *id) {  // scheduler.rs:423-434
    if (!s || !id) return;
    for (size_t i = 0; i < s->prefilling.size(); ++i)
        if (s->prefilling[i].id == id) {
            Seq q = std::move(s->prefilling[i]);
            s->prefilling.erase(s->prefilling.begin() + (ptrdiff_t)i);
            q.prefill_pending = false;
            s->decoding.push_back(std::move(q));
            return;
        }
}

void zk_sched_advance_prefill(zk_scheduler *s, const char *id) {  // scheduler.rs:437-457
    if (!s || !id) return;
    for (Seq &q : s->prefilling)
        if (q.id == id) {
            q.prefill_pos += q.chunk_size;
            q.chunk_size = 0;
            if (q.prefill_pos >= q.prompt.size()) zk_sched_promote_to_decoding(s, id);
            return;
        }
}

int zk_sched_finish(zk_scheduler *s, const char *id, size_t *prompt_len, size_t *output_len) {
    if (!s || !id) return 0;
    std::vector<Seq> *queue;
    size_t idx;
    if (!s->find_running(id, &queue, &idx)) return 0;  // scheduler.rs:396-420
    Seq q = std::move((*queue)[idx]);
    queue->erase(queue->begin() + (ptrdiff_t)idx);
    s->free_blocks(q);
    if (prompt_len) *prompt_len = q.prompt.size();
    if (output_len) *output_len = q.output.size();
    return 1;
}

int zk_sched_cancel(zk_scheduler *s, const char *id, size_t *prompt_len, size_t *output_len) {
    if (!s || !id) return ZK_CANCEL_NOT_FOUND;
    for (size_t i = 0; i < s->waiting.size(); ++i)  // scheduler.rs:460-469
        if (s->waiting[i].id == id) {
            if (prompt_len) *prompt_len = s->waiting[i].prompt.size();
            if (output_len) *output_len = 0;
            if (s->waiting[i].swapped) s->swap_used -= s->waiting[i].swap_blocks;
            s->waiting.erase(s->waiting.begin() + (ptrdiff_t)i);
            return ZK_CANCEL_WAS_WAITING;
        }
    return zk_sched_finish(s, id, prompt_len, output_len) ? ZK_CANCEL_WAS_RUNNING : ZK_CANCEL_NOT_FOUND;
}

int zk_sched_is_idle(const zk_scheduler *s) {
    return !s || (s->waiting.empty() && s->prefilling.empty() && s->decoding.empty());
}

int zk_sched_step_input(zk_scheduler *s, const char *id, int64_t *tokens, size_t *n) {
    if (!s || !id || !n) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_step_input: NULL argument");
    const Seq *q = s->find_running(id);
    if (!q) return zk::set_error(ZK_ERR_INTERNAL, std::string("Internal error: scheduler: no running seq ") + id);
    std::vector<int64_t> in;
    if (q->prefill_pending) {
        const size_t end = std::min(q->prefill_pos + q->chunk_size, q->prompt.size());
        in.assign(q->prompt.begin() + (ptrdiff_t)std::min(q->prefill_pos, end), q->prompt.begin() + (ptrdiff_t)end);
        if (q->final_chunk()) in.insert(in.end(), q->output.begin(), q->output.end());
    } else {
        if (q->output.empty())  // scheduler.rs:136-139 expects a generated token
            return zk::set_error(ZK_ERR_INTERNAL, "Internal error: decode step requires generated token");
        in.push_back(q->output.back());
    }
    const size_t cap = *n;
    *n = in.size();
    if (cap < in.size()) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_step_input: buffer too small");
    if (!in.empty()) std::copy(in.begin(), in.end(), tokens);
    return ZK_OK;
}

int zk_sched_seq_info(zk_scheduler *s, const char *id, zk_seq_info *info) {
    if (!s || !id || !info) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_sched_seq_info: NULL argument");
    const Seq *q = s->find_running(id);
    int state = ZK_SEQ_RUNNING;
    if (!q) {
        for (const Seq &w : s->waiting)
            if (w.id == id) q = &w;
        state = ZK_SEQ_WAITING;
    }
    if (!q) return zk::set_error(ZK_ERR_INTERNAL, std::string("Internal error: scheduler: unknown seq ") + id);
    info->state = state;
    info->is_prefill = q->prefill_pending;
    info->prompt_len = q->prompt.size();
    info->output_len = q->output.size();
    info->prefill_pos = q->prefill_pos;
    info->chunk_size = q->chunk_size;
    info->len = q->len();
    info->num_blocks = q->blocks.size();
    info->swapped = q->swapped ? 1 : 0;
    return ZK_OK;
}

}  // extern "C"

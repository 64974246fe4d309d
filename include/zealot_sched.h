/*
 * zealot_sched.h -- C ABI of the continuous-batching scheduler that feeds the
 * paged-KV path (host only: no call here touches a GPU).
 *
 * Restates src/scheduler.rs:156-478 (waiting queue by priority then arrival,
 * chunked prefill within a token budget, block top-up with preemption by
 * recompute) over a BlockManager that can be SHARED with the KV cache: the
 * reference's scheduler builds a private one (scheduler.rs:215) that no KV
 * code can see, so its block handles never reach the cache.  Here each batch
 * entry carries its sequence's handles (Sequence.blocks, scheduler.rs:60) and
 * zk_cache_bind_blocks turns them into the cache's block tables.
 *
 * Status codes and zk_last_error() are those of zealot_kv.h.
 */
#ifndef ZEALOT_SCHED_H
#define ZEALOT_SCHED_H

#include "zealot_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Priority (scheduler.rs:15-21; proto runtime.v1.Priority). */
typedef enum zk_priority {
    ZK_PRIORITY_LOWEST = 0,
    ZK_PRIORITY_MEDIUM = 1,
    ZK_PRIORITY_HIGH = 2,
    ZK_PRIORITY_HIGHEST = 3
} zk_priority;

/* SchedulerConfig (scheduler.rs:156-166). */
typedef struct zk_sched_config {
    size_t max_num_seqs;       /* running sequences (prefilling + decoding) */
    size_t block_size;         /* tokens per KV block */
    size_t num_gpu_blocks;     /* block pool capacity (admission control) */
    size_t max_prefill_tokens; /* prompt tokens per step */
    size_t prefill_chunk_size; /* prompt tokens per chunk */
    size_t swap_blocks;        /* host swap space in blocks (0: preempt by recompute only, the
                                  reference's policy); see zk_sched_output.swapped_out */
} zk_sched_config;

/* One batch entry of zk_sched_schedule: a snapshot of the sequence
 * (valid until the next zk_sched_schedule or zk_sched_destroy). */
typedef struct zk_sched_entry {
    const char *request_id;
    int is_prefill;       /* Sequence::is_prefill (scheduler.rs:142-144) */
    int is_final_chunk;   /* Sequence::is_final_chunk (scheduler.rs:150-152), prefill entries */
    size_t num_tokens;    /* tokens fed this step: the chunk (plus, on the final chunk of a
                             recompute, the preserved output tokens), or 1 when decoding */
    size_t tokens_before; /* KV tokens the sequence holds before this step */
    size_t len;           /* Sequence::len (scheduler.rs:115-121) */
    size_t num_blocks;    /* Sequence.blocks (scheduler.rs:60) */
    const zk_block_handle *blocks;
    size_t block_offset;  /* offset of `blocks` in zk_sched_output.blocks */
} zk_sched_entry;

/* ScheduleOutput (scheduler.rs:185-189): the batch (prefilling entries with a
 * chunk, then decoding ones) and the ids preempted this step (the runner drops
 * their state: ModelRunner::drop_state, engine.rs:20-22). */
typedef struct zk_sched_output {
    const zk_sched_entry *batch;
    size_t batch_len;
    const char *const *preempted;
    size_t num_preempted;
    const zk_block_handle *blocks; /* every entry's handles, packed in batch order */
    /* Preempted by swap this step: the runner moves their KV to host slots
     * (zk_cache_swap_out) BEFORE any write of this step, since their freed
     * blocks may already be another entry's.  Re-admitted this step: the
     * runner binds their new blocks and copies the KV back
     * (zk_cache_swap_in) before attention. */
    const char *const *swapped_out;
    size_t num_swapped_out;
    const char *const *swapped_in;
    size_t num_swapped_in;
} zk_sched_output;

typedef struct zk_scheduler zk_scheduler;

/* Scheduler::new (scheduler.rs:212-221).  bm == NULL: a private BlockManager
 * of cfg's size (the reference's behaviour); otherwise `bm` is shared (not
 * owned) and must have cfg's block_size and num_gpu_blocks. */
int zk_sched_create(const zk_sched_config *cfg, zk_block_manager *bm, zk_scheduler **out);
/* Returns the blocks of running sequences to a shared manager. */
void zk_sched_destroy(zk_scheduler *s);
zk_block_manager *zk_sched_block_manager(zk_scheduler *s);

/* A sequence made but not yet queued (Sequence, scheduler.rs:51-75). */
typedef struct zk_sequence zk_sequence;
/* make_sequence (scheduler.rs:225-253): SequenceTooLong when prompt_len +
 * max_tokens needs more blocks than the pool; the arrival number is taken
 * here.  Free with zk_sequence_destroy unless zk_sched_add takes it. */
int zk_sched_make_sequence(zk_scheduler *s, const char *request_id, const int64_t *prompt,
                           size_t prompt_len, size_t max_tokens, int priority, zk_sequence **out);
void zk_sequence_destroy(zk_sequence *seq);
/* add (scheduler.rs:255-257): queues and takes ownership of `seq`;
 * AlreadyExists (caller keeps ownership) for an id queued or running. */
int zk_sched_add(zk_scheduler *s, zk_sequence *seq);
/* schedule (scheduler.rs:267-344). */
int zk_sched_schedule(zk_scheduler *s, zk_sched_output *out);

/* Engine write-backs on a running sequence: output_tokens.push and
 * mark_prefilled (scheduler.rs:146-148). */
int zk_sched_push_token(zk_scheduler *s, const char *request_id, int64_t token);
int zk_sched_mark_prefilled(zk_scheduler *s, const char *request_id);
/* promote_to_decoding / advance_prefill (scheduler.rs:423-457); unknown ids
 * are ignored, as in the reference. */
void zk_sched_promote_to_decoding(zk_scheduler *s, const char *request_id);
void zk_sched_advance_prefill(zk_scheduler *s, const char *request_id);
/* finish (scheduler.rs:396-420): 1 and the lengths when the sequence was
 * running (its blocks freed), 0 otherwise. */
int zk_sched_finish(zk_scheduler *s, const char *request_id, size_t *prompt_len,
                    size_t *output_len);

/* cancel (scheduler.rs:460-469) -> CancelOutcome (scheduler.rs:191-197).
 * A swapped sequence cancelled while waiting is WasWaiting; the runner
 * releases its host slots (zk_cache_release_seq). */
typedef enum zk_cancel_outcome {
    ZK_CANCEL_NOT_FOUND = 0,
    ZK_CANCEL_WAS_WAITING = 1, /* prompt_len set, output_len 0 */
    ZK_CANCEL_WAS_RUNNING = 2  /* both set */
} zk_cancel_outcome;
int zk_sched_cancel(zk_scheduler *s, const char *request_id, size_t *prompt_len,
                    size_t *output_len);
/* is_idle (scheduler.rs:471-473). */
int zk_sched_is_idle(const zk_scheduler *s);

/* step_input (scheduler.rs:128-140) of a running sequence; *n in: capacity,
 * out: count.  Differs from the reference on multi-chunk recompute only: the
 * preserved output tokens follow the final chunk, not every chunk. */
int zk_sched_step_input(zk_scheduler *s, const char *request_id, int64_t *tokens, size_t *n);

/* Read-only view of a queued or running sequence. */
typedef enum zk_seq_state { ZK_SEQ_WAITING = 0, ZK_SEQ_RUNNING = 1 } zk_seq_state;
typedef struct zk_seq_info {
    int state;
    int is_prefill;
    size_t prompt_len, output_len, prefill_pos, chunk_size, len, num_blocks;
    int swapped; /* waiting with its KV in host slots */
} zk_seq_info;
int zk_sched_seq_info(zk_scheduler *s, const char *request_id, zk_seq_info *info);

#ifdef __cplusplus
}
#endif

#endif /* ZEALOT_SCHED_H */

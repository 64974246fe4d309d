/*
 * zealot_kv.h -- C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * This is the drop-in boundary a Rust HipModelRunner binds with `extern "C"`.
 * It replaces Zealot's GPU runtime layer for this path: src/kv_cache.rs
 * (KVCache), src/attention/cuda.rs (CudaAttention::paged_forward),
 * src/gpu_context.rs and src/buffer_pool.rs, plus the BlockManager of
 * src/block_manager.rs whose generation-gated handles it keeps.
 *
 * Conventions
 *  - Every function that can fail returns an int status (zk_status).  On
 *    failure zk_last_error() returns a message for the calling thread; messages
 *    match the reference's ZealotError Display strings (src/error.rs:3-46).
 *  - Device pointers are plain `void*` from hipMalloc (or any allocator);
 *    `stream` is a hipStream_t passed as `void*` (NULL = default stream).
 *    Kernel entry points are asynchronous on `stream`; they validate shapes on
 *    the host before launching and launch nothing when a check fails.
 *  - Pool layout (src/kv_cache.rs:41-50), element offset of
 *    (block, kv_head, token_in_block, dim):
 *        ((block * Hkv + kv_head) * block_size + token_in_block) * D + dim
 *    One block id indexes the pool of every layer (src/kv_cache.rs:241-253).
 *  - K/V inputs are token-major [T, Hkv, D] (src/kv_cache.rs:210-211).
 *  - Block tables are int32 [num_seqs, max_blocks_per_seq]; an entry < 0 ends
 *    the walk (src/attention/kernels/paged_attention.cu:66-67).
 */
#ifndef ZEALOT_KV_H
#define ZEALOT_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZK_ABI_VERSION 1

/* Status codes, one per ZealotError variant this path can raise
 * (src/error.rs:4-46), plus argument / HIP failures (reported by the
 * reference as ZealotError::Internal with a context prefix). */
typedef enum zk_status {
    ZK_OK = 0,
    ZK_ERR_BLOCK_ALREADY_ALLOCATED = 1, /* error.rs:5-6 */
    ZK_ERR_BLOCK_NOT_ALLOCATED = 2,     /* error.rs:8-9 */
    ZK_ERR_OUT_OF_BLOCKS = 3,           /* error.rs:11-12 */
    ZK_ERR_INVALID_BLOCK_SIZE = 4,      /* error.rs:14-15 */
    ZK_ERR_STALE_HANDLE = 5,            /* error.rs:23-28 */
    ZK_ERR_SEQUENCE_TOO_LONG = 6,       /* error.rs:36-37 */
    ZK_ERR_FAILED_PRECONDITION = 7,     /* error.rs:39-40 */
    ZK_ERR_ALREADY_EXISTS = 8,          /* error.rs:42-43 */
    ZK_ERR_INTERNAL = 9,                /* error.rs:45-46 */
    ZK_ERR_INVALID_ARGUMENT = 10,       /* shape/argument check (Internal in the reference) */
    ZK_ERR_HIP = 11                     /* HIP runtime failure (Internal in the reference) */
} zk_status;

typedef enum zk_dtype {
    ZK_F32 = 0,
    ZK_BF16 = 1,
    ZK_FP8_E4M3 = 2 /* OCP e4m3fn; pool elements only (no reference counterpart) */
} zk_dtype;

/* q-head -> kv-head mapping.  GROUPED is the kernel's
 * kv = h / (H / Hkv) (paged_attention.cu:32, :186); MODULO is the CPU runner's
 * kv = h % Hkv (model_runner_cpu.rs:295).  They agree for MHA. */
typedef enum zk_gqa_mapping { ZK_GQA_GROUPED = 0, ZK_GQA_MODULO = 1 } zk_gqa_mapping;

/* Message of the last failure on this thread ("" if none). */
const char *zk_last_error(void);
/* Status code of the last failure on this thread (ZK_OK if none) and the
 * fields of its ZealotError variant (src/error.rs:4-37), so a caller can
 * rebuild the typed error without parsing the message:
 *   ZK_ERR_STALE_HANDLE             {block_id, handle_gen, current_gen}
 *   ZK_ERR_OUT_OF_BLOCKS            {requested, available, 0}
 *   ZK_ERR_SEQUENCE_TOO_LONG        {required, capacity, 0}
 *   ZK_ERR_BLOCK_NOT_ALLOCATED,
 *   ZK_ERR_BLOCK_ALREADY_ALLOCATED,
 *   ZK_ERR_INVALID_BLOCK_SIZE       {value, 0, 0}
 *   every other code                {0, 0, 0} (the message carries the text)
 * fields may be NULL.  A failure that a call re-raises after cleaning up
 * (for example a BlockManager rejection inside a KVCache call) keeps its
 * code and fields. */
int zk_last_error_detail(uint64_t fields[3]);
int zk_abi_version(void);

/* ======================================================= BlockManager
 * src/block_manager.rs:16-164.  LIFO free list (first allocate returns id 0),
 * per-block refcount and generation (starting at 1, bumped when the last
 * reference is freed), StaleHandle on generation mismatch.  Thread-safe. */
typedef struct zk_block_manager zk_block_manager;
typedef struct zk_block_handle {
    uint64_t block_id;   /* BlockHandle.block_id, block_manager.rs:20 */
    uint64_t generation; /* BlockHandle.generation, block_manager.rs:23 */
} zk_block_handle;

/* BlockManager::create (block_manager.rs:88-104); InvalidBlockSize if block_size == 0. */
int zk_bm_create(size_t num_gpu_blocks, size_t block_size, zk_block_manager **out);
void zk_bm_destroy(zk_block_manager *bm);
/* try_allocate (block_manager.rs:108-122); OutOfBlocks when the pool is empty. */
int zk_bm_allocate(zk_block_manager *bm, zk_block_handle *out);
/* try_free (block_manager.rs:125-135); StaleHandle / BlockNotAllocated. */
int zk_bm_free(zk_block_manager *bm, zk_block_handle handle);
/* try_reference (block_manager.rs:140-144). */
int zk_bm_reference(zk_block_manager *bm, zk_block_handle handle);
/* available / free_blocks (block_manager.rs:70-73, :147-149). */
size_t zk_bm_available(const zk_block_manager *bm);
size_t zk_bm_num_gpu_blocks(const zk_block_manager *bm); /* block_manager.rs:75-78 */
size_t zk_bm_block_size(const zk_block_manager *bm);     /* block_manager.rs:80-83 */
/* check (block_manager.rs:151-164, private there): OK for a live handle;
 * BlockNotAllocated for an id out of range or a free block, StaleHandle on a
 * generation mismatch.  The KV cache uses it to reject stale handles it is
 * asked to bind. */
int zk_bm_check(zk_block_manager *bm, zk_block_handle handle);
/* Current refcount of a block (0 when free).  The reference keeps this
 * private (block_manager.rs:47); the KV cache needs it to decide copy-on-write. */
size_t zk_bm_refcount(const zk_block_manager *bm, uint64_t block_id);

/* ======================================================= kernel entry points
 * Stateless launches over caller-owned device buffers. */

/* KV append: scatter T token rows into the pools through a slot mapping.
 * Replaces the per-(token, head) cuMemcpyDtoD loops of KVCache::store_kv
 * (kv_cache.rs:229-274) and KVCache::append_kv (kv_cache.rs:316-344) with one
 * launch.  slot_mapping[t] = block_id * block_size + token_in_block; a negative
 * slot skips the token.  k, v: [T, Hkv, D] of src_dtype (F32 or BF16).
 * cache_dtype F32/BF16: the value is copied (converted if the dtypes differ);
 * FP8_E4M3: q = sat_rne_e4m3(x * (1 / scale)) with scale = {k,v}_scales
 * [token_row[t] * Hkv + h] (f32 division, round to nearest).  The scale
 * arguments must be NULL for non-fp8 pools. */
int zk_append(void *k_pool, void *v_pool, zk_dtype cache_dtype, const void *k, const void *v,
              zk_dtype src_dtype, const int64_t *slot_mapping, int64_t num_tokens,
              int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
              const float *k_scales, const float *v_scales, const int32_t *token_row,
              void *stream);

/* fp8 scales: scales[n * Hkv + h] = amax / 448 (1 if amax == 0) over tokens
 * [cu_seqlens[n], cu_seqlens[n+1]) of x ([T, Hkv, D], F32 or BF16).
 * cu_seqlens is a device int64 array of num_seqs + 1 entries. */
int zk_fp8_scales(const void *x, zk_dtype src_dtype, const int64_t *cu_seqlens, int num_seqs,
                  int num_kv_heads, int head_dim, float *scales, void *stream);

/* Block-table gather: pages -> contiguous token-major rows.  For sequence n,
 * its first ctx_lens[n] tokens (walk stops at a negative table entry, as
 * paged_attention.cu:63-83) land in rows [out_offsets[n], out_offsets[n] +
 * ctx_lens[n]) of k_out / v_out ([rows, Hkv, D], pool dtype, bit copy).
 * Rows after a sentinel (or an entry >= num_blocks) are left untouched. */
int zk_gather(const void *k_pool, const void *v_pool, zk_dtype dtype, const int32_t *block_tables,
              int max_blocks_per_seq, const int32_t *ctx_lens, const int64_t *out_offsets,
              int num_seqs, void *k_out, void *v_out, int num_kv_heads, int head_dim,
              int block_size, int64_t num_blocks, void *stream);

/* Copy-on-write block copy: for i < n, block dst[i] := block src[i] in every
 * pool of `pools` (host array of n_pools device pointers; pass each layer's K
 * and V pool).  block_bytes = block_size * Hkv * D * elt.  src/dst are device
 * int32 arrays.  No reference counterpart (the reference only has
 * BlockManager::try_reference, block_manager.rs:140-144). */
int zk_copy_blocks(void *const *pools, int n_pools, int64_t block_bytes, int64_t num_blocks,
                   const int32_t *src, const int32_t *dst, int64_t n, void *stream);

/* Split-K paged decode attention, batched over all sequences in one call.
 * Replaces CudaAttention::paged_forward (attention/cuda.rs:126-209) and the
 * paged_attention[_gqa]_kernel launches (paged_attention.cu:13-27, :151-165).
 *   q, out:  [num_seqs, num_heads, head_dim], dtype q_dtype (F32 or BF16)
 *   pools:   kv_dtype (F32, BF16 or FP8_E4M3)
 *   k_scales/v_scales: [num_seqs, Hkv] dequant scales, fp8 pools only
 *   scale:   softmax scale (the reference uses 1/sqrt(head_dim), cuda.rs:141)
 * num_blocks bounds the pool: a table entry outside [0, num_blocks) ends the
 * walk like a negative one (the reference kernel has no such check).
 * A sequence of length 0 yields a zero row.  workspace must hold
 * zk_paged_decode_workspace_size(...) bytes (device memory, 256-B aligned). */
size_t zk_paged_decode_workspace_size(int num_seqs, int num_heads, int head_dim,
                                      int max_blocks_per_seq, int block_size);
int zk_paged_decode(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                    zk_dtype kv_dtype, void *out, const int32_t *block_tables,
                    const int32_t *seq_lens, int num_seqs, int num_heads, int num_kv_heads,
                    int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                    float scale,
                    zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                    void *workspace, size_t workspace_bytes, void *stream);

/* zk_paged_decode without the workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * workspace is the library's own device scratch of ZK_DECODE_SCRATCH_BYTES
 * (64 MiB), one copy per GPU: it sits in a code object of its own, which the
 * HIP runtime loads on a GPU at the first call there (not when the library's
 * other kernels load), and is held until the process ends.  That first call
 * looks the scratch's address up, so make it outside graph capture; later
 * calls may be captured.  The call allocates nothing and creates no events.  A call
 * that needs more scratch than that (see zk_paged_decode_workspace_size; the
 * exact need depends on the batch) fails with ZK_ERR_INVALID_ARGUMENT and
 * launches nothing.  Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (different streams or host threads without
 * ordering) race.  Inputs, outputs and results are those of zk_paged_decode. */
#define ZK_DECODE_SCRATCH_BYTES (64u << 20)
int zk_paged_decode_noalloc(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                            zk_dtype kv_dtype, void *out, const int32_t *block_tables,
                            const int32_t *seq_lens, int num_seqs, int num_heads, int num_kv_heads,
                            int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                            float scale, zk_gqa_mapping mapping, const float *k_scales,
                            const float *v_scales, void *stream);

/* ======================================================= KVCache (stateful)
 * src/kv_cache.rs:51-356.  Owns per-layer K/V pools (one HBM slab) and
 * per-sequence device block tables.  Sequence ids are NUL-terminated strings. */
typedef struct zk_kv_cache zk_kv_cache;

/* KVCache::new (kv_cache.rs:66-102): zero-filled pools.  `max_seqs` bounds the
 * number of simultaneously registered sequences (their tables share one slab). */
int zk_cache_create(size_t num_blocks, size_t block_size, size_t num_layers, size_t num_kv_heads,
                    size_t head_dim, zk_dtype dtype, size_t max_seqs, size_t max_blocks_per_seq,
                    void *stream, zk_kv_cache **out);
void zk_cache_destroy(zk_kv_cache *c);
/* register_seq (kv_cache.rs:107-124): table of max_blocks entries set to -1. */
int zk_cache_register_seq(zk_kv_cache *c, const char *id, size_t max_blocks);
/* alloc_block (kv_cache.rs:127-161): allocate through `bm`, append to the table.
 * The device table row is written by the next call that needs it (a KV
 * write, the table pointer, fork, register, release), so a step's
 * allocations reach the device in one upload. */
int zk_cache_alloc_block(zk_kv_cache *c, const char *id, zk_block_manager *bm, size_t *block_id);
/* release_seq (kv_cache.rs:164-166).  Also frees the sequence's handles
 * through the BlockManager they came from (the reference leaks them). */
int zk_cache_release_seq(zk_kv_cache *c, const char *id);
/* Fork: `child` shares every block of `parent` (BlockManager reference per
 * block); the first write into a shared block copies it (all layers, K and V)
 * into a fresh block first.  No reference counterpart: the reference only has
 * the sharing primitive BlockManager::try_reference (block_manager.rs:140-144). */
int zk_cache_fork_seq(zk_kv_cache *c, const char *parent, const char *child);
/* store_kv (kv_cache.rs:212-276): n_tokens rows [n, Hkv, D] at start_token.
 * Fails with Internal "block_idx ... OOB" before writing anything if a
 * position has no block.  Writing the last layer advances cached_tokens to
 * max(cached_tokens, start_token + n_tokens). */
int zk_cache_store_kv(zk_kv_cache *c, size_t layer, const char *id, const void *k, const void *v,
                      zk_dtype src_dtype, size_t start_token, size_t n_tokens);
/* append_kv (kv_cache.rs:281-356): one token [Hkv, D] at cached_tokens;
 * writing the last layer advances cached_tokens / block_offset. */
int zk_cache_append_kv(zk_kv_cache *c, size_t layer, const char *id, const void *k,
                       const void *v, zk_dtype src_dtype);
/* Batched decode append for one layer: token i of k/v ([n, Hkv, D]) goes to
 * sequence ids[i] at its cached_tokens position (copy-on-write first where the
 * target block is shared); one launch for the whole batch.  Writing the last
 * layer advances each sequence by one token.  Batched form of append_kv
 * (kv_cache.rs:281-356) for a runner that steps all sequences together. */
int zk_cache_append_kv_batch(zk_kv_cache *c, size_t layer, const char *const *ids, int n,
                             const void *k, const void *v, zk_dtype src_dtype);
/* Batched write for one layer of a mixed prefill / decode step: sequence
 * ids[i] receives num_tokens[i] tokens (0 allowed) at its cached_tokens
 * position, packed in batch order in k/v ([sum num_tokens, Hkv, D]);
 * copy-on-write first where a target block is shared; one launch for the whole
 * batch.  Writing the last layer advances each sequence by its num_tokens[i].
 * Replaces the per-sequence store_kv / append_kv calls of the runner's step
 * (cuda_runner.rs:274-406, kv_cache.rs:206-356).  Fails before writing
 * anything if a position has no block (kv_cache.rs:234-239) or an id repeats.
 * src_token_stride: elements from one token's K (V) row block to the next
 * (0 = Hkv * D); with a fused QKV projection output [T, (H + 2 Hkv) * D], k
 * and v point at its K and V columns and the stride is (H + 2 Hkv) * D, so
 * the append reads them in place (no transpose or copy, cf. the head-major
 * transposes of cuda_runner.rs:373-392). */
int zk_cache_write_batch(zk_kv_cache *c, size_t layer, const char *const *ids,
                         const int32_t *num_tokens, int n, const void *k, const void *v,
                         zk_dtype src_dtype, int64_t src_token_stride);
/* No counterpart in the reference (whose runner runs three q/k/v sgemms and
 * then store_kv / append_kv per sequence, cuda_runner.rs:331-406): the fused
 * projection qkv = x . w_qkv^T (bf16 x [T, hidden], w_qkv [(H + 2 Hkv) D,
 * hidden] with q rows, then k, then v; T = sum num_tokens) and
 * zk_cache_write_batch of its K and V columns.  qkv ([T, (H + 2 Hkv) D]
 * bf16) receives at least the q columns, the input of the layer's attention
 * (row stride (H + 2 Hkv) D).  When zk_linear's plan for the projection keeps
 * a weight-streaming configuration with split k (as zk_linear_rms_norm
 * folds) and the pools are bf16, one kernel adds the split sums, writes the
 * q columns and stores K and V at their slots (the reduce kernel and the
 * append in one launch; qkv's K / V columns are then not written);
 * otherwise the projection writes qkv and the append reads it.  Pools and
 * q bit for bit the two-call sequence through the same configuration.  qkv
 * must not overlap x (rejected). */
int zk_cache_write_batch_qkv(zk_kv_cache *c, size_t layer, const char *const *ids,
                             const int32_t *num_tokens, int n, const void *x, const void *w_qkv,
                             int64_t hidden, int num_heads, void *qkv);
/* Block tables from the caller's handles: sequence ids[i]'s table becomes
 * blocks[o_i .. o_i + num_blocks[i]) (packed in batch order), registering the
 * sequence on first use.  This is how a scheduler that shares `bm` with the
 * cache hands over Sequence.blocks (scheduler.rs:60) instead of the cache
 * allocating its own (kv_cache.rs:127-164, which nothing in the reference
 * calls).  The handles stay the caller's: release_seq does not free them, and
 * fork_seq, alloc_block and a copy-on-write on a bound sequence fail.  All
 * checks run before anything changes: stale or free handles (zk_bm_check), a
 * table longer than max_blocks_per_seq, an id bound twice, an id the cache
 * allocated itself, fewer blocks than the written tokens need, and, when
 * tokens_before is given, a sequence whose cached_tokens differ from it (the
 * runner and the scheduler disagree).  One table-update launch per call. */
int zk_cache_bind_blocks(zk_kv_cache *c, zk_block_manager *bm, const char *const *ids, int n,
                         const zk_block_handle *blocks, const size_t *num_blocks,
                         const size_t *tokens_before);
/* ---- KV swap (docs/architecture.md:452-469: swap-out to CPU frees GPU
 * blocks, preemption prefers it to recompute; no reference code).
 * enable_swap: pinned host space of num_host_blocks slots, each holding one
 * block of every pool (2 * num_layers * block_size * Hkv * D elements).
 * swap_out: the written blocks of each sequence (ceil(tokens / block_size))
 * are staged through device memory in chunks and copied to host slots, one
 * DMA per run of consecutive slots; then the sequence's device blocks are
 * freed to its BlockManager (bound sequences: dropped, the caller frees its
 * handles) and its table cleared.  Its token counts stay; writes and
 * attention on it fail until swap_in.  OutOfBlocks (nothing moved) when the
 * host space is short.
 * swap_in: the cache allocates fresh blocks from `bm` (or the sequence's own
 * manager) for a sequence it owns, all or nothing; a bound sequence must have
 * been given its new handles with zk_cache_bind_blocks first.  The host data
 * is copied back into them and the host slots freed.  Asynchronous on the
 * cache stream like every other cache call; release_seq frees host slots. */
int zk_cache_enable_swap(zk_kv_cache *c, size_t num_host_blocks);
int zk_cache_swap_space(zk_kv_cache *c, size_t *total, size_t *free_blocks);
int zk_cache_swap_out(zk_kv_cache *c, const char *const *ids, int n);
int zk_cache_swap_in(zk_kv_cache *c, const char *const *ids, int n, zk_block_manager *bm);
int zk_cache_seq_swapped(zk_kv_cache *c, const char *id, int *swapped);
/* fp8 pools: set the per-(layer, kv_head) dequant scales of a sequence
 * (k_scales/v_scales: host arrays of num_layers * Hkv floats). */
int zk_cache_set_fp8_scales(zk_kv_cache *c, const char *id, const float *k_scales,
                            const float *v_scales);
/* Raw pointers (kv_cache.rs:188-204).  The table pointer call first applies
 * queued table writes on the cache stream. */
int zk_cache_block_table_ptr(zk_kv_cache *c, const char *id, const int32_t **out);
void *zk_cache_k_pool_ptr(zk_kv_cache *c, size_t layer);
void *zk_cache_v_pool_ptr(zk_kv_cache *c, size_t layer);
/* max_blocks (kv_cache.rs:184-186) and seq_state fields (kv_cache.rs:24-35). */
int zk_cache_max_blocks(zk_kv_cache *c, const char *id, size_t *out);
int zk_cache_seq_state(zk_kv_cache *c, const char *id, size_t *cached_tokens,
                       size_t *block_offset, size_t *num_blocks);
/* Host copy of a sequence's block ids (kv_cache.rs:28); *n in: capacity, out: count. */
int zk_cache_block_ids(zk_kv_cache *c, const char *id, int64_t *ids, size_t *n);
/* Batched decode for one layer over registered sequences `ids[0..n)`:
 * builds the batch's block tables / lengths and runs the paged decode
 * (zk_paged_decode; replaces the per-sequence paged_forward loop of
 * cuda_runner.rs:443-461).  Sequences forked from one prefix (fork_seq) whose
 * tables start with the same blocks are decoded in subgroups that read the
 * shared pages once (bf16 pools, MFMA shapes); no reference counterpart. */
int zk_cache_paged_decode(zk_kv_cache *c, size_t layer, const char *const *ids, int n,
                          const void *q, zk_dtype q_dtype, void *out, int num_heads, float scale,
                          zk_gqa_mapping mapping);
/* One decode step of one layer: zk_cache_append_kv_batch of k / v ([n, Hkv,
 * D], one token per sequence at its next position, copy-on-write of shared
 * tail blocks included) followed by zk_cache_paged_decode, with the same
 * results.  For bf16 pools and bf16 k / v on the MFMA decode shapes it is one
 * decode launch: the work item holding a sequence's last page stores the
 * token's K / V row into the pools and attends it from registers (the
 * per-layer append plus paged_forward of cuda_runner.rs:405-461); other
 * shapes run the two calls.  No single reference counterpart. */
int zk_cache_decode_append(zk_kv_cache *c, size_t layer, const char *const *ids, int n, const void *k,
                           const void *v, zk_dtype src_dtype, const void *q, zk_dtype q_dtype, void *out,
                           int num_heads, float scale, zk_gqa_mapping mapping);
/* Batched attention for one layer of a mixed step, after zk_cache_write_batch
 * wrote the step's tokens: the num_tokens[i] query rows of sequence ids[i]
 * (packed in batch order in q / out, [sum num_tokens, H, D]) are its last
 * num_tokens[i] tokens at this layer, attended causally over its pages (row t
 * sees positions [0, layer_len - num_tokens[i] + t], attention.cu:117-121).
 * One-row entries run as one paged decode (with prefix sharing), longer ones
 * as one chunked-prefill launch (zk_paged_prefill); shapes outside the
 * prefill kernel's run every chunk row as a decode.  Replaces the runner's
 * per-sequence paged_forward (cuda_runner.rs:438-461).  q rows are
 * q_token_stride elements apart (0 = H * D; a fused QKV output's row length
 * reads q in place); out rows are packed [rows, H, D]. */
int zk_cache_attention_batch(zk_kv_cache *c, size_t layer, const char *const *ids,
                             const int32_t *num_tokens, int n, const void *q, zk_dtype q_dtype,
                             int64_t q_token_stride, void *out, int num_heads, float scale,
                             zk_gqa_mapping mapping);
/* Prefix sharing of the last zk_cache_paged_decode: subgroups formed and the
 * pages they shared (sum over subgroups).  No reference counterpart. */
int zk_cache_decode_sharing(zk_kv_cache *c, int *subgroups, int64_t *shared_pages);

/* ================================================== chunked-prefill attention
 * Replaces CudaAttention::forward_gpu (attention/cuda.rs:56-110, the tiled
 * first-chunk kernel attention.cu:9-187) and the later-chunk paged_forward
 * call of cuda_runner.rs:443-461, which computes only the chunk's first row.
 * Sequence n's chunk has q rows cu_seqlens_q[n] .. cu_seqlens_q[n+1] (device,
 * int64; total_q == cu_seqlens_q[num_seqs]) at absolute positions
 * start_pos[n] + t (device, int32); its K/V are already in the pages (append
 * first).  causal != 0: row t attends to positions [0, start + t]
 * (attention.cu:117-121); causal == 0: to [0, start + len)
 * (CpuAttention::forward, attention/mod.rs:64-98).  q, out: [total_q, H, D],
 * f32 or bf16 (out has q's dtype).  The page walk stops at the first table
 * entry < 0 or >= num_blocks, as in zk_paged_decode.  Shapes: bf16 or fp8
 * pools, block_size 16, head_dim 64 or 128, H/Hkv in {1, 2, 4, 8},
 * max_blocks_per_seq <= 2048.  workspace: caller-owned, 256-B aligned, at
 * least zk_paged_prefill_workspace_size bytes.  Asynchronous on `stream`. */
size_t zk_paged_prefill_workspace_size(int num_seqs, int64_t total_q, int num_heads, int num_kv_heads);
int zk_paged_prefill(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                     zk_dtype kv_dtype, void *out, const int32_t *block_tables,
                     const int64_t *cu_seqlens_q, const int32_t *start_pos, int num_seqs,
                     int64_t total_q, int num_heads, int num_kv_heads, int head_dim, int block_size,
                     int max_blocks_per_seq, int64_t num_blocks, float scale, int causal,
                     zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                     void *workspace, size_t workspace_bytes, void *stream);

/* ======================================================= measurement
 * No reference counterpart (the reference's attention bench is a stub,
 * cuda_runner.rs:151-157).  When timing is on, every kernel this library
 * launches is bracketed by a pair of hipEvents on its stream; the query
 * synchronises on the recorded events and returns the launch count and total
 * milliseconds of one kernel name since the last reset.  Kernel names:
 * "append", "fp8_scales", "gather", "copy_blocks", "decode_seq_info",
 * "decode_plan", "decode_partials", "decode_reduce", "prefill_plan",
 * "prefill_attention", "stream_copy", "stream_read", "rms_norm", "silu_mul",
 * "add", "embedding", "linear", "swap_out", "swap_in". */
int zk_timing_enable(int on);
int zk_timing_reset(void);
int zk_timing_query(const char *kernel, int64_t *launches, double *total_ms);
/* Streaming copy of `bytes` (multiple of 16, 16-B aligned pointers): the
 * in-repo bandwidth yardstick and HBM-counter calibration kernel. */
int zk_stream_copy(void *dst, const void *src, size_t bytes, void *stream);
/* Streaming read of `bytes` (multiple of 16, 16-B aligned): the in-repo
 * read-bandwidth yardstick (the practical ceiling of an HBM-read-bound kernel
 * such as the decode).  `sink`: a device word the kernel may write. */
int zk_stream_read(const void *src, size_t bytes, uint32_t *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif

/*
 * zk_oracle.h -- CPU restatement of Zealot's paged-KV path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product (zealot_amd/, include/) never
 * links or calls it.
 *
 * Every function names the reference lines it restates.  Reference paths are
 * relative to the Zealot source tree (src/...).
 */
#ifndef ZK_ORACLE_H
#define ZK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of a pool or of an input tensor. */
enum { OR_F32 = 0, OR_BF16 = 1, OR_FP8_E4M3 = 2 };
/* q-head -> kv-head mappings. */
enum { OR_GQA_GROUPED = 0, OR_GQA_MODULO = 1 };

/* Scalar conversions. */
uint16_t or_bf16_from_f32(float f);  /* round-to-nearest-even, NaN stays NaN */
float or_f32_from_bf16(uint16_t b);
uint8_t or_e4m3_from_f32(float f);   /* OCP e4m3fn, RNE, saturating to +-448 */
float or_f32_from_e4m3(uint8_t c);

/* Chunked-prefill store, src/kv_cache.rs:212-276 (pool offset kv_cache.rs:245-247). */
int or_store_kv(void *k_pool, void *v_pool, int dtype, const void *k, const void *v,
                const int64_t *block_ids, int64_t n_block_ids, int64_t start_token,
                int64_t n_tokens, int num_kv_heads, int head_dim, int block_size);

/* or_store_kv over a batch of sequences (the CPU baseline's append leg);
 * threads > 1 runs the sequences on OpenMP threads. */
int or_store_kv_batch(void *k_pool, void *v_pool, int dtype, const void *k, const void *v,
                      const int64_t *block_ids, const int64_t *blk_off, const int64_t *tok_off,
                      const int64_t *start_token, int num_seqs, int num_kv_heads, int head_dim,
                      int block_size, int threads);

/* Slot-mapping append (store/append of kv_cache.rs:229-274 and 316-344 with
 * slot = block_ids[g / bs] * bs + g % bs precomputed).  Negative slots skip. */
int or_append_slots(void *k_pool, void *v_pool, int cache_dtype, const void *k, const void *v,
                    int src_dtype, const int64_t *slot_mapping, int64_t num_tokens,
                    int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                    const float *k_scales, const float *v_scales, const int32_t *token_row);

/* Per-(sequence, kv_head) fp8 scales: amax/448 over the tokens [cu[n], cu[n+1]). */
void or_fp8_scales(const void *x, int src_dtype, const int64_t *cu_seqlens, int num_seqs,
                   int num_kv_heads, int head_dim, float *scales);

/* Page walk (src/attention/kernels/paged_attention.cu:63-83): pages -> [ctx, Hkv, D]. */
int64_t or_gather(const void *pool, int dtype, const int32_t *block_table, int64_t max_blocks,
                  int64_t ctx_len, void *out, int num_kv_heads, int head_dim, int block_size);

/* Copy-on-write block copy over every pool (all layers, K and V). */
void or_copy_blocks(void *const *pools, int n_pools, int64_t block_bytes, const int32_t *src,
                    const int32_t *dst, int64_t n);

/* Decode attention, one query row per (seq, q-head); math of
 * src/attention/mod.rs:64-98, head mapping of paged_attention.cu:32 (grouped)
 * or model_runner_cpu.rs:295 (modulo).  q, out: [N, H, D] f32. */
int or_paged_decode(const float *q, const void *k_pool, const void *v_pool, int kv_dtype,
                    const float *k_scales, const float *v_scales, const int32_t *block_tables,
                    int64_t max_blocks, const int32_t *seq_lens, int num_seqs, int num_heads,
                    int num_kv_heads, int head_dim, int block_size, float scale, int mapping,
                    float *out, int threads);

/* Chunked-prefill attention: row t of sequence n's chunk (q rows
 * cu_seqlens_q[n] .. cu_seqlens_q[n+1], q/out [T, H, D] f32) sits at position
 * start_pos[n] + t and sees positions [0, start + t] (causal) or
 * [0, start + len) (not causal). */
int or_paged_prefill(const float *q, const void *k_pool, const void *v_pool, int kv_dtype,
                     const float *k_scales, const float *v_scales, const int32_t *block_tables,
                     int64_t max_blocks, const int64_t *cu_seqlens_q, const int32_t *start_pos, int num_seqs,
                     int num_heads, int num_kv_heads, int head_dim, int block_size, float scale, int mapping,
                     int causal, float *out, int threads);

/* Dense CPU attention, src/attention/mod.rs:31-103 verbatim semantics:
 * q, k, v, out are [S, H, n_pos, D] f32; non-causal softmax(QK^T*scale)V. */
int or_cpu_attention(const float *q, const float *k, const float *v, int num_seqs, int num_heads,
                     int head_dim, int max_seq_len, float *out);

/* src/attention/mod.rs:105-115. */
void or_matmul(const float *a, const float *b, int m, int k, int n, float *c);

/* src/model_runner_cpu.rs:286-304: [seq_len, kv_heads*d] -> [num_heads, seq_len, d]. */
void or_repeat_interleave_kv(const float *src, int kv_heads, int num_heads, int seq_len,
                             int head_dim, float *out);

#ifdef __cplusplus
}
#endif
/* dense ops around the path (rms_norm.cu, activation.cu, embedding.cu) */
void or_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t dim, float eps);
void or_silu_gate_mul(const float *gate, const float *up, float *out, int64_t n);
void or_add(const float *a, const float *b, float *out, int64_t n);
void or_embedding(const int64_t *ids, const float *table, float *out, int64_t n, int64_t dim);

#endif

/*
 * zk_oracle.c -- CPU restatement of Zealot's paged-KV path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline.  Nothing in the product links or calls this file.
 *
 * Arithmetic follows the reference's Rust CPU path: plain f32 operations in
 * source order, no fused multiply-add (Rust never contracts a*b+c; this file is
 * built with -ffp-contract=off), exp from the platform libm (Rust's f32::exp
 * calls the same expf).
 */
#include "zk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- scalars */

static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_bf16_from_f32(float f) {
    uint32_t u = bits_of(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float or_f32_from_bf16(uint16_t b) { return float_of((uint32_t)b << 16); }

/* OCP 8-bit floating point spec, E4M3 ("e4m3fn"): bias 7, no infinities,
 * NaN = S.1111.111, max finite 448 = S.1111.110, subnormals m * 2^-9.
 * Round to nearest even; magnitudes >= 448 (and infinities) saturate to 448;
 * NaN keeps its sign. */
uint8_t or_e4m3_from_f32(float f) {
    uint32_t u = bits_of(f);
    uint8_t s = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint8_t)(s | 0x7fu);
    if (a >= 0x43e00000u) return (uint8_t)(s | 0x7eu); /* |f| >= 448 */
    int e = (int)(a >> 23);                             /* biased f32 exponent */
    if (e >= 121) {                                     /* |f| >= 2^-6: e4m3 normal range */
        uint32_t mant = a & 0x7fffffu;
        uint32_t keep = mant >> 20, rem = mant & 0xfffffu;
        uint32_t up = (rem > 0x80000u) || (rem == 0x80000u && (keep & 1u));
        uint32_t v = (((uint32_t)(e - 120) << 3) | keep) + up; /* carry bumps the exponent */
        if (v > 0x7eu) v = 0x7eu;
        return (uint8_t)(s | v);
    }
    /* e4m3 subnormal: value = m * 2^-9; the f32 significand is sig * 2^(e-150). */
    uint32_t sig = e ? ((a & 0x7fffffu) | 0x800000u) : (a & 0x7fffffu);
    int sh = 141 - (e ? e : 1);
    if (sh >= 25) return s; /* below half of 2^-9 */
    uint32_t m = sig >> sh, rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint8_t)(s | m); /* m == 8 encodes the smallest normal */
}

float or_f32_from_e4m3(uint8_t c) {
    int e = (c >> 3) & 15, m = c & 7;
    float sg = (c & 0x80) ? -1.0f : 1.0f;
    if (e == 15 && m == 7) return sg * NAN;
    if (e == 0) return sg * ldexpf((float)m, -9);
    return sg * ldexpf((float)(8 + m), e - 10);
}

static size_t elt_size(int dt) { return dt == OR_F32 ? 4 : dt == OR_BF16 ? 2 : 1; }

static float load_elt(const void *base, int dt, int64_t i) {
    if (dt == OR_F32) return ((const float *)base)[i];
    if (dt == OR_BF16) return or_f32_from_bf16(((const uint16_t *)base)[i]);
    return or_f32_from_e4m3(((const uint8_t *)base)[i]);
}

/* ------------------------------------------------------------ append/store */

/* kv_cache.rs:229-274: for each token, (block_idx, token_in_block) from the
 * global position, OOB check against the sequence's block list, then one copy
 * of head_dim elements per kv head into
 * block_id*bs*Hkv*D + h*bs*D + token_in_block*D (kv_cache.rs:245-247). */
int or_store_kv(void *k_pool, void *v_pool, int dtype, const void *k, const void *v,
                const int64_t *block_ids, int64_t n_block_ids, int64_t start_token,
                int64_t n_tokens, int num_kv_heads, int head_dim, int block_size) {
    size_t es = elt_size(dtype);
    int64_t kv_data = (int64_t)num_kv_heads * head_dim;
    int64_t kv_block_stride = (int64_t)block_size * kv_data;
    for (int64_t t = 0; t < n_tokens; ++t) {
        int64_t g = start_token + t;
        int64_t block_idx = g / block_size, tib = g % block_size;
        if (block_idx >= n_block_ids) return -1; /* kv_cache.rs:234-239 */
        int64_t block_id = block_ids[block_idx];
        int64_t src_base = t * kv_data;
        for (int h = 0; h < num_kv_heads; ++h) {
            int64_t pool_off = block_id * kv_block_stride + (int64_t)h * block_size * head_dim +
                               tib * head_dim;
            int64_t src_off = src_base + (int64_t)h * head_dim;
            memcpy((char *)k_pool + pool_off * es, (const char *)k + src_off * es, head_dim * es);
            memcpy((char *)v_pool + pool_off * es, (const char *)v + src_off * es, head_dim * es);
        }
    }
    return 0;
}

/* The CPU baseline's append leg: or_store_kv for each of num_seqs sequences
 * (sequence n: its block ids block_ids[blk_off[n] .. blk_off[n+1]), tokens
 * k/v rows tok_off[n] .. tok_off[n+1] at start_token[n]), as the reference
 * runner would call KVCache::store_kv once per sequence
 * (cuda_runner.rs:405-431).  threads > 1 spreads the sequences over OpenMP
 * threads (the reference is single-threaded).  Returns the first failing
 * sequence's status (-1) or 0. */
int or_store_kv_batch(void *k_pool, void *v_pool, int dtype, const void *k, const void *v,
                      const int64_t *block_ids, const int64_t *blk_off, const int64_t *tok_off,
                      const int64_t *start_token, int num_seqs, int num_kv_heads, int head_dim,
                      int block_size, int threads) {
    size_t es = elt_size(dtype);
    int64_t row = (int64_t)num_kv_heads * head_dim * (int64_t)es;
    int rc = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(min : rc)
    for (int n = 0; n < num_seqs; ++n) {
        int r = or_store_kv(k_pool, v_pool, dtype, (const char *)k + tok_off[n] * row,
                            (const char *)v + tok_off[n] * row, block_ids + blk_off[n], blk_off[n + 1] - blk_off[n],
                            start_token[n], tok_off[n + 1] - tok_off[n], num_kv_heads, head_dim, block_size);
        if (r < rc) rc = r;
    }
    return rc;
}

static void put_row(void *pool, int cache_dt, int64_t pool_off, const void *src, int src_dt,
                    int64_t src_off, int head_dim, float inv_scale) {
    if (cache_dt == src_dt && cache_dt != OR_FP8_E4M3) {
        size_t es = elt_size(cache_dt);
        memcpy((char *)pool + pool_off * es, (const char *)src + src_off * es, head_dim * es);
        return;
    }
    if (cache_dt == OR_FP8_E4M3) {
        uint8_t *dst = (uint8_t *)pool + pool_off;
        for (int d = 0; d < head_dim; ++d) dst[d] = or_e4m3_from_f32(load_elt(src, src_dt, src_off + d) * inv_scale);
        return;
    }
    /* widening/narrowing between f32 and bf16 */
    for (int d = 0; d < head_dim; ++d) {
        float x = load_elt(src, src_dt, src_off + d);
        if (cache_dt == OR_F32) ((float *)pool)[pool_off + d] = x;
        else ((uint16_t *)pool)[pool_off + d] = or_bf16_from_f32(x);
    }
}

int or_append_slots(void *k_pool, void *v_pool, int cache_dtype, const void *k, const void *v,
                    int src_dtype, const int64_t *slot_mapping, int64_t num_tokens,
                    int num_kv_heads, int head_dim, int block_size, int64_t num_blocks,
                    const float *k_scales, const float *v_scales, const int32_t *token_row) {
    int64_t kv_data = (int64_t)num_kv_heads * head_dim;
    for (int64_t t = 0; t < num_tokens; ++t) {
        int64_t slot = slot_mapping[t];
        if (slot < 0) continue;
        int64_t block_id = slot / block_size, tib = slot % block_size;
        if (block_id >= num_blocks) return -1;
        for (int h = 0; h < num_kv_heads; ++h) {
            int64_t pool_off = block_id * block_size * kv_data + (int64_t)h * block_size * head_dim +
                               tib * head_dim;
            int64_t src_off = t * kv_data + (int64_t)h * head_dim;
            float ik = 1.0f, iv = 1.0f;
            if (cache_dtype == OR_FP8_E4M3) {
                int64_t r = (int64_t)token_row[t] * num_kv_heads + h;
                ik = 1.0f / k_scales[r];
                iv = 1.0f / v_scales[r];
            }
            put_row(k_pool, cache_dtype, pool_off, k, src_dtype, src_off, head_dim, ik);
            put_row(v_pool, cache_dtype, pool_off, v, src_dtype, src_off, head_dim, iv);
        }
    }
    return 0;
}

void or_fp8_scales(const void *x, int src_dtype, const int64_t *cu_seqlens, int num_seqs,
                   int num_kv_heads, int head_dim, float *scales) {
    for (int n = 0; n < num_seqs; ++n) {
        for (int h = 0; h < num_kv_heads; ++h) {
            float amax = 0.0f;
            for (int64_t t = cu_seqlens[n]; t < cu_seqlens[n + 1]; ++t) {
                int64_t off = (t * num_kv_heads + h) * (int64_t)head_dim;
                for (int d = 0; d < head_dim; ++d) amax = fmaxf(amax, fabsf(load_elt(x, src_dtype, off + d)));
            }
            scales[(int64_t)n * num_kv_heads + h] = amax > 0.0f ? amax / 448.0f : 1.0f;
        }
    }
}

/* ------------------------------------------------------------------ gather */

int64_t or_gather(const void *pool, int dtype, const int32_t *block_table, int64_t max_blocks,
                  int64_t ctx_len, void *out, int num_kv_heads, int head_dim, int block_size) {
    size_t es = elt_size(dtype);
    int64_t kv_block_stride = (int64_t)block_size * num_kv_heads * head_dim;
    for (int64_t t = 0; t < ctx_len; ++t) {
        int64_t tile = t / block_size;
        if (tile >= max_blocks) return t;
        int32_t blk = block_table[tile];
        if (blk < 0) return t; /* sentinel ends the walk, paged_attention.cu:66-67 */
        for (int h = 0; h < num_kv_heads; ++h) {
            int64_t off = (int64_t)blk * kv_block_stride + (int64_t)h * block_size * head_dim +
                          (t % block_size) * head_dim;
            memcpy((char *)out + ((t * num_kv_heads + h) * (int64_t)head_dim) * es,
                   (const char *)pool + off * es, head_dim * es);
        }
    }
    return ctx_len;
}

/* -------------------------------------------------------------- copy_blocks */

void or_copy_blocks(void *const *pools, int n_pools, int64_t block_bytes, const int32_t *src,
                    const int32_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        for (int p = 0; p < n_pools; ++p)
            memcpy((char *)pools[p] + (int64_t)dst[i] * block_bytes,
                   (const char *)pools[p] + (int64_t)src[i] * block_bytes, (size_t)block_bytes);
}

/* ------------------------------------------------------------------ decode */

/* One (seq, q-head) row: softmax(q K^T * scale) V over the seq's pages.
 * Score, max, exp-sum, normalise, weighted sum: attention/mod.rs:64-98 with
 * n_pos query rows reduced to the single decode row. */
static void decode_row(const float *q, const void *k_pool, const void *v_pool, int dt, float ks,
                       float vs, const int32_t *bt, int64_t max_blocks, int64_t ctx, int kvh,
                       int num_kv_heads, int head_dim, int block_size, float scale, float *out,
                       float *scores, float *vbuf) {
    int64_t kv_block_stride = (int64_t)block_size * num_kv_heads * head_dim;
    int64_t n = 0;
    for (int64_t j = 0; j < ctx; ++j) {
        int64_t tile = j / block_size;
        if (tile >= max_blocks || bt[tile] < 0) break; /* sentinel, paged_attention.cu:66-67 */
        int64_t off = (int64_t)bt[tile] * kv_block_stride + (int64_t)kvh * block_size * head_dim +
                      (j % block_size) * head_dim;
        float dot = 0.0f;
        for (int d = 0; d < head_dim; ++d) {
            float kd = load_elt(k_pool, dt, off + d);
            if (dt == OR_FP8_E4M3) kd = kd * ks;
            dot += q[d] * kd;
        }
        scores[j] = dot * scale;
        for (int d = 0; d < head_dim; ++d) {
            float vd = load_elt(v_pool, dt, off + d);
            if (dt == OR_FP8_E4M3) vd = vd * vs;
            vbuf[j * head_dim + d] = vd;
        }
        n = j + 1;
    }
    if (n == 0) { /* empty context: defined as a zero row */
        for (int d = 0; d < head_dim; ++d) out[d] = 0.0f;
        return;
    }
    float mx = -INFINITY;
    for (int64_t j = 0; j < n; ++j) mx = fmaxf(mx, scores[j]);
    float sum = 0.0f;
    for (int64_t j = 0; j < n; ++j) sum += expf(scores[j] - mx);
    for (int64_t j = 0; j < n; ++j) scores[j] = expf(scores[j] - mx) / sum;
    for (int d = 0; d < head_dim; ++d) {
        float acc = 0.0f;
        for (int64_t j = 0; j < n; ++j) acc += scores[j] * vbuf[j * head_dim + d];
        out[d] = acc;
    }
}

int or_paged_decode(const float *q, const void *k_pool, const void *v_pool, int kv_dtype,
                    const float *k_scales, const float *v_scales, const int32_t *block_tables,
                    int64_t max_blocks, const int32_t *seq_lens, int num_seqs, int num_heads,
                    int num_kv_heads, int head_dim, int block_size, float scale, int mapping,
                    float *out, int threads) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return -1;
    int64_t max_ctx = 0;
    for (int n = 0; n < num_seqs; ++n) if (seq_lens[n] > max_ctx) max_ctx = seq_lens[n];
    int group = num_heads / num_kv_heads;
    int64_t rows = (int64_t)num_seqs * num_heads;
    int err = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)(max_ctx + 1));
        float *vbuf = (float *)malloc(sizeof(float) * (size_t)(max_ctx + 1) * head_dim);
        if (!scores || !vbuf) {
            err = -2;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
            for (int64_t r = 0; r < rows; ++r) {
                int n = (int)(r / num_heads), h = (int)(r % num_heads);
                int kvh = mapping == OR_GQA_GROUPED ? h / group : h % num_kv_heads;
                float ks = k_scales ? k_scales[(int64_t)n * num_kv_heads + kvh] : 1.0f;
                float vs = v_scales ? v_scales[(int64_t)n * num_kv_heads + kvh] : 1.0f;
                decode_row(q + r * head_dim, k_pool, v_pool, kv_dtype, ks, vs,
                           block_tables + (int64_t)n * max_blocks, max_blocks, seq_lens[n], kvh,
                           num_kv_heads, head_dim, block_size, scale, out + r * head_dim, scores,
                           vbuf);
            }
        }
        free(scores);
        free(vbuf);
    }
    (void)threads;
    return err;
}

/* Chunked-prefill attention over pages: sequence n's chunk has query rows
 * cu_seqlens_q[n] .. cu_seqlens_q[n+1]; chunk row t sits at absolute position
 * start_pos[n] + t, and the chunk's own K/V are already in the pages.  Causal:
 * row t attends to positions [0, start + t] -- the per-element mask of
 * attention.cu:117-121 (k_pos > q_pos is excluded) carried over to a chunk
 * after `start` cached tokens.  Non-causal: every row attends to
 * [0, start + len), like CpuAttention::forward (attention/mod.rs:64-98).  Each
 * row is the decode row above with that many context tokens. */
int or_paged_prefill(const float *q, const void *k_pool, const void *v_pool, int kv_dtype,
                     const float *k_scales, const float *v_scales, const int32_t *block_tables,
                     int64_t max_blocks, const int64_t *cu_seqlens_q, const int32_t *start_pos, int num_seqs,
                     int num_heads, int num_kv_heads, int head_dim, int block_size, float scale, int mapping,
                     int causal, float *out, int threads) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return -1;
    int64_t max_ctx = 0;
    for (int n = 0; n < num_seqs; ++n) {
        int64_t c = start_pos[n] + (cu_seqlens_q[n + 1] - cu_seqlens_q[n]);
        if (c > max_ctx) max_ctx = c;
    }
    int group = num_heads / num_kv_heads;
    int64_t rows = cu_seqlens_q[num_seqs] * num_heads;
    int err = 0;
#ifdef _OPENMP
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
    {
        float *scores = (float *)malloc(sizeof(float) * (size_t)(max_ctx + 1));
        float *vbuf = (float *)malloc(sizeof(float) * (size_t)(max_ctx + 1) * head_dim);
        if (!scores || !vbuf) {
            err = -2;
        } else {
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
            for (int64_t r = 0; r < rows; ++r) {
                int64_t tok = r / num_heads;
                int h = (int)(r % num_heads);
                int n = 0;
                while (cu_seqlens_q[n + 1] <= tok) ++n;
                int64_t t = tok - cu_seqlens_q[n];
                int64_t len = cu_seqlens_q[n + 1] - cu_seqlens_q[n];
                int64_t ctx = causal ? start_pos[n] + t + 1 : start_pos[n] + len;
                int kvh = mapping == OR_GQA_GROUPED ? h / group : h % num_kv_heads;
                float ks = k_scales ? k_scales[(int64_t)n * num_kv_heads + kvh] : 1.0f;
                float vs = v_scales ? v_scales[(int64_t)n * num_kv_heads + kvh] : 1.0f;
                decode_row(q + r * head_dim, k_pool, v_pool, kv_dtype, ks, vs,
                           block_tables + (int64_t)n * max_blocks, max_blocks, ctx, kvh, num_kv_heads, head_dim,
                           block_size, scale, out + r * head_dim, scores, vbuf);
            }
        }
        free(scores);
        free(vbuf);
    }
    (void)threads;
    return err;
}

/* --------------------------------------------------- dense CPU attention */

int or_cpu_attention(const float *query, const float *key, const float *value, int num_seqs,
                     int num_heads, int head_dim, int max_seq_len, float *output) {
    int n_pos = max_seq_len, d_head = head_dim;
    float scale = 1.0f / sqrtf((float)d_head); /* attention/mod.rs:53 */
    float *scores = (float *)malloc(sizeof(float) * (size_t)n_pos * n_pos + 1);
    if (!scores) return -2;
    for (int s = 0; s < num_seqs; ++s)
        for (int h = 0; h < num_heads; ++h) {
            int64_t base = ((int64_t)(s * num_heads + h) * n_pos) * d_head;
            const float *q = query + base, *k = key + base, *v = value + base;
            float *out = output + base;
            for (int i = 0; i < n_pos; ++i)
                for (int j = 0; j < n_pos; ++j) {
                    float dot = 0.0f;
                    for (int d = 0; d < d_head; ++d) dot += q[i * d_head + d] * k[j * d_head + d];
                    scores[i * n_pos + j] = dot * scale;
                }
            for (int i = 0; i < n_pos; ++i) {
                float mx = -INFINITY;
                for (int j = 0; j < n_pos; ++j) mx = fmaxf(mx, scores[i * n_pos + j]);
                float sum = 0.0f;
                for (int j = 0; j < n_pos; ++j) sum += expf(scores[i * n_pos + j] - mx);
                for (int j = 0; j < n_pos; ++j) scores[i * n_pos + j] = expf(scores[i * n_pos + j] - mx) / sum;
            }
            for (int i = 0; i < n_pos; ++i)
                for (int d = 0; d < d_head; ++d) {
                    float acc = 0.0f;
                    for (int j = 0; j < n_pos; ++j) acc += scores[i * n_pos + j] * v[j * d_head + d];
                    out[i * d_head + d] = acc;
                }
        }
    free(scores);
    return 0;
}

void or_matmul(const float *a, const float *b, int m, int k, int n, float *c) {
    for (int i = 0; i < m * n; ++i) c[i] = 0.0f;
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j)
            for (int inner = 0; inner < k; ++inner) c[i * n + j] += a[i * k + inner] * b[inner * n + j];
}

void or_repeat_interleave_kv(const float *src, int kv_heads, int num_heads, int seq_len,
                             int head_dim, float *out) {
    for (int head = 0; head < num_heads; ++head) {
        int kh = head % kv_heads;
        for (int pos = 0; pos < seq_len; ++pos)
            for (int dim = 0; dim < head_dim; ++dim)
                out[(head * seq_len + pos) * head_dim + dim] = src[(pos * kv_heads + kh) * head_dim + dim];
    }
}

/* ------------------------------------------------------------ dense ops
 * rms_norm.cu:4-55: var = sum x^2 over the row; rms = rsqrt(var / dim + eps);
 * out = x * rms * w.  The sum runs in index order (the kernel's tree order
 * differs by rounding only). */
void or_rms_norm(const float *x, const float *w, float *out, int64_t rows, int64_t dim, float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        const float *xr = x + r * dim;
        float var = 0.0f;
        for (int64_t i = 0; i < dim; ++i) var += xr[i] * xr[i];
        const float rms = 1.0f / sqrtf(var / (float)dim + eps);
        for (int64_t i = 0; i < dim; ++i) out[r * dim + i] = xr[i] * rms * w[i];
    }
}

/* activation.cu:4-12: out = (g / (1 + exp(-g))) * u. */
void or_silu_gate_mul(const float *gate, const float *up, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = gate[i];
        out[i] = (g / (1.0f + expf(-g))) * up[i];
    }
}

/* activation.cu:14-20. */
void or_add(const float *a, const float *b, float *out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* embedding.cu:4-22: out[t] = table[ids[t]] (ids must be in range). */
void or_embedding(const int64_t *ids, const float *table, float *out, int64_t n, int64_t dim) {
    for (int64_t t = 0; t < n; ++t)
        for (int64_t i = 0; i < dim; ++i) out[t * dim + i] = table[ids[t] * dim + i];
}


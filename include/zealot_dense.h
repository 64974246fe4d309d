/*
 * zealot_dense.h -- C ABI of the dense ops around the paged-KV path (gfx950):
 * the elementwise / normalisation kernels and projections of a Llama layer
 * that the reference runner launches around its KV calls
 * (src/cuda_runner.rs:287-660).  Asynchronous on `stream`; shapes are checked
 * on the host first and nothing is launched when a check fails.  Tensors are
 * row-major, f32 or bf16 (zk_dtype of zealot_kv.h) with f32 arithmetic.
 */
#ifndef ZEALOT_DENSE_H
#define ZEALOT_DENSE_H

#include "zealot_kv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RMSNorm (attention/kernels/rms_norm.cu:4-55):
 *   out[i] = s[r] * rsqrt(mean(s[r]^2) + eps) * weight
 * over rows r = rows ? rows[i] : i (i < num_rows), with s = x, or, when
 * `residual` is given, s = x + residual (the reference's add_kernel,
 * activation.cu:14-20, fused in) written to residual_out[i] (which may be
 * `residual` itself).  dim <= 32768 (bf16) / 16384 (f32) for 16-byte rows,
 * <= 4096 otherwise.  out / residual_out are packed [num_rows, dim]; out may
 * be x when rows is NULL. */
int zk_rms_norm(const void *x, const void *residual, const void *weight, void *out,
                void *residual_out, const int64_t *rows, int64_t num_rows, int64_t dim, float eps,
                zk_dtype dtype, void *stream);

/* silu_gate_mul (activation.cu:4-12): out[r, c] = silu(gate[r, c]) * up[r, c]
 * with silu(g) = g / (1 + exp(-g)); gate / up rows are gate_stride /
 * up_stride elements apart (0 = cols), so the halves of a fused gate|up
 * projection [rows, 2 * cols] feed it in place. */
int zk_silu_mul(const void *gate, const void *up, void *out, int64_t rows, int64_t cols,
                int64_t gate_stride, int64_t up_stride, zk_dtype dtype, void *stream);

/* add_kernel (activation.cu:14-20): out = a + b over n elements. */
int zk_add(const void *a, const void *b, void *out, int64_t n, zk_dtype dtype, void *stream);

/* embedding_gather_kernel (embedding.cu:4-22): out[t] = table[ids[t]]
 * (ids: device int64 [num_tokens]); an id outside [0, vocab) gives a zero row
 * (the reference reads out of bounds). */
int zk_embedding(const int64_t *ids, const void *table, void *out, int64_t num_tokens, int64_t vocab,
                 int64_t dim, zk_dtype dtype, void *stream);

/* Projection y[m, n] = x[m, k] . w[n, k]^T (w in nn.Linear layout), the
 * product of every cublasSgemm_v2 site (attention/cublas.rs:72-114;
 * cuda_runner.rs:331-369, :483-495, :531-559, :577-589, :627-639), with
 * f32 accumulation, on hipBLASLt or (bf16, m <= 64) on this library's
 * weight-streaming kernel (zk_linear_skinny): the fastest is chosen per shape
 * (see zk_linear_tuning).  in_dtype F32 -> out F32; in_dtype BF16 ->
 * out BF16 or F32 (e.g. f32 logits).  Each (device, stream) has its own
 * workspaces (up to 8 streams a device; a ninth replaces the least recently
 * used one after a device synchronization), so calls on different streams
 * may overlap. */
int zk_linear(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, zk_dtype in_dtype,
              zk_dtype out_dtype, void *stream);
/* No counterpart in the reference: the weight-streaming kernel zk_linear's
 * tuning may pick for bf16 products with m <= 64, called directly (for
 * tests, and callers that want it without tuning).  x, w bf16, y f32 or bf16,
 * all 16-byte aligned.  Workgroups own tile_rows (64 or 128) weight rows and
 * k / splits of k: needs n % tile_rows == 0, k % (128 * splits) == 0,
 * splits <= 64 and splits * m * n * 4 <= 32 MiB.  With splits > 1 the
 * ranges' sums are added in range order by a second kernel (the result does
 * not depend on scheduling), in the stream's own workspace as for
 * zk_linear. */
int zk_linear_skinny(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, zk_dtype out_dtype,
                     int tile_rows, int splits, void *stream);
/* No counterpart in the reference (which launches its GEMM, add_kernel and
 * rms_norm_kernel one after the other, cuda_runner.rs:483-529): the
 * projection y = x . w^T (bf16, as zk_linear) followed by
 * zk_rms_norm(y, residual, norm_weight, out, residual_out, NULL rows), bit for
 * bit, with y itself not kept.  When zk_linear's tuning finds the
 * weight-streaming kernel with split k as fast as its choice, to within the
 * launch this saves, the norm kernel adds the split-k sums as it reads its
 * rows (two launches instead of three); otherwise the projection writes `out`
 * and the norm runs in place.  residual_out may be residual; dim n % 8 == 0
 * and <= 32768 for the fused form. */
int zk_linear_rms_norm(const void *x, const void *w, int64_t m, int64_t n, int64_t k, const void *residual,
                       const void *norm_weight, float eps, void *out, void *residual_out, void *stream);
/* No counterpart in the reference (which launches gate and up sgemms and
 * silu_gate_mul_kernel, cuda_runner.rs:531-571): act[m, inter] = silu(gate) *
 * up for x[m, k] (bf16) against w[2 inter, k] whose rows hold gate and up
 * interleaved in blocks of 16 -- rows 32 b .. 32 b + 15 are gate rows
 * 16 b .. 16 b + 15, the next 16 the up rows of the same columns -- bit for
 * bit zk_linear(x, w) followed by SiLU * up of the rounded outputs.  When
 * zk_linear's tuning keeps the weight-streaming kernel with 128-row tiles and
 * no split for (m, 2 inter, k), that kernel's waves hold the gate and up
 * outputs of the same columns and write act directly (one launch); otherwise
 * the projection goes to gu [m, 2 inter] (bf16, always required: the tuning
 * also writes there) and a second kernel forms act.  inter % 16 == 0. */
int zk_linear_silu_mul(const void *x, const void *w, void *act, int64_t m, int64_t inter, int64_t k, void *gu,
                       void *stream);
/* No counterpart in the reference: what zk_linear's plan for (m, n, k,
 * dtypes) on the current device runs, once a call has made it:
 * choice = {splits, tile_rows, fused_splits, fused_rows}; splits 0 means
 * hipBLASLt, else the weight-streaming kernel with that split of k and
 * tile; fused_* is what zk_linear_rms_norm runs (fused_splits 0: the
 * projection as zk_linear, then the norm). */
int zk_linear_choice(int64_t m, int64_t n, int64_t k, zk_dtype in_dtype, zk_dtype out_dtype, int choice[4]);

/* Tiled weights.  No counterpart in the reference, whose weights stay in
 * nn.Linear layout for cuBLAS (model_loader.rs:241, cuda_runner.rs:331-639):
 * the layout the weight-streaming kernel reads with contiguous 1 KiB loads,
 * [k / 128][n / 16][16 rows][16 units of 8 bf16], unit u of row r holding
 * columns 8 (u ^ r) .. 8 (u ^ r) + 7 of its 128-column chunk.  A model
 * converts its large decode-time weights once at load; the products below
 * read them 17-19 % faster than row-major weights on the Llama-3-8B
 * gate|up and lm_head shapes, bit for bit the same results as the
 * weight-streaming kernel on the row-major weights (same configuration).
 * The tiled products run on that kernel only (no hipBLASLt), for any m: up
 * to 64 rows of x per pass over the weights, so they suit decode-sized m.
 * All operands 16-byte aligned. */
/* wt = row-major bf16 w [n, k] tiled; n % 16 == 0, k % 128 == 0, w and wt
 * must not overlap. */
int zk_weight_tile(const void *w, void *wt, int64_t n, int64_t k, void *stream);
/* zk_linear for bf16 x and tiled weights (y bf16 or f32): the fastest
 * configuration of the weight-streaming kernel (tile rows, split of k) is
 * timed on first use of (m, n, k, out_dtype) as zk_linear times its
 * candidates.  Needs n % 64 == 0 and k % 128 == 0. */
int zk_linear_tiled(const void *x, const void *wt, void *y, int64_t m, int64_t n, int64_t k, zk_dtype out_dtype,
                    void *stream);
/* zk_linear_rms_norm (same arguments, bf16) for tiled weights. */
int zk_linear_rms_norm_tiled(const void *x, const void *wt, int64_t m, int64_t n, int64_t k, const void *residual,
                             const void *norm_weight, float eps, void *out, void *residual_out, void *stream);
/* zk_linear_silu_mul for the tiled form of the interleaved gate|up weight
 * [2 inter, k]: always one launch (the kernel's 128-row tiles hold gate and
 * up of the same columns), so no projection buffer; inter % 64 == 0. */
int zk_linear_silu_mul_tiled(const void *x, const void *wt, void *act, int64_t m, int64_t inter, int64_t k,
                             void *stream);
/* zk_linear_choice for the plan zk_linear_tiled / zk_linear_rms_norm_tiled
 * made for (m, n, k, out_dtype): {splits, tile_rows, fused_splits,
 * fused_rows}. */
int zk_linear_tiled_choice(int64_t m, int64_t n, int64_t k, zk_dtype out_dtype, int choice[4]);

/* No counterpart in the reference.  Pins the split-k configuration that
 * zk_linear_rms_norm[_tiled] and zk_cache_write_batch_qkv fold for the plan
 * an earlier call made for (m, n, k, dtypes; tiled: the tiled plan):
 * fused_splits > 1 ranges of k over tiles of fused_rows weight rows, or
 * fused_splits 0 for none (the projection, then its consumer).  For callers
 * that fix a configuration they measured, and for tests that must run the
 * folded kernels whatever the tuning chose.  ZK_ERR_INVALID_ARGUMENT if no
 * plan exists yet or the configuration does not fit the shape. */
int zk_linear_pin_split(int64_t m, int64_t n, int64_t k, zk_dtype in_dtype, zk_dtype out_dtype, int tiled,
                        int fused_splits, int fused_rows);

/* On (default): the first call of each (m, n, k, dtypes) times hipBLASLt's
 * candidate algorithms on its operands (synchronizing the stream once) and
 * keeps the fastest.  Off: the heuristic's first choice, no synchronization
 * (for callers under stream capture). */
int zk_linear_tuning(int on);

#ifdef __cplusplus
}
#endif

#endif /* ZEALOT_DENSE_H */

// zk_common.h -- shared host/device helpers of the gfx950 paged-KV library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/zealot_kv.h"
#include "zk_error.h"

namespace zk {

#define ZK_HIP_CHECK(expr, ctx)                                                         \
    do {                                                                                \
        hipError_t e_ = (expr);                                                         \
        if (e_ != hipSuccess)                                                           \
            return ::zk::set_error(ZK_ERR_HIP, std::string("Internal error: ") + (ctx) + \
                                                   ": " + hipGetErrorString(e_));       \
    } while (0)

// While one exists on a thread, that thread's launches are not timed (entry
// points that must not create hipEvents, such as the no-allocation decode).
struct TimingSuspend {
    TimingSuspend();
    ~TimingSuspend();
    TimingSuspend(const TimingSuspend &) = delete;
    TimingSuspend &operator=(const TimingSuspend &) = delete;
};

// Brackets one kernel launch with hipEvents when timing is enabled
// (zk_timing_enable) and not suspended on this thread; a no-op otherwise.
class KernelTimer {
  public:
    KernelTimer(const char *name, hipStream_t stream);
    ~KernelTimer();
    KernelTimer(const KernelTimer &) = delete;
    KernelTimer &operator=(const KernelTimer &) = delete;

  private:
    const char *name_;
    hipStream_t stream_;
    hipEvent_t start_ = nullptr, stop_ = nullptr;
    bool active_ = false;
};

// zk_append with the source's token stride (elements from one token's K row
// block to the next; 0 = Hkv * D, the packed layout): K/V can be read in
// place from a fused projection output.
int append(void *k_pool, void *v_pool, zk_dtype cache_dtype, const void *k, const void *v, zk_dtype src_dtype,
           int64_t src_token_stride, const int64_t *slot_mapping, int64_t num_tokens, int num_kv_heads, int head_dim,
           int block_size, int64_t num_blocks, const float *k_scales, const float *v_scales, const int32_t *token_row,
           void *stream);
// A fused q/k/v projection's split-k sums (partial: [splits][rows][cols]
// f32, cols = qcols + 2 Hkv D) added in range order and rounded to bf16 as
// the projection's reduce kernel does: the q columns to q_out (bf16, row
// stride ldq elements), the K and V columns into the bf16 pools at
// slot_mapping[row] -- one launch for the reduce and the append.
int append_split_sums(void *k_pool, void *v_pool, const float *partial, int splits, int64_t rows, int64_t cols,
                      void *q_out, int64_t ldq, int64_t qcols, const int64_t *slot_mapping, int num_kv_heads,
                      int head_dim, int block_size, int64_t num_blocks, void *stream);
// y = x . w^T (bf16, zk_linear's plan for the shape) left as split-k sums
// when the plan keeps a weight-streaming configuration with split k beside
// its choice (the one zk_linear_rms_norm folds) and x, w, y are 16-byte
// aligned with n % 8 == 0: consume(partial, splits) then runs, still under
// the projection's lock (the sums, [splits][m][n] f32, sit in the stream's
// workspace), y is not written and *fused is set; otherwise y holds the
// product and *fused is false.
struct SplitSumsConsumer {
    virtual int operator()(const float *partial, int splits) const = 0;
};
int linear_split_sums(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, hipStream_t stream,
                      const SplitSumsConsumer &consume, bool *fused);
// Swap staging (kv_ops.hip): blocks[i] of each of the num_pools pools at
// slab + p * pool_bytes <-> staging[(i * num_pools + p) * block_bytes ...]
// (to_staging: pools -> staging, else staging -> pools).
int swap_stage(char *slab, size_t pool_bytes, size_t block_bytes, int num_pools, const int32_t *blocks, int n,
               char *staging, int64_t num_blocks, bool to_staging, hipStream_t stream);
// Internal launcher (kv_ops.hip): base[pairs[i].x] = pairs[i].y for i < n,
// offsets checked on the device against `limit`.  Used by the KV cache to
// apply a batch of block-table updates in one launch.
int scatter_i32(int32_t *base, int64_t limit, const int2 *pairs, int n, hipStream_t stream);

// Shared-prefix description for the paged decode (device arrays, see the
// Params comment in paged_decode.hip); total_shared_pages is the host-side
// sum of sg_pages, used to size the shared partitions.
struct PrefixGroups {
    const int32_t *seq_pb;      // [N] shared pages of each sequence (0: none)
    const int32_t *sg_members;  // [num_sg][32] batch indices, padded with -1
    const int32_t *sg_pages;
    int num_sg;
    long total_shared_pages;
};
// zk_paged_decode with optional shared prefixes (pg may be null), an
// optional device map from sequence to q / out row (q_rows may be null), the
// q row stride in elements (0 = H * D; out rows stay H * D apart) and, for
// callers that built the tables themselves (every entry below a length is a
// valid block id), trusted_tables: the page walk that finds the first
// invalid entry is skipped.  reuse_plan: the previous call on this workspace
// and stream had the same lengths, tables, prefix groups and shapes (another
// layer of the same step), so its work items stand and planning is skipped.
// append (fused append; bf16 MFMA shapes with trusted tables only): row n
// of append->k / ->v (bf16 [Hkv, D], row_bytes apart) is sequence n's token
// at position seq_lens[n] - 1; the decode stores it into the pools and
// attends it (that page must not be a shared-prefix page).  head_set: the
// caller's record of which queue-head set the next launch on this workspace
// uses when it reuses the plan (0 after a planning launch's successor
// flips it); null: every launch plans.  max_waves > 0 caps the persistent
// grid of the MFMA path (0: one wave per SIMD); a plan is reused only by
// launches with the same cap.
struct AppendRows {
    const void *k, *v;
    int64_t row_bytes;
};
int paged_decode(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                 void *out, const int32_t *block_tables, const int32_t *seq_lens, int num_seqs, int num_heads,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                 float scale, zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                 void *workspace, size_t workspace_bytes, void *stream, const PrefixGroups *pg,
                 const int32_t *q_rows, int64_t q_stride = 0, bool trusted_tables = false, bool reuse_plan = false,
                 const AppendRows *append = nullptr, int *head_set = nullptr, int max_waves = 0);
// Whether paged_decode can take a fused append for this shape.
bool paged_decode_fuses_append(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads);
// zk_paged_prefill with the chunk rows of sequence n given as a device
// offset and length (q_off[n], q_len[n]) instead of cu_seqlens_q; total_q is
// an upper bound of the rows; q rows are q_stride elements apart (0 = H * D).
// max_groups > 0 caps the persistent grid (two-wave workgroups; 0: two per
// CU, every SIMD), leaving SIMDs to a kernel that runs beside it.
int paged_prefill_rows(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                       void *out, const int32_t *block_tables, const int64_t *q_off, const int32_t *q_len,
                       const int32_t *start_pos, int num_seqs, int64_t total_q, int num_heads, int num_kv_heads,
                       int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks, float scale,
                       int causal, zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                       void *workspace, size_t workspace_bytes, void *stream, int64_t q_stride = 0,
                       int max_groups = 0);
// Weight-streaming product y[m, n] = x[m, k] . w[n, k]^T for bf16 x / w and
// m <= 64 (any m with tiled weights, in blocks of 64 columns), output f32 or
// bf16: workgroups own tiles of tile_rows (64 or 128) weight rows and
// k / splits of k; needs n % tile_rows == 0 and k % (128 * splits) == 0.
// With splits > 1 the ranges' sums go through `partial` (at least
// skinny_linear_partial_bytes) and are added in range order by a second
// kernel; calls sharing a workspace must not overlap.  tiled: w in the
// layout tile_weight writes, else row-major.
bool skinny_linear_ok(int64_t m, int64_t n, int64_t k, int tile_rows, int splits, bool tiled = false);
size_t skinny_linear_partial_bytes(int64_t m, int64_t n, int splits);
int skinny_linear(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, bool f32_out, int tile_rows,
                  int splits, void *partial, size_t partial_bytes, hipStream_t stream, bool reduce = true,
                  bool tiled = false);
// y = x . w^T with w's rows gate / up interleaved in blocks of 16 (n = 2 I),
// written as act[m, I] = silu(gate) * up of the bf16-rounded outputs: the
// skinny kernel with 128-row tiles and no split, bf16, m <= 64 (any m with
// tiled weights).
int skinny_linear_silu(const void *x, const void *w, void *act, int64_t m, int64_t n, int64_t k, hipStream_t stream,
                       bool tiled = false);
// wt = row-major bf16 w [n, k] in the tiled layout of the weight-streaming
// kernel: [k / 128][n / 16][16 rows][16 units of 8], unit u of row r holding
// columns 8 (u ^ r) .. of the chunk.  n % 16 == 0, k % 128 == 0, no overlap.
bool tile_weight_ok(int64_t n, int64_t k);
int tile_weight(const void *w, void *wt, int64_t n, int64_t k, hipStream_t stream);
// act[r, c] = silu(gu[r, g(c)]) * gu[r, g(c) + 16], g(c) = 32 (c / 16) + c % 16:
// SiLU * up over a [rows, 2 inter] projection output whose gate / up columns
// are interleaved in blocks of 16 (bf16, inter % 16 == 0).
int silu_mul_blocked(const void *gu, void *act, int64_t rows, int64_t inter, hipStream_t s);
// RMSNorm (with the residual add, as zk_rms_norm) of the bf16 rows
// y = bf16(sum over ranges of partial[range][row]) that skinny_linear with
// splits > 1 and reduce == false leaves in `partial` ([splits][rows][dim]
// f32): bit for bit the reduce kernel's y followed by zk_rms_norm.  bf16,
// dim % 8 == 0 and <= 32768, 16-byte aligned.
bool rms_norm_partials_ok(int64_t rows, int64_t dim);
int rms_norm_partials(const float *partial, int splits, const void *residual, const void *weight, void *out,
                      void *residual_out, int64_t rows, int64_t dim, float eps, hipStream_t s);
size_t paged_decode_workspace(int num_seqs, int num_heads, int head_dim, int max_blocks_per_seq, int block_size,
                              bool shared);
// Device address of the current device's ZK_DECODE_SCRATCH_BYTES scratch of
// zk_paged_decode_noalloc (noalloc_scratch.hip); the first call on a device
// loads the array there.
int noalloc_scratch(void **out);
// Whether paged_decode runs shared-prefix items for this shape (otherwise pg
// is ignored and every sequence reads its whole table).
bool paged_decode_shares_prefixes(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads);
// Longest block table (pages per sequence) paged_prefill accepts.
constexpr int kPrefillMaxPages = 2048;
// Whether paged_prefill / paged_prefill_rows run this shape (the MFMA kernel's
// shapes: bf16 or fp8 pools, block_size 16, head_dim 64 or 128, H/Hkv in {1,2,4,8}).
bool paged_prefill_supported(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads);

inline int elt_size(int dt) { return dt == ZK_F32 ? 4 : dt == ZK_BF16 ? 2 : 1; }
inline bool valid_dtype(int dt) { return dt == ZK_F32 || dt == ZK_BF16 || dt == ZK_FP8_E4M3; }

// ----------------------------------------------------------- device helpers
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// bf16 <-> f32.  A bf16 value is the high half of the f32 with the same value.
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;                 // round to nearest even
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Exclusive prefix sum of one int per thread over a 1024-thread workgroup:
// a shuffle scan inside each of the 16 waves, then the wave totals through
// `wsum` (16 ints of LDS) after one barrier.  Every thread must call it.
// Returns the sum of the values of the threads before this one; *total gets
// the sum over the workgroup.
__device__ __forceinline__ int block_exclusive_scan_1024(int v, int *wsum, int *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o);
        if (lane >= o) incl += u;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int s = wsum[w];
        before += w < wave ? s : 0;
        all += s;
    }
    *total = all;
    return before + incl - v;
}

// Sum of N consecutive f32x4 over the k ranges of a split-k product:
// acc[q] = p[q] + p[plane + q] + ... in range order (the order every reduce
// of these sums uses, so results do not depend on which kernel adds them).
// The first kFoldLoads ranges are loaded before any addition, so a fold of up
// to that many ranges costs one memory round trip, not one per range.  The
// loads are unconditional (a range past `splits` re-reads range 0, a cache
// hit whose value is not used): guarded loads make the compiler wait for each
// group before the next.  The sum selects instead of adding zero, which keeps
// a -0 sum's sign.  FOLD (at most kFoldLoads) lowers the up-front loads for a
// caller that knows `splits` is small: loads past `splits` are wasted issue.
constexpr int kFoldLoads = 8;
__device__ __forceinline__ size_t fold_offset(int r, int splits, size_t plane) {
    return r < splits ? (size_t)r * plane : 0;
}
template <int N, int FOLD = kFoldLoads>
__device__ __forceinline__ void sum_ranges(const f32x4 *p, size_t plane, int splits, f32x4 (&acc)[N]) {
    f32x4 t[FOLD][N];
#pragma unroll
    for (int r = 0; r < FOLD; ++r)
#pragma unroll
        for (int q = 0; q < N; ++q) t[r][q] = p[fold_offset(r, splits, plane) + q];
#pragma unroll
    for (int q = 0; q < N; ++q) acc[q] = t[0][q];
#pragma unroll
    for (int r = 1; r < FOLD; ++r)
#pragma unroll
        for (int q = 0; q < N; ++q) acc[q] = r < splits ? acc[q] + t[r][q] : acc[q];
    for (int r = FOLD; r < splits; ++r)
#pragma unroll
        for (int q = 0; q < N; ++q) acc[q] += p[(size_t)r * plane + q];
}

// f32 -> OCP e4m3 (e4m3fn), round to nearest even, saturating at +-448, NaN
// keeps its sign as S.1111.111.  The gfx950 converter rounds in-range values
// to nearest even; clamping first makes it saturate, and NaN is patched.
__device__ __forceinline__ float clamp448(float x) { return fminf(fmaxf(x, -448.0f), 448.0f); }
__device__ __forceinline__ uint32_t nan_code(float x) {
    return (__float_as_uint(x) >> 24 & 0x80u) | 0x7fu;
}
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(a), clamp448(b), 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(c), clamp448(d), w, true);
    uint32_t r = (uint32_t)w;
    if (__builtin_expect(a != a || b != b || c != c || d != d, 0)) {
        if (a != a) r = (r & 0xffffff00u) | nan_code(a);
        if (b != b) r = (r & 0xffff00ffu) | (nan_code(b) << 8);
        if (c != c) r = (r & 0xff00ffffu) | (nan_code(c) << 16);
        if (d != d) r = (r & 0x00ffffffu) | (nan_code(d) << 24);
    }
    return r;
}
// Four e4m3 bytes -> four f32 (exact).
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float *o) {
    f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}
// Four e4m3 bytes -> four bf16 packed in two dwords, by gfx950's scaled
// converter with scale 1 (v_cvt_scalef32_pk_bf16_fp8, two values per
// instruction): exact, every e4m3 value is a bf16 value.
__device__ __forceinline__ u32x2 e4m3x4_to_bf16x4(uint32_t w) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    const bf16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
    return u32x2{__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi)};
}

}  // namespace zk

// kv_ops.hip -- KV append (slot-mapping scatter), fp8 scales, block-table
// gather and copy-on-write block copy for gfx950.
//
// All four are HBM-bound byte movers.  Each lane moves 16-byte vectors
// (global_load/store_dwordx4); a thread issues all of its loads before its
// stores so several 16-B requests per lane are in flight.
//
// Pool layout (src/kv_cache.rs:41-50): a (block, kv_head) page is block_size
// contiguous rows of head_dim elements, so a token row of one head is
// row_bytes = head_dim * elt contiguous bytes at
//   ((block * Hkv + head) * block_size + token_in_block) * row_bytes.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "zk_common.h"

using namespace zk;

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint4 ld16(const void *p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ void st16(void *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }
// Streaming (nontemporal) 16-byte accesses: every byte is touched once, so
// the hint keeps the moved data from displacing useful lines in L2 / MALL
// (measured ~12% faster than plain accesses for the chunked-prefill append).
__device__ __forceinline__ uint4 ld16_nt(const void *p) {
    const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return uint4{w[0], w[1], w[2], w[3]};
}
__device__ __forceinline__ void st16_nt(void *p, uint4 v) {
    const u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4 *>(p));
}

// ------------------------------------------------------------------ append
// Same-dtype append: one thread per 16-B chunk, chunks numbered (token, K|V,
// head, chunk) so a wavefront reads one token's contiguous K (or V) rows and
// writes whole 16-B-aligned pieces of the destination rows.  One chunk per
// thread (rather than several) keeps the most wavefronts in flight.
__global__ void __launch_bounds__(kThreads)
append_copy_kernel(const char *__restrict__ k, const char *__restrict__ v, char *__restrict__ k_pool,
                   char *__restrict__ v_pool, const int64_t *__restrict__ slots, uint32_t total,
                   uint32_t chunks_per_row, uint32_t hkv, uint32_t row_bytes, uint32_t block_size,
                   int64_t num_slots, uint64_t src_token_bytes) {
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= total) return;
    const uint32_t c = idx % chunks_per_row;
    uint32_t r = idx / chunks_per_row;
    const uint32_t h = r % hkv;
    r /= hkv;
    const uint32_t kv = r & 1u;
    const uint32_t t = r >> 1;
    const int64_t slot = slots[t];
    const size_t src_off = (size_t)t * src_token_bytes + (size_t)h * row_bytes + (size_t)c * 16;
    const uint4 data = ld16_nt((kv ? v : k) + src_off);
    if (slot < 0 || slot >= num_slots) return;
    const int64_t blk = slot / block_size, tib = slot % block_size;
    st16_nt((kv ? v_pool : k_pool) + (((size_t)blk * hkv + h) * block_size + (size_t)tib) * row_bytes +
                (size_t)c * 16,
            data);
}

// A fused q/k/v projection's split-k sums straight into the pools: y[t, c] =
// bf16(sum over ranges r, in order, of partial[r][t][c]) (the sum the
// projection's reduce kernel would store), one thread per 8 columns of a
// row; q columns [0, qcols) go to q_out (row stride ldq), the K and V
// columns (Hkv * D each, after them) to the bf16 pools at slot_mapping[t],
// bit for bit the reduce kernel followed by the append of its K / V columns.
// FOLD: ranges loaded up front (splits rounded up to 2, 4 or 8).
template <int FOLD>
__global__ void __launch_bounds__(kThreads)
append_split_sums_kernel(const float *__restrict__ partial, int splits, uint32_t rows, uint32_t cols8,
                         uint16_t *__restrict__ q_out, uint64_t ldq, uint32_t qcols, char *__restrict__ k_pool,
                         char *__restrict__ v_pool, const int64_t *__restrict__ slots, uint32_t hkv, uint32_t head_dim,
                         uint32_t block_size, int64_t num_slots) {
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= rows * cols8) return;
    const uint32_t t = idx / cols8, c = 8 * (idx % cols8);
    const size_t plane = (size_t)rows * cols8 * 8;
    const f32x4 *p = reinterpret_cast<const f32x4 *>(partial + (size_t)t * cols8 * 8 + c);
    const int64_t slot = c < qcols ? 0 : slots[t];  // loaded beside the sums
    f32x4 ab[2];
    sum_ranges<2, FOLD>(p, plane / 4, splits, ab);
    const f32x4 a = ab[0], b = ab[1];
    const uint4 v = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
    if (c < qcols) {
        st16(q_out + (size_t)t * ldq + c, v);
        return;
    }
    if (slot < 0 || slot >= num_slots) return;
    const uint32_t kc = c - qcols, kd = hkv * head_dim, kvc = kc < kd ? kc : kc - kd;
    const uint32_t h = kvc / head_dim, d = kvc % head_dim;
    const int64_t blk = slot / block_size, tib = slot % block_size;
    st16_nt((kc < kd ? k_pool : v_pool) +
                ((((size_t)blk * hkv + h) * block_size + (size_t)tib) * head_dim + d) * sizeof(uint16_t),
            v);
}

// The same copy when the chunks per row, the kv-heads, the row bytes and the
// block size are all powers of two (16-token blocks, 2^k heads, 256-byte bf16
// rows: the usual paged layout): shifts and masks instead of the divisions,
// which left the copy VALU-bound.
__global__ void __launch_bounds__(kThreads)
append_copy_pow2_kernel(const char *__restrict__ k, const char *__restrict__ v, char *__restrict__ k_pool,
                        char *__restrict__ v_pool, const int64_t *__restrict__ slots, uint32_t total, uint32_t cpr_log2,
                        uint32_t hkv_log2, uint32_t row_log2, uint32_t bs_log2, int64_t num_slots,
                        uint64_t src_token_bytes) {
    const uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= total) return;
    const uint32_t c = idx & ((1u << cpr_log2) - 1u);
    uint32_t r = idx >> cpr_log2;
    const uint32_t h = r & ((1u << hkv_log2) - 1u);
    r >>= hkv_log2;
    const uint32_t kv = r & 1u;
    const uint32_t t = r >> 1;
    const int64_t slot = slots[t];
    const size_t src_off = (size_t)t * src_token_bytes + ((size_t)h << row_log2) + (size_t)c * 16;
    const uint4 data = ld16_nt((kv ? v : k) + src_off);
    if (slot < 0 || slot >= num_slots) return;
    const uint64_t blk = (uint64_t)slot >> bs_log2, tib = (uint64_t)slot & ((1u << bs_log2) - 1u);
    const uint64_t row = (((blk << hkv_log2) + h) << bs_log2) + tib;
    st16_nt((kv ? v_pool : k_pool) + (row << row_log2) + (size_t)c * 16, data);
}

// The same copy with the work laid out by token, for power-of-two shapes
// whose token moves 64..512 16-byte chunks (K and V rows of every head: 256
// for 8 heads of 256-byte rows): a workgroup of 512 threads moves
// 512 / chunks tokens, each wave lies inside one token, so the token's slot
// is one scalar value (readfirstlane of a uniform load) and the destination
// splits into a scalar row base plus a per-lane offset fixed by threadIdx.
// Measured on C3 (64 x 512 tokens, 8 heads x 128 bf16): 49.9 vs 50.5-51.4 us
// for append_copy_pow2_kernel; one or four tokens per workgroup, or one
// thread moving a chunk of K and of V, were no faster.
constexpr int kTokenBlock = 512;
__global__ void __launch_bounds__(kTokenBlock)
append_token_kernel(const char *__restrict__ k, const char *__restrict__ v, char *__restrict__ k_pool,
                    char *__restrict__ v_pool, const int64_t *__restrict__ slots, uint32_t num_tokens,
                    uint32_t tt_log2, uint32_t cpr_log2, uint32_t hkv_log2, uint32_t row_log2, uint32_t bs_log2,
                    int64_t num_slots, uint64_t src_token_bytes) {
    const uint32_t r = threadIdx.x & ((1u << tt_log2) - 1u);
    const uint32_t t = blockIdx.x * (kTokenBlock >> tt_log2) + (threadIdx.x >> tt_log2);
    if (t >= num_tokens) return;
    const uint32_t half = tt_log2 - 1;  // K chunks of a token: Hkv * chunks per row
    const uint32_t kv = r >> half, h = (r >> cpr_log2) & ((1u << hkv_log2) - 1u), c = r & ((1u << cpr_log2) - 1u);
    const int64_t sl = slots[t];  // the same for the whole wave
    const int64_t slot = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(sl >> 32)) << 32) |
                                   (uint32_t)__builtin_amdgcn_readfirstlane((int)sl));
    const uint4 data = ld16_nt((kv ? v : k) + (size_t)t * src_token_bytes + ((size_t)(r & ((1u << half) - 1u)) << 4));
    if (slot < 0 || slot >= num_slots) return;
    const uint64_t blk = (uint64_t)slot >> bs_log2, tib = (uint64_t)slot & ((1u << bs_log2) - 1u);
    const uint64_t base = (((blk << hkv_log2) << bs_log2) + tib) << row_log2;
    st16_nt((kv ? v_pool : k_pool) + base + ((uint64_t)h << (bs_log2 + row_log2)) + (c << 4), data);
}

// Quantising append into an fp8 pool: one 16-element chunk per index; the
// source chunk is 32 B (bf16) or 64 B (f32), the destination chunk 16 B.
template <int SRC>  // ZK_BF16 or ZK_F32
__global__ void __launch_bounds__(kThreads)
append_fp8_kernel(const char *__restrict__ k, const char *__restrict__ v, uint8_t *__restrict__ k_pool,
                  uint8_t *__restrict__ v_pool, const int64_t *__restrict__ slots,
                  const float *__restrict__ k_scales, const float *__restrict__ v_scales,
                  const int32_t *__restrict__ token_row, uint32_t total, uint32_t chunks_per_row,
                  uint32_t hkv, uint32_t head_dim, uint32_t block_size, int64_t num_slots,
                  uint64_t src_token_elems) {
    uint32_t idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= total) return;
    uint32_t c = idx % chunks_per_row;
    uint32_t r = idx / chunks_per_row;
    uint32_t h = r % hkv;
    r /= hkv;
    uint32_t kv = r & 1u;
    uint32_t t = r >> 1;
    int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) return;
    float s = (kv ? v_scales : k_scales)[(size_t)token_row[t] * hkv + h];
    float inv = 1.0f / s;  // IEEE division, identical to the host's
    size_t elem = (size_t)t * src_token_elems + (size_t)h * head_dim + (size_t)c * 16;
    float x[16];
    if (SRC == ZK_BF16) {
        const char *src = (kv ? v : k) + elem * 2;
        uint4 a = ld16_nt(src), b = ld16_nt(src + 16);
        uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[2 * i] = bf16lo(w[i]);
            x[2 * i + 1] = bf16hi(w[i]);
        }
    } else {
        const char *src = (kv ? v : k) + elem * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint4 a = ld16_nt(src + 16 * i);
            x[4 * i] = __uint_as_float(a.x);
            x[4 * i + 1] = __uint_as_float(a.y);
            x[4 * i + 2] = __uint_as_float(a.z);
            x[4 * i + 3] = __uint_as_float(a.w);
        }
    }
    uint4 o;
    o.x = e4m3x4(x[0] * inv, x[1] * inv, x[2] * inv, x[3] * inv);
    o.y = e4m3x4(x[4] * inv, x[5] * inv, x[6] * inv, x[7] * inv);
    o.z = e4m3x4(x[8] * inv, x[9] * inv, x[10] * inv, x[11] * inv);
    o.w = e4m3x4(x[12] * inv, x[13] * inv, x[14] * inv, x[15] * inv);
    int64_t blk = slot / block_size, tib = slot % block_size;
    uint8_t *dst = (kv ? v_pool : k_pool) +
                   (((size_t)blk * hkv + h) * block_size + (size_t)tib) * head_dim + (size_t)c * 16;
    st16_nt(dst, o);
}

// Element-wise append for shapes whose rows are not 16-B multiples and for
// f32<->bf16 conversion on the way into the pool.
__global__ void __launch_bounds__(kThreads)
append_elem_kernel(const void *__restrict__ k, const void *__restrict__ v, void *__restrict__ k_pool,
                   void *__restrict__ v_pool, int src_dt, int cache_dt,
                   const int64_t *__restrict__ slots, const float *__restrict__ k_scales,
                   const float *__restrict__ v_scales, const int32_t *__restrict__ token_row,
                   uint64_t total, uint32_t hkv, uint32_t head_dim, uint32_t block_size,
                   int64_t num_slots, uint64_t src_token_elems) {
    uint64_t idx = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (idx >= total) return;
    uint64_t d = idx % head_dim;
    uint64_t r = idx / head_dim;
    uint64_t h = r % hkv;
    r /= hkv;
    uint32_t kv = (uint32_t)(r & 1u);
    uint64_t t = r >> 1;
    int64_t slot = slots[t];
    if (slot < 0 || slot >= num_slots) return;
    uint64_t src_i = t * src_token_elems + h * head_dim + d;
    const void *src = kv ? v : k;
    int64_t blk = slot / block_size, tib = slot % block_size;
    uint64_t dst_i = (((uint64_t)blk * hkv + h) * block_size + (uint64_t)tib) * head_dim + d;
    void *pool = kv ? v_pool : k_pool;
    if (src_dt == cache_dt) {
        if (cache_dt == ZK_F32) ((float *)pool)[dst_i] = ((const float *)src)[src_i];
        else ((uint16_t *)pool)[dst_i] = ((const uint16_t *)src)[src_i];
        return;
    }
    float x = src_dt == ZK_F32 ? ((const float *)src)[src_i]
                               : __uint_as_float((uint32_t)((const uint16_t *)src)[src_i] << 16);
    if (cache_dt == ZK_F32) {
        ((float *)pool)[dst_i] = x;
    } else if (cache_dt == ZK_BF16) {
        ((uint16_t *)pool)[dst_i] = (uint16_t)f32_to_bf16_bits(x);
    } else {
        float s = (kv ? v_scales : k_scales)[(size_t)token_row[t] * hkv + h];
        float inv = 1.0f / s;
        ((uint8_t *)pool)[dst_i] = (uint8_t)(e4m3x4(x * inv, 0.f, 0.f, 0.f) & 0xffu);
    }
}

// ------------------------------------------------------------- fp8 scales
// One workgroup per (sequence, kv head); each thread takes whole token rows
// (head_dim values) so every lane has a row's worth of loads in flight.
__global__ void __launch_bounds__(kThreads)
fp8_scales_kernel(const void *__restrict__ x, int src_dt, const int64_t *__restrict__ cu,
                  uint32_t hkv, uint32_t head_dim, float *__restrict__ scales) {
    __shared__ float red[kThreads / 64];
    const uint32_t n = blockIdx.x, h = blockIdx.y;
    const int64_t t0 = cu[n], t1 = cu[n + 1];
    const uint32_t es = src_dt == ZK_F32 ? 4 : 2;
    const bool vec = ((head_dim * es) % 16) == 0 && (((uintptr_t)x) & 15u) == 0;
    float amax = 0.0f;
    for (int64_t t = t0 + threadIdx.x; t < t1; t += kThreads) {
        const size_t off = ((size_t)t * hkv + h) * head_dim;
        if (vec) {
            const uint4 *row = reinterpret_cast<const uint4 *>((const char *)x + off * es);
            const uint32_t n16 = head_dim * es / 16;
            for (uint32_t c = 0; c < n16; ++c) {
                const uint4 w = row[c];
                const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (src_dt == ZK_F32) {
                        amax = fmaxf(amax, fabsf(__uint_as_float(ws[j])));
                    } else {
                        amax = fmaxf(amax, fabsf(bf16lo(ws[j])));
                        amax = fmaxf(amax, fabsf(bf16hi(ws[j])));
                    }
                }
            }
        } else {
            for (uint32_t d = 0; d < head_dim; ++d) {
                const float val = src_dt == ZK_F32 ? ((const float *)x)[off + d]
                                                   : __uint_as_float((uint32_t)((const uint16_t *)x)[off + d] << 16);
                amax = fmaxf(amax, fabsf(val));
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) {
        float m = red[0];
        for (int i = 1; i < kThreads / 64; ++i) m = fmaxf(m, red[i]);
        scales[(size_t)n * hkv + h] = m > 0.0f ? m / 448.0f : 1.0f;
    }
}

// ------------------------------------------------------------------ gather
// One workgroup per (page index j, sequence n).  The walk stops at the first
// table entry that is negative or >= num_blocks (paged_attention.cu:66-67),
// so page j is copied only when entries 0..j are all valid.
__global__ void __launch_bounds__(kThreads)
gather_kernel(const char *__restrict__ k_pool, const char *__restrict__ v_pool,
              const int32_t *__restrict__ bt, uint32_t max_blocks, const int32_t *__restrict__ ctx,
              const int64_t *__restrict__ out_off, char *__restrict__ k_out, char *__restrict__ v_out,
              uint32_t hkv, uint32_t row_bytes, uint32_t block_size, int64_t num_blocks, bool vec16) {
    uint32_t j = blockIdx.x, n = blockIdx.y;
    int64_t len = ctx[n];
    if ((int64_t)j * block_size >= len) return;
    const int32_t *row = bt + (size_t)n * max_blocks;
    int bad = 0;
    for (uint32_t i = threadIdx.x; i <= j; i += kThreads) {
        int32_t b = row[i];
        bad |= (b < 0) | ((int64_t)b >= num_blocks);
    }
    if (__syncthreads_or(bad)) return;
    int64_t blk = row[j];
    int64_t rem = len - (int64_t)j * block_size;
    uint32_t nt = rem < (int64_t)block_size ? (uint32_t)rem : block_size;
    size_t dst_row0 = (size_t)(out_off[n] + (int64_t)j * block_size);
    if (vec16) {
        uint32_t cpr = row_bytes >> 4;
        uint32_t total = 2u * nt * hkv * cpr;
        for (uint32_t i = threadIdx.x; i < total; i += kThreads) {
            uint32_t c = i % cpr, r = i / cpr;
            uint32_t h = r % hkv;
            r /= hkv;
            uint32_t t = r % nt, kv = r / nt;
            const char *src = (kv ? v_pool : k_pool) +
                              (((size_t)blk * hkv + h) * block_size + t) * row_bytes + (size_t)c * 16;
            char *dst = (kv ? v_out : k_out) + ((dst_row0 + t) * hkv + h) * row_bytes + (size_t)c * 16;
            st16_nt(dst, ld16_nt(src));
        }
    } else {
        uint32_t total = 2u * nt * hkv * row_bytes;
        for (uint32_t i = threadIdx.x; i < total; i += kThreads) {
            uint32_t c = i % row_bytes, r = i / row_bytes;
            uint32_t h = r % hkv;
            r /= hkv;
            uint32_t t = r % nt, kv = r / nt;
            (kv ? v_out : k_out)[((dst_row0 + t) * hkv + h) * row_bytes + c] =
                (kv ? v_pool : k_pool)[(((size_t)blk * hkv + h) * block_size + t) * row_bytes + c];
        }
    }
}

// ------------------------------------------------------------- copy blocks
constexpr int kMaxPoolsPerLaunch = 64;
struct PoolArgs {
    char *p[kMaxPoolsPerLaunch];
};

// One workgroup per (pair i, pool p): block dst[i] := block src[i].  Sources
// are read with the default cache policy: the forks of one parent copy the
// same source block, and the nontemporal hint made the re-reads of a source
// that another fork had just fetched slower (C4's copy: 76 -> 44 us with the
// default policy, every byte still read from HBM once).  The destinations are
// written once, nontemporal.
__global__ void __launch_bounds__(kThreads)
copy_blocks_kernel(PoolArgs pools, const int32_t *__restrict__ src, const int32_t *__restrict__ dst,
                   uint64_t block_bytes, int64_t num_blocks) {
    uint32_t i = blockIdx.x, p = blockIdx.y;
    int64_t s = src[i], d = dst[i];
    if (s < 0 || d < 0 || s >= num_blocks || d >= num_blocks) return;
    char *base = pools.p[p];
    const char *from = base + (size_t)s * block_bytes;
    char *to = base + (size_t)d * block_bytes;
    if ((block_bytes & 15u) == 0 && ((uintptr_t)base & 15u) == 0) {
        uint64_t n16 = block_bytes >> 4;
        uint64_t i0 = threadIdx.x;
        for (; i0 + 3 * kThreads < n16; i0 += 4 * kThreads) {
            uint4 a = ld16(from + 16 * i0), b = ld16(from + 16 * (i0 + kThreads));
            uint4 c = ld16(from + 16 * (i0 + 2 * kThreads)), e = ld16(from + 16 * (i0 + 3 * kThreads));
            st16_nt(to + 16 * i0, a);
            st16_nt(to + 16 * (i0 + kThreads), b);
            st16_nt(to + 16 * (i0 + 2 * kThreads), c);
            st16_nt(to + 16 * (i0 + 3 * kThreads), e);
        }
        for (; i0 < n16; i0 += kThreads) st16_nt(to + 16 * i0, ld16(from + 16 * i0));
    } else {
        for (uint64_t b = threadIdx.x; b < block_bytes; b += kThreads) to[b] = from[b];
    }
}

// The same copy for blocks made of whole 4 KiB pieces (every paged layout of
// 16-token blocks with 256-byte rows): one 16-byte chunk per thread, a
// workgroup per (pair, piece, pool) -- the fastest copy shape measured.
__global__ void __launch_bounds__(kThreads)
copy_blocks_piece_kernel(PoolArgs pools, const int32_t *__restrict__ src, const int32_t *__restrict__ dst,
                         uint64_t block_bytes, int64_t num_blocks, uint32_t pieces) {
    const uint32_t i = blockIdx.x / pieces, piece = blockIdx.x % pieces, p = blockIdx.y;
    const int64_t s = src[i], d = dst[i];
    if (s < 0 || d < 0 || s >= num_blocks || d >= num_blocks) return;
    char *base = pools.p[p];
    const size_t off = (size_t)piece * (16 * kThreads) + 16 * (size_t)threadIdx.x;
    st16_nt(base + (size_t)d * block_bytes + off, ld16(base + (size_t)s * block_bytes + off));
}

// Swap staging: block blocks[i] of every pool (pool p at slab + p *
// pool_bytes) <-> staging row (i * num_pools + p) * block_bytes, so one
// sequence's blocks of all layers, K and V, are one contiguous staging range
// for a single host DMA.  Workgroup (i, p); out-of-range ids are skipped.
__global__ void __launch_bounds__(kThreads)
swap_stage_kernel(char *__restrict__ slab, uint64_t pool_bytes, uint64_t block_bytes, const int32_t *__restrict__ blocks,
                  char *__restrict__ staging, int64_t num_blocks, int to_staging) {
    const uint32_t i = blockIdx.x, p = blockIdx.y, np = gridDim.y;
    const int64_t b = blocks[i];
    if (b < 0 || b >= num_blocks) return;
    char *pool = slab + (size_t)p * pool_bytes + (size_t)b * block_bytes;
    char *stage = staging + ((size_t)i * np + p) * block_bytes;
    const char *from = to_staging ? pool : stage;
    char *to = to_staging ? stage : pool;
    const uint64_t n16 = block_bytes >> 4;
    uint64_t i0 = threadIdx.x;
    for (; i0 + 3 * kThreads < n16; i0 += 4 * kThreads) {
        uint4 a = ld16_nt(from + 16 * i0), c = ld16_nt(from + 16 * (i0 + kThreads));
        uint4 d = ld16_nt(from + 16 * (i0 + 2 * kThreads)), e = ld16_nt(from + 16 * (i0 + 3 * kThreads));
        st16_nt(to + 16 * i0, a);
        st16_nt(to + 16 * (i0 + kThreads), c);
        st16_nt(to + 16 * (i0 + 2 * kThreads), d);
        st16_nt(to + 16 * (i0 + 3 * kThreads), e);
    }
    for (; i0 < n16; i0 += kThreads) st16_nt(to + 16 * i0, ld16_nt(from + 16 * i0));
}

// Streaming copy (bandwidth yardstick).
__global__ void __launch_bounds__(kThreads)
stream_copy_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst, uint64_t n16) {
    // one 16-byte chunk per thread, non-temporal both ways: the fastest of
    // the copy shapes measured on MI355X with data larger than the caches
    // (grid-stride loops with 4 chunks per lane, plain or NT, came 3-8 %
    // slower)
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n16) st16_nt(dst + i, ld16_nt(src + i));
}

// Streaming read (the read-bandwidth yardstick): persistent one-wave
// workgroups, one per CU, sweep the buffer in 8 KiB chunks interleaved over
// the waves (chunk c belongs to wave c % grid, so the whole grid advances
// through the buffer together), each wave keeping three chunks in flight by
// global_load_lds_dwordx4 (nontemporal, no VGPRs; the LDS copies are never
// read).  Measured on MI355X against one contiguous range per 256-thread
// workgroup with four 16-B register loads per lane in flight (the previous
// yardstick): 7.44 vs 7.05 TB/s on 2.5 GiB and 7.45 vs 6.69 TB/s on 4.9 GiB;
// deeper or shallower rings, 2-4 KiB chunks and 2-4 waves per CU were 1-15 %
// slower.  The tail (bytes % 8 KiB) goes through 16-byte register loads.
constexpr int kReadChunk = 8192, kReadStages = 3;
typedef __attribute__((address_space(3))) void lds_void_t;
template <int N>
__device__ __forceinline__ void read_wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__global__ void __launch_bounds__(64)
stream_read_kernel(const char *__restrict__ src, uint64_t bytes, uint32_t *__restrict__ sink) {
    constexpr int L = kReadChunk / 1024;  // loads per chunk
    __shared__ __attribute__((aligned(16))) char ring[kReadStages][kReadChunk];
    const int lane = threadIdx.x;
    const uint64_t nch = bytes / kReadChunk, step = gridDim.x;
    auto issue = [&](uint64_t c, int s) {
        const char *g = src + c * kReadChunk + lane * 16;
#pragma unroll
        for (int j = 0; j < L; ++j)
            __builtin_amdgcn_global_load_lds(g + 1024 * j, (lds_void_t *)(ring[s] + 1024 * j), 16, 0, /*NT*/ 2);
    };
    uint64_t c = blockIdx.x;
#pragma unroll
    for (int j = 0; j < kReadStages - 1; ++j)
        if (c + j * step < nch) issue(c + j * step, j);
    int s = kReadStages - 1;
    for (; c < nch; c += step, s = s == kReadStages - 1 ? 0 : s + 1) {
        if (c + (kReadStages - 1) * step < nch) {
            issue(c + (kReadStages - 1) * step, s);
            read_wait_vmcnt<(kReadStages - 1) * L>();  // chunk c has landed
        } else {
            read_wait_vmcnt<0>();
        }
    }
    // tail bytes after the whole chunks, folded into a word that is stored
    // only when it equals a value it cannot take for the yardstick's inputs
    uint32_t acc = 0;
    for (uint64_t i = nch * kReadChunk / 16 + (uint64_t)blockIdx.x * 64 + lane; i < bytes / 16; i += step * 64) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(src) + i);
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (acc == 0x9e3779b9u) sink[0] = 1u;
}

// Block-table update: one entry per thread.
__global__ void __launch_bounds__(kThreads)
scatter_i32_kernel(int32_t *__restrict__ base, int64_t limit, const int2 *__restrict__ pairs, int n) {
    int i = blockIdx.x * kThreads + threadIdx.x;
    if (i < n) {
        int2 e = pairs[i];
        if (e.x >= 0 && e.x < limit) base[e.x] = e.y;
    }
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: ") + what + ": " + hipGetErrorString(e));
    return ZK_OK;
}

}  // namespace

int zk::scatter_i32(int32_t *base, int64_t limit, const int2 *pairs, int n, hipStream_t stream) {
    if (n <= 0) return ZK_OK;
    scatter_i32_kernel<<<(n + kThreads - 1) / kThreads, kThreads, 0, stream>>>(base, limit, pairs, n);
    return check_launch("KVCache block-table update");
}

extern "C" {

int zk_append(void *k_pool, void *v_pool, zk_dtype cache_dtype, const void *k, const void *v,
              zk_dtype src_dtype, const int64_t *slot_mapping, int64_t num_tokens, int num_kv_heads,
              int head_dim, int block_size, int64_t num_blocks, const float *k_scales,
              const float *v_scales, const int32_t *token_row, void *stream) {
    return zk::append(k_pool, v_pool, cache_dtype, k, v, src_dtype, 0, slot_mapping, num_tokens, num_kv_heads,
                      head_dim, block_size, num_blocks, k_scales, v_scales, token_row, stream);
}

}  // extern "C"

int zk::append_split_sums(void *k_pool, void *v_pool, const float *partial, int splits, int64_t rows,
                          int64_t cols, void *q_out, int64_t ldq, int64_t qcols, const int64_t *slot_mapping,
                          int num_kv_heads, int head_dim, int block_size, int64_t num_blocks, void *stream) {
    if (rows <= 0) return ZK_OK;
    const int64_t kd = (int64_t)num_kv_heads * head_dim;
    if (splits < 1 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 || block_size <= 0 || num_blocks <= 0 ||
        qcols < 0 || qcols % 8 || cols != qcols + 2 * kd || ldq < qcols || rows * (cols / 8) >= (1ll << 31))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append_split_sums: bad shape");
    if (!k_pool || !v_pool || !partial || !slot_mapping || (qcols > 0 && !q_out))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append_split_sums: NULL pointer");
    if ((((uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)partial | (uintptr_t)q_out) & 15u) || (ldq % 8))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append_split_sums: unaligned operand");
    hipStream_t s = (hipStream_t)stream;
    const uint32_t cols8 = (uint32_t)(cols / 8), total = (uint32_t)(rows * cols8);
    KernelTimer timer("append", s);
    auto kernel = splits <= 2 ? append_split_sums_kernel<2>
                  : splits <= 4 ? append_split_sums_kernel<4>
                                : append_split_sums_kernel<kFoldLoads>;
    kernel<<<(total + kThreads - 1) / kThreads, kThreads, 0, s>>>(
        partial, splits, (uint32_t)rows, cols8, (uint16_t *)q_out, (uint64_t)ldq, (uint32_t)qcols, (char *)k_pool,
        (char *)v_pool, slot_mapping, (uint32_t)num_kv_heads, (uint32_t)head_dim, (uint32_t)block_size,
        num_blocks * block_size);
    return check_launch("zk_append_split_sums");
}

int zk::append(void *k_pool, void *v_pool, zk_dtype cache_dtype, const void *k, const void *v, zk_dtype src_dtype,
               int64_t src_token_stride, const int64_t *slot_mapping, int64_t num_tokens, int num_kv_heads,
               int head_dim, int block_size, int64_t num_blocks, const float *k_scales, const float *v_scales,
               const int32_t *token_row, void *stream) {
    if (!valid_dtype(cache_dtype) || (src_dtype != ZK_F32 && src_dtype != ZK_BF16))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: unsupported dtype");
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_blocks <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: bad shape");
    if (num_tokens == 0) return ZK_OK;
    if (!k_pool || !v_pool || !k || !v || !slot_mapping)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: NULL pointer");
    bool fp8 = cache_dtype == ZK_FP8_E4M3;
    if (fp8 && (!k_scales || !v_scales || !token_row))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: fp8 pool needs scales and token_row");
    if (!fp8 && (k_scales || v_scales || token_row))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: scales given for a non-fp8 pool");
    const int64_t row_elems = (int64_t)num_kv_heads * head_dim;
    if (src_token_stride == 0) src_token_stride = row_elems;
    if (src_token_stride < row_elems)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: source token stride below Hkv * D");
    hipStream_t s = (hipStream_t)stream;
    int64_t num_slots = num_blocks * block_size;
    uint32_t row_bytes = (uint32_t)head_dim * elt_size(cache_dtype);
    uint64_t total_rows = (uint64_t)num_tokens * 2 * num_kv_heads;
    const uint64_t src_token_bytes = (uint64_t)src_token_stride * elt_size(src_dtype);
    bool aligned = (((uintptr_t)k | (uintptr_t)v | (uintptr_t)k_pool | (uintptr_t)v_pool) & 15u) == 0 &&
                   (src_token_bytes % 16) == 0;
    if (aligned && cache_dtype == src_dtype && (row_bytes % 16) == 0 && total_rows * (row_bytes / 16) < (1ull << 31)) {
        uint32_t cpr = row_bytes / 16;
        uint32_t total = (uint32_t)(total_rows * cpr);
        uint32_t grid = (total + kThreads - 1) / kThreads;
        auto pow2 = [](uint64_t x) { return x > 0 && (x & (x - 1)) == 0; };
        auto log2u = [](uint64_t x) { return (uint32_t)__builtin_ctzll(x); };
        KernelTimer timer("append", s);
        const uint64_t tt = 2ull * cpr * (uint64_t)num_kv_heads;  // 16-byte chunks per token
        if (pow2(cpr) && pow2((uint64_t)num_kv_heads) && pow2(block_size) && tt >= 64 && tt <= kTokenBlock) {
            const uint64_t per = kTokenBlock / tt;
            append_token_kernel<<<(uint32_t)(((uint64_t)num_tokens + per - 1) / per), kTokenBlock, 0, s>>>(
                (const char *)k, (const char *)v, (char *)k_pool, (char *)v_pool, slot_mapping, (uint32_t)num_tokens,
                log2u(tt), log2u(cpr), log2u((uint64_t)num_kv_heads), log2u(row_bytes), log2u((uint64_t)block_size),
                num_slots, src_token_bytes);
        } else if (pow2(cpr) && pow2((uint64_t)num_kv_heads) && pow2(block_size))
            append_copy_pow2_kernel<<<grid, kThreads, 0, s>>>(
                (const char *)k, (const char *)v, (char *)k_pool, (char *)v_pool, slot_mapping, total, log2u(cpr),
                log2u((uint64_t)num_kv_heads), log2u(row_bytes), log2u((uint64_t)block_size), num_slots,
                src_token_bytes);
        else
            append_copy_kernel<<<grid, kThreads, 0, s>>>((const char *)k, (const char *)v, (char *)k_pool,
                                                         (char *)v_pool, slot_mapping, total, cpr, num_kv_heads,
                                                         row_bytes, block_size, num_slots, src_token_bytes);
        return check_launch("zk_append");
    }
    if (aligned && fp8 && (head_dim % 16) == 0 && total_rows * (head_dim / 16) < (1ull << 31)) {
        uint32_t cpr = head_dim / 16;
        uint32_t total = (uint32_t)(total_rows * cpr);
        uint32_t grid = (total + kThreads - 1) / kThreads;
        KernelTimer timer("append", s);
        if (src_dtype == ZK_BF16)
            append_fp8_kernel<ZK_BF16><<<grid, kThreads, 0, s>>>(
                (const char *)k, (const char *)v, (uint8_t *)k_pool, (uint8_t *)v_pool, slot_mapping,
                k_scales, v_scales, token_row, total, cpr, num_kv_heads, head_dim, block_size, num_slots,
                (uint64_t)src_token_stride);
        else
            append_fp8_kernel<ZK_F32><<<grid, kThreads, 0, s>>>(
                (const char *)k, (const char *)v, (uint8_t *)k_pool, (uint8_t *)v_pool, slot_mapping,
                k_scales, v_scales, token_row, total, cpr, num_kv_heads, head_dim, block_size, num_slots,
                (uint64_t)src_token_stride);
        return check_launch("zk_append");
    }
    uint64_t total = total_rows * (uint64_t)head_dim;
    uint64_t grid = (total + kThreads - 1) / kThreads;
    if (grid > 0x7fffffffull)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_append: too many tokens for one launch");
    KernelTimer timer("append", s);
    append_elem_kernel<<<(uint32_t)grid, kThreads, 0, s>>>(k, v, k_pool, v_pool, src_dtype, cache_dtype,
                                                           slot_mapping, k_scales, v_scales, token_row,
                                                           total, num_kv_heads, head_dim, block_size,
                                                           num_slots, (uint64_t)src_token_stride);
    return check_launch("zk_append");
}

int zk::swap_stage(char *slab, size_t pool_bytes, size_t block_bytes, int num_pools, const int32_t *blocks, int n,
                   char *staging, int64_t num_blocks, bool to_staging, hipStream_t stream) {
    if (n <= 0) return ZK_OK;
    if ((block_bytes & 15u) || (pool_bytes & 15u) || (((uintptr_t)slab | (uintptr_t)staging) & 15u))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap: blocks must be 16-byte multiples");
    if (num_pools <= 0 || num_pools > 65535)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: KVCache swap: bad pool count");
    KernelTimer timer(to_staging ? "swap_out" : "swap_in", stream);
    swap_stage_kernel<<<dim3((unsigned)n, (unsigned)num_pools), kThreads, 0, stream>>>(
        slab, pool_bytes, block_bytes, blocks, staging, num_blocks, to_staging ? 1 : 0);
    return check_launch("KVCache swap");
}

extern "C" {

int zk_fp8_scales(const void *x, zk_dtype src_dtype, const int64_t *cu_seqlens, int num_seqs,
                  int num_kv_heads, int head_dim, float *scales, void *stream) {
    if (src_dtype != ZK_F32 && src_dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_fp8_scales: unsupported dtype");
    if (num_seqs < 0 || num_kv_heads <= 0 || head_dim <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_fp8_scales: bad shape");
    if (num_seqs == 0) return ZK_OK;
    if (!x || !cu_seqlens || !scales)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_fp8_scales: NULL pointer");
    dim3 grid(num_seqs, num_kv_heads);
    KernelTimer timer("fp8_scales", (hipStream_t)stream);
    fp8_scales_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(x, src_dtype, cu_seqlens, num_kv_heads,
                                                                 head_dim, scales);
    return check_launch("zk_fp8_scales");
}

int zk_gather(const void *k_pool, const void *v_pool, zk_dtype dtype, const int32_t *block_tables,
              int max_blocks_per_seq, const int32_t *ctx_lens, const int64_t *out_offsets, int num_seqs,
              void *k_out, void *v_out, int num_kv_heads, int head_dim, int block_size,
              int64_t num_blocks, void *stream) {
    if (!valid_dtype(dtype))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_gather: unsupported dtype");
    if (num_seqs < 0 || max_blocks_per_seq <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_gather: bad shape");
    if (num_seqs == 0) return ZK_OK;
    if (!k_pool || !v_pool || !block_tables || !ctx_lens || !out_offsets || !k_out || !v_out)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_gather: NULL pointer");
    dim3 grid(max_blocks_per_seq, num_seqs);
    uint32_t row_bytes = (uint32_t)head_dim * elt_size(dtype);
    bool vec16 = (row_bytes % 16) == 0 &&
                 (((uintptr_t)k_pool | (uintptr_t)v_pool | (uintptr_t)k_out | (uintptr_t)v_out) & 15u) == 0;
    KernelTimer timer("gather", (hipStream_t)stream);
    gather_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(
        (const char *)k_pool, (const char *)v_pool, block_tables, max_blocks_per_seq, ctx_lens,
        out_offsets, (char *)k_out, (char *)v_out, num_kv_heads, row_bytes, block_size, num_blocks, vec16);
    return check_launch("zk_gather");
}

int zk_copy_blocks(void *const *pools, int n_pools, int64_t block_bytes, int64_t num_blocks,
                   const int32_t *src, const int32_t *dst, int64_t n, void *stream) {
    if (n < 0 || n_pools < 0 || block_bytes <= 0 || num_blocks <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_copy_blocks: bad shape");
    if (n == 0 || n_pools == 0) return ZK_OK;
    if (!pools || !src || !dst)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_copy_blocks: NULL pointer");
    if (n > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_copy_blocks: too many pairs");
    for (int p0 = 0; p0 < n_pools; p0 += kMaxPoolsPerLaunch) {
        int np = n_pools - p0 < kMaxPoolsPerLaunch ? n_pools - p0 : kMaxPoolsPerLaunch;
        PoolArgs a{};
        for (int i = 0; i < np; ++i) {
            if (!pools[p0 + i])
                return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_copy_blocks: NULL pool");
            a.p[i] = (char *)pools[p0 + i];
        }
        KernelTimer timer("copy_blocks", (hipStream_t)stream);
        const uint64_t piece = 16 * kThreads;
        bool aligned = true;
        for (int j = 0; j < np; ++j) aligned = aligned && ((uintptr_t)a.p[j] & 15u) == 0;
        if (aligned && block_bytes % piece == 0 && (uint64_t)n * (block_bytes / piece) < (1ull << 31)) {
            const uint32_t pieces = (uint32_t)(block_bytes / piece);
            copy_blocks_piece_kernel<<<dim3((uint32_t)n * pieces, np), kThreads, 0, (hipStream_t)stream>>>(
                a, src, dst, (uint64_t)block_bytes, num_blocks, pieces);
        } else {
            copy_blocks_kernel<<<dim3((uint32_t)n, np), kThreads, 0, (hipStream_t)stream>>>(
                a, src, dst, (uint64_t)block_bytes, num_blocks);
        }
        if (int rc = check_launch("zk_copy_blocks")) return rc;
    }
    return ZK_OK;
}

int zk_stream_copy(void *dst, const void *src, size_t bytes, void *stream) {
    if (bytes == 0) return ZK_OK;
    if (!dst || !src || (bytes & 15u) || (((uintptr_t)dst | (uintptr_t)src) & 15u))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_stream_copy: needs 16-B aligned pointers and size");
    uint64_t n16 = bytes / 16;
    if (n16 >= (1ull << 31) * kThreads)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_stream_copy: too large");
    uint32_t grid = (uint32_t)((n16 + kThreads - 1) / kThreads);
    KernelTimer timer("stream_copy", (hipStream_t)stream);
    stream_copy_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>((const uint4 *)src, (uint4 *)dst, n16);
    return check_launch("zk_stream_copy");
}

int zk_stream_read(const void *src, size_t bytes, uint32_t *sink, void *stream) {
    if (bytes == 0) return ZK_OK;
    if (!src || !sink || (bytes & 15u) || ((uintptr_t)src & 15u))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_stream_read: needs a 16-B aligned pointer and size, and a sink");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    KernelTimer timer("stream_read", (hipStream_t)stream);
    stream_read_kernel<<<(uint32_t)cus, 64, 0, (hipStream_t)stream>>>((const char *)src, (uint64_t)bytes, sink);
    return check_launch("zk_stream_read");
}

}  // extern "C"

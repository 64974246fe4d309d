// paged_decode.hip -- split-K paged decode attention for gfx950.
//
// One query row per (sequence, q-head) attends to the sequence's pages
// (src/attention/kernels/paged_attention.cu:13-291 computes the same thing
// with one serial thread per workgroup).  The context of every (sequence,
// kv-head) is cut into partitions of `part_pages` pages; one wavefront owns
// one partition of one kv-head and serves all G = H/Hkv query heads that share
// it, so every K/V byte is read from HBM exactly once.  Partials (running max
// m, sum l, unnormalised o) of sequences with more than one partition are
// merged by a log-sum-exp reduce kernel.
//
// Kernels
//   seq_info_kernel   effective length: the page walk stops at the first table
//                     entry that is < 0 or >= num_blocks (paged_attention.cu:66-67)
//   plan_kernel       prefix sums of partitions -> work items; resets the queue
//   decode_mfma_kernel  bf16 / fp8 pools, D in {64,128}, G in {1,2,4,8}:
//       persistent one-wave workgroups pull (sequence, partition, kv-head)
//       items from an atomic queue (no tail of short waves), stream each page
//       through LDS with global_load_lds, and run QK^T on MFMA, softmax and PV
//       on the VALU with DPP broadcasts (details at the kernel).
//   decode_generic_kernel  any dtype / D <= 256 / G <= 16 (fp32 pools):
//       one wavefront per (partition, kv-head, sequence); token-per-lane QK on
//       the VALU, readlane-broadcast PV.
//   decode_reduce_kernel  log-sum-exp merge of the partitions.
// Softmax runs in the log2 domain: scores are pre-multiplied by
// scale * log2(e) and exponentiated with exp2 (the FlashAttention trick).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <utility>

#include "zk_common.h"

using namespace zk;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// Pages per work item.  ZEALOT_DECODE_PART_PAGES (1..64) overrides; otherwise
// an item covers ~128 KiB of K+V: 16 pages of bf16 D=128, 32 of fp8 D=128.
int part_pages_env() {
    static int v = [] {
        const char *e = std::getenv("ZEALOT_DECODE_PART_PAGES");
        int p = e ? std::atoi(e) : 0;
        return p < 0 ? 0 : (p > 64 ? 64 : p);
    }();
    return v;
}
int part_pages_for(int kv_dtype, int head_dim, int block_size) {
    if (int e = part_pages_env()) return e;
    const long page_bytes = (long)block_size * head_dim * (kv_dtype == ZK_FP8_E4M3 ? 1 : 2);
    long p = (128 * 1024) / (2 * page_bytes);
    return (int)(p < 16 ? 16 : (p > 64 ? 64 : p));
}
// Smallest partition any path uses (sizes the workspace): every path uses at
// least 16 pages unless ZEALOT_DECODE_PART_PAGES asks for fewer.
int min_part_pages(int head_dim, int block_size) {
    (void)head_dim;
    (void)block_size;
    const int e = part_pages_env();
    return e ? e : 16;
}

struct Params {
    const void *q;
    const char *k_pool;
    const char *v_pool;
    void *out;
    const int32_t *bt;
    const int32_t *seq_lens;
    const float *k_scales;
    const float *v_scales;
    int32_t *eff_len;     // [N] length after the page walk
    int32_t *item_start;  // [N + 1] first work item of each sequence (MFMA path)
    int2 *item_map;       // [N * MP] work item -> (sequence, partition) (MFMA path)
    int32_t *work;        // [2] total items, queue head (MFMA path)
    float2 *ml;   // [N][H][MP] (m, l), log2 domain
    float *po;    // [N][H][MP][D]
    int num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks, part_pages, max_parts;
    int64_t num_blocks;
    float scale_log2;  // softmax scale * log2(e)
    int grouped;       // 1: kv = h / G, 0: kv = h % Hkv
    int q_f32;         // Q / out dtype: 1 f32, 0 bf16
};

__device__ __forceinline__ int qhead_of(const Params &p, int kvh, int j, int G) {
    return p.grouped ? kvh * G + j : kvh + j * p.num_kv_heads;
}

__device__ __forceinline__ float load_q(const Params &p, size_t i) {
    return p.q_f32 ? ((const float *)p.q)[i]
                   : __uint_as_float((uint32_t)((const uint16_t *)p.q)[i] << 16);
}
__device__ __forceinline__ void store_out(const Params &p, size_t i, float x) {
    if (p.q_f32) ((float *)p.out)[i] = x;
    else ((uint16_t *)p.out)[i] = (uint16_t)f32_to_bf16_bits(x);
}

__device__ __forceinline__ int num_parts_for(const Params &p, int len) {
    int pages = (len + p.block_size - 1) / p.block_size;
    return (pages + p.part_pages - 1) / p.part_pages;
}

// ------------------------------------------------------------ seq info
__global__ void __launch_bounds__(kWave) seq_info_kernel(Params p) {
    int n = blockIdx.x;
    int len = p.seq_lens[n];
    if (len < 0) len = 0;
    int cap = p.max_blocks * p.block_size;
    if (len > cap) len = cap;
    int pages = (len + p.block_size - 1) / p.block_size;
    const int32_t *row = p.bt + (size_t)n * p.max_blocks;
    int first_bad = pages;
    for (int i0 = 0; i0 < pages && first_bad == pages; i0 += 8 * kWave) {
        int32_t b[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // eight independent loads in flight per lane
            const int i = i0 + j * kWave + (int)threadIdx.x;
            b[j] = i < pages ? row[i] : 0;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = i0 + j * kWave + (int)threadIdx.x;
            if (i < pages && (b[j] < 0 || (int64_t)b[j] >= p.num_blocks)) first_bad = min(first_bad, i);
        }
        for (int o = 32; o > 0; o >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, o));
    }
    if (threadIdx.x == 0) p.eff_len[n] = min(len, first_bad * p.block_size);
}

// ------------------------------------------------------------ helpers
template <int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (f(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, N>{});
}

// Value of head H's lane inside this lane's G-lane group of its 16-lane row.
template <int G, int H>
__device__ __forceinline__ float head_bcast(float v) {
    if constexpr (G == 1) {
        return v;
    } else if constexpr (G == 2) {
        constexpr int ctl = H == 0 ? 0xA0 : 0xF5;  // quad_perm [H,H,2+H,2+H]
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctl, 0xF, 0xF, false));
    } else if constexpr (G == 4) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), H * 0x55, 0xF, 0xF, false));
    } else {
        static_assert(G == 8, "G must be 1, 2, 4 or 8");
        // ds_swizzle bit mode inside 32-lane halves: src = (lane & 0x18) | H
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x18 | (H << 5)));
    }
}

__device__ __forceinline__ float xor16(float v) {
    // ds_swizzle bit mode: src = lane ^ 16 within 32-lane halves
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (0x10 << 10)));
}
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// ------------------------------------------------------------ work plan
// A work item is (sequence, partition, kv-head).  The host picks the
// partition length (part_pages, up to kMaxItemPages) so the queue holds a few
// items per wave; plan_kernel sizes pairs from the effective lengths of
// seq_info_kernel and lists the (sequence, partition) pairs longest
// first (counting sort on the page count) so that the persistent waves, which
// take items in queue order, perform greedy longest-processing-time-first
// scheduling.  Item i is pair i / Hkv, kv-head i % Hkv.  The kernel also
// resets the queue head.
constexpr int kMaxItemPages = 1024;

__device__ __forceinline__ int pair_pages(const Params &p, int n, int k) {
    const int pages = (p.eff_len[n] + p.block_size - 1) / p.block_size;
    return max(0, min(p.part_pages, pages - k * p.part_pages));
}

__global__ void __launch_bounds__(1024) plan_kernel(Params p, int num_seqs) {
    constexpr int kBins = kMaxItemPages + 1;  // page counts 0 .. kMaxItemPages
    __shared__ int hist[2048];                // bin j = kMaxItemPages - pages (longest first)
    __shared__ int sums[1024];
    const int t = threadIdx.x;
    hist[2 * t] = 0;
    hist[2 * t + 1] = 0;
    __syncthreads();
    int local = 0;
    for (int n = t; n < num_seqs; n += 1024) {
        const int np = max(1, num_parts_for(p, p.eff_len[n]));
        local += np;
        for (int k = 0; k < np; ++k) atomicAdd(&hist[kMaxItemPages - pair_pages(p, n, k)], 1);
    }
    __syncthreads();
    // exclusive scan of the bins, two per thread (block scan of the pair sums)
    const int a = hist[2 * t], b = hist[2 * t + 1];
    sums[t] = a + b;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
        const int v = t >= o ? sums[t - o] : 0;
        __syncthreads();
        sums[t] += v;
        __syncthreads();
    }
    const int base = sums[t] - (a + b);
    __syncthreads();
    hist[2 * t] = base;
    hist[2 * t + 1] = base + a;
    const int total_pairs = sums[1023];
    __syncthreads();
    for (int n = t; n < num_seqs; n += 1024) {
        const int np = max(1, num_parts_for(p, p.eff_len[n]));
        for (int k = 0; k < np; ++k) {
            const int pos = atomicAdd(&hist[kMaxItemPages - pair_pages(p, n, k)], 1);
            p.item_map[pos] = make_int2(n, k);
        }
    }
    (void)local;
    (void)kBins;
    if (t == 0) {
        p.work[0] = total_pairs * p.num_kv_heads;  // total items
        p.work[1] = 0;                             // queue head
    }
}

// ------------------------------------------------------------ MFMA kernel
typedef __attribute__((address_space(3))) void lds_void;

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (global_load_lds_dwordx4; no VGPRs, counted by vmcnt).  Cache policy NT
// (nontemporal, aux bit 1): every K/V byte is read exactly once, and the
// streaming hint measured ~9% faster than the default policy on C2.
constexpr int kCachePolicyNT = 2;
__device__ __forceinline__ void g2l16(const void *g, lds_void *l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, kCachePolicyNT);
}
// s_waitcnt vmcnt(N) alone (gfx9 encoding: expcnt 7 and lgkmcnt 15 mean "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

template <int BYTES>
struct LdsVec;
template <>
struct LdsVec<16> { typedef u32x4 T; };
template <>
struct LdsVec<8> { typedef u32x2 T; };
template <>
struct LdsVec<4> { typedef uint32_t T; };

// Persistent split-K decode for bf16 / fp8 pools, D in {64, 128}, block_size 16,
// G = H/Hkv in {1, 2, 4, 8}.  The grid holds a fixed number of one-wave
// workgroups; each loops over work items.  Per item, the partition's pages
// stream through two LDS stages per wave: every page (K and V, 16 rows of
// D elements each) arrives by global_load_lds_dwordx4, 1 KiB contiguous per
// instruction, so the next page is in flight while this one is computed.
//   K stage layout: 16-byte chunk c of row r sits at chunk slot
//     r * CPR + (c ^ (r % CPR)), so the MFMA fragment reads (16 rows, same c)
//     hit distinct LDS banks.
//   V stage layout: natural [row][D].
// Scores: QK^T on v_mfma_f32_16x16x32_bf16 with A = K rows (tokens), B = the G
// query heads replicated over the 16 columns; lane l gets tokens 4*(l/16)+i of
// head (l%16)%G.  PV: each lane accumulates D/16 dims of all G heads for the
// four tokens 4*(l/16)+r, taking the other heads' weights by DPP/ds_swizzle
// broadcasts; each 16-lane row keeps its own online-softmax state and the
// rows merge once per item.
template <int KV, int D, int G>
__global__ void __launch_bounds__(kWave) decode_mfma_kernel(Params p) {
    constexpr int BS = 16;
    constexpr int ELT = KV == ZK_BF16 ? 2 : 1;
    constexpr int DG = D / 4;            // head dims per 16-lane row in QK
    constexpr int KK = DG / 8;           // MFMA k-steps
    constexpr int DV = D / 16;           // dims per lane in PV
    constexpr int RB = D * ELT;          // bytes per token row
    constexpr int CPR = RB / 16;         // 16-byte chunks per row
    constexpr int PAGE = BS * RB;        // bytes per (block, kv-head) page
    constexpr int LPK = PAGE / 1024;     // global_load_lds per page of K (or V)
    constexpr int LPP = 2 * LPK;         // per page, K and V
    constexpr int KBYTES = DG * ELT;     // K fragment bytes per lane per page
    constexpr int KCH = KBYTES / 16;     // ... in 16-byte chunks
    constexpr int VBYTES = DV * ELT;     // V bytes per lane per token row
    static_assert(PAGE % 1024 == 0 && KBYTES % 16 == 0, "page shape");
    typedef typename LdsVec<VBYTES>::T vrow_t;
    __shared__ __attribute__((aligned(16))) char lds[2][2][PAGE];  // [stage][K|V]
    __shared__ int32_t bids[kMaxItemPages];                         // this item's block ids

    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    const int H = p.num_heads, Hkv = p.num_kv_heads;
    const int my_head = col % G;

    // per-lane byte offsets, fixed for the whole kernel
    uint32_t kg[LPK], vg[LPK];  // global offsets inside a page
#pragma unroll
    for (int j = 0; j < LPK; ++j) {
        const int q = 64 * j + lane, row = q / CPR, c = (q % CPR) ^ (row % CPR);
        kg[j] = row * RB + c * 16;
        vg[j] = q * 16;
    }
    uint32_t kl[KCH];  // LDS offsets of this lane's K fragment chunks
#pragma unroll
    for (int f = 0; f < KCH; ++f) {
        const int row = col, c = grp * KCH + f;
        kl[f] = (row * CPR + (c ^ (row % CPR))) * 16;
    }
    const uint32_t vl = (uint32_t)((4 * grp) * RB + col * VBYTES);  // + r * RB

    const int total = p.work[0];
    int item = 0;
    if (lane == 0) item = atomicAdd(&p.work[1], 1);
    item = __builtin_amdgcn_readfirstlane(item);
    while (item < total) {
        int next = 0;
        if (lane == 0) next = atomicAdd(&p.work[1], 1);  // older than this item's page loads
        const int kvh = item % Hkv;
        const int2 np_pair = p.item_map[item / Hkv];
        const int n = np_pair.x, part = np_pair.y;
        const int len = p.eff_len[n];  // walk already cut at the first invalid entry
        const int pages = (len + BS - 1) / BS;
        const int nparts = (pages + p.part_pages - 1) / p.part_pages;
        const int page0 = part * p.part_pages;
        const int np = nparts > 0 ? min(p.part_pages, pages - page0) : 0;
        const int32_t *row = p.bt + (size_t)n * p.max_blocks;

        // Q fragment (B operand): column col -> head col % G
        bf16x8 qf[KK];
        {
            const size_t qb = ((size_t)n * H + qhead_of(p, kvh, my_head, G)) * D + (size_t)grp * DG;
            if (p.q_f32) {
                const float *qq = (const float *)p.q + qb;
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    u32x4 w;
#pragma unroll
                    for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(qq[8 * kk + 2 * j], qq[8 * kk + 2 * j + 1]);
                    qf[kk] = __builtin_bit_cast(bf16x8, w);
                }
            } else {
                const uint16_t *qq = (const uint16_t *)p.q + qb;
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) qf[kk] = *reinterpret_cast<const bf16x8 *>(qq + 8 * kk);
            }
        }
        float sl2 = p.scale_log2, vscale = 1.0f;
        if constexpr (KV == ZK_FP8_E4M3) {
            sl2 *= p.k_scales[(size_t)n * Hkv + kvh];
            vscale = p.v_scales[(size_t)n * Hkv + kvh];
        }
        for (int i0 = 0; i0 < np; i0 += 8 * kWave) {  // eight independent loads per lane per round
            int32_t b[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave + lane;
                b[j] = i < np ? row[page0 + i] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave + lane;
                if (i < np) bids[i] = b[j];
            }
        }
        wait_lgkmcnt0();  // this wave's LDS writes are visible to its own reads
        const char *kbase = p.k_pool + ((size_t)kvh * PAGE);
        const char *vbase = p.v_pool + ((size_t)kvh * PAGE);
        const size_t block_bytes = (size_t)PAGE * Hkv;

        auto issue = [&](int pi, int s) {
            const int blk = __builtin_amdgcn_readfirstlane(bids[pi]);
            const char *kp = kbase + (size_t)blk * block_bytes;
            const char *vp = vbase + (size_t)blk * block_bytes;
#pragma unroll
            for (int j = 0; j < LPK; ++j) g2l16(kp + kg[j], (lds_void *)(lds[s][0] + 1024 * j));
#pragma unroll
            for (int j = 0; j < LPK; ++j) g2l16(vp + vg[j], (lds_void *)(lds[s][1] + 1024 * j));
        };

        float o[G][DV];
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int d = 0; d < DV; ++d) o[h][d] = 0.0f;
        float m_run = -INFINITY, l_run = 0.0f;

        auto page = [&](int pi, int s) {
            if (pi + 1 < np) wait_vmcnt<LPP>();  // page pi landed, pi + 1 may still fly
            else wait_vmcnt<0>();
            uint32_t kw[KBYTES / 4];
#pragma unroll
            for (int f = 0; f < KCH; ++f) {
                const u32x4 c4 = *reinterpret_cast<const u32x4 *>(lds[s][0] + kl[f]);
#pragma unroll
                for (int j = 0; j < 4; ++j) kw[4 * f + j] = c4[j];
            }
            vrow_t vr[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) vr[r] = *reinterpret_cast<const vrow_t *>(lds[s][1] + vl + r * RB);
            wait_lgkmcnt0();
            if (pi + 2 < np) issue(pi + 2, s);  // the stage is free again

            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                u32x4 w;
                if constexpr (KV == ZK_BF16) {
                    w = u32x4{kw[4 * kk], kw[4 * kk + 1], kw[4 * kk + 2], kw[4 * kk + 3]};
                } else {
                    const u32x2 lo2 = e4m3x4_to_bf16x4(kw[2 * kk]), hi2 = e4m3x4_to_bf16x4(kw[2 * kk + 1]);
                    w = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
                }
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w), qf[kk], acc, 0, 0, 0);
            }
            const int tok0 = (page0 + pi) * BS + 4 * grp;
            float sc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[i] = (tok0 + i < len) ? acc[i] * sl2 : -INFINITY;

            float v[4][DV];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                uint32_t w[VBYTES / 4];
                __builtin_memcpy(w, &vr[r], VBYTES);
                if constexpr (KV == ZK_BF16) {
#pragma unroll
                    for (int j = 0; j < DV / 2; ++j) {
                        v[r][2 * j] = bf16lo(w[j]);
                        v[r][2 * j + 1] = bf16hi(w[j]);
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < DV / 4; ++j) e4m3x4_to_f32(w[j], &v[r][4 * j]);
                }
            }
            if (tok0 + 4 > len) {  // partial last page: stale rows must not reach O
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (tok0 + r >= len)
#pragma unroll
                        for (int d = 0; d < DV; ++d) v[r][d] = 0.0f;
            }

            const float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            const float m_new = fmaxf(m_run, mx);
            float alpha, pr[4];
            if (m_new == -INFINITY) {
                alpha = 1.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) pr[i] = 0.0f;
            } else {
                alpha = exp2_fast(m_run - m_new);
#pragma unroll
                for (int i = 0; i < 4; ++i) pr[i] = exp2_fast(sc[i] - m_new);
            }
            l_run = l_run * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
            m_run = m_new;
            static_for<G>([&](auto hc) {
                constexpr int h = decltype(hc)::value;
                const float a_h = head_bcast<G, h>(alpha);
                float ph[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) ph[r] = head_bcast<G, h>(pr[r]);
#pragma unroll
                for (int d = 0; d < DV; ++d) {
                    float x = o[h][d] * a_h;
                    x = fmaf(ph[0], v[0][d], x);
                    x = fmaf(ph[1], v[1][d], x);
                    x = fmaf(ph[2], v[2][d], x);
                    x = fmaf(ph[3], v[3][d], x);
                    o[h][d] = x;
                }
            });
        };

        if (np > 0) issue(0, 0);
        if (np > 1) issue(1, 1);
        for (int pi = 0; pi < np; pi += 2) {
            page(pi, 0);
            if (pi + 1 < np) page(pi + 1, 1);
        }

        // merge the four 16-lane rows
        float M = fmaxf(m_run, xor16(m_run));
        M = fmaxf(M, xor32(M));
        const float f = (m_run == -INFINITY) ? 0.0f : exp2_fast(m_run - M);
        float lsum = l_run * f;
        lsum += xor16(lsum);
        lsum += xor32(lsum);
        static_for<G>([&](auto hc) {
            constexpr int h = decltype(hc)::value;
            const float f_h = head_bcast<G, h>(f);
#pragma unroll
            for (int d = 0; d < DV; ++d) {
                float x = o[h][d] * f_h;
                x += xor16(x);
                x += xor32(x);
                o[h][d] = x * vscale;
            }
        });
        // lanes 0..15 hold o[h][col*DV + d]; lane h < G holds (M, lsum) of head h
        if (nparts <= 1) {
            static_for<G>([&](auto hc) {
                constexpr int h = decltype(hc)::value;
                const float l_h = head_bcast<G, h>(lsum);
                const float inv = l_h > 0.0f ? 1.0f / l_h : 0.0f;
                if (grp == 0) {
                    const size_t ob = ((size_t)n * H + qhead_of(p, kvh, h, G)) * D + (size_t)col * DV;
                    if (p.q_f32) {
#pragma unroll
                        for (int d = 0; d < DV; ++d) ((float *)p.out)[ob + d] = o[h][d] * inv;
                    } else {
#pragma unroll
                        for (int d = 0; d < DV; ++d) ((uint16_t *)p.out)[ob + d] = (uint16_t)f32_to_bf16_bits(o[h][d] * inv);
                    }
                }
            });
        } else {
            static_for<G>([&](auto hc) {
                constexpr int h = decltype(hc)::value;
                const size_t slot = ((size_t)n * H + qhead_of(p, kvh, h, G)) * p.max_parts + part;
                if (grp == 0) {
                    float *dst = p.po + slot * D + (size_t)col * DV;
#pragma unroll
                    for (int d = 0; d < DV; ++d) dst[d] = o[h][d];
                }
                if (lane == h) p.ml[slot] = make_float2(M, lsum);
            });
        }
        item = __builtin_amdgcn_readfirstlane(next);
    }
}

// ------------------------------------------------------------ generic kernel
// One wavefront per (partition, kv-head, sequence).  Lane = token for QK
// (64-token chunks), lane = dim for PV with readlane broadcasts of p.
constexpr int kMaxG = 16;
constexpr int kMaxDSlots = 4;  // D <= 256

template <int KV>
__device__ __forceinline__ float load_kv(const char *pool, size_t i) {
    if constexpr (KV == ZK_F32) return ((const float *)pool)[i];
    else if constexpr (KV == ZK_BF16) return __uint_as_float((uint32_t)((const uint16_t *)pool)[i] << 16);
    else {
        f32x2 r = __builtin_amdgcn_cvt_pk_f32_fp8((int)((const uint8_t *)pool)[i], false);
        return r[0];
    }
}

template <int KV>
__global__ void __launch_bounds__(kWave) decode_generic_kernel(Params p) {
    __shared__ float q_s[kMaxG * 256];
    const int part = blockIdx.x, kvh = blockIdx.y, n = blockIdx.z;
    const int lane = threadIdx.x;
    const int len = p.eff_len[n];
    const int nparts = num_parts_for(p, len);
    if (part >= (nparts > 0 ? nparts : 1)) return;
    const int H = p.num_heads, Hkv = p.num_kv_heads, D = p.head_dim, BS = p.block_size;
    const int G = H / Hkv;

    for (int i = lane; i < G * D; i += kWave) {
        int j = i / D, d = i % D;
        q_s[i] = load_q(p, ((size_t)n * H + qhead_of(p, kvh, j, G)) * D + d);
    }
    __syncthreads();
    float ks = 1.0f, vs = 1.0f;
    if constexpr (KV == ZK_FP8_E4M3) {
        ks = p.k_scales[(size_t)n * Hkv + kvh];
        vs = p.v_scales[(size_t)n * Hkv + kvh];
    }
    const float sl2 = p.scale_log2 * ks;

    float m[kMaxG], l[kMaxG], o[kMaxG][kMaxDSlots];
#pragma unroll
    for (int j = 0; j < kMaxG; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.0f;
#pragma unroll
        for (int c = 0; c < kMaxDSlots; ++c) o[j][c] = 0.0f;
    }
    const int t_begin = part * p.part_pages * BS;
    const int t_end = min(len, t_begin + p.part_pages * BS);
    const int32_t *btrow = p.bt + (size_t)n * p.max_blocks;
    const size_t rows_per_block = (size_t)Hkv * BS;

    for (int t0 = t_begin; t0 < t_end; t0 += kWave) {
        const int t = t0 + lane;
        const bool valid = t < t_end;
        size_t row = 0;
        if (valid) row = ((size_t)btrow[t / BS] * rows_per_block + (size_t)kvh * BS + t % BS);
        float s[kMaxG];
#pragma unroll
        for (int j = 0; j < kMaxG; ++j) s[j] = 0.0f;
        if (valid) {
            for (int d = 0; d < D; ++d) {
                float kd = load_kv<KV>(p.k_pool, row * D + d);
#pragma unroll
                for (int j = 0; j < kMaxG; ++j)
                    if (j < G) s[j] = fmaf(q_s[j * D + d], kd, s[j]);
            }
        }
        float pj[kMaxG];
#pragma unroll
        for (int j = 0; j < kMaxG; ++j) {
            if (j >= G) break;
            float sj = valid ? s[j] * sl2 : -INFINITY;
            float mx = sj;
            for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            float m_new = fmaxf(m[j], mx);  // at least one valid token: finite
            float alpha = exp2f(m[j] - m_new);
            float pv = valid ? exp2f(sj - m_new) : 0.0f;
            float ps = pv;
            for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off);
            l[j] = l[j] * alpha + ps;
            m[j] = m_new;
#pragma unroll
            for (int c = 0; c < kMaxDSlots; ++c) o[j][c] *= alpha;
            pj[j] = pv;
        }
        const int nvalid = min(kWave, t_end - t0);
        for (int i = 0; i < nvalid; ++i) {
            size_t row_i = ((size_t)(uint32_t)__builtin_amdgcn_readlane((int)(row & 0xffffffffu), i)) |
                           ((size_t)(uint32_t)__builtin_amdgcn_readlane((int)(row >> 32), i) << 32);
            float vd[kMaxDSlots];
#pragma unroll
            for (int c = 0; c < kMaxDSlots; ++c) {
                int d = lane + c * kWave;
                vd[c] = d < D ? load_kv<KV>(p.v_pool, row_i * D + d) : 0.0f;
            }
#pragma unroll
            for (int j = 0; j < kMaxG; ++j) {
                if (j >= G) break;
                float pi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj[j]), i));
#pragma unroll
                for (int c = 0; c < kMaxDSlots; ++c) o[j][c] = fmaf(pi, vd[c], o[j][c]);
            }
        }
    }

#pragma unroll
    for (int j = 0; j < kMaxG; ++j) {
        if (j >= G) break;
        const int qh = qhead_of(p, kvh, j, G);
        if (nparts <= 1) {
            const float inv = l[j] > 0.0f ? 1.0f / l[j] : 0.0f;
#pragma unroll
            for (int c = 0; c < kMaxDSlots; ++c) {
                int d = lane + c * kWave;
                if (d < D) store_out(p, ((size_t)n * H + qh) * D + d, o[j][c] * vs * inv);
            }
        } else {
            const size_t slot = ((size_t)n * H + qh) * p.max_parts + part;
#pragma unroll
            for (int c = 0; c < kMaxDSlots; ++c) {
                int d = lane + c * kWave;
                if (d < D) p.po[slot * D + d] = o[j][c] * vs;
            }
            if (lane == 0) p.ml[slot] = make_float2(m[j], l[j]);
        }
    }
}

// ------------------------------------------------------------ reduce
// One wavefront per (q-head, sequence): o = sum_p w_p o_p / sum_p w_p l_p with
// w_p = 2^(m_p - M).  Lane i owns partition i's weight; the weighted sum walks
// the partitions eight at a time so 16 loads per lane are in flight.
__global__ void __launch_bounds__(kWave) decode_reduce_kernel(Params p) {
    const int h = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const int len = p.eff_len[n];
    const int nparts = num_parts_for(p, len);
    if (nparts <= 1) return;
    const int D = p.head_dim;
    const size_t base = ((size_t)n * p.num_heads + h) * p.max_parts;
    float M = -INFINITY;
    for (int i = lane; i < nparts; i += kWave) M = fmaxf(M, p.ml[base + i].x);
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    float L = 0.0f;
    for (int i = lane; i < nparts; i += kWave) {
        const float2 v = p.ml[base + i];
        L += v.x == -INFINITY ? 0.0f : v.y * exp2f(v.x - M);
    }
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // d = lane + 64 * c, D <= 256
    for (int c0 = 0; c0 < nparts; c0 += kWave) {
        float w = 0.0f;
        if (c0 + lane < nparts) {
            const float2 v = p.ml[base + c0 + lane];
            w = v.x == -INFINITY ? 0.0f : exp2f(v.x - M);
        }
        const int cnt = min(kWave, nparts - c0);
        for (int i0 = 0; i0 < cnt; i0 += 8) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int i = i0 + u;
                if (i < cnt) {
                    const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), i));
                    const float *src = p.po + (base + c0 + i) * D;
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (lane + 64 * c < D) acc[c] = fmaf(wi, src[lane + 64 * c], acc[c]);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
        if (lane + 64 * c < D) store_out(p, ((size_t)n * p.num_heads + h) * D + lane + 64 * c, acc[c] * inv);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
    size_t eff, items, map, work, ml, po, total;
};
WsLayout ws_layout(int num_seqs, int num_heads, int head_dim, int max_parts) {
    WsLayout w;
    w.eff = 0;
    w.items = align256(sizeof(int32_t) * (size_t)num_seqs);
    w.map = w.items + align256(sizeof(int32_t) * ((size_t)num_seqs + 1));
    w.work = w.map + align256(sizeof(int2) * (size_t)num_seqs * max_parts);
    w.ml = w.work + 256;
    size_t slots = (size_t)num_seqs * num_heads * max_parts;
    w.po = w.ml + align256(sizeof(float2) * slots);
    w.total = w.po + align256(sizeof(float) * slots * head_dim);
    return w;
}

int max_parts_for(int max_blocks, int part_pages) { return (max_blocks + part_pages - 1) / part_pages; }

int waves_per_simd_config() {
    static int v = [] {
        const char *e = std::getenv("ZEALOT_DECODE_WAVES_PER_SIMD");
        int w = e ? std::atoi(e) : 1;
        return w < 1 ? 1 : (w > 8 ? 8 : w);
    }();
    return v;
}

// Persistent grid: waves_per_simd one-wave workgroups per SIMD (4 SIMDs per CU).
// Partition length for the persistent kernel: enough (sequence, partition)
// pairs for ~ZEALOT_DECODE_ITEMS_PER_WAVE (default 6) items per wave, at least
// 16 pages, at most kMaxItemPages.
int items_per_wave_config() {
    static int v = [] {
        const char *e = std::getenv("ZEALOT_DECODE_ITEMS_PER_WAVE");
        int w = e ? std::atoi(e) : 6;
        return w < 1 ? 1 : (w > 64 ? 64 : w);
    }();
    return v;
}

int persistent_grid();

int mfma_part_pages(int num_seqs, int num_kv_heads, int max_blocks) {
    if (int e = part_pages_env()) return e;
    const long waves = persistent_grid();
    const long pairs = (items_per_wave_config() * waves + num_kv_heads - 1) / num_kv_heads;
    const long per_seq = (pairs + num_seqs - 1) / num_seqs;
    long pp = (max_blocks + per_seq - 1) / per_seq;
    pp = (pp + 15) / 16 * 16;
    return (int)(pp < 16 ? 16 : (pp > kMaxItemPages ? kMaxItemPages : pp));
}

int persistent_grid() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus * 4 * waves_per_simd_config();
}

template <int KV, int D>
bool launch_mfma_g(const Params &p, int grid, hipStream_t s, int G) {
    switch (G) {
        case 1: decode_mfma_kernel<KV, D, 1><<<grid, kWave, 0, s>>>(p); return true;
        case 2: decode_mfma_kernel<KV, D, 2><<<grid, kWave, 0, s>>>(p); return true;
        case 4: decode_mfma_kernel<KV, D, 4><<<grid, kWave, 0, s>>>(p); return true;
        case 8: decode_mfma_kernel<KV, D, 8><<<grid, kWave, 0, s>>>(p); return true;
        default: return false;
    }
}

template <int KV>
bool launch_mfma(const Params &p, int grid, hipStream_t s, int G) {
    if (p.head_dim == 128) return launch_mfma_g<KV, 128>(p, grid, s, G);
    return launch_mfma_g<KV, 64>(p, grid, s, G);
}

bool mfma_supported(int kv_dtype, int head_dim, int block_size, int G) {
    return (kv_dtype == ZK_BF16 || kv_dtype == ZK_FP8_E4M3) && block_size == 16 &&
           (head_dim == 128 || head_dim == 64) && (G == 1 || G == 2 || G == 4 || G == 8);
}

int check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: ") + what + ": " + hipGetErrorString(e));
    return ZK_OK;
}

}  // namespace

extern "C" {

size_t zk_paged_decode_workspace_size(int num_seqs, int num_heads, int head_dim, int max_blocks_per_seq,
                                      int block_size) {
    if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_blocks_per_seq <= 0) return 256;
    return ws_layout(num_seqs, num_heads, head_dim,
                     max_parts_for(max_blocks_per_seq, min_part_pages(head_dim, block_size)))
        .total;
}

int zk_paged_decode(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                    zk_dtype kv_dtype, void *out, const int32_t *block_tables, const int32_t *seq_lens,
                    int num_seqs, int num_heads, int num_kv_heads, int head_dim, int block_size,
                    int max_blocks_per_seq, int64_t num_blocks, float scale, zk_gqa_mapping mapping,
                    const float *k_scales, const float *v_scales, void *workspace, size_t workspace_bytes,
                    void *stream) {
    if (q_dtype != ZK_F32 && q_dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: q dtype must be f32 or bf16");
    if (!valid_dtype(kv_dtype))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: unsupported kv dtype");
    if (num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
        max_blocks_per_seq <= 0 || num_blocks <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: bad shape");
    if (num_heads % num_kv_heads != 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: num_heads must be a multiple of num_kv_heads");
    if (mapping != ZK_GQA_GROUPED && mapping != ZK_GQA_MODULO)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: bad gqa mapping");
    const int G = num_heads / num_kv_heads;
    if (head_dim > 256 || G > kMaxG)
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: head_dim <= 256 and H/Hkv <= 16 required");
    if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: context too long");
    if (num_seqs == 0) return ZK_OK;
    if (!q || !k_pool || !v_pool || !out || !block_tables || !seq_lens || !workspace)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: NULL pointer");
    const bool fp8 = kv_dtype == ZK_FP8_E4M3;
    if (fp8 != (k_scales != nullptr && v_scales != nullptr))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: fp8 pools need k/v scales, other pools none");
    const bool use_mfma = mfma_supported(kv_dtype, head_dim, block_size, G);
    const int part_pages = use_mfma ? mfma_part_pages(num_seqs, num_kv_heads, max_blocks_per_seq)
                                    : part_pages_for(ZK_F32, head_dim, block_size);
    const int max_parts = max_parts_for(max_blocks_per_seq, part_pages);
    WsLayout w = ws_layout(num_seqs, num_heads, head_dim, max_parts);
    if (workspace_bytes < w.total || ((uintptr_t)workspace & 255u))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: workspace too small or not 256-B aligned (need " +
                             std::to_string(w.total) + " bytes)");

    Params p;
    p.q = q;
    p.k_pool = (const char *)k_pool;
    p.v_pool = (const char *)v_pool;
    p.out = out;
    p.bt = block_tables;
    p.seq_lens = seq_lens;
    p.k_scales = k_scales;
    p.v_scales = v_scales;
    char *ws = (char *)workspace;
    p.eff_len = (int32_t *)(ws + w.eff);
    p.item_start = (int32_t *)(ws + w.items);
    p.item_map = (int2 *)(ws + w.map);
    p.work = (int32_t *)(ws + w.work);
    p.ml = (float2 *)(ws + w.ml);
    p.po = (float *)(ws + w.po);
    p.num_seqs = num_seqs;
    p.num_heads = num_heads;
    p.num_kv_heads = num_kv_heads;
    p.head_dim = head_dim;
    p.block_size = block_size;
    p.max_blocks = max_blocks_per_seq;
    p.part_pages = part_pages;
    p.max_parts = max_parts;
    p.num_blocks = num_blocks;
    p.scale_log2 = scale * kLog2e;
    p.grouped = mapping == ZK_GQA_GROUPED ? 1 : 0;
    p.q_f32 = q_dtype == ZK_F32 ? 1 : 0;

    hipStream_t s = (hipStream_t)stream;
    {
        KernelTimer timer("decode_seq_info", s);
        seq_info_kernel<<<num_seqs, kWave, 0, s>>>(p);
    }
    if (int rc = check_launch("zk_paged_decode seq_info")) return rc;
    if (use_mfma) {
        {
            KernelTimer timer("decode_plan", s);
            plan_kernel<<<1, 1024, 0, s>>>(p, num_seqs);
        }
        if (int rc = check_launch("zk_paged_decode plan")) return rc;
        KernelTimer timer("decode_partials", s);
        const int grid = persistent_grid();
        if (kv_dtype == ZK_BF16) launch_mfma<ZK_BF16>(p, grid, s, G);
        else launch_mfma<ZK_FP8_E4M3>(p, grid, s, G);
    } else {
        KernelTimer timer("decode_partials", s);
        dim3 grid(max_parts, num_kv_heads, num_seqs);
        if (kv_dtype == ZK_F32) decode_generic_kernel<ZK_F32><<<grid, kWave, 0, s>>>(p);
        else if (kv_dtype == ZK_BF16) decode_generic_kernel<ZK_BF16><<<grid, kWave, 0, s>>>(p);
        else decode_generic_kernel<ZK_FP8_E4M3><<<grid, kWave, 0, s>>>(p);
    }
    if (int rc = check_launch("zk_paged_decode partials")) return rc;
    if (max_parts > 1) {
        dim3 rgrid(num_heads, num_seqs);
        KernelTimer timer("decode_reduce", s);
        decode_reduce_kernel<<<rgrid, kWave, 0, s>>>(p);
        if (int rc = check_launch("zk_paged_decode reduce")) return rc;
    }
    return ZK_OK;
}

}  // extern "C"

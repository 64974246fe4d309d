// paged_decode.hip -- split-K paged decode attention for gfx950.
//
// One query row per (sequence, q-head) attends to the sequence's pages
// (src/attention/kernels/paged_attention.cu:13-291 computes the same thing
// with one serial thread per workgroup).  The context of every (sequence,
// kv-head) is cut into partitions of `part_pages` pages; one wavefront owns
// one partition of one kv-head and serves all G = H/Hkv query heads that share
// it, so every K/V byte is read from HBM exactly once.  Sequences forked from
// one prefix (the KV cache passes their subgroups) read the shared pages once
// per subgroup as well.  Partials (running max m, sum l, unnormalised o) of
// sequences with more than one partition are merged by a log-sum-exp reduce.
//
// Kernels
//   seq_info_kernel   effective length: the page walk stops at the first table
//                     entry that is < 0 or >= num_blocks (paged_attention.cu:66-67)
//   plan_kernel       partitions -> work-item descriptors, longest first;
//                     resets the queue
//   decode_mfma_kernel  bf16 / fp8 pools, D in {64,128}, G in {1,2,4,8}:
//       persistent one-wave workgroups take (sequence or subgroup, partition,
//       kv-head) items from an atomic queue (no tail of short waves), stream
//       each page through LDS with global_load_lds, and run QK^T and PV on
//       MFMA with a lazily rescaled softmax (details at the kernel).
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

constexpr int kSgStride = 32;  // member slots per prefix subgroup (query rows of one shared item)

// Work queues of the persistent MFMA decode (Params::queues of them, 1 or
// kQueues): item i belongs to queue i % queues, and workgroup w takes its
// items from queue w % queues (with 8 queues, the XCD it runs on when
// workgroups are dispatched round-robin over the 8 XCDs).  Each head sits on
// its own 128-byte line.  One queue balances best (a global
// longest-first order); batches of shared-prefix items, many of equal length
// that finish at the same moment, use eight, so their claims go to eight
// lines instead of one, whose atomics the L2 serialises.
constexpr int kQueues = 8;
constexpr int kQueueStride = 32;  // int32 slots between heads
// Two sets of queue heads: a launch takes its items through set
// Params::head_set and puts the other set back to its start values, which
// the launch after it (same workspace, same stream) then uses; the plan
// kernel sets both.  So launches that reuse a plan (the layers of one step)
// need no kernel of their own to reset the heads.
constexpr size_t kWorkBytes = sizeof(int32_t) * kQueueStride * (2 * kQueues + 1);

struct Params {
    const void *q;        // [rows, H, D]; sequence n's row is q_rows[n] (n when q_rows is null)
    const char *k_pool;
    const char *v_pool;
    void *out;
    const int32_t *bt;
    const int32_t *seq_lens;
    const float *k_scales;
    const float *v_scales;
    const int32_t *q_rows;  // optional: q / out row of each sequence
    int64_t q_stride;       // elements between consecutive q rows (out rows: H * D)
    int trusted;            // tables hold valid ids up to every length: no page walk
    int32_t *eff_len;     // [N] length after the page walk
    int4 *items;          // [N * MP][2] work-item descriptors, longest first (MFMA path):
                          //   {n, part, first page, pages} of a sequence's own pages or
                          //   {-1 - g, part, member 0, pages} of subgroup g's shared pages,
                          //   then the block ids of the item's first kDescPages pages
    int32_t *work;        // total items at [0]; the head of queue j of set s at
                          // [kQueueStride * (1 + j + s * kQueues)] (MFMA path)
    int num_waves;        // persistent grid: wave w starts with item w
    int queues;           // work queues in use (1 or kQueues)
    int head_set;         // the set of queue heads this launch claims from (0 or 1)
    // Fused append (MFMA bf16 path; null when unused): the step's K / V row
    // of sequence n, kv-head h, at new_k / new_v + n * new_row_bytes + h * D * 2,
    // is the token at position len - 1; the item holding the sequence's last
    // page stores it into the pools and attends it from registers.
    const char *new_k;
    const char *new_v;
    int64_t new_row_bytes;
    float2 *ml;   // [N][H][MP] (m, l), log2 domain
    float *po;    // [N][H][MP][D]
    // Shared prefixes (MFMA bf16 path; all null when unused): sequence n's
    // first seq_pb[n] pages are the same blocks as every other member of its
    // prefix subgroup.  Subgroup g has members sg_members[g * kSgStride + i]
    // (batch indices, at most 32 / G, padded with -1) and sg_pages[g] shared
    // full pages.  Partial slots of a member: shared parts first, then its
    // private parts.
    const int32_t *seq_pb;
    const int32_t *sg_members;
    const int32_t *sg_pages;
    int num_sg, shared_part_pages;
    int num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks, part_pages, max_parts;
    int64_t num_blocks;
    float scale_log2;  // softmax scale * log2(e)
    int grouped;       // 1: kv = h / G, 0: kv = h % Hkv
    int q_f32;         // Q / out dtype: 1 f32, 0 bf16
};

__device__ __forceinline__ size_t qrow(const Params &p, int n) { return p.q_rows ? (size_t)p.q_rows[n] : (size_t)n; }

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
__device__ __forceinline__ int prefix_pages_of(const Params &p, int n) { return p.seq_pb ? p.seq_pb[n] : 0; }
// Partitions of sequence n's shared prefix (computed by its subgroup's items).
__device__ __forceinline__ int shared_parts_of(const Params &p, int n) {
    const int pb = prefix_pages_of(p, n);
    return pb > 0 ? (pb + p.shared_part_pages - 1) / p.shared_part_pages : 0;
}
// Partitions of the pages after the shared prefix (the sequence's own items).
__device__ __forceinline__ int private_parts_of(const Params &p, int n) {
    const int pages = (p.eff_len[n] + p.block_size - 1) / p.block_size;
    const int rest = pages - prefix_pages_of(p, n);
    return rest > 0 ? (rest + p.part_pages - 1) / p.part_pages : 0;
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
// Lane l ^ 16 / l ^ 32's value, on the VALU: v_permlane16_swap exchanges the
// odd 16-lane rows of its first operand with the even rows of its second, and
// v_permlane32_swap the upper half of the first with the lower half of the
// second; with both operands v, a lane's partner value lands in the second
// result on the even rows (lower half) and in the first elsewhere.  (Unlike
// ds_swizzle / ds_bpermute they are not LDS instructions, so they never wait
// behind outstanding LDS or scalar loads.)
__device__ __forceinline__ float xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Two f32 -> packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2_t));
}

// Lazy-rescale slack of the shared-prefix softmax, in log2 units.
constexpr float kRescaleSlack = 8.0f;

// ------------------------------------------------------------ work plan
// A work item is (sequence or prefix subgroup, partition, kv-head).  The host
// picks the partition length (part_pages, up to kMaxItemPages) so the queue
// holds a few items per wave; plan_kernel sizes pairs from the effective
// lengths of seq_info_kernel and lists them longest first (counting sort on
// the page count) as self-contained descriptors (first page and page count
// included), so that the persistent waves, which take items in queue order,
// perform greedy longest-processing-time-first scheduling and start an item
// with one descriptor load.  Item i is pair i / Hkv, kv-head i % Hkv; wave w
// takes item w first, then pulls from the queue, whose head the kernel sets.
constexpr int kMaxItemPages = 1024;
// Block ids carried in a work-item descriptor (the first pages of the item).
constexpr int kDescPages = 4;

// Pages in flight per wave in the MFMA decode (LDS stages of K + V).
#ifndef ZK_DECODE_STAGES
#define ZK_DECODE_STAGES 2
#endif
constexpr int kStages = ZK_DECODE_STAGES;

__device__ __forceinline__ int pair_pages(const Params &p, int n, int k) {
    const int pages = (p.eff_len[n] + p.block_size - 1) / p.block_size - prefix_pages_of(p, n);
    return max(0, min(p.part_pages, pages - k * p.part_pages));
}
// Items of sequence n: its private partitions; a sequence with neither shared
// nor private pages still gets one (it writes the zero row).
__device__ __forceinline__ int private_items_of(const Params &p, int n) {
    const int np = private_parts_of(p, n);
    return shared_parts_of(p, n) == 0 ? max(1, np) : np;
}
__device__ __forceinline__ int shared_pair_pages(const Params &p, int g, int k) {
    return max(0, min(p.shared_part_pages, p.sg_pages[g] - k * p.shared_part_pages));
}

// At most 64 VGPRs a lane, so that its 16 waves fit beside attention waves
// already resident (four a SIMD beside one decode or prefill wave).
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8)))
plan_kernel(Params p, int num_seqs) {
    __shared__ int hist[2048];  // bin j = kMaxItemPages - pages (longest first)
    __shared__ int wsum[16];
    const int t = threadIdx.x;
    hist[2 * t] = 0;
    hist[2 * t + 1] = 0;
    if (p.trusted) {  // the caller built the tables: the walk would reach every length
        const int cap = p.max_blocks * p.block_size;
        for (int n = t; n < num_seqs; n += 1024) p.eff_len[n] = min(max(p.seq_lens[n], 0), cap);
        __threadfence_block();
    }
    __syncthreads();
    for (int n = t; n < num_seqs; n += 1024) {
        const int np = private_items_of(p, n);
        for (int k = 0; k < np; ++k) atomicAdd(&hist[kMaxItemPages - pair_pages(p, n, k)], 1);
    }
    for (int g = t; g < p.num_sg; g += 1024) {
        const int np = (p.sg_pages[g] + p.shared_part_pages - 1) / p.shared_part_pages;
        for (int k = 0; k < np; ++k) atomicAdd(&hist[kMaxItemPages - shared_pair_pages(p, g, k)], 1);
    }
    __syncthreads();
    // exclusive scan of the bins, two per thread (each thread rewrites only
    // its own two, so no barrier between reading and writing them)
    const int a = hist[2 * t], b = hist[2 * t + 1];
    int total_pairs;
    const int base = zk::block_exclusive_scan_1024(a + b, wsum, &total_pairs);
    hist[2 * t] = base;
    hist[2 * t + 1] = base + a;
    __syncthreads();
    // an item's descriptor carries the block ids of its first pages, so the
    // decode issues them without waiting for the item's table entries
    auto first_blocks = [&](const int32_t *row, int pages) {
        int b[kDescPages];
#pragma unroll
        for (int j = 0; j < kDescPages; ++j) b[j] = j < pages ? row[j] : 0;
        return make_int4(b[0], b[1], b[2], b[3]);
    };
    for (int n = t; n < num_seqs; n += 1024) {
        const int np = private_items_of(p, n);
        for (int k = 0; k < np; ++k) {
            const int np = pair_pages(p, n, k);
            const int pos = atomicAdd(&hist[kMaxItemPages - np], 1);
            const int first = prefix_pages_of(p, n) + k * p.part_pages;
            p.items[2 * pos] = make_int4(n, k, first, np);
            p.items[2 * pos + 1] = first_blocks(p.bt + (size_t)n * p.max_blocks + first, np);
        }
    }
    for (int g = t; g < p.num_sg; g += 1024) {
        const int np = (p.sg_pages[g] + p.shared_part_pages - 1) / p.shared_part_pages;
        const int n0 = p.sg_members[(size_t)g * kSgStride];
        // pages member 0's walk reaches (all unless its table is cut inside the prefix)
        const int valid = min(p.sg_pages[g], p.eff_len[n0] / p.block_size);
        for (int k = 0; k < np; ++k) {
            const int pos = atomicAdd(&hist[kMaxItemPages - shared_pair_pages(p, g, k)], 1);
            const int pages = max(0, min(p.shared_part_pages, valid - k * p.shared_part_pages));
            p.items[2 * pos] = make_int4(-1 - g, k, n0, pages);  // negative: subgroup item
            p.items[2 * pos + 1] =
                first_blocks(p.bt + (size_t)n0 * p.max_blocks + (size_t)k * p.shared_part_pages, pages);
        }
    }
    if (t == 0) {
        p.work[0] = total_pairs * p.num_kv_heads;  // total items
    }
    if (t < p.queues) {  // queue heads, both sets: wave w takes item w statically, w < num_waves
        p.work[kQueueStride * (1 + t)] = (p.num_waves - t + p.queues - 1) / p.queues;
        p.work[kQueueStride * (1 + t + kQueues)] = (p.num_waves - t + p.queues - 1) / p.queues;
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
// stream through kStages LDS stages per wave: every page (K and V, 16 rows of
// D elements each) arrives by global_load_lds_dwordx4, 1 KiB contiguous per
// instruction, so the next page is in flight while this one is computed.
//   K stage layout: 16-byte chunk c of row r sits at chunk slot
//     r * CPR + (c ^ (r % CPR)), so the MFMA fragment reads (16 rows, same c)
//     hit distinct LDS banks.
//   V stage layout: natural [row][D].
// An item computes the query rows held in the columns of T 16-column MFMA
// tiles: a sequence's own partition has the G heads of one kv-head (T = 1,
// columns >= G idle); a prefix subgroup's shared partition has member-major
// rows, G heads per member (T = 2, up to 32 rows), so one read of a shared
// page serves every member.
//   QK^T  v_mfma_f32_16x16x32_bf16, A = the page's 16 K rows (tokens), B = the
//         tile's query rows; lane (grp, col) gets tokens 4*grp+i of row col.
//   softmax  one reference max per row, shared by the 4 lane groups and moved
//         lazily: only when a score exceeds it by kRescaleSlack (always on the
//         first page), so weights stay <= 2^kRescaleSlack, the 16 tokens of a
//         page share a scale, and most pages leave the accumulators alone.
//   PV    O^T[dims x rows] += V^T[dims x 16 tokens] * P^T[16 tokens x rows] on
//         v_mfma_f32_16x16x16_bf16: P^T is the score fragment in bf16; lane
//         (grp, col) reads DT = D/16 consecutive dims of the token rows
//         4*grp+i (fp8 pools: converted to bf16, exactly) and v_perm
//         transposes them into DT A operands, so A row m of tile dt is dim
//         DT*m + dt.
// fp8 pools: the K scale folds into the softmax scale, the V scale into the
// result.
template <int KV, int D, int G>
__global__ void __launch_bounds__(kWave) decode_mfma_kernel(Params p) {
    constexpr int BS = 16;
    constexpr int ELT = KV == ZK_BF16 ? 2 : 1;
    constexpr int DG = D / 4;            // head dims per lane group in QK
    constexpr int KK = DG / 8;           // MFMA k-steps
    constexpr int DT = D / 16;           // PV dim tiles = dims per lane per V row
    constexpr int RB = D * ELT;          // bytes per token row
    constexpr int CPR = RB / 16;         // 16-byte chunks per row
    constexpr int PAGE = BS * RB;        // bytes per (block, kv-head) page
    constexpr int LPK = PAGE / 1024;     // global_load_lds per page of K (or V)
    constexpr int LPP = 2 * LPK;         // per page, K and V
    constexpr int KBYTES = DG * ELT;     // K fragment bytes per lane per page
    constexpr int KCH = KBYTES / 16;     // ... in 16-byte chunks
    constexpr int VTB = DT * ELT;        // V bytes per lane per token row
    static_assert(PAGE % 1024 == 0 && KBYTES % 16 == 0 && DT % 2 == 0, "page shape");
    typedef typename LdsVec<VTB>::T vtrow_t;
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    __shared__ __attribute__((aligned(16))) char lds[kStages][2][PAGE];  // [stage][K|V]
    __shared__ int32_t bids[kMaxItemPages];                              // this item's block ids

    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    const int H = p.num_heads, Hkv = p.num_kv_heads;

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
    const uint32_t vt_off = (uint32_t)((4 * grp) * RB + col * VTB);  // + i * RB

    // Wait until page pi of an np-page item has landed in LDS: the pages
    // issued after it (up to kStages - 1) may still be in flight.
    auto wait_page = [&](int pi, int np) {
        const int ahead = min(kStages - 1, np - 1 - pi);
        static_assert(kStages >= 2 && kStages <= 4, "pipeline depth");
        if (ahead <= 0) wait_vmcnt<0>();
        else if (ahead == 1) wait_vmcnt<LPP>();
        else if (ahead == 2) wait_vmcnt<(kStages > 2 ? 2 * LPP : 0)>();
        else wait_vmcnt<(kStages > 3 ? 3 * LPP : 0)>();
    };

    int next = 0;
    // Claims the next item.  Called once per item, in the iteration that
    // issues the item's last page (right after the first issues for items of
    // at most kStages pages), so the atomic's round trip overlaps the item's
    // last pages.  (Claiming at the start of an item instead lets every wave
    // holding a long item reserve a short one it only starts much later,
    // while waves that finish their short items find the queue empty: with
    // mixed item lengths that left a tail of late short items.)
    const int nq = p.queues, xq = blockIdx.x % nq;
    auto head = [&](int q) { return p.work + kQueueStride * (1 + q + p.head_set * kQueues); };
    // the other set of heads back to its start for the next launch on this
    // workspace (no wave of this launch touches it)
    if (blockIdx.x == 0 && lane < nq)
        p.work[kQueueStride * (1 + lane + (1 - p.head_set) * kQueues)] = (p.num_waves - lane + nq - 1) / nq;
    auto claim_next = [&]() {
        if (lane == 0) next = atomicAdd(head(xq), 1);
    };

    // Data the kernel only reads (descriptors, subgroup members, lengths,
    // scales) goes through constant-space views: scalar loads, counted by
    // lgkmcnt, so they never hold up the page stream's vmcnt waits.
    typedef const __attribute__((address_space(4))) int32_t *cint_t;
    typedef const __attribute__((address_space(4))) float *cfloat_t;
    const cint_t citems = (cint_t)p.items;
    // descriptor of pair k: 8 ints (two int4)
    auto load_desc = [&](int k, int4 &a, int4 &b) {
        const cint_t c = citems + 8 * (size_t)k;
        a = make_int4(c[0], c[1], c[2], c[3]);
        b = make_int4(c[4], c[5], c[6], c[7]);
    };

    // Block ids of an item's pages kStages .. np-1 into LDS (bids[i] = table
    // entry i; the first pages' ids come with the descriptor), eight
    // independent loads in flight per lane.  The LDS writes wait for their
    // loads, which retires every earlier load of the item (Q fragments, the
    // first pages) too, so the page loop starts with nothing pending in the
    // compiler's view.  (LDS-DMA staging of the ids, or register loads still
    // pending at the loop, make the compiler wait for vmcnt(0) inside the
    // page loop, which drains the page stream every page.)
    auto stage_bids = [&](const int32_t *row, int np) {
        for (int i0 = kStages; i0 < np; i0 += 8 * kWave) {
            int32_t b[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave + lane;
                b[j] = i < np ? row[i] : 0;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = i0 + j * kWave + lane;
                if (i < np) bids[i] = b[j];
            }
        }
        wait_lgkmcnt0();  // this wave's LDS writes are visible to its own reads
    };

    // B fragment of query row (n, qh): this lane group's DG dims as KK bf16x8.
    auto load_q = [&](size_t qr, int qh, bf16x8 *qf) {
        const size_t qb = qr * (size_t)p.q_stride + (size_t)qh * D + (size_t)grp * DG;
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
    };

    const int total = *(cint_t)p.work;
    // The next item and its descriptor, loaded while the current item's last
    // page is computed (the claim has returned by then).  The scalar load is
    // issued by inline asm: a plain load, whose result is only used after the
    // page loop, is moved past the loop by the compiler; the asm keeps it in
    // the last iteration, and desc_ready() waits for it (lgkmcnt) and hands
    // the registers on.
    typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
    int nx = 0;
    i32x8 nraw = {0, 0, 0, 0, 0, 0, 0, 0};
    bool have_next = false;
    // (claims past the last item read a descriptor the item loop then
    // ignores: the index is clamped to the descriptor array)
    const int desc_cap = p.num_seqs * p.max_parts;
    auto fetch_next = [&]() {
        nx = __builtin_amdgcn_readfirstlane(next) * nq + xq;
        if (nx >= total) {
            // own queue done: take from the others (a plain load first, so
            // exhausted queues cost no atomic)
            int got = total;
            if (lane == 0)
                for (int j = 1; j < nq && got >= total; ++j) {
                    const int q = (xq + j) % nq;
                    if (__hip_atomic_load(head(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) * nq + q >= total)
                        continue;
                    const int idx = atomicAdd(head(q), 1) * nq + q;
                    if (idx < total) got = idx;
                }
            nx = __builtin_amdgcn_readfirstlane(got);
        }
        const int k = __builtin_amdgcn_readfirstlane(min(nx / Hkv, desc_cap - 1));
        asm volatile("s_load_dwordx8 %0, %1, 0x0" : "=s"(nraw) : "s"(p.items + 2 * (size_t)k) : "memory");
        have_next = true;
    };
    auto desc_ready = [&](int4 &a, int4 &b) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(nraw)::"memory");
        a = make_int4(nraw[0], nraw[1], nraw[2], nraw[3]);
        b = make_int4(nraw[4], nraw[5], nraw[6], nraw[7]);
    };

    // q / out row of sequence n
    auto q_row = [&](int n) -> size_t { return p.q_rows ? (size_t)((cint_t)p.q_rows)[n] : (size_t)n; };

    // Attention of T tiles of query rows (qf) over pages [page0, page0 + np)
    // of table `trow` for kv-head kvh; tokens at positions >= len are masked.
    // trow points at the table entry of page page0; blk0 holds the block ids
    // of the first kDescPages pages.
    // Leaves O^T (o), the rows' reference max (m) and sum (l, all 4 lane
    // groups) for the caller to write.  fuse_tib >= 0 (fused append): the
    // last page's row fuse_tib is the step's token, nrow in this wave's
    // registers (lane c < CPR: chunk c of K, CPR <= lane < 2 CPR: of V); it is
    // written into the page's LDS copy once that has landed, and to the pools
    // at byte offset row_dst of the K / V pool.
    auto attend = [&]<int T>(const bf16x8 (&qf)[T][KK], const int32_t *trow, int4 blk0, int page0, int np, int len,
                             int kvh, float sl2, f32x4 (&o)[DT][T], float (&m)[T], float (&l)[T], int fuse_tib,
                             u32x4 nrow, size_t row_dst) {
        const char *kbase = p.k_pool + ((size_t)kvh * PAGE);
        const char *vbase = p.v_pool + ((size_t)kvh * PAGE);
        const size_t block_bytes = (size_t)PAGE * Hkv;
        auto issue_blk = [&](int blk, int s) {
            const char *kp = kbase + (size_t)blk * block_bytes;
            const char *vp = vbase + (size_t)blk * block_bytes;
#pragma unroll
            for (int j = 0; j < LPK; ++j) g2l16(kp + kg[j], (lds_void *)(lds[s][0] + 1024 * j));
#pragma unroll
            for (int j = 0; j < LPK; ++j) g2l16(vp + vg[j], (lds_void *)(lds[s][1] + 1024 * j));
        };
#pragma unroll
        for (int t = 0; t < T; ++t) {
            m[t] = -INFINITY;
            l[t] = 0.0f;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        auto page = [&](int pi, int s) {
            wait_page(pi, np);
            if constexpr (KV == ZK_BF16) {
                if (fuse_tib >= 0 && pi == np - 1) {  // the step's token over the page's stale row
                    if (lane < CPR)
                        *reinterpret_cast<u32x4 *>(lds[s][0] + (fuse_tib * CPR + (lane ^ (fuse_tib % CPR))) * 16) =
                            nrow;
                    else if (lane < 2 * CPR)
                        *reinterpret_cast<u32x4 *>(lds[s][1] + fuse_tib * RB + (lane - CPR) * 16) = nrow;
                    if (lane < 2 * CPR)
                        __builtin_nontemporal_store(
                            nrow, reinterpret_cast<u32x4 *>((char *)(lane < CPR ? p.k_pool : p.v_pool) + row_dst));
                }
            }
            uint32_t kw[KBYTES / 4];
#pragma unroll
            for (int f = 0; f < KCH; ++f) {
                const u32x4 c4 = *reinterpret_cast<const u32x4 *>(lds[s][0] + kl[f]);
#pragma unroll
                for (int j = 0; j < 4; ++j) kw[4 * f + j] = c4[j];
            }
            vtrow_t vt[4];  // token rows 4*grp+i, dims DT*col .. DT*col+DT-1
#pragma unroll
            for (int i = 0; i < 4; ++i) vt[i] = *reinterpret_cast<const vtrow_t *>(lds[s][1] + vt_off + i * RB);
            const int nb = bids[min(pi + kStages, kMaxItemPages - 1)];
            // The stage is free once its reads are done: the empty asm needs
            // their results, so the compiler's own lgkmcnt wait lands here
            // (it does not count an explicit s_waitcnt as completing them and
            // would wait again at the MFMAs, behind the prefetch below).
#pragma unroll
            for (int j = 0; j < KBYTES / 4; ++j) asm volatile("" ::"v"(kw[j]));
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" ::"v"(vt[i]));
            asm volatile("" ::"v"(nb));
            if (pi + kStages < np) issue_blk(__builtin_amdgcn_readfirstlane(nb), s);
            if (pi == np - 1 - kStages) claim_next();
            if (pi == np - 1) fetch_next();

            f32x4 sacc[T];
#pragma unroll
            for (int t = 0; t < T; ++t) sacc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) {
                u32x4 w;
                if constexpr (KV == ZK_BF16) {
                    w = u32x4{kw[4 * kk], kw[4 * kk + 1], kw[4 * kk + 2], kw[4 * kk + 3]};
                } else {
                    const u32x2 lo2 = e4m3x4_to_bf16x4(kw[2 * kk]), hi2 = e4m3x4_to_bf16x4(kw[2 * kk + 1]);
                    w = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
                }
#pragma unroll
                for (int t = 0; t < T; ++t)
                    sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w), qf[t][kk],
                                                                      sacc[t], 0, 0, 0);
            }
            // V rows as bf16 pairs: w[i][j] = dims (2j, 2j+1) of token row 4*grp+i
            uint32_t w[4][DT / 2];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (KV == ZK_BF16) {
                    __builtin_memcpy(w[i], &vt[i], 2 * DT);
                } else {
                    uint32_t b8[DT / 4];
                    __builtin_memcpy(b8, &vt[i], DT);
#pragma unroll
                    for (int j = 0; j < DT / 4; ++j) {
                        const u32x2 c2 = e4m3x4_to_bf16x4(b8[j]);
                        w[i][2 * j] = c2[0];
                        w[i][2 * j + 1] = c2[1];
                    }
                }
            }
            const int tok0 = (page0 + pi) * BS + 4 * grp;
            if (tok0 + 4 > len) {  // partial last page: stale rows must not reach O
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (tok0 + i >= len)
#pragma unroll
                        for (int j = 0; j < DT / 2; ++j) w[i][j] = 0u;
            }
            s16x4 va[DT];  // element i of tile dt = V[4*grp+i][DT*col+dt]
#pragma unroll
            for (int j = 0; j < DT / 2; ++j) {
                const u32x2 lo{__builtin_amdgcn_perm(w[1][j], w[0][j], 0x05040100u),
                               __builtin_amdgcn_perm(w[3][j], w[2][j], 0x05040100u)};
                const u32x2 hi{__builtin_amdgcn_perm(w[1][j], w[0][j], 0x07060302u),
                               __builtin_amdgcn_perm(w[3][j], w[2][j], 0x07060302u)};
                va[2 * j] = __builtin_bit_cast(s16x4, lo);
                va[2 * j + 1] = __builtin_bit_cast(s16x4, hi);
            }
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float sc[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) sc[i] = tok0 + i < len ? sacc[t][i] * sl2 : -INFINITY;
                const float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                // lazy rescale (wave-uniform branch): the new reference is the
                // row max over the page's 16 tokens (all four lane groups)
                if (__builtin_amdgcn_ballot_w64(mx > m[t] + kRescaleSlack)) {
                    float cm = fmaxf(mx, xor16(mx));
                    cm = fmaxf(cm, xor32(cm));
                    const float m_new = fmaxf(m[t], cm);
                    const float alpha = m_new == -INFINITY ? 1.0f : exp2_fast(m[t] - m_new);
                    l[t] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][t] *= alpha;
                    m[t] = m_new;
                }
                float pr[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) pr[i] = exp2_fast(sc[i] - m[t]);
                l[t] += (pr[0] + pr[1]) + (pr[2] + pr[3]);
                const s16x4 pb = __builtin_bit_cast(s16x4, u32x2{bf16x2_rne(pr[0], pr[1]), bf16x2_rne(pr[2], pr[3])});
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    o[dt][t] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va[dt], pb, o[dt][t], 0, 0, 0);
            }
        };
        // the first pages straight from the descriptor, then the other ids
        static_assert(kStages <= kDescPages, "descriptor carries the first kStages block ids");
        const int b0[4] = {blk0.x, blk0.y, blk0.z, blk0.w};
#pragma unroll
        for (int j = 0; j < kStages; ++j)
            if (j < np) issue_blk(b0[j], j);
        stage_bids(trow, np);
        // Q is complete before the loop on every path (see stage_bids)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) asm volatile("" ::"v"(qf[t][kk]));
        // and so is the fused row
        asm volatile("" ::"v"(nrow[0]), "v"(nrow[1]), "v"(nrow[2]), "v"(nrow[3]));
        if (np <= kStages) claim_next();
        // one page per iteration (a single loop-carried accumulator set)
        for (int pi = 0, st = 0; pi < np; ++pi, st = (st + 1 == kStages ? 0 : st + 1)) page(pi, st);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            l[t] += xor16(l[t]);
            l[t] += xor32(l[t]);
        }
    };

    // Lane (grp, col) holds dims DT*(4*grp+i)+dt, i < 4, dt < DT, of row col:
    // four runs of DT consecutive floats.
    auto store_row_f32 = [&](float *dst, const f32x4 (&o)[DT][2], int t, float scale) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) v[dt] = o[dt][t][i] * scale;
            __builtin_memcpy(dst + DT * (4 * grp + i), v, sizeof(v));
        }
    };
    // a partial slot and its (m, l), for decode_reduce_kernel
    auto store_partial = [&](size_t slot, const f32x4 (&o)[DT][2], int t, float scale, float m_, float l_) {
        store_row_f32(p.po + slot * D, o, t, scale);
        if (grp == 0) p.ml[slot] = make_float2(m_, l_);
    };
    const u32x4 no_row = {0u, 0u, 0u, 0u};

    int item = blockIdx.x;  // first item static, the rest from the queue
    int4 d0 = make_int4(0, 0, 0, 0), d1 = make_int4(0, 0, 0, 0);
    if (item < total) load_desc(item / Hkv, d0, d1);
    while (item < total) {
        const int kvh = item % Hkv;
        have_next = false;
        if (KV == ZK_BF16 && d0.x < 0) {
            // shared-prefix partition of subgroup sg: up to 32 rows, member-major
            const int sg = -1 - d0.x, part = d0.y, n0 = d0.z, np = d0.w;
            const int page0 = part * p.shared_part_pages;
            // members (batch indices) of the subgroup, by scalar loads; lane
            // (grp, col) serves row r = 16 t + col, member r / G
            constexpr int NM = kSgStride / G;
            const cint_t cmem = (cint_t)(p.sg_members + (size_t)sg * kSgStride);
            int mem_s[NM];
#pragma unroll
            for (int j = 0; j < NM; ++j) mem_s[j] = cmem[j];
            bf16x8 qf[2][KK];
            int nm[2];  // member of this lane's row in tile t, or -1
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int r = 16 * t + col;
                int v = mem_s[0];
#pragma unroll
                for (int j = 1; j < NM; ++j) v = r / G == j ? mem_s[j] : v;
                nm[t] = v;
                if (nm[t] >= 0) load_q(q_row(nm[t]), qhead_of(p, kvh, r % G, G), qf[t]);
                else
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) qf[t][kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
            }
            f32x4 o[DT][2];
            float m[2], l[2];
            attend.template operator()<2>(qf, p.bt + (size_t)n0 * p.max_blocks + page0, d1, page0, np, 0x7fffffff,
                                          kvh, p.scale_log2, o, m, l, -1, no_row, 0);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int r = 16 * t + col;
                if (nm[t] >= 0) {
                    const size_t slot = ((size_t)nm[t] * H + qhead_of(p, kvh, r % G, G)) * p.max_parts + part;
                    store_partial(slot, o, t, 1.0f, m[t], l[t]);
                }
            }
        } else {
            // a sequence's own partition: rows 0..G-1 are its heads of kv-head kvh
            const int n = d0.x, part = d0.y, page0 = d0.z, np = d0.w;
            const int len = ((cint_t)p.eff_len)[n];  // walk already cut at the first invalid entry
            const int pb = p.seq_pb ? ((cint_t)p.seq_pb)[n] : 0;
            const int ns = pb > 0 ? (pb + p.shared_part_pages - 1) / p.shared_part_pages : 0;
            const int rest = (len + p.block_size - 1) / p.block_size - pb;
            const int nparts = rest > 0 ? (rest + p.part_pages - 1) / p.part_pages : 0;
            const int qh = qhead_of(p, kvh, col % G, G);
            const size_t qr = q_row(n);
            bf16x8 qf[1][KK];
            if (col < G) load_q(qr, qh, qf[0]);
            else
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) qf[0][kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
            float sl2 = p.scale_log2, vscale = 1.0f;
            if constexpr (KV == ZK_FP8_E4M3) {
                sl2 *= ((cfloat_t)p.k_scales)[(size_t)n * Hkv + kvh];
                vscale = ((cfloat_t)p.v_scales)[(size_t)n * Hkv + kvh];
            }
            // fused append: the item holding the sequence's last page
            int fuse_tib = -1;
            u32x4 nrow = no_row;
            size_t row_dst = 0;
            if constexpr (KV == ZK_BF16) {
                if (p.new_k && len > 0 && np > 0 && page0 + np == (len + BS - 1) / BS) {
                    fuse_tib = (len - 1) % BS;
                    const int blk = ((cint_t)p.bt)[(size_t)n * p.max_blocks + (len - 1) / BS];
                    const int c = lane % CPR;
                    row_dst = ((size_t)blk * Hkv + kvh) * PAGE + (size_t)fuse_tib * RB + (size_t)c * 16;
                    if (lane < 2 * CPR)
                        nrow = *reinterpret_cast<const u32x4 *>((lane < CPR ? p.new_k : p.new_v) +
                                                                (size_t)n * p.new_row_bytes + (size_t)kvh * RB + c * 16);
                }
            }
            f32x4 o[DT][1];
            float m[1], l[1];
            attend.template operator()<1>(qf, p.bt + (size_t)n * p.max_blocks + page0, d1, page0, np, len, kvh, sl2,
                                          o, m, l, fuse_tib, nrow, row_dst);
            if (col < G) {
                if (ns == 0 && nparts <= 1) {  // the whole context: write the output row
                    const float inv = l[0] > 0.0f ? vscale / l[0] : 0.0f;
                    const size_t ob = (qr * H + qh) * D;
                    if (p.q_f32) {
                        f32x4 o2[DT][2];
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) o2[dt][0] = o[dt][0];
                        store_row_f32((float *)p.out + ob, o2, 0, inv);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            uint32_t v[DT / 2];
#pragma unroll
                            for (int j = 0; j < DT / 2; ++j)
                                v[j] = bf16x2_rne(o[2 * j][0][i] * inv, o[2 * j + 1][0][i] * inv);
                            __builtin_memcpy((uint16_t *)p.out + ob + DT * (4 * grp + i), v, sizeof(v));
                        }
                    }
                } else {
                    const size_t slot = ((size_t)n * H + qh) * p.max_parts + ns + part;
                    f32x4 o2[DT][2];
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o2[dt][0] = o[dt][0];
                    store_partial(slot, o2, 0, vscale, m[0], l[0]);
                }
            }
        }
        if (!have_next) fetch_next();  // an item without pages
        item = nx;
        desc_ready(d0, d1);
        // consumed: a constant until the next fetch, so the descriptor's
        // scalar registers are not kept across the next item's prologue
        nraw = i32x8{0, 0, 0, 0, 0, 0, 0, 0};
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
        q_s[i] = load_q(p, qrow(p, n) * (size_t)p.q_stride + (size_t)qhead_of(p, kvh, j, G) * D + d);
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
                if (d < D) store_out(p, (qrow(p, n) * H + qh) * D + d, o[j][c] * vs * inv);
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
    const int ns = shared_parts_of(p, n);
    const int nparts = ns + private_parts_of(p, n);
    if (ns == 0 && nparts <= 1) return;  // written by the partition kernel
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
        if (lane + 64 * c < D) store_out(p, (qrow(p, n) * p.num_heads + h) * D + lane + 64 * c, acc[c] * inv);
}

// The same merge for D = 4 * LP (D in {64, 128, 256}): LP lanes hold a
// partition's partial output as one float4 each, so one load instruction
// covers 64 / LP partitions and all of a sequence's partitions are in flight
// at once (the loop above waits for each group of eight).  Lane i reads
// partition i's (m, l) once for the maximum, the sum and its weight; the
// first 64 * U0 / LP partials are loaded beside the (m, l), so after the
// lengths a row of up to that many partitions needs one more memory round
// trip, not two.
template <int D>
__global__ void __launch_bounds__(kWave) decode_reduce_vec_kernel(Params p) {
    constexpr int LP = D / 4, P = kWave / LP, U = 16;  // lanes per partition, partitions per load, loads per lane
    constexpr int U0 = 4;  // loads per lane issued with the (m, l): few, so that four waves fit a SIMD
    static_assert(D % 4 == 0 && kWave % LP == 0, "partition layout");
    const int h = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const int ns = shared_parts_of(p, n);
    const int nparts = ns + private_parts_of(p, n);
    if (ns == 0 && nparts <= 1) return;  // written by the partition kernel
    const size_t base = ((size_t)n * p.num_heads + h) * p.max_parts;
    const float2 none = make_float2(-INFINITY, 0.0f);
    const int sub = lane / LP, j = lane % LP;  // partition slot within a load, float4 index
    // the first P * U0 partials go out with the (m, l) loads: one round trip
    // instead of two (they do not depend on the maximum)
    const int cnt0 = min(kWave, nparts);
    f32x4 x0[U0];
#pragma unroll
    for (int u = 0; u < U0; ++u) {
        const int i = P * u + sub;
        x0[u] = i < cnt0 ? *reinterpret_cast<const f32x4 *>(p.po + (base + i) * D + 4 * j) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float2 ml0 = lane < nparts ? p.ml[base + lane] : none;
    float M = ml0.x;
    for (int i = lane + kWave; i < nparts; i += kWave) M = fmaxf(M, p.ml[base + i].x);
    for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
    auto weight = [&](float2 v) { return v.x == -INFINITY ? 0.0f : exp2f(v.x - M); };
    float L = ml0.y * weight(ml0);
    for (int i = lane + kWave; i < nparts; i += kWave) {
        const float2 v = p.ml[base + i];
        L += v.y * weight(v);
    }
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nparts; c0 += kWave) {  // weights of partitions c0 .. c0 + 63 in lanes
        const float w = weight(c0 == 0 ? ml0 : (c0 + lane < nparts ? p.ml[base + c0 + lane] : none));
        const int cnt = min(kWave, nparts - c0);
        for (int i0 = 0; i0 < cnt; i0 += P * U) {
            f32x4 x[U];
            float wi[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int i = i0 + P * u + sub;
                wi[u] = __shfl(w, min(i, kWave - 1));
                if (c0 == 0 && i0 == 0 && u < U0) x[u] = x0[u];
                else x[u] = i < cnt ? *reinterpret_cast<const f32x4 *>(p.po + (base + c0 + i) * D + 4 * j)
                                    : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (i0 + P * u + sub < cnt)
#pragma unroll
                    for (int c = 0; c < 4; ++c) acc[c] = fmaf(wi[u], x[u][c], acc[c]);
        }
    }
    // the P partition slots of a load sit LP lanes apart
#pragma unroll
    for (int off = LP; off < kWave; off <<= 1)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[c] += __shfl_xor(acc[c], off);
    if (sub == 0)
#pragma unroll
        for (int c = 0; c < 4; ++c) store_out(p, (qrow(p, n) * p.num_heads + h) * D + 4 * j + c, acc[c] * inv);
}

// One wave per (kv-head, sequence): the G query heads of the kv-head at once
// (LPH = 64 / G lanes a head, F = G * D / 64 floats a lane), so a launch has
// Hkv / H of the waves of decode_reduce_vec_kernel.  Each lane reads its
// head's (m, l) of every partition itself (no cross-lane reductions) and the
// first C partitions' partials with them, one memory round trip; partitions
// are added in slot order.
template <int D, int G>
__global__ void __launch_bounds__(kWave) decode_reduce_kv_kernel(Params p) {
    constexpr int LPH = kWave / G, F = G * D / kWave, F4 = F / 4;
    constexpr int C = 8;  // partitions loaded with the (m, l)
    static_assert(F % 4 == 0 && kWave % G == 0, "lane layout");
    const int kvh = blockIdx.x, n = blockIdx.y, lane = threadIdx.x;
    const int ns = shared_parts_of(p, n);
    const int nparts = ns + private_parts_of(p, n);
    if (ns == 0 && nparts <= 1) return;  // written by the partition kernel
    const int hh = lane / LPH, d0 = (lane % LPH) * F;
    const int qh = qhead_of(p, kvh, hh, G);
    const size_t base = ((size_t)n * p.num_heads + qh) * p.max_parts;
    float2 ml[C];
    f32x4 x[C][F4];
#pragma unroll
    for (int i = 0; i < C; ++i) {
        if (i < nparts) {
            ml[i] = p.ml[base + i];
#pragma unroll
            for (int k = 0; k < F4; ++k) x[i][k] = *reinterpret_cast<const f32x4 *>(p.po + (base + i) * D + d0 + 4 * k);
        } else {
            ml[i] = make_float2(-INFINITY, 0.0f);
        }
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < C; ++i) M = fmaxf(M, ml[i].x);
    for (int i = C; i < nparts; ++i) M = fmaxf(M, p.ml[base + i].x);
    auto weight = [&](float2 v) { return v.x == -INFINITY ? 0.0f : exp2f(v.x - M); };
    float L = 0.0f;
    f32x4 acc[F4];
#pragma unroll
    for (int k = 0; k < F4; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < C; ++i)
        if (i < nparts) {
            const float w = weight(ml[i]);
            L += ml[i].y * w;
#pragma unroll
            for (int k = 0; k < F4; ++k)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[k][c] = fmaf(w, x[i][k][c], acc[k][c]);
        }
    for (int i = C; i < nparts; ++i) {
        const float2 v = p.ml[base + i];
        const float w = weight(v);
        L += v.y * w;
#pragma unroll
        for (int k = 0; k < F4; ++k) {
            const f32x4 y = *reinterpret_cast<const f32x4 *>(p.po + (base + i) * D + d0 + 4 * k);
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[k][c] = fmaf(w, y[c], acc[k][c]);
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const size_t ob = (qrow(p, n) * p.num_heads + qh) * D + d0;
    if (p.q_f32) {
#pragma unroll
        for (int k = 0; k < F4; ++k) {
            const f32x4 y = acc[k] * inv;
            __builtin_memcpy((float *)p.out + ob + 4 * k, &y, sizeof(y));
        }
    } else {
        uint32_t v[F / 2];
#pragma unroll
        for (int k = 0; k < F4; ++k) {
            v[2 * k] = bf16x2_rne(acc[k][0] * inv, acc[k][1] * inv);
            v[2 * k + 1] = bf16x2_rne(acc[k][2] * inv, acc[k][3] * inv);
        }
        __builtin_memcpy((uint16_t *)p.out + ob, v, sizeof(v));
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
    size_t eff, items, map, work, ml, po, total;
};
WsLayout ws_layout(int num_seqs, int num_heads, int head_dim, int max_parts) {
    WsLayout w;
    w.eff = 0;
    w.items = align256(sizeof(int32_t) * (size_t)num_seqs);
    w.map = w.items;
    w.work = w.map + align256(2 * sizeof(int4) * (size_t)num_seqs * max_parts);
    w.ml = w.work + align256(kWorkBytes);
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

int mfma_part_pages(int num_seqs, int num_kv_heads, int max_blocks, long waves) {
    if (int e = part_pages_env()) return e;
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

// Pages per shared-prefix item: about one item per two waves over all
// subgroups' pages, so half the waves stream the shared pages (two query-row
// tiles each) while the rest run the sequences' own items; measured best on
// forked-prefix batches.  ZEALOT_DECODE_SHARED_PART_PAGES (16..1024) overrides.
int shared_part_pages_for(long total_shared_pages, int num_kv_heads, long waves) {
    static const int env = [] {
        const char *e = std::getenv("ZEALOT_DECODE_SHARED_PART_PAGES");
        const int v = e ? std::atoi(e) : 0;
        return v <= 0 ? 0 : (v < 16 ? 16 : (v > kMaxItemPages ? kMaxItemPages : v));
    }();
    if (env) return env;
    const long half = waves / 2;
    long pp = (total_shared_pages * num_kv_heads + half - 1) / half;
    pp = (pp + 15) / 16 * 16;
    return (int)(pp < 16 ? 16 : (pp > kMaxItemPages ? kMaxItemPages : pp));
}

}  // namespace

size_t zk::paged_decode_workspace(int num_seqs, int num_heads, int head_dim, int max_blocks_per_seq,
                                  int block_size, bool shared) {
    if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_blocks_per_seq <= 0) return 256;
    return ws_layout(num_seqs, num_heads, head_dim,
                     max_parts_for(max_blocks_per_seq, min_part_pages(head_dim, block_size)) + (shared ? 1 : 0))
        .total;
}

bool zk::paged_decode_shares_prefixes(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads) {
    return kv_dtype == ZK_BF16 && num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
           mfma_supported(kv_dtype, head_dim, block_size, num_heads / num_kv_heads);
}

bool zk::paged_decode_fuses_append(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads) {
    return zk::paged_decode_shares_prefixes(kv_dtype, head_dim, block_size, num_heads, num_kv_heads);
}

namespace {

// Host-side argument checks of zk_paged_decode (no device work).
int check_decode_args(zk_dtype q_dtype, zk_dtype kv_dtype, int num_seqs, int num_heads, int num_kv_heads,
                      int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                      zk_gqa_mapping mapping) {
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
    if (head_dim > 256 || num_heads / num_kv_heads > kMaxG)
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: head_dim <= 256 and H/Hkv <= 16 required");
    if ((int64_t)max_blocks_per_seq * block_size > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: context too long");
    return ZK_OK;
}

// Which kernel a call runs, how it cuts the contexts and the workspace it
// needs (arguments already checked).
struct DecodeShape {
    bool use_mfma, shared;
    int part_pages, shared_pages, max_parts, waves;
    WsLayout w;
};
// max_waves > 0 caps the MFMA path's persistent grid (partitions are sized
// for the waves that run them).
DecodeShape decode_shape(zk_dtype kv_dtype, int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                         int block_size, int max_blocks_per_seq, const PrefixGroups *pg, int max_waves = 0) {
    DecodeShape d;
    const int G = num_heads / num_kv_heads;
    d.use_mfma = mfma_supported(kv_dtype, head_dim, block_size, G);
    d.waves = persistent_grid();
    if (max_waves > 0 && max_waves < d.waves) d.waves = max_waves;
    d.part_pages = d.use_mfma ? mfma_part_pages(num_seqs, num_kv_heads, max_blocks_per_seq, d.waves)
                              : part_pages_for(ZK_F32, head_dim, block_size);
    d.shared = pg && pg->num_sg > 0 &&
               paged_decode_shares_prefixes(kv_dtype, head_dim, block_size, num_heads, num_kv_heads);
    d.shared_pages = d.shared ? shared_part_pages_for(pg->total_shared_pages, num_kv_heads, d.waves) : 0;
    // slot stride: a sequence's shared and private partitions together
    d.max_parts = d.shared ? max_parts_for(max_blocks_per_seq, min_part_pages(head_dim, block_size)) + 1
                           : max_parts_for(max_blocks_per_seq, d.part_pages);
    d.w = ws_layout(num_seqs, num_heads, head_dim, d.max_parts);
    return d;
}

}  // namespace

int zk::paged_decode(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                     void *out, const int32_t *block_tables, const int32_t *seq_lens, int num_seqs, int num_heads,
                     int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                     float scale, zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                     void *workspace, size_t workspace_bytes, void *stream, const PrefixGroups *pg,
                     const int32_t *q_rows, int64_t q_stride, bool trusted_tables, bool reuse_plan,
                     const AppendRows *append, int *head_set, int max_waves) {
    if (int rc = check_decode_args(q_dtype, kv_dtype, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                                   max_blocks_per_seq, num_blocks, mapping))
        return rc;
    if (num_seqs == 0) return ZK_OK;
    if (!q || !k_pool || !v_pool || !out || !block_tables || !seq_lens || !workspace)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode: NULL pointer");
    const bool fp8 = kv_dtype == ZK_FP8_E4M3;
    if (fp8 != (k_scales != nullptr && v_scales != nullptr))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: fp8 pools need k/v scales, other pools none");
    const int G = num_heads / num_kv_heads;
    if (pg && pg->num_sg > 0 && (!pg->seq_pb || !pg->sg_members || !pg->sg_pages) &&
        paged_decode_shares_prefixes(kv_dtype, head_dim, block_size, num_heads, num_kv_heads))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: paged decode: NULL prefix-group array");
    const DecodeShape ds = decode_shape(kv_dtype, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                                        max_blocks_per_seq, pg, max_waves);
    const bool use_mfma = ds.use_mfma, shared = ds.shared;
    if (append && (!use_mfma || kv_dtype != ZK_BF16 || !trusted_tables || !append->k || !append->v ||
                   append->row_bytes < (int64_t)num_kv_heads * head_dim * 2 || (append->row_bytes & 15) ||
                   (((uintptr_t)append->k | (uintptr_t)append->v) & 15u)))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: paged decode: fused append needs the bf16 MFMA path, trusted tables and "
                         "16-byte aligned rows");
    const int part_pages = ds.part_pages, shared_pages = ds.shared_pages, max_parts = ds.max_parts;
    const WsLayout &w = ds.w;
    if (workspace_bytes < w.total || ((uintptr_t)workspace & 255u))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_decode: workspace too small or not 256-B aligned (need " +
                             std::to_string(w.total) + " bytes)");

    Params p{};
    p.q = q;
    p.k_pool = (const char *)k_pool;
    p.v_pool = (const char *)v_pool;
    p.out = out;
    p.bt = block_tables;
    p.seq_lens = seq_lens;
    p.k_scales = k_scales;
    p.v_scales = v_scales;
    p.q_rows = q_rows;
    p.q_stride = q_stride > 0 ? q_stride : (int64_t)num_heads * head_dim;
    p.trusted = trusted_tables ? 1 : 0;
    char *ws = (char *)workspace;
    p.eff_len = (int32_t *)(ws + w.eff);
    p.items = (int4 *)(ws + w.map);
    p.work = (int32_t *)(ws + w.work);
    p.num_waves = use_mfma ? ds.waves : 0;
    p.queues = shared ? kQueues : 1;
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
    p.seq_pb = shared ? pg->seq_pb : nullptr;
    p.sg_members = shared ? pg->sg_members : nullptr;
    p.sg_pages = shared ? pg->sg_pages : nullptr;
    p.num_sg = shared ? pg->num_sg : 0;
    p.shared_part_pages = shared ? shared_pages : 1;
    p.scale_log2 = scale * kLog2e;
    p.grouped = mapping == ZK_GQA_GROUPED ? 1 : 0;
    p.q_f32 = q_dtype == ZK_F32 ? 1 : 0;
    if (append) {
        p.new_k = (const char *)append->k;
        p.new_v = (const char *)append->v;
        p.new_row_bytes = append->row_bytes;
    }

    hipStream_t s = (hipStream_t)stream;
    reuse_plan = reuse_plan && use_mfma;
    if (!(use_mfma && (trusted_tables || reuse_plan))) {  // trusted MFMA launches: the plan sets the lengths
        {
            KernelTimer timer("decode_seq_info", s);
            seq_info_kernel<<<num_seqs, kWave, 0, s>>>(p);
        }
        if (int rc = check_launch("zk_paged_decode seq_info")) return rc;
    }
    const bool reduce = max_parts > 1 || shared;
    if (use_mfma) {
        // a launch reusing the plan claims from the head set the launch
        // before it put back
        reuse_plan = reuse_plan && head_set;
        p.head_set = reuse_plan ? (*head_set & 1) : 0;
        if (!reuse_plan) {
            {
                KernelTimer timer("decode_plan", s);
                plan_kernel<<<1, 1024, 0, s>>>(p, num_seqs);
            }
            if (int rc = check_launch("zk_paged_decode plan")) return rc;
        }
        {
            KernelTimer timer("decode_partials", s);
            const int grid = p.num_waves;
            if (kv_dtype == ZK_BF16) launch_mfma<ZK_BF16>(p, grid, s, G);
            else launch_mfma<ZK_FP8_E4M3>(p, grid, s, G);
        }
        if (int rc = check_launch("zk_paged_decode partials")) return rc;
        if (head_set) *head_set = p.head_set ^ 1;
    } else {
        KernelTimer timer("decode_partials", s);
        dim3 grid(max_parts, num_kv_heads, num_seqs);
        if (kv_dtype == ZK_F32) decode_generic_kernel<ZK_F32><<<grid, kWave, 0, s>>>(p);
        else if (kv_dtype == ZK_BF16) decode_generic_kernel<ZK_BF16><<<grid, kWave, 0, s>>>(p);
        else decode_generic_kernel<ZK_FP8_E4M3><<<grid, kWave, 0, s>>>(p);
    }
    if (int rc = check_launch("zk_paged_decode partials")) return rc;
    if (reduce) {
        dim3 rgrid(num_heads, num_seqs);
        KernelTimer timer("decode_reduce", s);
        const dim3 kgrid(num_kv_heads, num_seqs);
        if (head_dim == 128 && G == 4) decode_reduce_kv_kernel<128, 4><<<kgrid, kWave, 0, s>>>(p);
        else if (head_dim == 128 && G == 8) decode_reduce_kv_kernel<128, 8><<<kgrid, kWave, 0, s>>>(p);
        else if (head_dim == 128 && G == 2) decode_reduce_kv_kernel<128, 2><<<kgrid, kWave, 0, s>>>(p);
        else if (head_dim == 128) decode_reduce_vec_kernel<128><<<rgrid, kWave, 0, s>>>(p);
        else if (head_dim == 64) decode_reduce_vec_kernel<64><<<rgrid, kWave, 0, s>>>(p);
        else if (head_dim == 256) decode_reduce_vec_kernel<256><<<rgrid, kWave, 0, s>>>(p);
        else decode_reduce_kernel<<<rgrid, kWave, 0, s>>>(p);
        if (int rc = check_launch("zk_paged_decode reduce")) return rc;
    }
    return ZK_OK;
}

// ------------------------------------------------------------ no-allocation decode
// zk_paged_decode_noalloc's workspace is the device array of
// noalloc_scratch.hip (zk::noalloc_scratch), reserved on a GPU by the first
// call there.

extern "C" {

size_t zk_paged_decode_workspace_size(int num_seqs, int num_heads, int head_dim, int max_blocks_per_seq,
                                      int block_size) {
    return zk::paged_decode_workspace(num_seqs, num_heads, head_dim, max_blocks_per_seq, block_size, false);
}

int zk_paged_decode(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                    zk_dtype kv_dtype, void *out, const int32_t *block_tables, const int32_t *seq_lens,
                    int num_seqs, int num_heads, int num_kv_heads, int head_dim, int block_size,
                    int max_blocks_per_seq, int64_t num_blocks, float scale, zk_gqa_mapping mapping,
                    const float *k_scales, const float *v_scales, void *workspace, size_t workspace_bytes,
                    void *stream) {
    return zk::paged_decode(q, q_dtype, k_pool, v_pool, kv_dtype, out, block_tables, seq_lens, num_seqs,
                            num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_blocks, scale,
                            mapping, k_scales, v_scales, workspace, workspace_bytes, stream, nullptr, nullptr);
}

int zk_paged_decode_noalloc(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                            zk_dtype kv_dtype, void *out, const int32_t *block_tables, const int32_t *seq_lens,
                            int num_seqs, int num_heads, int num_kv_heads, int head_dim, int block_size,
                            int max_blocks_per_seq, int64_t num_blocks, float scale, zk_gqa_mapping mapping,
                            const float *k_scales, const float *v_scales, void *stream) {
    if (int rc = check_decode_args(q_dtype, kv_dtype, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
                                   max_blocks_per_seq, num_blocks, mapping))
        return rc;
    if (num_seqs == 0) return ZK_OK;
    const size_t need =
        decode_shape(kv_dtype, num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq, nullptr)
            .w.total;
    if (need > (size_t)ZK_DECODE_SCRATCH_BYTES)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_decode_noalloc: the call needs " +
                                                      std::to_string(need) + " bytes of scratch, the maximum is " +
                                                      std::to_string((size_t)ZK_DECODE_SCRATCH_BYTES));
    void *ws = nullptr;
    if (int rc = zk::noalloc_scratch(&ws)) return rc;
    zk::TimingSuspend no_events;  // per-kernel timing would create hipEvents
    return zk::paged_decode(q, q_dtype, k_pool, v_pool, kv_dtype, out, block_tables, seq_lens, num_seqs, num_heads,
                            num_kv_heads, head_dim, block_size, max_blocks_per_seq, num_blocks, scale, mapping,
                            k_scales, v_scales, ws, (size_t)ZK_DECODE_SCRATCH_BYTES, stream, nullptr, nullptr);
}

}  // extern "C"

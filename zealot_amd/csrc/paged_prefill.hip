// paged_prefill.hip -- chunked-prefill attention over paged K/V for gfx950.
//
// A prompt chunk of C tokens of sequence n, whose K/V are already in the
// pages behind start_pos[n] cached tokens, attends to its context: chunk row t
// (absolute position start + t) sees positions [0, start + t] when causal --
// the per-element mask of src/attention/kernels/attention.cu:117-121, there
// applied to a first chunk held outside the pages -- or [0, start + C) when
// not (CpuAttention::forward, src/attention/mod.rs:64-98).  This replaces the
// reference's first-chunk tiled kernel (attention/cuda.rs:56-110) and its later
// chunks, for which cuda_runner.rs:443-461 runs the one-query decode kernel.
//
// Kernels
//   prefill_plan_kernel  one workgroup: effective context per sequence (the
//       page walk stops at the first table entry < 0 or >= num_blocks, as in
//       the decode), then work items (sequence, query tile, kv-head) in one
//       queue per XCD: every tile of a (sequence, kv-head) goes to the same
//       XCD, (n * Hkv + kvh) mod 8, so the tiles reading the same pages share
//       that XCD's L2; within a queue the groups run longest first (counting
//       sort on their last tile's pages) and a group's tiles back to back,
//       longest first.
//   prefill_mfma_kernel<KV, D, G>  bf16 / fp8 pools, D in {64, 128}, G in
//       {1, 2, 4, 8}, block_size 16: persistent four-wave workgroups (one wave
//       a SIMD, two workgroups a CU, so two waves share each SIMD) take items
//       from their XCD's queue (workgroups are dispatched round-robin over the
//       8 XCDs), then from the others' when it runs dry.  An item holds 128
//       query rows -- TQ = 128/G chunk tokens x the G heads of one kv-head,
//       token-major -- and each wave computes 64 of them as four 16-column
//       MFMA tiles, so each K/V page read into LDS serves all 128 rows.  Pages
//       stream through LDS in pairs (global_load_lds, a ring of four stages,
//       each wave loading one page of every pair); QK^T and PV run on MFMA with
//       a lazily rescaled softmax (see paged_decode.hip), software-pipelined
//       one pair deep; every column carries its own visibility limit.
// Rows write their outputs directly (no split over keys): an item reads the
// pages up to its last row's limit, so the causal triangle costs half.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdint>
#include <string>

#include "zk_common.h"

using namespace zk;

namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;
constexpr int kWaves = 4;             // waves per workgroup, one per SIMD
constexpr int kWavesPerSimd = 2;      // workgroups per CU: two waves share each SIMD
constexpr int kWaveRows = 32;         // query rows per wave (2 MFMA tiles)
constexpr int kRows = kWaves * kWaveRows;  // query rows per item
constexpr int kTiles = kWaveRows / 16;
constexpr int kStages = 4;            // page pairs in LDS: the one computed on, the rest in flight
static_assert((kStages & (kStages - 1)) == 0 && kStages >= 3, "stage ring");
constexpr int kMaxBins = zk::kPrefillMaxPages;  // LDS block ids per item; plan-kernel bins
constexpr int kXcds = 8;                         // XCDs of an MI355X
constexpr int kXcdBins = kMaxBins / kXcds;       // longest-first bins per XCD queue
constexpr int kQueueStride = 32;                 // ints between XCD queue heads (128 B)
constexpr float kRescaleSlack = 8.0f;  // lazy-rescale slack, log2 units

struct PParams {
    const void *q;        // [T, H, D]
    const char *k_pool;
    const char *v_pool;
    void *out;            // [T, H, D], dtype of q
    const int32_t *bt;    // [N, max_blocks]
    const int64_t *cu_q;  // [N + 1] chunk rows per sequence (or, when q_off is set,
    const int64_t *q_off; //  sequence n's rows are q_off[n] .. q_off[n] + q_len[n])
    const int32_t *q_len;
    int64_t q_stride;     // elements between consecutive q rows (out rows: H * D)
    const int32_t *start; // [N] cached tokens before each chunk
    const float *k_scales;
    const float *v_scales;
    int32_t *eff;         // [N] context after the page walk
    int4 *items;          // {n, query tile, pages, kv-head}, per-XCD segments
    int32_t *work;        // [0] total items; XCD x at 64 + 32 x: segment start, end, queue head
    int num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_blocks, tq, num_groups, max_items;
    int64_t num_blocks;
    float scale_log2;
    int grouped, q_f32, causal;
};

__device__ __forceinline__ int chunk_len(const PParams &p, int n) {
    return p.q_off ? p.q_len[n] : (int)(p.cu_q[n + 1] - p.cu_q[n]);
}
__device__ __forceinline__ int64_t chunk_row0(const PParams &p, int n) { return p.q_off ? p.q_off[n] : p.cu_q[n]; }

__device__ __forceinline__ int qhead_of(const PParams &p, int kvh, int j, int G) {
    return p.grouped ? kvh * G + j : kvh + j * p.num_kv_heads;
}

// Pages a query tile reads: up to its last row's visibility limit.
__device__ __forceinline__ int tile_pages(const PParams &p, int n, int qt) {
    const int len = chunk_len(p, n);
    const int last = min(len, (qt + 1) * p.tq);  // rows of the tile end here
    const int lim = p.causal ? p.start[n] + last : p.start[n] + len;
    const int vis = min(lim, p.eff[n]);
    return (vis + p.block_size - 1) / p.block_size;
}

// At most 64 VGPRs a lane (eight waves a SIMD): in a mixed step this kernel
// starts while the decode's waves (about 200 VGPRs) hold half of every CU,
// and its 16 waves need four per SIMD beside them; with more registers it
// could not be placed until the decode ended, and the chunks' attention would
// run after the decode instead of beside it.
__global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8)))
prefill_plan_kernel(PParams p) {
    __shared__ int hist[kMaxBins];
    __shared__ int wsum[16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    hist[2 * t] = 0;
    hist[2 * t + 1] = 0;
    // effective contexts: one wave per sequence, the first 512 table entries
    // of two sequences in flight at once (eight unconditional loads a lane
    // each, the index clamped into the row), longer walks in further rounds
    constexpr int kSeqsAtOnce = 2;
    const int cap = p.max_blocks * p.block_size;
    for (int n0 = wave; n0 < p.num_seqs; n0 += 16 * kSeqsAtOnce) {
        int32_t b[kSeqsAtOnce][8];
        int len[kSeqsAtOnce], pages[kSeqsAtOnce];
#pragma unroll
        for (int q = 0; q < kSeqsAtOnce; ++q) {
            const int n = min(n0 + 16 * q, p.num_seqs - 1);
            len[q] = max(0, min(p.start[n] + chunk_len(p, n), cap));
            pages[q] = (len[q] + p.block_size - 1) / p.block_size;
            const int32_t *row = p.bt + (size_t)n * p.max_blocks;
#pragma unroll
            for (int j = 0; j < 8; ++j) b[q][j] = row[min(j * kWave + lane, max(pages[q] - 1, 0))];
        }
#pragma unroll
        for (int q = 0; q < kSeqsAtOnce; ++q) {
            const int n = n0 + 16 * q;
            if (n >= p.num_seqs) break;
            int first_bad = pages[q];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int i = j * kWave + lane;
                if (i < pages[q] && (b[q][j] < 0 || (int64_t)b[q][j] >= p.num_blocks)) first_bad = min(first_bad, i);
            }
            for (int o = 32; o > 0; o >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, o));
            const int32_t *row = p.bt + (size_t)n * p.max_blocks;
            for (int i0 = 8 * kWave; i0 < pages[q] && first_bad == pages[q]; i0 += 8 * kWave) {
                int32_t c[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) c[j] = row[min(i0 + j * kWave + lane, pages[q] - 1)];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int i = i0 + j * kWave + lane;
                    if (i < pages[q] && (c[j] < 0 || (int64_t)c[j] >= p.num_blocks)) first_bad = min(first_bad, i);
                }
                for (int o = 32; o > 0; o >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, o));
            }
            if (lane == 0) p.eff[n] = min(len[q], first_bad * p.block_size);
        }
    }
    __threadfence_block();
    __syncthreads();
    const int Hkv = p.num_kv_heads;
    // group (n, kvh) -> XCD queue x, longest group first within the queue
    auto key = [&](int n, int kvh, int tiles) {
        const int x = (n * Hkv + kvh) % kXcds;
        const int maxp = tiles > 0 ? tile_pages(p, n, tiles - 1) : 0;
        return x * kXcdBins + kXcdBins - 1 - min(maxp / 8, kXcdBins - 1);
    };
    const int groups = p.num_seqs * Hkv;  // one thread per (n, kvh)
    for (int g = t; g < groups; g += 1024) {
        const int n = g / Hkv, kvh = g % Hkv;
        const int tiles = (chunk_len(p, n) + p.tq - 1) / p.tq;
        if (tiles > 0) atomicAdd(&hist[key(n, kvh, tiles)], tiles);
    }
    __syncthreads();
    // exclusive scan of the bins, two per thread (each thread rewrites only
    // its own two, so no barrier between reading and writing them)
    const int a = hist[2 * t], b = hist[2 * t + 1];
    int total;
    const int base = zk::block_exclusive_scan_1024(a + b, wsum, &total);
    hist[2 * t] = base;
    hist[2 * t + 1] = base + a;
    __syncthreads();
    if (t < kXcds) {  // segment of each XCD queue; its first waves take items statically
        const int start = hist[t * kXcdBins], end = t + 1 < kXcds ? hist[(t + 1) * kXcdBins] : total;
        int32_t *w = p.work + 64 + kQueueStride * t;
        w[0] = start;
        w[1] = end;
        w[2] = start + p.num_groups / kXcds;
    }
    __syncthreads();
    for (int g = t; g < groups; g += 1024) {
        const int n = g / Hkv, kvh = g % Hkv;
        const int tiles = (chunk_len(p, n) + p.tq - 1) / p.tq;
        if (tiles == 0) continue;
        const int pos = atomicAdd(&hist[key(n, kvh, tiles)], tiles);
        for (int j = 0; j < tiles; ++j) {  // the group's tiles back to back, longest first
            const int qt = tiles - 1 - j;
            p.items[pos + j] = make_int4(n, qt, tile_pages(p, n, qt), kvh);
        }
    }
    if (t == 0) p.work[0] = total;
}

typedef __attribute__((address_space(3))) void lds_void;
// Default cache policy: the tiles of one sequence read the same pages, and
// keeping them in L2 / MALL measured 17% faster than streaming them (NT).
constexpr int kCachePolicy = 0;
__device__ __forceinline__ void g2l16(const void *g, lds_void *l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, kCachePolicy);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }
// workgroup barrier without the fences of __syncthreads (those would wait for
// every load in flight); the memory clobber keeps LDS accesses on their side
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ float xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1f | (0x10 << 10)));
}
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32); }
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2_t));
}
typedef short v4i16 __attribute__((ext_vector_type(4)));
template <int BYTES>
struct LdsVec;
template <>
struct LdsVec<16> { typedef u32x4 T; };
template <>
struct LdsVec<8> { typedef u32x2 T; };
template <>
struct LdsVec<4> { typedef uint32_t T; };

template <int KV, int D, int G>
// At most 256 registers a lane (two waves a SIMD): the operands stay in
// VGPRs, so the kernel uses no AGPRs.
__global__ void __launch_bounds__(kWave * kWaves) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd)))
prefill_mfma_kernel(PParams p) {
    constexpr int BS = 16;
    constexpr int ELT = KV == ZK_BF16 ? 2 : 1;
    constexpr int DG = D / 4;         // head dims per lane group in QK
    constexpr int KK = DG / 8;        // MFMA k-steps
    constexpr int DT = D / 16;        // PV dim tiles = dims per lane per V row
    constexpr int RB = D * ELT;       // bytes per token row
    constexpr int CPR = RB / 16;      // 16-byte chunks per row
    constexpr int PAGE = BS * RB;     // bytes per (block, kv-head) page
    constexpr int LPK = PAGE / 1024;  // global_load_lds per page of K (or V)
    constexpr int PARTS = 4 / kWaves;  // (page, K|V) parts of a pair each wave loads
    constexpr int LPW = PARTS * LPK;   // loads per wave and pair
    constexpr int KBYTES = DG * ELT;
    constexpr int KCH = KBYTES / 16;
    constexpr int VTB = DT * ELT;
    constexpr int T = kTiles;
    static_assert(PAGE % 1024 == 0 && KBYTES % 16 == 0 && DT % 2 == 0, "page shape");
    typedef typename LdsVec<VTB>::T vtrow_t;
    __shared__ __attribute__((aligned(16))) char lds[kStages][2][2][PAGE];  // [stage][page of the pair][K|V]
    __shared__ int item_bcast;

    // wave w computes rows 32 w .. 32 w + 31 of every item and loads one
    // (page, K|V) part of every pair; every wave reads both pages
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave, col = lane & 15, grp = lane >> 4;
    const int H = p.num_heads, Hkv = p.num_kv_heads;
    uint32_t kg[LPK], vg[LPK];
#pragma unroll
    for (int j = 0; j < LPK; ++j) {
        const int q = 64 * j + lane, row = q / CPR, c = (q % CPR) ^ (row % CPR);
        kg[j] = row * RB + c * 16;
        // bf16 V: chunk c of row r sits at slot c ^ 2 (r mod CPR/2), so the
        // transposed reads below hit distinct banks; fp8 V stays natural
        vg[j] = KV == ZK_BF16 ? row * RB + ((q % CPR) ^ ((row % (CPR / 2)) << 1)) * 16 : q * 16;
    }
    uint32_t kl[KCH];
#pragma unroll
    for (int f = 0; f < KCH; ++f) {
        const int row = col, c = grp * KCH + f;
        kl[f] = (row * CPR + (c ^ (row % CPR))) * 16;
    }
    const uint32_t vt_off = (uint32_t)((4 * grp) * RB + col * VTB);
    // bf16 V^T fragments by ds_read_b64_tr_b16: in each 16-lane group, lane
    // j names 4 dims of key 4 grp + j / 4 and lane c receives dim c of those
    // 4 keys.  Dim tile dt of a page: vtr_base ^ (32 dt) (the XOR only moves
    // the swizzled slot).
    const uint32_t vtr_base = [&] {
        const int j = col, r = 4 * grp + j / 4;
        return (uint32_t)(r * RB + 32 * (r % (CPR / 2)) + 16 * ((j % 4) / 2) + 8 * (j % 2));
    }();

    // this wave's XCD queue (round-robin dispatch); its first item is static
    const int xcd = blockIdx.x % kXcds;
    const int32_t *myq = p.work + 64 + kQueueStride * xcd;
    int item = myq[0] + (int)blockIdx.x / kXcds;
    if (item >= myq[1]) item = -1;
    int next = -1;
    // thread 0: next item from this XCD's queue, else from the others'
    auto claim = [&]() {
        for (int k = 0; k < kXcds; ++k) {
            int32_t *wq = p.work + 64 + kQueueStride * ((xcd + k) % kXcds);
            if (__hip_atomic_load(&wq[2], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= wq[1]) continue;
            const int v = atomicAdd(&wq[2], 1);
            if (v < wq[1]) return v;
        }
        return -1;
    };
    // thread 0's item id to both waves, once both are done with the last
    // item (its LDS stages and the broadcast slot)
    auto bcast = [&](int v) {
        wg_barrier();
        if (threadIdx.x == 0) item_bcast = v;
        wait_lgkmcnt0();
        wg_barrier();
        return __builtin_amdgcn_readfirstlane(item_bcast);
    };
    if (item < 0) item = bcast(threadIdx.x == 0 ? claim() : -1);
    while (item >= 0) {
        const int4 desc = p.items[item];
        const int n = desc.x, qt = desc.y, np = desc.z, kvh = desc.w;
        const int len = chunk_len(p, n), st = p.start[n], eff = p.eff[n];
        const int64_t row0 = chunk_row0(p, n) + (int64_t)qt * p.tq;  // first q row of the item

        // rows: column col of this wave's tile t is item row r = 64 w + 16 t + col
        // = token r / G, head r % G
        bf16x8 qf[T][KK];
        int lim[T];       // keys at positions < lim[t] are visible to this lane's row
        bool real[T];     // the row is a chunk token (not padding past the chunk)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int r = kWaveRows * w + 16 * t + col, tok = qt * p.tq + r / G;
            real[t] = tok < len;
            const int tok_c = min(tok, len - 1);  // padding rows see what the last row sees
            lim[t] = min(p.causal ? st + tok_c + 1 : st + len, eff);
            if (real[t]) {
                const size_t qb = (size_t)(row0 + r / G) * (size_t)p.q_stride + (size_t)qhead_of(p, kvh, r % G, G) * D +
                                  (size_t)grp * DG;
                if (p.q_f32) {
                    const float *qq = (const float *)p.q + qb;
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) {
                        u32x4 w;
#pragma unroll
                        for (int j = 0; j < 4; ++j) w[j] = pack_bf16x2(qq[8 * kk + 2 * j], qq[8 * kk + 2 * j + 1]);
                        qf[t][kk] = __builtin_bit_cast(bf16x8, w);
                    }
                } else {
                    const uint16_t *qq = (const uint16_t *)p.q + qb;
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) qf[t][kk] = *reinterpret_cast<const bf16x8 *>(qq + 8 * kk);
                }
            } else {
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) qf[t][kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
            }
        }
        // the Q fragments are ready here (their loads' wait stays out of the
        // page loop)
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+v"(qf[t][kk]));
        float sl2 = p.scale_log2, vscale = 1.0f;
        if constexpr (KV == ZK_FP8_E4M3) {
            sl2 *= p.k_scales[(size_t)n * Hkv + kvh];
            vscale = p.v_scales[(size_t)n * Hkv + kvh];
        }
        // block ids by scalar loads (a constant-space view of the table: the
        // kernel never writes it)
        typedef const __attribute__((address_space(4))) int32_t *ctab_t;
        const ctab_t trow = (ctab_t)(p.bt + (size_t)n * p.max_blocks);
        const char *kbase = p.k_pool + ((size_t)kvh * PAGE);
        const char *vbase = p.v_pool + ((size_t)kvh * PAGE);
        const size_t block_bytes = (size_t)PAGE * Hkv;
        // Pages go through LDS in pairs: 32 keys per PV step feed the
        // 16x16x32 MFMA (the 16x16x16 form runs at half its rate).  Wave w
        // loads the K (w even) or V (w odd) of page w / 2 of every pair into
        // the pair's stage.  A missing second
        // page (odd page count) is loaded as a copy of the first, so every
        // wave issues the same loads per pair; its keys lie past every row's
        // limit and its V rows are zeroed below.
        // this wave's page of pair pj (waves 2 h and 2 h + 1 load page h's K
        // and V)
        static_assert(PARTS == 1, "a wave loads one (page, K|V) part of each pair");
        auto page_of = [&](int pj) { return trow[min(2 * pj + (w >> 1), np - 1)]; };
        // blk = page_of(pj), read one pair ahead: waiting for a scalar load
        // also waits for every LDS read issued before it
        auto issue = [&](int pj, int blk) {
            const int stg = pj & (kStages - 1);
#pragma unroll
            for (int q = 0; q < PARTS; ++q) {
                const int part = PARTS * w + q, kind = part & 1, pg = part >> 1;  // this wave's page, K or V
                const char *src = (kind ? vbase : kbase) + (size_t)blk * block_bytes;
#pragma unroll
                for (int j = 0; j < LPK; ++j)
                    g2l16(src + (kind ? vg[j] : kg[j]), (lds_void *)(lds[stg][pg][kind] + 1024 * j));
            }
        };
        f32x4 o[DT][T];
        // m: the rows' reference max (log2 units); lsum: every element of
        // column col holds the row's sum of weights (MFMA with a ones operand)
        float m[T];
        f32x4 lsum[T];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            m[t] = -INFINITY;
            lsum[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) o[dt][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
        const int npair = (np + 1) / 2;
        // V rows at or past vlim are zeroed: stale rows past the context and a
        // missing second page (its LDS holds another page's bytes, which may
        // not even be finite as fp8)
        const int vlim = min(eff, np * BS);
        // pairs every row sees whole: both pages below the item's first row's
        // limit (rows are token-major, limits grow with the row)
        const int open = min(p.causal ? st + qt * p.tq + 1 : st + len, eff) / BS / 2;

        // K of pair pj as MFMA A operands
        auto read_k = [&](int pj, bf16x8 (&kop)[2][KK]) {
            const int stg = pj & (kStages - 1);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t kw[KBYTES / 4];
#pragma unroll
                for (int f = 0; f < KCH; ++f) {
                    const u32x4 c4 = *reinterpret_cast<const u32x4 *>(lds[stg][h][0] + kl[f]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) kw[4 * f + j] = c4[j];
                }
#pragma unroll
                for (int kk = 0; kk < KK; ++kk) {
                    u32x4 w4;
                    if constexpr (KV == ZK_BF16) {
                        w4 = u32x4{kw[4 * kk], kw[4 * kk + 1], kw[4 * kk + 2], kw[4 * kk + 3]};
                    } else {
                        const u32x2 lo2 = e4m3x4_to_bf16x4(kw[2 * kk]), hi2 = e4m3x4_to_bf16x4(kw[2 * kk + 1]);
                        w4 = u32x4{lo2[0], lo2[1], hi2[0], hi2[1]};
                    }
                    kop[h][kk] = __builtin_bit_cast(bf16x8, w4);
                }
            }
        };
        // V^T of pair pj as MFMA A operands: k slots 8 grp + i (i < 4) are
        // keys 4 grp + i of the first page, 8 grp + 4 + i those of the second,
        // as in P^T.  ZERO: rows at or past vlim are zeroed.
        auto read_v = [&]<bool ZERO>(int pj, u32x4 (&va)[DT]) {
            const int stg = pj & (kStages - 1);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int key0 = (2 * pj + h) * BS + 4 * grp;  // position of this lane's first key
                if constexpr (KV == ZK_BF16) {
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) {
                        const u32x2 t2 = __builtin_bit_cast(
                            u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) v4i16 *)(lds[stg][h][1] + (vtr_base ^ (32 * dt)))));
                        va[dt][2 * h] = t2[0];
                        va[dt][2 * h + 1] = t2[1];
                    }
                    if (ZERO && key0 + 4 > vlim) {
                        const uint32_t lo = (key0 >= vlim ? 0u : 0xffffu) | (key0 + 1 >= vlim ? 0u : 0xffff0000u);
                        const uint32_t hi = (key0 + 2 >= vlim ? 0u : 0xffffu) | (key0 + 3 >= vlim ? 0u : 0xffff0000u);
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) {
                            va[dt][2 * h] &= lo;
                            va[dt][2 * h + 1] &= hi;
                        }
                    }
                } else {
                    vtrow_t vt[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        vt[i] = *reinterpret_cast<const vtrow_t *>(lds[stg][h][1] + vt_off + i * RB);
                    uint32_t w[4][DT / 2];  // V rows as bf16 pairs
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        uint32_t b8[DT / 4];
                        __builtin_memcpy(b8, &vt[i], DT);
#pragma unroll
                        for (int j = 0; j < DT / 4; ++j) {
                            const u32x2 c2 = e4m3x4_to_bf16x4(b8[j]);
                            w[i][2 * j] = c2[0];
                            w[i][2 * j + 1] = c2[1];
                        }
                    }
                    if (ZERO && key0 + 4 > vlim) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (key0 + i >= vlim)
#pragma unroll
                                for (int j = 0; j < DT / 2; ++j) w[i][j] = 0u;
                    }
#pragma unroll
                    for (int j = 0; j < DT / 2; ++j) {
                        va[2 * j][2 * h] = __builtin_amdgcn_perm(w[1][j], w[0][j], 0x05040100u);
                        va[2 * j][2 * h + 1] = __builtin_amdgcn_perm(w[3][j], w[2][j], 0x05040100u);
                        va[2 * j + 1][2 * h] = __builtin_amdgcn_perm(w[1][j], w[0][j], 0x07060302u);
                        va[2 * j + 1][2 * h + 1] = __builtin_amdgcn_perm(w[3][j], w[2][j], 0x07060302u);
                    }
                }
            }
        };
        // raw scores of the pair being turned into weights (the scale sits in
        // the exponent); -inf past a row's limit
        float scb[2][T][8];  // double buffer: pair j's scores and pair j + 1's
        // masks of pair pj's raw scores (pairs from open on): keys at or past a
        // row's limit get -inf
        auto mask_scores = [&](int pj, const f32x4 (&sacc)[2][T], float (&out)[T][8]) {
            const int key0a = 2 * pj * BS + 4 * grp, key0b = key0a + BS;
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    out[t][i] = key0a + i < lim[t] ? sacc[0][t][i] : -INFINITY;
                    out[t][4 + i] = key0b + i < lim[t] ? sacc[1][t][i] : -INFINITY;
                }
        };
        auto lane_max = [&](const float (&v)[8]) {
            return fmaxf(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])), fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7])));
        };
        if (npair > 0) issue(0, page_of(0));
        if (threadIdx.x == 0) next = claim();  // overlaps the first pairs' round trip
        for (int i = 1; i < min(npair, kStages - 1); ++i) issue(i, page_of(i));
        int nblk = npair > 0 ? page_of(kStages - 1) : 0;  // the next refill's page
        // pair 0's scores set the rows' reference maxima (key 0 is visible to
        // every row, so they are finite)
        if (npair > 0) {
            const int behind = min(npair - 1, kStages - 2);
            if (behind >= 2) wait_vmcnt<2 * LPW>();
            else if (behind == 1) wait_vmcnt<LPW>();
            else wait_vmcnt<0>();
            wg_barrier();
            bf16x8 kop[2][KK];
            read_k(0, kop);
            f32x4 sacc[2][T];
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    sacc[h][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk)
                        sacc[h][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[h][kk], qf[t][kk], sacc[h][t], 0, 0, 0);
                }
            mask_scores(0, sacc, scb[0]);
#pragma unroll
            for (int t = 0; t < T; ++t) {
                float cm = lane_max(scb[0][t]) * sl2;
                cm = fmaxf(cm, xor16(cm));
                m[t] = fmaxf(cm, xor32(cm));
            }
        }
        // Iteration j: the weights of pair j (P) go through PV while pair
        // j + 1's scores run on the MFMA pipe -- the exponentials of one pair
        // issue between the score MFMAs of the next, the next pair's maxima
        // between this pair's PV MFMAs.  A rescale, when a maximum grew, is
        // applied after PV and before the next pair's weights.  IN: pairs j
        // and j + 1 are open and pair j + 3 exists (no masks, no tests).  P:
        // the buffer of scb holding pair j's scores; IN iterations run in
        // pairs that alternate it, so pair j + 1's scores are produced in the
        // other buffer, not copied over the one being read.
        auto iter = [&]<bool IN, int P>(int j) {
            float (&sc)[T][8] = scb[P];
            float (&sn)[T][8] = scb[IN ? 1 - P : P];
            const bool nxt = IN || j + 1 < npair;
            if (nxt) {
                // this wave's part of pair j + 1 is in once only pair j + 2's
                // loads may fly; the barrier brings the other wave's part and
                // says both have left pair j - 1, whose stage takes pair j + 3
                if (IN || j + 2 < npair) wait_vmcnt<LPW>();
                else wait_vmcnt<0>();
                wg_barrier();
            }
            // K of pair j + 1 first (the score MFMAs need it first), then V of
            // pair j; both are pinned only where the MFMAs take them, so the
            // LDS reads all issue before the first wait
            bf16x8 kop[2][KK];
            if (nxt) read_k(j + 1, kop);
            u32x4 va[DT];
            if (IN || 2 * (j + 1) * BS <= vlim) read_v.template operator()<false>(j, va);
            else read_v.template operator()<true>(j, va);
            if (IN || j + kStages - 1 < npair) {
                issue(j + kStages - 1, nblk);
                nblk = page_of(j + kStages);
            }

            f32x4 sacc[2][T];  // pair j + 1's scores
            bf16x8 pb[T];      // pair j's weights
            if (nxt)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+v"(kop[h][kk]));
#pragma unroll
            for (int t = 0; t < T; ++t) {
                if (nxt)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        sacc[h][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                        for (int kk = 0; kk < KK; ++kk)
                            sacc[h][t] =
                                __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[h][kk], qf[t][kk], sacc[h][t], 0, 0, 0);
                    }
                float pr[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) pr[i] = exp2_fast(fmaf(sc[t][i], sl2, -m[t]));
                pb[t] = __builtin_bit_cast(bf16x8, u32x4{bf16x2_rne(pr[0], pr[1]), bf16x2_rne(pr[2], pr[3]),
                                                         bf16x2_rne(pr[4], pr[5]), bf16x2_rne(pr[6], pr[7])});
            }
            float mx[T];
            bool grow = false;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) asm volatile("" : "+v"(va[dt]));
#pragma unroll
            for (int t = 0; t < T; ++t) {
                lsum[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[t], lsum[t], 0, 0, 0);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
                    o[dt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, va[dt]), pb[t], o[dt][t],
                                                                       0, 0, 0);
            }
            if (nxt) {
                if constexpr (IN) {
#pragma unroll
                    for (int t = 0; t < T; ++t)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            sn[t][i] = sacc[0][t][i];
                            sn[t][4 + i] = sacc[1][t][i];
                        }
                } else {
                    mask_scores(j + 1, sacc, sn);
                }
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    mx[t] = lane_max(sn[t]) * sl2;
                    grow |= mx[t] > m[t] + kRescaleSlack;
                }
            }
            // lazy rescale (rare past the first pairs): O and the sums follow
            // the new maxima before pair j + 1's weights are formed
            if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
                for (int t = 0; t < T; ++t) {
                    float cm = fmaxf(mx[t], xor16(mx[t]));
                    cm = fmaxf(cm, xor32(cm));
                    const float m_new = fmaxf(m[t], cm);
                    const float alpha = exp2_fast(m[t] - m_new);
                    lsum[t] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt) o[dt][t] *= alpha;
                    m[t] = m_new;
                }
            }
        };
        const int in_end = min(open - 1, npair - (kStages - 1));  // iterations j < in_end are IN
        int j = 0;
        for (; j + 1 < in_end; j += 2) {  // two iterations a trip: the score buffers swap roles, no copies
            iter.template operator()<true, 0>(j);
            iter.template operator()<true, 1>(j + 1);
        }
        if (j < in_end) {
            iter.template operator()<true, 0>(j++);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < 8; ++i) scb[0][t][i] = scb[1][t][i];
        }
        for (; j < npair; ++j) iter.template operator()<false, 0>(j);

        // rows of this lane: item row 64 w + 16 t + col, dims 16 dt + 4 grp + i
        // (bf16 pools, transposed V reads) or DT (4 grp + i) + dt (fp8 pools)
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float lt = lsum[t][0];  // the row's total (every element holds it)
            if (!real[t]) continue;
            const int r = kWaveRows * w + 16 * t + col;
            const float inv = lt > 0.0f ? vscale / lt : 0.0f;
            const size_t ob = ((size_t)(row0 + r / G) * H + qhead_of(p, kvh, r % G, G)) * D;
            if constexpr (KV == ZK_BF16) {
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    const size_t od = ob + 16 * dt + 4 * grp;
                    if (p.q_f32) {
                        const f32x4 v = o[dt][t] * inv;
                        __builtin_memcpy((float *)p.out + od, &v, sizeof(v));
                    } else {
                        const uint32_t v[2] = {bf16x2_rne(o[dt][t][0] * inv, o[dt][t][1] * inv),
                                               bf16x2_rne(o[dt][t][2] * inv, o[dt][t][3] * inv)};
                        __builtin_memcpy((uint16_t *)p.out + od, v, sizeof(v));
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (p.q_f32) {
                        float v[DT];
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) v[dt] = o[dt][t][i] * inv;
                        __builtin_memcpy((float *)p.out + ob + DT * (4 * grp + i), v, sizeof(v));
                    } else {
                        uint32_t v[DT / 2];
#pragma unroll
                        for (int j = 0; j < DT / 2; ++j)
                            v[j] = bf16x2_rne(o[2 * j][t][i] * inv, o[2 * j + 1][t][i] * inv);
                        __builtin_memcpy((uint16_t *)p.out + ob + DT * (4 * grp + i), v, sizeof(v));
                    }
                }
            }
        }
        item = bcast(next);
    }
}

template <int KV, int D>
bool launch_g(const PParams &p, hipStream_t s, int G) {
    switch (G) {
        case 1: prefill_mfma_kernel<KV, D, 1><<<p.num_groups, kWave * kWaves, 0, s>>>(p); return true;
        case 2: prefill_mfma_kernel<KV, D, 2><<<p.num_groups, kWave * kWaves, 0, s>>>(p); return true;
        case 4: prefill_mfma_kernel<KV, D, 4><<<p.num_groups, kWave * kWaves, 0, s>>>(p); return true;
        case 8: prefill_mfma_kernel<KV, D, 8><<<p.num_groups, kWave * kWaves, 0, s>>>(p); return true;
        default: return false;
    }
}

// persistent workgroups: kWavesPerSimd waves a SIMD
int persistent_groups() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus * kWavesPerSimd * 4 / kWaves;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kWorkBytes = 2048;  // total + 8 XCD queues of 128 B

// Workspace: eff[N] | work (kWorkBytes: total, 8 XCD queues) | items[max_items * Hkv] (int4).
int max_items_for(int num_seqs, int64_t total_q, int num_heads, int num_kv_heads) {
    const int G = num_kv_heads > 0 ? std::max(1, num_heads / num_kv_heads) : 1;
    const int tq = std::max(1, kRows / G);
    const int64_t m = (total_q + tq - 1) / tq + num_seqs;
    return (int)std::min<int64_t>(m, 0x3fffffff);
}

int prefill_impl(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                 void *out, const int32_t *block_tables, const int64_t *cu_seqlens_q, const int64_t *q_off,
                 const int32_t *q_len, const int32_t *start_pos, int num_seqs, int64_t total_q, int num_heads,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                 float scale, int causal, zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                 void *workspace, size_t workspace_bytes, void *stream, int64_t q_stride, int max_groups);

}  // namespace

int zk::paged_prefill_rows(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool,
                           zk_dtype kv_dtype, void *out, const int32_t *block_tables, const int64_t *q_off,
                           const int32_t *q_len, const int32_t *start_pos, int num_seqs, int64_t total_q,
                           int num_heads, int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq,
                           int64_t num_blocks, float scale, int causal, zk_gqa_mapping mapping,
                           const float *k_scales, const float *v_scales, void *workspace, size_t workspace_bytes,
                           void *stream, int64_t q_stride, int max_groups) {
    if (!q_off || !q_len)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: paged prefill: NULL row offsets");
    return prefill_impl(q, q_dtype, k_pool, v_pool, kv_dtype, out, block_tables, nullptr, q_off, q_len, start_pos,
                        num_seqs, total_q, num_heads, num_kv_heads, head_dim, block_size, max_blocks_per_seq,
                        num_blocks, scale, causal, mapping, k_scales, v_scales, workspace, workspace_bytes, stream,
                        q_stride, max_groups);
}

extern "C" {

size_t zk_paged_prefill_workspace_size(int num_seqs, int64_t total_q, int num_heads, int num_kv_heads) {
    if (num_seqs <= 0 || total_q < 0) return 256;
    return align256(sizeof(int32_t) * (size_t)num_seqs) + kWorkBytes +
           align256(sizeof(int4) * (size_t)max_items_for(num_seqs, total_q, num_heads, num_kv_heads) *
                    (size_t)num_kv_heads);
}

int zk_paged_prefill(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                     void *out, const int32_t *block_tables, const int64_t *cu_seqlens_q, const int32_t *start_pos,
                     int num_seqs, int64_t total_q, int num_heads, int num_kv_heads, int head_dim, int block_size,
                     int max_blocks_per_seq, int64_t num_blocks, float scale, int causal, zk_gqa_mapping mapping,
                     const float *k_scales, const float *v_scales, void *workspace, size_t workspace_bytes,
                     void *stream) {
    if (num_seqs > 0 && total_q > 0 && !cu_seqlens_q)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_prefill: NULL pointer");
    return prefill_impl(q, q_dtype, k_pool, v_pool, kv_dtype, out, block_tables, cu_seqlens_q, nullptr, nullptr,
                        start_pos, num_seqs, total_q, num_heads, num_kv_heads, head_dim, block_size,
                        max_blocks_per_seq, num_blocks, scale, causal, mapping, k_scales, v_scales, workspace,
                        workspace_bytes, stream, 0, 0);
}

}  // extern "C"

namespace {

int prefill_impl(const void *q, zk_dtype q_dtype, const void *k_pool, const void *v_pool, zk_dtype kv_dtype,
                 void *out, const int32_t *block_tables, const int64_t *cu_seqlens_q, const int64_t *q_off,
                 const int32_t *q_len, const int32_t *start_pos, int num_seqs, int64_t total_q, int num_heads,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks_per_seq, int64_t num_blocks,
                 float scale, int causal, zk_gqa_mapping mapping, const float *k_scales, const float *v_scales,
                 void *workspace, size_t workspace_bytes, void *stream, int64_t q_stride, int max_groups) {
    if (q_dtype != ZK_F32 && q_dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_prefill: q dtype must be f32 or bf16");
    if (num_seqs < 0 || total_q < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
        max_blocks_per_seq <= 0 || num_blocks <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_prefill: bad shape");
    if (num_heads % num_kv_heads != 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_prefill: num_heads must be a multiple of num_kv_heads");
    if (mapping != ZK_GQA_GROUPED && mapping != ZK_GQA_MODULO)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_prefill: bad gqa mapping");
    const int G = num_heads / num_kv_heads;
    if (!zk::paged_prefill_supported(kv_dtype, head_dim, block_size, num_heads, num_kv_heads))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_prefill: needs bf16 or fp8 pools, block_size 16, head_dim 64 "
                         "or 128 and H/Hkv in {1, 2, 4, 8}");
    if (max_blocks_per_seq > kMaxBins)  // an item stages its block ids in LDS
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_prefill: max_blocks_per_seq above " + std::to_string(kMaxBins));
    if (num_seqs == 0 || total_q == 0) return ZK_OK;
    if (!q || !k_pool || !v_pool || !out || !block_tables || !start_pos || !workspace)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_paged_prefill: NULL pointer");
    const bool fp8 = kv_dtype == ZK_FP8_E4M3;
    if (fp8 != (k_scales != nullptr && v_scales != nullptr))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_prefill: fp8 pools need k/v scales, other pools none");
    const size_t need = zk_paged_prefill_workspace_size(num_seqs, total_q, num_heads, num_kv_heads);
    if (workspace_bytes < need || ((uintptr_t)workspace & 255u))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_paged_prefill: workspace too small or not 256-B aligned (need " +
                             std::to_string(need) + " bytes)");
    PParams p;
    p.q = q;
    p.k_pool = (const char *)k_pool;
    p.v_pool = (const char *)v_pool;
    p.out = out;
    p.bt = block_tables;
    p.cu_q = cu_seqlens_q;
    p.q_off = q_off;
    p.q_len = q_len;
    p.q_stride = q_stride > 0 ? q_stride : (int64_t)num_heads * head_dim;
    p.start = start_pos;
    p.k_scales = k_scales;
    p.v_scales = v_scales;
    char *ws = (char *)workspace;
    p.eff = (int32_t *)ws;
    p.work = (int32_t *)(ws + align256(sizeof(int32_t) * (size_t)num_seqs));
    p.items = (int4 *)(ws + align256(sizeof(int32_t) * (size_t)num_seqs) + kWorkBytes);
    p.num_seqs = num_seqs;
    p.num_heads = num_heads;
    p.num_kv_heads = num_kv_heads;
    p.head_dim = head_dim;
    p.block_size = block_size;
    p.max_blocks = max_blocks_per_seq;
    p.tq = kRows / G;
    // a whole number of workgroups per XCD queue
    p.num_groups = persistent_groups();
    if (max_groups >= kXcds) p.num_groups = std::min(p.num_groups, max_groups / kXcds * kXcds);
    p.max_items = max_items_for(num_seqs, total_q, num_heads, num_kv_heads);
    p.num_blocks = num_blocks;
    p.scale_log2 = scale * kLog2e;
    p.grouped = mapping == ZK_GQA_GROUPED ? 1 : 0;
    p.q_f32 = q_dtype == ZK_F32 ? 1 : 0;
    p.causal = causal ? 1 : 0;
    hipStream_t s = (hipStream_t)stream;
    {
        KernelTimer timer("prefill_plan", s);
        prefill_plan_kernel<<<1, 1024, 0, s>>>(p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: zk_paged_prefill plan: ") + hipGetErrorString(e));
    {
        KernelTimer timer("prefill_attention", s);
        if (kv_dtype == ZK_BF16) {
            if (head_dim == 128) launch_g<ZK_BF16, 128>(p, s, G);
            else launch_g<ZK_BF16, 64>(p, s, G);
        } else {
            if (head_dim == 128) launch_g<ZK_FP8_E4M3, 128>(p, s, G);
            else launch_g<ZK_FP8_E4M3, 64>(p, s, G);
        }
    }
    e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: zk_paged_prefill: ") + hipGetErrorString(e));
    return ZK_OK;
}

}  // namespace

bool zk::paged_prefill_supported(int kv_dtype, int head_dim, int block_size, int num_heads, int num_kv_heads) {
    if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return false;
    const int G = num_heads / num_kv_heads;
    return (kv_dtype == ZK_BF16 || kv_dtype == ZK_FP8_E4M3) && block_size == 16 &&
           (head_dim == 64 || head_dim == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

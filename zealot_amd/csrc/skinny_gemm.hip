// skinny_gemm.hip -- y[m, n] = x[m, k] . w[n, k]^T for m <= 64 (a decode
// step's projections) in bf16 with f32 accumulation, on MFMA.
//
// With at most 64 activation rows the product does at most 64 flops per
// weight byte, far below what the matrix cores sustain: it is bound by
// streaming w from HBM once.  The kernel is built around that stream:
//  - a workgroup owns a tile of 64 or 128 weight rows (four waves of one or
//    two 16-row MFMA tiles each) and a range of k / splits;
//  - weights and activations move to LDS by DMA (global_load_lds) in chunks
//    of 128 k, in a ring of three or four chunks (as deep as 160 KiB of LDS
//    allows): each wave fetches its own weight rows (nontemporal: every
//    weight byte is used once), and the chunk's x[0:m] is fetched once per
//    workgroup and shared by the four waves;
//  - every DMA reads whole 256-byte row segments, each lane fetching column
//    c ^ (row % 16) of its segment, so the MFMA operand reads (16 rows, one
//    column) hit 16 different bank groups;
//  - waits are explicit (the chunks issued after the awaited one stay in
//    flight), with one barrier per chunk;
//  - splits == 1: the waves write y; splits > 1: each range's sums go to a
//    workspace [splits][m][n] and skinny_reduce_kernel adds them in range
//    order, so the result does not depend on scheduling (or the RMSNorm
//    that follows the product adds them as it reads its rows: reduce ==
//    false, for zk_linear_rms_norm).
// Weights come row-major (nn.Linear layout) or tiled (tile_weight_kernel):
// [k / 128][n / 16][16 rows][16 units of 8 bf16], unit u of row r holding
// columns 8 (u ^ r) .. 8 (u ^ r) + 7 of the 128-column chunk, i.e. each
// 16 x 128 block exactly as the DMA leaves it in LDS.  Tiled, every DMA
// instruction reads 1 KiB of contiguous weights (row-major: four 256-byte
// segments k apart), and at any moment the grid streams one contiguous
// n x 256-byte slab: 17-19 % faster on the large projections.  With tiled
// weights m may exceed 64: blockIdx.y takes the columns 64 y .. 64 y + 63.
// MFMA 16x16x32 bf16 operand layout: lane l holds A[l % 16][8 (l / 16) + j]
// and B[8 (l / 16) + j][l % 16] for j < 8, and receives
// D[4 (l / 16) + r][l % 16] for r < 4.  A = weight rows, B = x^T, so lane l
// ends with y[column l % 16][rows 4 (l / 16) .. + 3] of each 16 x 16 tile.
#include <hip/hip_runtime.h>

#include "zk_common.h"

namespace {

using zk::bf16x8;
using zk::f32x4;
using zk::u32x4;
using zk::sum_ranges;

constexpr int kThreads = 256;  // four waves
constexpr int kChunk = 128;    // k per chunk: four MFMA k-steps, 256 bytes of a row

struct SkinnyArgs {
    const uint16_t *x;
    const uint16_t *w;
    void *y;
    float *partial;  // [splits][m][n] when splits > 1
    int m, n, k, kr, splits;  // kr = k / splits, the k range of a workgroup
};

__device__ __forceinline__ u32x4 ld_nt(const uint16_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

__device__ __forceinline__ void store4(void *y, bool f32, size_t at, f32x4 v) {
    if (f32) {
        *reinterpret_cast<f32x4 *>((float *)y + at) = v;
    } else {
        const zk::u32x2 o = {zk::pack_bf16x2(v[0], v[1]), zk::pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<zk::u32x2 *>((uint16_t *)y + at) = o;
    }
}

typedef __attribute__((address_space(3))) void lds_void;
// Weights stream with the nontemporal policy: every byte is read once.
constexpr int kWeightPolicy = 2;
template <int POLICY>
__device__ __forceinline__ void g2l16(const void *g, lds_void *l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, POLICY);
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
// workgroup barrier without the fences of __syncthreads (those would wait for
// every load in flight); the memory clobber keeps LDS accesses on their side
__device__ __forceinline__ void wg_barrier() { asm volatile("s_barrier" ::: "memory"); }

// LDS ring depth: four chunks where they fit in 160 KiB, else three.
constexpr int ring_depth(int mt, int rf) { return 4 * (64 * rf + 16 * mt) * 256 <= 163840 ? 4 : 3; }

// MT: 16-row tiles of x (ceil(m / 16), at most 4); RF: 16-row weight tiles per
// wave; TILED: the weight layout above, else row-major.
// SILU (RF = 2, no split, bf16 out): W holds gate and up rows interleaved in
// blocks of 16 (rows 32 b .. 32 b + 15 gate rows 16 b .., the next 16 the up
// rows of the same columns), so a wave's two tiles are the gate and up
// outputs of 16 columns, lane by lane; the wave writes
// y[m, n / 2] = silu(gate) * up instead of both (the value silu_mul_kernel
// computes from the rounded projection).
template <int MT, int RF, bool F32, bool SILU = false, bool TILED = false>
__global__ void __launch_bounds__(kThreads) skinny_linear_kernel(SkinnyArgs a) {
    constexpr int D = ring_depth(MT, RF);
    constexpr int WU = 16 * RF * 16;         // 16-byte units of a wave's weight chunk
    constexpr int XU = 16 * MT * 16;         // units of the workgroup's x chunk
    constexpr int WQ = WU / 64, XQ = XU / 64 / 4;  // DMA instructions a wave issues per chunk
    constexpr int L = WQ + XQ;
    static_assert(L * (D - 2) <= 63, "vmcnt range");
    __shared__ u32x4 lds[D * (4 * WU + XU)];
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tiles_n = a.n / (64 * RF);
    const int rt = blockIdx.x % tiles_n, s = blockIdx.x / tiles_n;
    const int r16 = lane & 15, g = lane >> 4;
    const size_t k = (size_t)a.k;
    const size_t kbeg = (size_t)s * a.kr;
    const int row0 = rt * 64 * RF + wv * 16 * RF;
    // this workgroup's columns of y (rows of x): 64 cb .. 64 cb + mb - 1
    const int cb = blockIdx.y, mb = min(64, a.m - 64 * cb);
    const uint16_t *xblk = a.x + (size_t)64 * cb * k;
    u32x4 *wring = lds + wv * WU;       // slot c: + c * (4 WU + XU)
    u32x4 *xring = lds + 4 * WU;

    // DMA q of a chunk moves rows 4 q .. 4 q + 3 of the tile (64 lanes, 16
    // lanes a row): lane l stores 16-byte unit l of the instruction, i.e.
    // row 4 q + l / 16 at column c' = l % 16, and fetches the row's column
    // c' ^ (row % 16) -- a permutation of one 256-byte segment per row, so
    // every DMA reads four whole segments, and the operand reads (16 rows,
    // one column) hit 16 different bank groups.
    // (tiled weights: the same units, in that order in memory already)
    const uint16_t *wsrc[WQ], *xsrc[XQ];
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int r = 4 * q + (lane >> 4), c = (lane & 15) ^ (r & 15);
        if constexpr (TILED)
            wsrc[q] = a.w + (((size_t)(kbeg / kChunk) * (a.n / 16) + (row0 + r) / 16) * 16 + ((row0 + r) & 15)) * kChunk +
                      8 * (lane & 15);
        else
            wsrc[q] = a.w + (size_t)(row0 + r) * k + kbeg + 8 * c;
    }
#pragma unroll
    for (int j = 0; j < XQ; ++j) {
        const int r = 4 * (wv * XQ + j) + (lane >> 4), c = (lane & 15) ^ (r & 15);
        xsrc[j] = xblk + (size_t)min(r, mb - 1) * k + kbeg + 8 * c;
    }
    // weight elements between consecutive chunks of a row
    const size_t wstep = TILED ? (size_t)a.n * kChunk : (size_t)kChunk;
    auto issue = [&](int c) {
        const int slot = c % D, off = c * kChunk;
        u32x4 *wl = wring + slot * (4 * WU + XU), *xl = xring + slot * (4 * WU + XU);
#pragma unroll
        for (int q = 0; q < WQ; ++q) g2l16<kWeightPolicy>(wsrc[q] + c * wstep, (lds_void *)(wl + 64 * q));
#pragma unroll
        for (int j = 0; j < XQ; ++j) g2l16<0>(xsrc[j] + off, (lds_void *)(xl + 64 * (wv * XQ + j)));
    };

    f32x4 acc[RF][MT];
#pragma unroll
    for (int f = 0; f < RF; ++f)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[f][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nchunks = a.kr / kChunk;
    for (int c = 0; c < D - 1 && c < nchunks; ++c) issue(c);
    for (int c = 0; c < nchunks; ++c) {
        // chunk c is in once only the D - 2 chunks issued after it may fly;
        // the barrier brings the other waves' parts of x and says every wave
        // has left chunk c - 1, whose slot takes chunk c + D - 1
        const int ahead = min(D - 2, nchunks - 1 - c);
        if (ahead >= 2) wait_vmcnt<2 * L>();
        else if (ahead == 1) wait_vmcnt<L>();
        else wait_vmcnt<0>();
        wg_barrier();
        const int slot = c % D;
        const u32x4 *wl = wring + slot * (4 * WU + XU), *xl = xring + slot * (4 * WU + XU);
        // k-step i: A rows 16 f + r16 and B rows 16 t + r16 at column 4 i + g
        bf16x8 av[RF][4], bv[MT][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int col = (4 * i + g) ^ r16;
#pragma unroll
            for (int f = 0; f < RF; ++f) av[f][i] = __builtin_bit_cast(bf16x8, wl[(16 * f + r16) * 16 + col]);
#pragma unroll
            for (int t = 0; t < MT; ++t) bv[t][i] = __builtin_bit_cast(bf16x8, xl[(16 * t + r16) * 16 + col]);
        }
        if (c + D - 1 < nchunks) issue(c + D - 1);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int f = 0; f < RF; ++f)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[f][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[f][i], bv[t][i], acc[f][t], 0, 0, 0);
    }

    // lane: column t * 16 + r16, rows row0 + 16 f + 4 g .. + 3
    if constexpr (SILU) {
        static_assert(RF == 2 && !F32, "gate and up tiles of one wave, bf16 out");
        const int inter = a.n / 2, c0 = (row0 / 32) * 16 + 4 * g;
        auto rounded = [](float x) { return __uint_as_float(zk::f32_to_bf16_bits(x) << 16); };
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int col = t * 16 + r16;
            if (col < mb) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gt = rounded(acc[0][t][e]), up = rounded(acc[1][t][e]);
                    v[e] = (gt / (1.0f + expf(-gt))) * up;
                }
                const zk::u32x2 o = {zk::pack_bf16x2(v[0], v[1]), zk::pack_bf16x2(v[2], v[3])};
                *reinterpret_cast<zk::u32x2 *>((uint16_t *)a.y + (size_t)(64 * cb + col) * inter + c0) = o;
            }
        }
        return;
    }
    void *out = a.splits == 1 ? a.y : (void *)(a.partial + (size_t)s * a.m * a.n);
    const bool f32 = F32 || a.splits > 1;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int col = t * 16 + r16;
        if (col < mb)
#pragma unroll
            for (int f = 0; f < RF; ++f)
                store4(out, f32, (size_t)(64 * cb + col) * a.n + row0 + 16 * f + 4 * g, acc[f][t]);
    }
}

// y[i] = sum over ranges s (in order) of partial[s][i], four outputs a thread.
template <bool F32>
__global__ void __launch_bounds__(kThreads) skinny_reduce_kernel(const float *__restrict__ partial, void *y,
                                                                 size_t quads, int splits) {
    const size_t q = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (q >= quads) return;
    const f32x4 *p = reinterpret_cast<const f32x4 *>(partial) + q;
    f32x4 v[1];
    sum_ranges(p, quads, splits, v);
    store4(y, F32, 4 * q, v[0]);
}

// grid: (weight tiles x splits, 64-column blocks of y)
dim3 grid_of(const SkinnyArgs &a, int tile_rows) {
    return dim3((uint32_t)(a.n / tile_rows) * a.splits, (uint32_t)((a.m + 63) / 64));
}

template <int MT, int RF, bool TILED>
void launch(const SkinnyArgs &a, bool f32, hipStream_t stream) {
    const dim3 grid = grid_of(a, 64 * RF);
    if (f32 || a.splits > 1)
        skinny_linear_kernel<MT, RF, true, false, TILED><<<grid, kThreads, 0, stream>>>(a);
    else
        skinny_linear_kernel<MT, RF, false, false, TILED><<<grid, kThreads, 0, stream>>>(a);
}

template <int RF, bool TILED>
void launch_rf(const SkinnyArgs &a, bool f32, hipStream_t stream) {
    switch ((a.m + 15) / 16) {
        case 1: launch<1, RF, TILED>(a, f32, stream); break;
        case 2: launch<2, RF, TILED>(a, f32, stream); break;
        case 3: launch<3, RF, TILED>(a, f32, stream); break;
        default: launch<4, RF, TILED>(a, f32, stream); break;
    }
}

template <int MT, bool TILED>
void launch_silu(const SkinnyArgs &a, hipStream_t stream) {
    skinny_linear_kernel<MT, 2, false, true, TILED><<<grid_of(a, 128), kThreads, 0, stream>>>(a);
}

// wt = the tiled layout of row-major w [n, k] (bf16): one 16-byte unit a
// thread, unit (j, b, r, u) of wt = columns 128 j + 8 (u ^ r) .. + 7 of row
// 16 b + r.
__global__ void __launch_bounds__(kThreads) tile_weight_kernel(const u32x4 *__restrict__ w, u32x4 *__restrict__ wt,
                                                               uint32_t nb, uint32_t kj, size_t units) {
    const size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= units) return;
    const uint32_t u = (uint32_t)(i & 15), r = (uint32_t)((i >> 4) & 15);
    const size_t jb = i >> 8;  // j * nb + b
    const uint32_t b = (uint32_t)(jb % nb), j = (uint32_t)(jb / nb);
    const size_t row = (size_t)b * 16 + r;
    wt[i] = w[row * ((size_t)kj * 16) + (size_t)j * 16 + (u ^ r)];
}

}  // namespace

namespace zk {

int skinny_linear_silu(const void *x, const void *w, void *act, int64_t m, int64_t n, int64_t k, hipStream_t stream,
                       bool tiled) {
    if (!skinny_linear_ok(m, n, k, 128, 1, tiled))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_silu_mul: unsupported shape");
    if (!x || !w || !act)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_silu_mul: NULL pointer");
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)act) & 15)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_silu_mul: operands not 16-byte aligned");
    SkinnyArgs a{(const uint16_t *)x, (const uint16_t *)w, act, nullptr, (int)m, (int)n, (int)k, (int)k, 1};
    if (tiled) {
        switch ((m + 15) / 16) {
            case 1: launch_silu<1, true>(a, stream); break;
            case 2: launch_silu<2, true>(a, stream); break;
            case 3: launch_silu<3, true>(a, stream); break;
            default: launch_silu<4, true>(a, stream); break;
        }
    } else {
        switch ((m + 15) / 16) {
            case 1: launch_silu<1, false>(a, stream); break;
            case 2: launch_silu<2, false>(a, stream); break;
            case 3: launch_silu<3, false>(a, stream); break;
            default: launch_silu<4, false>(a, stream); break;
        }
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: zk_linear_silu_mul: ") + hipGetErrorString(e));
    return ZK_OK;
}

bool skinny_linear_ok(int64_t m, int64_t n, int64_t k, int tile_rows, int splits, bool tiled) {
    return m >= 1 && m <= (tiled ? 64 * (int64_t)65535 : 64) && (tile_rows == 64 || tile_rows == 128) &&
           n >= tile_rows && n % tile_rows == 0 &&
           n <= 0x7fffffff && splits >= 1 && splits <= 64 && k > 0 && k <= 0x7fffffff &&
           k % ((int64_t)kChunk * splits) == 0 && (n / tile_rows) * (int64_t)splits <= 0x7fffffff;
}

size_t skinny_linear_partial_bytes(int64_t m, int64_t n, int splits) {
    return splits <= 1 ? 0 : (size_t)splits * m * n * sizeof(float);
}

int skinny_linear(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, bool f32_out, int tile_rows,
                  int splits, void *partial, size_t partial_bytes, hipStream_t stream, bool reduce, bool tiled) {
    if (!skinny_linear_ok(m, n, k, tile_rows, splits, tiled))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_skinny: unsupported shape");
    if (!x || !w || (!y && (reduce || splits == 1)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_skinny: NULL pointer");
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) & 15)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_skinny: operands not 16-byte aligned");
    if (splits > 1 && (!partial || ((uintptr_t)partial & 15) ||
                       partial_bytes < skinny_linear_partial_bytes(m, n, splits)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_skinny: workspace too small");
    SkinnyArgs a{(const uint16_t *)x, (const uint16_t *)w, y, (float *)partial,
                 (int)m, (int)n, (int)k, (int)(k / splits), splits};
    if (tiled) {
        if (tile_rows == 64) launch_rf<1, true>(a, f32_out, stream);
        else launch_rf<2, true>(a, f32_out, stream);
    } else {
        if (tile_rows == 64) launch_rf<1, false>(a, f32_out, stream);
        else launch_rf<2, false>(a, f32_out, stream);
    }
    if (splits > 1 && reduce) {
        const size_t quads = (size_t)m * n / 4;
        const uint32_t blocks = (uint32_t)((quads + kThreads - 1) / kThreads);
        if (f32_out)
            skinny_reduce_kernel<true><<<blocks, kThreads, 0, stream>>>((const float *)partial, y, quads, splits);
        else
            skinny_reduce_kernel<false><<<blocks, kThreads, 0, stream>>>((const float *)partial, y, quads, splits);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: zk_linear_skinny: ") + hipGetErrorString(e));
    return ZK_OK;
}

bool tile_weight_ok(int64_t n, int64_t k) {
    // one workgroup per 16 x 128 block: the grid's x extent
    return n > 0 && k > 0 && n % 16 == 0 && k % kChunk == 0 && n <= 0x7fffffff && k <= 0x7fffffff &&
           (n / 16) * (k / kChunk) <= 0x7fffffffll;
}

int tile_weight(const void *w, void *wt, int64_t n, int64_t k, hipStream_t stream) {
    if (!tile_weight_ok(n, k))
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_weight_tile: needs n % 16 == 0 and k % 128 == 0");
    if (!w || !wt) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_weight_tile: NULL pointer");
    if (((uintptr_t)w | (uintptr_t)wt) & 15)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_weight_tile: operands not 16-byte aligned");
    const size_t bytes = (size_t)n * k * 2;
    if ((const char *)w < (const char *)wt + bytes && (const char *)wt < (const char *)w + bytes)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_weight_tile: w and wt overlap");
    const size_t units = bytes / 16;
    tile_weight_kernel<<<(uint32_t)((units + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
        (const u32x4 *)w, (u32x4 *)wt, (uint32_t)(n / 16), (uint32_t)(k / kChunk), units);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(ZK_ERR_HIP, std::string("Internal error: zk_weight_tile: ") + hipGetErrorString(e));
    return ZK_OK;
}

}  // namespace zk

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
//   decode_mfma_kernel  bf16 / fp8 pools, D in {64,128}, G in {1,2,4,8}:
//       QK^T on MFMA (v_mfma_f32_16x16x32_bf16): A = one 16-token page of K
//       (rows = tokens, loaded straight from HBM, 16 B per lane), B = the G
//       query heads replicated over the 16 columns.  Lane l then holds the
//       scores of tokens 4*(l/16)+i (i<4) for head (l%16)%G, which are exactly
//       the tokens whose V rows the same lane loads for the PV product, so P
//       never leaves the lane's 16-lane row: the other heads' weights arrive by
//       DPP quad_perm (G<=4) or ds_swizzle (G=8) broadcasts.  Each 16-lane row
//       keeps its own online-softmax state; rows merge once per partition.
//   decode_generic_kernel  any dtype / D <= 256 / G <= 16 (fp32 pools):
//       token-per-lane QK on the VALU, readlane-broadcast PV.
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

int part_pages_config() {
    static int v = [] {
        const char *e = std::getenv("ZEALOT_DECODE_PART_PAGES");
        int p = e ? std::atoi(e) : 32;
        if (p < 1) p = 1;
        if (p > 64) p = 64;
        return p;
    }();
    return v;
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
    int32_t *eff_len;
    float2 *ml;   // [N][H][MP] (m, l), log2 domain
    float *po;    // [N][H][MP][D]
    int num_heads, num_kv_heads, head_dim, block_size, max_blocks, part_pages, max_parts;
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
    for (int i = threadIdx.x; i < pages; i += kWave) {
        int32_t b = row[i];
        if (b < 0 || (int64_t)b >= p.num_blocks) { first_bad = i; break; }
    }
    for (int o = 32; o > 0; o >>= 1) first_bad = min(first_bad, __shfl_xor(first_bad, o));
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

// ------------------------------------------------------------ MFMA kernel
// KV: ZK_BF16 or ZK_FP8_E4M3.  Template D (64 or 128), G (1, 2, 4, 8).
template <int KV, int D, int G>
__global__ void __launch_bounds__(kWave) decode_mfma_kernel(Params p) {
    constexpr int BS = 16;          // tokens per page (block_size)
    constexpr int DG = D / 4;       // dims per 16-lane row in the QK operand
    constexpr int KK = DG / 8;      // MFMA steps over the head dim
    constexpr int DV = D / 16;      // dims per lane in the PV product
    constexpr int ELT = KV == ZK_BF16 ? 2 : 1;
    constexpr int KBYTES = DG * ELT;  // K bytes per lane per page
    constexpr int VBYTES = DV * ELT;  // V bytes per lane per token row
    static_assert(KBYTES % 16 == 0 || KBYTES == 8, "K fragment size");

    const int part = blockIdx.x, kvh = blockIdx.y, n = blockIdx.z;
    const int lane = threadIdx.x;
    const int col = lane & 15, grp = lane >> 4;
    const int len = p.eff_len[n];
    const int pages = (len + BS - 1) / BS;
    const int nparts = (pages + p.part_pages - 1) / p.part_pages;
    if (part >= (nparts > 0 ? nparts : 1)) return;
    const int H = p.num_heads, Hkv = p.num_kv_heads;

    // ---- Q fragments (B operand): column col -> head col % G
    const int my_head = col % G;
    bf16x8 qf[KK];
    {
        const size_t qb = ((size_t)n * H + qhead_of(p, kvh, my_head, G)) * D + (size_t)grp * DG;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            uint32_t w[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float a = load_q(p, qb + 8 * kk + 2 * j), b = load_q(p, qb + 8 * kk + 2 * j + 1);
                w[j] = p.q_f32 ? pack_bf16x2(a, b) : (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
            }
            u32x4 v = {w[0], w[1], w[2], w[3]};
            qf[kk] = __builtin_bit_cast(bf16x8, v);
        }
    }
    float sl2 = p.scale_log2;
    float vscale = 1.0f;
    if constexpr (KV == ZK_FP8_E4M3) {
        sl2 *= p.k_scales[(size_t)n * Hkv + kvh];
        vscale = p.v_scales[(size_t)n * Hkv + kvh];
    }

    const int page0 = part * p.part_pages;
    const int np = nparts > 0 ? min(p.part_pages, pages - page0) : 0;
    // Block ids of this partition: lane i holds page page0 + i.
    const int32_t *btrow = p.bt + (size_t)n * p.max_blocks + page0;
    int bid_lane = lane < np ? btrow[lane] : 0;

    const size_t page_elems = (size_t)BS * D;
    const size_t head_stride = page_elems;             // (block, head) page
    const size_t block_stride = page_elems * Hkv;      // block
    const char *kbase = p.k_pool + ((size_t)kvh * head_stride) * ELT;
    const char *vbase = p.v_pool + ((size_t)kvh * head_stride) * ELT;
    // lane offsets inside a page (bytes)
    const size_t k_lane_off = ((size_t)col * D + (size_t)grp * DG) * ELT;
    const size_t v_lane_off = ((size_t)(4 * grp) * D + (size_t)col * DV) * ELT;

    typedef uint32_t kfrag_t __attribute__((ext_vector_type(KBYTES / 4)));
    typedef uint32_t vrow_t __attribute__((ext_vector_type(VBYTES >= 4 ? VBYTES / 4 : 1)));
    kfrag_t kcur, knext;
    vrow_t vcur[4], vnext[4];

    auto load_page = [&](int pi, kfrag_t &kf, vrow_t *vr) {
        int blk = __builtin_amdgcn_readlane(bid_lane, pi);
        const char *kp = kbase + (size_t)blk * block_stride * ELT + k_lane_off;
        const char *vp = vbase + (size_t)blk * block_stride * ELT + v_lane_off;
        kf = *reinterpret_cast<const kfrag_t *>(kp);
#pragma unroll
        for (int r = 0; r < 4; ++r) vr[r] = *reinterpret_cast<const vrow_t *>(vp + (size_t)r * D * ELT);
    };

    float o[G][DV];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < DV; ++d) o[h][d] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    if (np > 0) load_page(0, kcur, vcur);
    for (int pi = 0; pi < np; ++pi) {
        if (pi + 1 < np) load_page(pi + 1, knext, vnext);

        // ---- scores: S[token 4*grp + i][col] for i < 4
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            bf16x8 a;
            if constexpr (KV == ZK_BF16) {
                u32x4 w = {kcur[4 * kk], kcur[4 * kk + 1], kcur[4 * kk + 2], kcur[4 * kk + 3]};
                a = __builtin_bit_cast(bf16x8, w);
            } else {
                u32x2 lo = e4m3x4_to_bf16x4(kcur[2 * kk]);
                u32x2 hi = e4m3x4_to_bf16x4(kcur[2 * kk + 1]);
                u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
                a = __builtin_bit_cast(bf16x8, w);
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[kk], acc, 0, 0, 0);
        }
        const int tok0 = (page0 + pi) * BS + 4 * grp;
        float s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] = (tok0 + i < len) ? acc[i] * sl2 : -INFINITY;

        // ---- V rows of tokens 4*grp + r, dims col*DV .. +DV (as f32)
        float v[4][DV];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (KV == ZK_BF16) {
#pragma unroll
                for (int j = 0; j < DV / 2; ++j) {
                    v[r][2 * j] = bf16lo(vcur[r][j]);
                    v[r][2 * j + 1] = bf16hi(vcur[r][j]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < DV / 4; ++j) e4m3x4_to_f32(vcur[r][j], &v[r][4 * j]);
            }
        }
        if (tok0 + 4 > len) {  // partial last page: stale rows must not reach O
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (tok0 + r >= len)
#pragma unroll
                    for (int d = 0; d < DV; ++d) v[r][d] = 0.0f;
        }

        // ---- online softmax, per 16-lane row, for head my_head
        float mx = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        float m_new = fmaxf(m_run, mx);
        float alpha, pr[4];
        if (m_new == -INFINITY) {
            alpha = 1.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[i] = 0.0f;
        } else {
            alpha = exp2_fast(m_run - m_new);
#pragma unroll
            for (int i = 0; i < 4; ++i) pr[i] = exp2_fast(s[i] - m_new);
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

        if (pi + 1 < np) {
            kcur = knext;
#pragma unroll
            for (int r = 0; r < 4; ++r) vcur[r] = vnext[r];
        }
    }

    // ---- merge the four 16-lane rows
    float M = fmaxf(m_run, xor16(m_run));
    M = fmaxf(M, xor32(M));
    float f = (m_run == -INFINITY) ? 0.0f : exp2_fast(m_run - M);
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

    // Lanes 0..15 now hold o[h][col*DV + d]; lanes h < G hold (M, lsum) of head h.
    if (nparts <= 1) {
        static_for<G>([&](auto hc) {
            constexpr int h = decltype(hc)::value;
            const float l_h = head_bcast<G, h>(lsum);
            const float inv = l_h > 0.0f ? 1.0f / l_h : 0.0f;
            if (grp == 0) {
                const size_t ob = ((size_t)n * H + qhead_of(p, kvh, h, G)) * D + (size_t)col * DV;
#pragma unroll
                for (int d = 0; d < DV; ++d) store_out(p, ob + d, o[h][d] * inv);
            }
        });
    } else {
        static_for<G>([&](auto hc) {
            constexpr int h = decltype(hc)::value;
            const int qh = qhead_of(p, kvh, h, G);
            const size_t slot = ((size_t)n * H + qh) * p.max_parts + part;
            if (grp == 0) {
                float *dst = p.po + slot * D + (size_t)col * DV;
#pragma unroll
                for (int d = 0; d < DV; ++d) dst[d] = o[h][d];
            }
            if (lane == h) p.ml[slot] = make_float2(M, lsum);
        });
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
// One wavefront per (q-head, sequence): o = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p.
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
        float2 v = p.ml[base + i];
        L += v.x == -INFINITY ? 0.0f : v.y * exp2f(v.x - M);
    }
    for (int off = 32; off > 0; off >>= 1) L += __shfl_xor(L, off);
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    for (int d = lane; d < D; d += kWave) {
        float acc = 0.0f;
        for (int i = 0; i < nparts; ++i) {
            float2 v = p.ml[base + i];
            float w = v.x == -INFINITY ? 0.0f : exp2f(v.x - M);
            acc = fmaf(w, p.po[(base + i) * D + d], acc);
        }
        store_out(p, ((size_t)n * p.num_heads + h) * D + d, acc * inv);
    }
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
    size_t eff, ml, po, total;
};
WsLayout ws_layout(int num_seqs, int num_heads, int head_dim, int max_parts) {
    WsLayout w;
    w.eff = 0;
    w.ml = align256(sizeof(int32_t) * (size_t)num_seqs);
    size_t slots = (size_t)num_seqs * num_heads * max_parts;
    w.po = w.ml + align256(sizeof(float2) * slots);
    w.total = w.po + align256(sizeof(float) * slots * head_dim);
    return w;
}

int max_parts_for(int max_blocks, int part_pages) { return (max_blocks + part_pages - 1) / part_pages; }

template <int KV, int D, int G>
void launch_mfma(const Params &p, dim3 grid, hipStream_t s) {
    decode_mfma_kernel<KV, D, G><<<grid, kWave, 0, s>>>(p);
}

template <int KV, int D>
bool dispatch_g(const Params &p, dim3 grid, hipStream_t s, int G) {
    switch (G) {
        case 1: launch_mfma<KV, D, 1>(p, grid, s); return true;
        case 2: launch_mfma<KV, D, 2>(p, grid, s); return true;
        case 4: launch_mfma<KV, D, 4>(p, grid, s); return true;
        case 8: launch_mfma<KV, D, 8>(p, grid, s); return true;
        default: return false;
    }
}

template <int KV>
bool dispatch_mfma(const Params &p, dim3 grid, hipStream_t s, int G) {
    if (p.block_size != 16) return false;
    if (p.head_dim == 128) return dispatch_g<KV, 128>(p, grid, s, G);
    if (p.head_dim == 64) return dispatch_g<KV, 64>(p, grid, s, G);
    return false;
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
    (void)block_size;
    if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_blocks_per_seq <= 0) return 256;
    return ws_layout(num_seqs, num_heads, head_dim, max_parts_for(max_blocks_per_seq, part_pages_config()))
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
    const int part_pages = part_pages_config();
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
    p.ml = (float2 *)(ws + w.ml);
    p.po = (float *)(ws + w.po);
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

    dim3 grid(max_parts, num_kv_heads, num_seqs);
    bool done = false;
    {
    KernelTimer timer("decode_partials", s);
    if (kv_dtype == ZK_BF16) done = dispatch_mfma<ZK_BF16>(p, grid, s, G);
    else if (kv_dtype == ZK_FP8_E4M3) done = dispatch_mfma<ZK_FP8_E4M3>(p, grid, s, G);
    if (!done) {
        if (kv_dtype == ZK_F32) decode_generic_kernel<ZK_F32><<<grid, kWave, 0, s>>>(p);
        else if (kv_dtype == ZK_BF16) decode_generic_kernel<ZK_BF16><<<grid, kWave, 0, s>>>(p);
        else decode_generic_kernel<ZK_FP8_E4M3><<<grid, kWave, 0, s>>>(p);
    }
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

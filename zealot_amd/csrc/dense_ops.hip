// dense_ops.hip -- the elementwise / row-reduction ops around the paged-KV
// path, for gfx950: RMSNorm (optionally fused with the residual add that
// precedes it), SiLU(gate) * up, add and the embedding-row gather.
//
// Semantics of src/attention/kernels/rms_norm.cu:4-55 (out = x *
// rsqrt(mean(x^2) + eps) * w), activation.cu:4-20 (silu_gate_mul, add) and
// embedding.cu:4-22 (row gather by int64 token id); f32 or bf16 tensors with
// f32 arithmetic.  All are HBM-bound: every lane moves 16-byte vectors and
// each element is read and written once.
//
// Fusions (no reference counterpart):
//  - add + RMSNorm: s = x + residual is written back as the new residual and
//    normalised in the same pass (the reference launches add_kernel, then
//    rms_norm_kernel on its output).  For bf16 the norm uses the rounded sum,
//    the value the next layer reads.
//  - RMSNorm over selected rows (row index array): the final norm of the last
//    token of each sequence without a gather copy.
//  - SiLU * up reads gate and up through row strides, so a fused gate|up
//    projection output [T, 2 * inter] feeds it in place.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "zk_common.h"

using namespace zk;

namespace {

constexpr int kThreads = 256;

template <typename T> struct Vec;  // VEC elements in one 16-byte load
template <> struct Vec<float> {
    static constexpr int N = 4;
};
template <> struct Vec<uint16_t> {  // bf16 bits
    static constexpr int N = 8;
};

__device__ __forceinline__ void load_vec(const float *p, float *x) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(p);
    x[0] = v[0]; x[1] = v[1]; x[2] = v[2]; x[3] = v[3];
}
__device__ __forceinline__ void store_vec(float *p, const float *x) {
    *reinterpret_cast<f32x4 *>(p) = f32x4{x[0], x[1], x[2], x[3]};
}
__device__ __forceinline__ void load_vec(const uint16_t *p, float *x) {
    const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = bf16lo(v[i]);
        x[2 * i + 1] = bf16hi(v[i]);
    }
}
__device__ __forceinline__ void store_vec(uint16_t *p, const float *x) {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    *reinterpret_cast<u32x4 *>(p) = v;
}
// value as stored in T (the rounding a bf16 tensor applies)
__device__ __forceinline__ float stored(float x, const float *) { return x; }
__device__ __forceinline__ float stored(float x, const uint16_t *) {
    return __uint_as_float(f32_to_bf16_bits(x) << 16);
}
__device__ __forceinline__ float load1(const float *p) { return *p; }
__device__ __forceinline__ float load1(const uint16_t *p) { return __uint_as_float((uint32_t)*p << 16); }
__device__ __forceinline__ void store1(float *p, float x) { *p = x; }
__device__ __forceinline__ void store1(uint16_t *p, float x) { *p = (uint16_t)f32_to_bf16_bits(x); }

// Sum over the 256 threads of a workgroup.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) s += red[w];
    return s;
}

// ---------------------------------------------------------------- RMSNorm
// One workgroup per output row; each thread keeps its MAXV vectors of the
// row in registers between the sum of squares and the scaled write.
// in_row = rows ? rows[blockIdx.x] : blockIdx.x selects the input row;
// residual (optional) is added first and the sum written to res_out.  A
// workgroup reads its whole row before the reduction and writes after it, so
// out may be x (without row selection) and res_out may be residual.
// PART: the input row is not read from x but is the projection output a
// split-k skinny product leaves as f32 sums [splits][rows][dim] in `partial`:
// x = T(sum over ranges, in range order), the value its reduce kernel would
// have stored (VEC > 1 only).  FOLD: the ranges loaded up front (at least
// `splits` where the register budget allows: a range past `splits` is a
// wasted load instruction).
template <typename T, int VEC, int MAXV, bool PART = false, int FOLD = kFoldLoads>
__global__ void __launch_bounds__(kThreads)
rms_norm_kernel(const T *x, const T *residual, const T *__restrict__ w, T *out, T *res_out,
                const int64_t *__restrict__ rows, int dim, float eps,  // out may be x, res_out residual
                const float *__restrict__ partial = nullptr, int splits = 0) {
    __shared__ float red[kThreads / 64];
    const int64_t r_in = rows ? rows[blockIdx.x] : (int64_t)blockIdx.x;
    const T *xr = PART ? nullptr : x + (size_t)r_in * dim;
    const T *rr = residual ? residual + (size_t)r_in * dim : nullptr;
    float v[MAXV][VEC], wv[MAXV][VEC];
    float ss = 0.0f;
    if constexpr (PART) {
        static_assert(VEC % 4 == 0, "f32x4 sums");
        constexpr int N4 = VEC / 4;
        // ranges loaded up front, within a budget of 32 16-byte loads a thread
        constexpr int FB = 32 / (MAXV * N4);
        constexpr int FL = FB < 1 ? 1 : FB > FOLD ? FOLD : FB;
        const size_t plane4 = (size_t)gridDim.x * dim / 4;
        f32x4 t[MAXV][FL][N4];
        float a[MAXV][VEC];
        // every load of the row before any arithmetic: the first FL ranges'
        // sums, the residual and the weights in one memory round trip
        // (no branch around a load: a lane past the row's end re-reads its
        // start, a range past `splits` range 0, the residual without rr the
        // weights; unused values, but guarded loads make the compiler wait)
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int i0 = (j * kThreads + (int)threadIdx.x) * VEC, i = i0 < dim ? i0 : 0;
            const f32x4 *pp = reinterpret_cast<const f32x4 *>(partial + (size_t)r_in * dim + i);
#pragma unroll
            for (int r = 0; r < FL; ++r)
#pragma unroll
                for (int q = 0; q < N4; ++q) t[j][r][q] = pp[fold_offset(r, splits, plane4) + q];
            load_vec((rr ? rr : w) + i, a[j]);
            load_vec(w + i, wv[j]);
        }
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int i = (j * kThreads + (int)threadIdx.x) * VEC;
            if (i < dim) {
                const f32x4 *pp = reinterpret_cast<const f32x4 *>(partial + (size_t)r_in * dim + i);
                f32x4 acc[N4];
#pragma unroll
                for (int q = 0; q < N4; ++q) acc[q] = t[j][0][q];
#pragma unroll
                for (int r = 1; r < FL; ++r)
#pragma unroll
                    for (int q = 0; q < N4; ++q) acc[q] = r < splits ? acc[q] + t[j][r][q] : acc[q];
                for (int r = FL; r < splits; ++r)  // range order, as the reduce kernel adds them
#pragma unroll
                    for (int q = 0; q < N4; ++q) acc[q] += pp[(size_t)r * plane4 + q];
#pragma unroll
                for (int e = 0; e < VEC; ++e) v[j][e] = stored(acc[e / 4][e % 4], (const T *)nullptr);
                if (rr) {
#pragma unroll
                    for (int e = 0; e < VEC; ++e) v[j][e] = stored(v[j][e] + a[j][e], (const T *)nullptr);
                    store_vec(res_out + (size_t)blockIdx.x * dim + i, v[j]);
                }
#pragma unroll
                for (int e = 0; e < VEC; ++e) ss += v[j][e] * v[j][e];
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int i = (j * kThreads + (int)threadIdx.x) * VEC;
            if (i < dim) {
                // the weights load with the row (not after the reduction): one
                // memory round trip per launch instead of two
                if (VEC > 1) load_vec(w + i, wv[j]);
                else wv[j][0] = load1(w + i);
                if (VEC > 1) {
                    load_vec(xr + i, v[j]);
                    if (rr) {
                        float a[VEC];
                        load_vec(rr + i, a);
#pragma unroll
                        for (int e = 0; e < VEC; ++e) v[j][e] = stored(v[j][e] + a[e], (const T *)nullptr);
                        store_vec(res_out + (size_t)blockIdx.x * dim + i, v[j]);
                    }
                } else {
                    v[j][0] = load1(xr + i);
                    if (rr) {
                        v[j][0] = stored(v[j][0] + load1(rr + i), (const T *)nullptr);
                        store1(res_out + (size_t)blockIdx.x * dim + i, v[j][0]);
                    }
                }
#pragma unroll
                for (int e = 0; e < VEC; ++e) ss += v[j][e] * v[j][e];
            }
        }
    }
    const float inv = rsqrtf(block_sum(ss, red) / (float)dim + eps);
    T *orow = out + (size_t)blockIdx.x * dim;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int i = (j * kThreads + (int)threadIdx.x) * VEC;
        if (i < dim) {
            float o[VEC];
#pragma unroll
            for (int e = 0; e < VEC; ++e) o[e] = v[j][e] * inv * wv[j][e];
            if (VEC > 1) store_vec(orow + i, o);
            else store1(orow + i, o[0]);
        }
    }
}

// ---------------------------------------------------------- SiLU * up, add
// BLOCKED: gate and up are the column blocks of one projection output whose
// gate / up columns alternate in blocks of 16: output column c reads gate
// column 32 (c / 16) + c % 16 and up column 16 after it (VEC divides 16).
template <typename T, int VEC, bool BLOCKED = false>
__global__ void __launch_bounds__(kThreads)
silu_mul_kernel(const T *__restrict__ gate, const T *__restrict__ up, T *__restrict__ out, int64_t rows, int cols,
                int64_t gate_stride, int64_t up_stride) {
    const int64_t per_row = cols / VEC;
    const int64_t total = rows * per_row;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t r = idx / per_row;
        const int c = (int)(idx - r * per_row) * VEC;
        const int gc = BLOCKED ? (c / 16) * 32 + c % 16 : c, uc = BLOCKED ? gc + 16 : c;
        float g[VEC], u[VEC], o[VEC];
        if (VEC > 1) {
            load_vec(gate + r * gate_stride + gc, g);
            load_vec(up + r * up_stride + uc, u);
        } else {
            g[0] = load1(gate + r * gate_stride + gc);
            u[0] = load1(up + r * up_stride + uc);
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) o[e] = (g[e] / (1.0f + expf(-g[e]))) * u[e];
        if (VEC > 1) store_vec(out + r * cols + c, o);
        else store1(out + r * cols + c, o[0]);
    }
}

template <typename T, int VEC>
__global__ void __launch_bounds__(kThreads)
add_kernel(const T *__restrict__ a, const T *__restrict__ b, T *__restrict__ out, int64_t n) {
    const int64_t nv = n / VEC;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < nv; idx += (int64_t)gridDim.x * kThreads) {
        float x[VEC], y[VEC];
        if (VEC > 1) {
            load_vec(a + idx * VEC, x);
            load_vec(b + idx * VEC, y);
        } else {
            x[0] = load1(a + idx);
            y[0] = load1(b + idx);
        }
#pragma unroll
        for (int e = 0; e < VEC; ++e) x[e] += y[e];
        if (VEC > 1) store_vec(out + idx * VEC, x);
        else store1(out + idx, x[0]);
    }
}

// ----------------------------------------------------------------- embedding
// One workgroup per token; an id outside [0, vocab) yields a zero row.
__global__ void __launch_bounds__(kThreads)
embedding_kernel(const int64_t *__restrict__ ids, const char *__restrict__ table, char *__restrict__ out,
                 int64_t vocab, int64_t row_bytes, int vec) {
    const int64_t id = ids[blockIdx.x];
    const bool ok = id >= 0 && id < vocab;
    const char *src = table + (ok ? id : 0) * row_bytes;
    char *dst = out + (int64_t)blockIdx.x * row_bytes;
    if (vec) {
        for (int64_t o = (int64_t)threadIdx.x * 16; o < row_bytes; o += kThreads * 16) {
            u32x4 v = ok ? *reinterpret_cast<const u32x4 *>(src + o) : u32x4{0, 0, 0, 0};
            *reinterpret_cast<u32x4 *>(dst + o) = v;
        }
    } else {
        for (int64_t o = threadIdx.x; o < row_bytes; o += kThreads) dst[o] = ok ? src[o] : 0;
    }
}

int grid_for(int64_t work) {
    // enough workgroups to cover 8 per CU on 256 CUs, the rest by grid stride
    const int64_t g = (work + kThreads - 1) / kThreads;
    return (int)std::max<int64_t>(1, std::min<int64_t>(g, 2048));
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int check(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(ZK_ERR_HIP, std::string("Internal error: ") + what + ": " + hipGetErrorString(e));
    return ZK_OK;
}

template <typename T, int VEC, int MAXV>
void launch_norm(int rows_n, const void *x, const void *res, const void *w, void *out, void *res_out,
                 const int64_t *rows, int dim, float eps, hipStream_t s) {
    rms_norm_kernel<T, VEC, MAXV><<<rows_n, kThreads, 0, s>>>((const T *)x, (const T *)res, (const T *)w, (T *)out,
                                                               (T *)res_out, rows, dim, eps);
}

template <typename T>
int norm_dispatch(int rows_n, const void *x, const void *res, const void *w, void *out, void *res_out,
                  const int64_t *rows, int dim, float eps, hipStream_t s) {
    constexpr int V = Vec<T>::N;
    const bool vec = dim % V == 0 && aligned16(x) && aligned16(w) && aligned16(out) && (!res || aligned16(res)) &&
                     (!res_out || aligned16(res_out));
    const int per = vec ? V : 1;
    const int chunks = (dim + kThreads * per - 1) / (kThreads * per);
    if (vec) {
        if (chunks <= 1) launch_norm<T, V, 1>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else if (chunks <= 2) launch_norm<T, V, 2>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else if (chunks <= 4) launch_norm<T, V, 4>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else if (chunks <= 8) launch_norm<T, V, 8>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else if (chunks <= 16) launch_norm<T, V, 16>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else return -1;
    } else {
        if (chunks <= 4) launch_norm<T, 1, 4>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else if (chunks <= 16) launch_norm<T, 1, 16>(rows_n, x, res, w, out, res_out, rows, dim, eps, s);
        else return -1;
    }
    return 0;
}

template <int MAXV, int FOLD>
void launch_norm_fold(int rows_n, const float *partial, int splits, const void *res, const void *w, void *out,
                      void *res_out, int dim, float eps, hipStream_t s) {
    rms_norm_kernel<uint16_t, 8, MAXV, true, FOLD><<<rows_n, kThreads, 0, s>>>(
        nullptr, (const uint16_t *)res, (const uint16_t *)w, (uint16_t *)out, (uint16_t *)res_out, nullptr, dim, eps,
        partial, splits);
}

// ranges loaded up front: splits rounded up to 2, 4 or 8
template <int MAXV>
void launch_norm_partials(int rows_n, const float *partial, int splits, const void *res, const void *w, void *out,
                          void *res_out, int dim, float eps, hipStream_t s) {
    if (splits <= 2) launch_norm_fold<MAXV, 2>(rows_n, partial, splits, res, w, out, res_out, dim, eps, s);
    else if (splits <= 4) launch_norm_fold<MAXV, 4>(rows_n, partial, splits, res, w, out, res_out, dim, eps, s);
    else launch_norm_fold<MAXV, kFoldLoads>(rows_n, partial, splits, res, w, out, res_out, dim, eps, s);
}

}  // namespace

namespace zk {

int silu_mul_blocked(const void *gu, void *act, int64_t rows, int64_t inter, hipStream_t s) {
    if (rows < 0 || inter <= 0 || inter % 16 || !gu || !act)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: blocked silu_mul: bad arguments");
    if (rows == 0) return ZK_OK;
    const int grid_v = grid_for(rows * inter / 8), grid_1 = grid_for(rows * inter);
    if (aligned16(gu) && aligned16(act))
        silu_mul_kernel<uint16_t, 8, true><<<grid_v, kThreads, 0, s>>>(
            (const uint16_t *)gu, (const uint16_t *)gu, (uint16_t *)act, rows, (int)inter, 2 * inter, 2 * inter);
    else
        silu_mul_kernel<uint16_t, 1, true><<<grid_1, kThreads, 0, s>>>(
            (const uint16_t *)gu, (const uint16_t *)gu, (uint16_t *)act, rows, (int)inter, 2 * inter, 2 * inter);
    return check("blocked silu_mul");
}

bool rms_norm_partials_ok(int64_t rows, int64_t dim) {
    return rows >= 1 && rows <= 0x7fffffff && dim >= 8 && dim % 8 == 0 && dim <= 32768;
}

int rms_norm_partials(const float *partial, int splits, const void *residual, const void *weight, void *out,
                      void *residual_out, int64_t rows, int64_t dim, float eps, hipStream_t s) {
    if (!rms_norm_partials_ok(rows, dim) || splits < 1 || !partial || !weight || !out ||
        (residual && !residual_out))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: rms_norm over split-k sums: bad arguments");
    if (!aligned16(partial) || !aligned16(weight) || !aligned16(out) || (residual && !aligned16(residual)) ||
        (residual_out && !aligned16(residual_out)))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: rms_norm over split-k sums: not 16-byte aligned");
    const int chunks = (int)((dim + kThreads * 8 - 1) / (kThreads * 8));
    const int r = (int)rows, d = (int)dim;
    if (chunks <= 1) launch_norm_partials<1>(r, partial, splits, residual, weight, out, residual_out, d, eps, s);
    else if (chunks <= 2) launch_norm_partials<2>(r, partial, splits, residual, weight, out, residual_out, d, eps, s);
    else if (chunks <= 4) launch_norm_partials<4>(r, partial, splits, residual, weight, out, residual_out, d, eps, s);
    else if (chunks <= 8) launch_norm_partials<8>(r, partial, splits, residual, weight, out, residual_out, d, eps, s);
    else launch_norm_partials<16>(r, partial, splits, residual, weight, out, residual_out, d, eps, s);
    return check("rms_norm over split-k sums");
}

}  // namespace zk

extern "C" {

int zk_rms_norm(const void *x, const void *residual, const void *weight, void *out, void *residual_out,
                const int64_t *rows, int64_t num_rows, int64_t dim, float eps, zk_dtype dtype, void *stream) {
    if (dtype != ZK_F32 && dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_rms_norm: dtype must be f32 or bf16");
    if (num_rows < 0 || dim <= 0 || dim > (1 << 24) || num_rows > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_rms_norm: bad shape");
    if (num_rows == 0) return ZK_OK;
    if (!x || !weight || !out || (residual && !residual_out))
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_rms_norm: NULL pointer");
    hipStream_t s = (hipStream_t)stream;
    KernelTimer timer("rms_norm", s);
    const int rc = dtype == ZK_BF16
                       ? norm_dispatch<uint16_t>((int)num_rows, x, residual, weight, out, residual_out, rows, (int)dim,
                                                 eps, s)
                       : norm_dispatch<float>((int)num_rows, x, residual, weight, out, residual_out, rows, (int)dim,
                                              eps, s);
    if (rc)
        return set_error(ZK_ERR_INVALID_ARGUMENT,
                         "Internal error: zk_rms_norm: dim " + std::to_string(dim) +
                             " too large (at most 32768 bf16 / 16384 f32 elements with 16-byte rows, 4096 otherwise)");
    return check("zk_rms_norm");
}

int zk_silu_mul(const void *gate, const void *up, void *out, int64_t rows, int64_t cols, int64_t gate_stride,
                int64_t up_stride, zk_dtype dtype, void *stream) {
    if (dtype != ZK_F32 && dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_silu_mul: dtype must be f32 or bf16");
    if (rows < 0 || cols <= 0 || cols > 0x7fffffff)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_silu_mul: bad shape");
    if (gate_stride == 0) gate_stride = cols;
    if (up_stride == 0) up_stride = cols;
    if (gate_stride < cols || up_stride < cols)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_silu_mul: row stride below cols");
    if (rows == 0) return ZK_OK;
    if (!gate || !up || !out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_silu_mul: NULL pointer");
    hipStream_t s = (hipStream_t)stream;
    KernelTimer timer("silu_mul", s);
    const int V = dtype == ZK_BF16 ? 8 : 4;
    const bool vec = cols % V == 0 && gate_stride % V == 0 && up_stride % V == 0 && aligned16(gate) &&
                     aligned16(up) && aligned16(out);
    const int grid = grid_for(rows * (vec ? cols / V : cols));
    if (dtype == ZK_BF16) {
        if (vec)
            silu_mul_kernel<uint16_t, 8><<<grid, kThreads, 0, s>>>((const uint16_t *)gate, (const uint16_t *)up,
                                                                   (uint16_t *)out, rows, (int)cols, gate_stride,
                                                                   up_stride);
        else
            silu_mul_kernel<uint16_t, 1><<<grid, kThreads, 0, s>>>((const uint16_t *)gate, (const uint16_t *)up,
                                                                   (uint16_t *)out, rows, (int)cols, gate_stride,
                                                                   up_stride);
    } else {
        if (vec)
            silu_mul_kernel<float, 4><<<grid, kThreads, 0, s>>>((const float *)gate, (const float *)up, (float *)out,
                                                                rows, (int)cols, gate_stride, up_stride);
        else
            silu_mul_kernel<float, 1><<<grid, kThreads, 0, s>>>((const float *)gate, (const float *)up, (float *)out,
                                                                rows, (int)cols, gate_stride, up_stride);
    }
    return check("zk_silu_mul");
}

int zk_add(const void *a, const void *b, void *out, int64_t n, zk_dtype dtype, void *stream) {
    if (dtype != ZK_F32 && dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_add: dtype must be f32 or bf16");
    if (n < 0) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_add: bad shape");
    if (n == 0) return ZK_OK;
    if (!a || !b || !out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_add: NULL pointer");
    hipStream_t s = (hipStream_t)stream;
    KernelTimer timer("add", s);
    const int V = dtype == ZK_BF16 ? 8 : 4;
    const bool vec = n % V == 0 && aligned16(a) && aligned16(b) && aligned16(out);
    const int grid = grid_for(vec ? n / V : n);
    if (dtype == ZK_BF16) {
        if (vec) add_kernel<uint16_t, 8><<<grid, kThreads, 0, s>>>((const uint16_t *)a, (const uint16_t *)b,
                                                                   (uint16_t *)out, n);
        else add_kernel<uint16_t, 1><<<grid, kThreads, 0, s>>>((const uint16_t *)a, (const uint16_t *)b,
                                                              (uint16_t *)out, n);
    } else {
        if (vec) add_kernel<float, 4><<<grid, kThreads, 0, s>>>((const float *)a, (const float *)b, (float *)out, n);
        else add_kernel<float, 1><<<grid, kThreads, 0, s>>>((const float *)a, (const float *)b, (float *)out, n);
    }
    return check("zk_add");
}

int zk_embedding(const int64_t *ids, const void *table, void *out, int64_t num_tokens, int64_t vocab, int64_t dim,
                 zk_dtype dtype, void *stream) {
    if (dtype != ZK_F32 && dtype != ZK_BF16)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_embedding: dtype must be f32 or bf16");
    if (num_tokens < 0 || num_tokens > 0x7fffffff || vocab <= 0 || dim <= 0)
        return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_embedding: bad shape");
    if (num_tokens == 0) return ZK_OK;
    if (!ids || !table || !out) return set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_embedding: NULL pointer");
    hipStream_t s = (hipStream_t)stream;
    KernelTimer timer("embedding", s);
    const int64_t row_bytes = dim * elt_size(dtype);
    const bool vec = row_bytes % 16 == 0 && aligned16(table) && aligned16(out);
    embedding_kernel<<<(unsigned)num_tokens, kThreads, 0, s>>>(ids, (const char *)table, (char *)out, vocab,
                                                               row_bytes, vec ? 1 : 0);
    return check("zk_embedding");
}

}  // extern "C"

// gemm.cpp -- the dense projections around the paged-KV path on hipBLASLt.
//
// y[m, n] = x[m, k] . w[n, k]^T (nn.Linear weight layout), the product every
// cublasSgemm_v2 site of the reference computes (attention/cublas.rs:72-114,
// called at cuda_runner.rs:331-369 q/k/v, :483-495 o_proj, :531-559 gate/up,
// :577-589 down, :627-639 lm_head).  Row-major x / w / y map onto hipBLASLt's
// column-major "TN" problem: C^T[n, m] = op(W)[n, k] . X^T[k, m] with
// op(W) = transpose of W stored k x n, X^T stored k x m, both with leading
// dimension k.  Inputs f32 or bf16 (both operands alike), output f32 or bf16,
// f32 accumulation.  A plan (descriptors + an algorithm) is cached per
// (device, m, n, k, dtypes); the workspaces are per (device, stream), so
// calls on different streams may overlap.  On first use of a
// shape the heuristic's 16 first candidates are timed on the caller's
// operands and the fastest kept.  Skinny products over large weights (m <=
// 256, n k >= 4M: a decode step's projections, HBM-bound on the weights) get
// a deeper search: every algorithm hipBLASLt has for the problem (sampled
// down when the product is long) is timed with the weights warm in the
// caches, and the 12 fastest again with the caches flushed before each run,
// as the weights of a model's layers are when they stream from HBM; the
// fastest cold one is kept.  For bf16 products with m <= 64 the candidates
// also hold this library's weight-streaming kernel (skinny_gemm.hip) at each
// split of k it supports; when it wins, the fastest hipBLASLt algorithm is
// kept beside it for operands that are not 16-byte aligned.
// zk_linear_tuning(0) keeps the heuristic's first instead (e.g. under graph
// capture, where nothing may synchronize).
// Tiled weights (zk_weight_tile: the layout the weight-streaming kernel
// reads with contiguous 1 KiB loads) have their own plans, over the
// weight-streaming kernel's configurations only, timed as above with the
// caches flushed; with more than 64 rows of x the kernel covers them in
// blocks of 64 (the weights stream once per block).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <utility>
#include <vector>

#include "../../include/zealot_dense.h"
#include "zk_common.h"

namespace {

constexpr size_t kWorkspace = 64ull << 20;
constexpr int kCandidates = 16;           // heuristic candidates
constexpr int kFinalists = 12;            // re-timed with cold caches
constexpr size_t kFlushBytes = 512ull << 20;  // > the 256 MiB MALL
constexpr double kWarmBudgetMs = 400.0;   // warm timing budget per shape
constexpr size_t kSkinnyPartial = 32ull << 20;  // split-k sums of the skinny kernel
const int kSkinnySplits[] = {1, 2, 4, 7, 8, 14, 16, 28};
const int kSkinnyRows[] = {64, 128};
// What folding a projection's split-k sum into the RMSNorm after it saves:
// the reduce kernel's launch (about 4 us of a small kernel on the stream).
constexpr float kFuseMarginMs = 0.004f;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};  // hipBLASLt's fastest
    size_t ws = 0;
    int splits = 0;                // > 0: the skinny kernel with this split of k
    int tile_rows = 0;             // and tiles of this many weight rows
    // zk_linear_rms_norm: the skinny configuration with splits > 1 whose
    // sums the norm kernel adds (fused_splits 0: none within kFuseMarginMs of
    // the fastest)
    int fused_splits = 0, fused_rows = 0;
    bool tiled = false;            // a plan for tiled weights (skinny kernel only)
};

// Workspaces of one stream: hipBLASLt's, and the skinny kernel's split-k
// sums (allocated when a plan first needs them).
struct Scratch {
    void *blas = nullptr;
    void *partial = nullptr;
    uint64_t used = 0;  // last use, for eviction
};
constexpr size_t kMaxStreams = 8;  // streams per device that keep their workspaces

struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    std::map<hipStream_t, Scratch> scratch;
    uint64_t clock = 0;
    std::map<std::tuple<int64_t, int64_t, int64_t, int, int, bool>, Plan> plans;  // (m, n, k, in, out, tiled)
};

std::mutex g_mu;
std::map<int, DeviceState> g_dev;
bool g_tune = true;  // time the heuristic's candidates on first use of a shape

hipDataType hip_type(zk_dtype d) { return d == ZK_BF16 ? HIP_R_16BF : HIP_R_32F; }

int fail(const char *what, hipblasStatus_t st) {
    return zk::set_error(ZK_ERR_HIP, std::string("Internal error: zk_linear: ") + what + " (hipBLASLt status " +
                                         std::to_string((int)st) + ")");
}

int device_state(DeviceState **out) {
    int dev = 0;
    ZK_HIP_CHECK(hipGetDevice(&dev), "zk_linear device");
    DeviceState &d = g_dev[dev];
    if (!d.handle) {
        hipblasStatus_t st = hipblasLtCreate(&d.handle);
        if (st != HIPBLAS_STATUS_SUCCESS) {
            d.handle = nullptr;
            return fail("hipblasLtCreate", st);
        }
    }
    *out = &d;
    return ZK_OK;
}

// The workspaces of `stream` on this device, created on first use.  A ninth
// stream takes the place of the least recently used one, whose memory is
// freed once the device has drained (a synchronization: not for callers
// under stream capture, who use one stream).
int scratch_for(DeviceState &d, hipStream_t stream, bool partial, Scratch **out) {
    auto it = d.scratch.find(stream);
    if (it == d.scratch.end()) {
        if (d.scratch.size() >= kMaxStreams) {
            auto lru = d.scratch.begin();
            for (auto j = d.scratch.begin(); j != d.scratch.end(); ++j)
                if (j->second.used < lru->second.used) lru = j;
            ZK_HIP_CHECK(hipDeviceSynchronize(), "zk_linear workspace eviction");
            (void)hipFree(lru->second.blas);
            if (lru->second.partial) (void)hipFree(lru->second.partial);
            d.scratch.erase(lru);
        }
        Scratch sc;
        ZK_HIP_CHECK(hipMalloc(&sc.blas, kWorkspace), "zk_linear workspace");
        it = d.scratch.emplace(stream, sc).first;
    }
    Scratch &sc = it->second;
    if (partial && !sc.partial) ZK_HIP_CHECK(hipMalloc(&sc.partial, kSkinnyPartial), "zk_linear skinny workspace");
    sc.used = ++d.clock;
    *out = &sc;
    return ZK_OK;
}

// The problem of one zk_linear call.
struct Problem {
    const void *x, *w;
    void *y;
    int64_t m, n, k;
    bool f32_out;
    bool tiled = false;  // w in the weight-streaming kernel's tiled layout
};

int run_skinny(const Scratch &sc, const Problem &q, int tile_rows, int splits, hipStream_t stream) {
    return zk::skinny_linear(q.x, q.w, q.y, q.m, q.n, q.k, q.f32_out, tile_rows, splits, sc.partial,
                             sc.partial ? kSkinnyPartial : 0, stream, /*reduce=*/true, q.tiled);
}

bool skinny_fits(int64_t m, int64_t n, int64_t k, int tile_rows, int splits, bool tiled = false) {
    return zk::skinny_linear_ok(m, n, k, tile_rows, splits, tiled) &&
           zk::skinny_linear_partial_bytes(m, n, splits) <= kSkinnyPartial;
}

// Reads a buffer larger than the last-level cache with ordinary (allocating)
// loads, so the next GEMM finds its weights in HBM only.
__global__ void __launch_bounds__(256) flush_kernel(const uint4 *__restrict__ p, size_t n16, uint32_t *sink) {
    uint4 acc = {0u, 0u, 0u, 0u};
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) {
        const uint4 v = p[i];
        acc.x ^= v.x;
        acc.y ^= v.y;
        acc.z ^= v.z;
        acc.w ^= v.w;
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u) sink[0] = 1u;
}

struct Cand {
    hipblasLtMatmulAlgo_t algo;
    size_t ws;
    int splits;     // > 0: the skinny kernel
    int tile_rows;
};

// Picks the candidate to keep (see the file comment), the fastest hipBLASLt
// one (best_blas, -1 if none ran) and the fastest skinny one with splits > 1
// if it is within kFuseMarginMs of the kept one (best_split, else -1).  The
// first n_always candidates are always timed.  The output y is overwritten
// by every timed run and finally by the real call.
int pick_fastest(DeviceState &d, const Scratch &sc, Plan &p, const std::vector<Cand> &cands, const Problem &q,
                 size_t n_always, hipStream_t stream, bool cold, int *best, int *best_blas, int *best_split) {
    hipEvent_t e0, e1;
    ZK_HIP_CHECK(hipEventCreate(&e0), "zk_linear tuning");
    ZK_HIP_CHECK(hipEventCreate(&e1), "zk_linear tuning");
    const float alpha = 1.0f, beta = 0.0f;
    auto run = [&](const Cand &c) {
        if (c.splits) return run_skinny(sc, q, c.tile_rows, c.splits, stream) == ZK_OK;
        return hipblasLtMatmul(d.handle, p.desc, &alpha, q.w, p.a, q.x, p.b, &beta, q.y, p.c, q.y, p.c, &c.algo,
                               sc.blas, c.ws, stream) == HIPBLAS_STATUS_SUCCESS;
    };
    auto timed = [&](const Cand &c, int reps, float *ms) {
        (void)hipEventRecord(e0, stream);
        bool ok = true;
        for (int r = 0; r < reps && ok; ++r) ok = run(c);
        (void)hipEventRecord(e1, stream);
        if (hipEventSynchronize(e1) != hipSuccess || !ok) return false;
        return hipEventElapsedTime(ms, e0, e1) == hipSuccess;
    };
    // warm: the heuristic's candidates first; the rest sampled evenly when
    // all of them would take longer than the budget
    std::vector<std::pair<float, int>> warm;
    size_t stride = 1;
    for (size_t i = 0; i < cands.size(); i += (i < n_always ? 1 : stride)) {
        float ms = 0.0f;
        if (!run(cands[i]) || !timed(cands[i], 2, &ms)) continue;
        warm.push_back({ms / 2, (int)i});
        if (warm.size() == 1) {
            const double runs = kWarmBudgetMs / std::max(1e-3, 3.0 * ms / 2);
            stride = std::max<size_t>(1, (size_t)((double)cands.size() / std::max(1.0, runs)));
        }
    }
    if (warm.empty()) {
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        return zk::set_error(ZK_ERR_HIP, "Internal error: zk_linear: no hipBLASLt algorithm ran");
    }
    std::sort(warm.begin(), warm.end());
    *best = warm[0].second;
    *best_blas = -1;
    *best_split = -1;
    for (auto &t : warm)
        if (!cands[t.second].splits) {
            *best_blas = t.second;
            break;
        }
    for (auto &t : warm)
        if (cands[t.second].splits > 1) {
            if (t.first <= warm[0].first + kFuseMarginMs) *best_split = t.second;
            break;
        }
    // cold: flush the caches before each run of the finalists
    void *flush = nullptr;
    if (cold && warm.size() > 1 && hipMalloc(&flush, kFlushBytes) == hipSuccess) {
        // the finalists: the warm fastest, and the skinny kernel's three
        // fastest configurations (warm, the weights partly sit in the
        // last-level cache, which flatters other algorithms more)
        std::vector<std::pair<float, int>> fin(warm.begin(), warm.begin() + std::min<size_t>(kFinalists, warm.size()));
        int skinny_added = 0;
        for (size_t i = 0; i < warm.size() && skinny_added < 3; ++i)
            if (cands[warm[i].second].splits) {
                ++skinny_added;
                if (i >= fin.size()) fin.push_back(warm[i]);
            }
        float best_ms = 1e30f, blas_ms = 1e30f, split_ms = 1e30f;
        int split_at = -1;
        for (size_t f = 0; f < fin.size(); ++f) {
            float total = 0.0f;
            bool ok = true;
            for (int r = 0; r < 3 && ok; ++r) {
                flush_kernel<<<1024, 256, 0, stream>>>((const uint4 *)flush, kFlushBytes / 16,
                                                       (uint32_t *)((char *)flush + kFlushBytes - 16));
                float ms = 0.0f;
                ok = timed(cands[fin[f].second], 1, &ms);
                total += ms;
            }
            if (ok && total < best_ms) {
                best_ms = total;
                *best = fin[f].second;
            }
            if (ok && !cands[fin[f].second].splits && total < blas_ms) {
                blas_ms = total;
                *best_blas = fin[f].second;
            }
            if (ok && cands[fin[f].second].splits > 1 && total < split_ms) {
                split_ms = total;
                split_at = fin[f].second;
            }
        }
        // three runs each: the margin counts three times
        *best_split = split_ms <= best_ms + 3 * kFuseMarginMs ? split_at : -1;
        (void)hipStreamSynchronize(stream);
        (void)hipFree(flush);
    }
    (void)hipGetLastError();
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ZK_OK;
}

int make_plan(DeviceState &d, Scratch &sc, int64_t m, int64_t n, int64_t k, zk_dtype in, zk_dtype out, const void *x,
              const void *w, void *y, hipStream_t stream, bool tune, Plan **res) {
    auto key = std::make_tuple(m, n, k, (int)in, (int)out, false);
    auto it = d.plans.find(key);
    if (it != d.plans.end()) {
        *res = &it->second;
        return ZK_OK;
    }
    Plan p;
    hipblasStatus_t st = hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtMatmulDescCreate", st);
    hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
    st = hipblasLtMatrixLayoutCreate(&p.a, hip_type(in), (uint64_t)k, (uint64_t)n, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.b, hip_type(in), (uint64_t)k, (uint64_t)m, k);
    if (st == HIPBLAS_STATUS_SUCCESS) st = hipblasLtMatrixLayoutCreate(&p.c, hip_type(out), (uint64_t)n, (uint64_t)m, n);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtMatrixLayoutCreate", st);
    hipblasLtMatmulPreference_t pref;
    st = hipblasLtMatmulPreferenceCreate(&pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtMatmulPreferenceCreate", st);
    uint64_t ws = kWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t heur[kCandidates];
    int found = 0;
    st = hipblasLtMatmulAlgoGetHeuristic(d.handle, p.desc, p.a, p.b, p.c, p.c, pref, kCandidates, heur, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || found == 0)
        return fail("no hipBLASLt algorithm for this shape", st == HIPBLAS_STATUS_SUCCESS ? HIPBLAS_STATUS_NOT_SUPPORTED : st);
    std::vector<Cand> cands;
    for (int i = 0; i < found; ++i)
        if (heur[i].state == HIPBLAS_STATUS_SUCCESS && heur[i].workspaceSize <= kWorkspace)
            cands.push_back({heur[i].algo, heur[i].workspaceSize, 0, 0});
    if (cands.empty()) return fail("no hipBLASLt algorithm fits the workspace", HIPBLAS_STATUS_NOT_SUPPORTED);
    int best = 0, best_blas = 0, best_split = -1;
    const bool deep = m <= 256 && n * k >= (int64_t)1 << 22;
    const Problem q{x, w, y, m, n, k, out == ZK_F32};
    const bool aligned = (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) & 15) == 0;
    if (tune && deep && in == ZK_BF16 && aligned &&
        (sc.partial || hipMalloc(&sc.partial, kSkinnyPartial) == hipSuccess))
        for (int rows : kSkinnyRows)
            for (int sp : kSkinnySplits)
                if (skinny_fits(m, n, k, rows, sp)) cands.push_back({hipblasLtMatmulAlgo_t{}, 0, sp, rows});
    const size_t n_always = cands.size();  // the heuristic's and the skinny kernel's
    if (tune && deep) {
        // the heuristic's order is not the fastest for the skinny (decode)
        // shapes: every algorithm the library has for the problem is a candidate
        std::vector<hipblasLtMatmulHeuristicResult_t> all;
        if (hipblaslt_ext::getAllAlgos(d.handle, hipblaslt_ext::GemmType::HIPBLASLT_GEMM, ta, tb, hip_type(in),
                                       hip_type(in), hip_type(out), hip_type(out), HIPBLAS_COMPUTE_32F,
                                       all) == HIPBLAS_STATUS_SUCCESS) {
            const float alpha = 1.0f, beta = 0.0f;
            for (auto &r : all) {
                size_t wsz = 0;
                if (hipblaslt_ext::matmulIsAlgoSupported(d.handle, p.desc, &alpha, p.a, p.b, &beta, p.c, p.c, r.algo,
                                                         wsz) == HIPBLAS_STATUS_SUCCESS &&
                    wsz <= kWorkspace)
                    cands.push_back({r.algo, wsz, 0, 0});
            }
        }
    }
    if (tune && cands.size() > 1)
        if (int rc = pick_fastest(d, sc, p, cands, q, n_always, stream, deep, &best, &best_blas, &best_split))
            return rc;
    if (best_blas < 0) best_blas = 0;  // candidate 0 is the heuristic's first
    p.splits = cands[best].splits;
    p.tile_rows = cands[best].tile_rows;
    if (best_split >= 0) {
        p.fused_splits = cands[best_split].splits;
        p.fused_rows = cands[best_split].tile_rows;
    }
    p.algo = cands[best_blas].algo;
    p.ws = cands[best_blas].ws;
    *res = &(d.plans[key] = p);
    return ZK_OK;
}

// The plan for tiled weights: the weight-streaming kernel's configurations
// (tile rows x splits that fit the shape and the split-k workspace), the
// fastest kept as make_plan keeps its, with the fastest split one for
// zk_linear_rms_norm_tiled beside it.
int make_tiled_plan(DeviceState &d, Scratch &sc, int64_t m, int64_t n, int64_t k, zk_dtype out, const void *x,
                    const void *w, void *y, hipStream_t stream, bool tune, Plan **res) {
    auto key = std::make_tuple(m, n, k, (int)ZK_BF16, (int)out, true);
    auto it = d.plans.find(key);
    if (it != d.plans.end()) {
        *res = &it->second;
        return ZK_OK;
    }
    std::vector<Cand> cands;
    for (int rows : {128, 64})  // 128-row tiles first: the untuned choice
        for (int sp : kSkinnySplits)
            if (skinny_fits(m, n, k, rows, sp, true)) cands.push_back({hipblasLtMatmulAlgo_t{}, 0, sp, rows});
    if (cands.empty())
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_tiled: unsupported shape");
    if (!sc.partial) ZK_HIP_CHECK(hipMalloc(&sc.partial, kSkinnyPartial), "zk_linear skinny workspace");
    Plan p;
    p.tiled = true;
    int best = 0, best_blas = -1, best_split = -1;
    if (tune && cands.size() > 1) {
        Problem q{x, w, y, m, n, k, out == ZK_F32, true};
        if (int rc = pick_fastest(d, sc, p, cands, q, cands.size(), stream, true, &best, &best_blas, &best_split))
            return rc;
    }
    p.splits = cands[best].splits;
    p.tile_rows = cands[best].tile_rows;
    if (best_split >= 0) {
        p.fused_splits = cands[best_split].splits;
        p.fused_rows = cands[best_split].tile_rows;
    }
    *res = &(d.plans[key] = p);
    return ZK_OK;
}

// Runs the plan's choice for y = x . w^T (the caller holds g_mu).
int run_plan(DeviceState &d, Scratch *sc, const Plan *p, const void *x, const void *w, void *y, int64_t m, int64_t n,
             int64_t k, zk_dtype out_dtype, hipStream_t stream) {
    const float alpha = 1.0f, beta = 0.0f;
    if (p->splits && (p->tiled || (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) & 15) == 0)) {
        if (int rc = scratch_for(d, stream, p->splits > 1, &sc)) return rc;
        zk::KernelTimer timer("linear", stream);
        return run_skinny(*sc, Problem{x, w, y, m, n, k, out_dtype == ZK_F32, p->tiled}, p->tile_rows, p->splits,
                          stream);
    }
    zk::KernelTimer timer("linear", stream);
    hipblasStatus_t st = hipblasLtMatmul(d.handle, p->desc, &alpha, w, p->a, x, p->b, &beta, y, p->c, y, p->c,
                                         &p->algo, sc->blas, p->ws, stream);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtMatmul", st);
    return ZK_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" {

int zk_linear(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, zk_dtype in_dtype,
              zk_dtype out_dtype, void *stream) {
    if ((in_dtype != ZK_F32 && in_dtype != ZK_BF16) || (out_dtype != ZK_F32 && out_dtype != ZK_BF16))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear: dtypes must be f32 or bf16");
    if (in_dtype == ZK_F32 && out_dtype != ZK_F32)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear: f32 inputs give f32 outputs");
    if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear: bad shape");
    if (m == 0) return ZK_OK;
    if (!x || !w || !y) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear: NULL pointer");
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    Scratch *sc;
    if (int rc = scratch_for(*d, (hipStream_t)stream, false, &sc)) return rc;
    Plan *p;
    if (int rc = make_plan(*d, *sc, m, n, k, in_dtype, out_dtype, x, w, y, (hipStream_t)stream, g_tune, &p))
        return rc;
    return run_plan(*d, sc, p, x, w, y, m, n, k, out_dtype, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// zk_linear_rms_norm over row-major or tiled weights.
int linear_rms_norm(const void *x, const void *w, bool tiled, int64_t m, int64_t n, int64_t k, const void *residual,
                    const void *norm_weight, float eps, void *out, void *residual_out, void *stream) {
    if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_rms_norm: bad shape");
    if (m == 0) return ZK_OK;
    if (!x || !w || !norm_weight || !out || (residual && !residual_out))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_rms_norm: NULL pointer");
    if (tiled && !(aligned16(x) && aligned16(w) && aligned16(out)))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_rms_norm_tiled: operands not 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    {
        std::lock_guard<std::mutex> g(g_mu);
        DeviceState *d;
        if (int rc = device_state(&d)) return rc;
        Scratch *sc;
        if (int rc = scratch_for(*d, s, false, &sc)) return rc;
        Plan *p;
        if (int rc = tiled ? make_tiled_plan(*d, *sc, m, n, k, ZK_BF16, x, w, out, s, g_tune, &p)
                           : make_plan(*d, *sc, m, n, k, ZK_BF16, ZK_BF16, x, w, out, s, g_tune, &p))
            return rc;
        const bool fuse = p->fused_splits > 1 && skinny_fits(m, n, k, p->fused_rows, p->fused_splits, tiled) &&
                          zk::rms_norm_partials_ok(m, n) && aligned16(x) && aligned16(w) && aligned16(out) &&
                          aligned16(norm_weight) && (!residual || (aligned16(residual) && aligned16(residual_out)));
        if (fuse) {  // the skinny kernel's split-k sums go straight into the norm kernel
            if (int rc = scratch_for(*d, s, true, &sc)) return rc;
            {
                zk::KernelTimer timer("linear", s);
                if (int rc = zk::skinny_linear(x, w, nullptr, m, n, k, false, p->fused_rows, p->fused_splits,
                                               sc->partial, kSkinnyPartial, s, /*reduce=*/false, tiled))
                    return rc;
            }
            zk::KernelTimer timer("rms_norm", s);
            return zk::rms_norm_partials((const float *)sc->partial, p->fused_splits, residual, norm_weight, out,
                                         residual_out, m, n, eps, s);
        }
        if (int rc = run_plan(*d, sc, p, x, w, out, m, n, k, ZK_BF16, s)) return rc;
    }
    // the projection's output sits in `out`, which the norm overwrites in place
    return zk_rms_norm(out, residual, norm_weight, out, residual_out, nullptr, m, n, eps, ZK_BF16, stream);
}

// Shape / pointer checks of the tiled products (bf16 x and wt, y bf16 or f32).
int tiled_args(const char *what, const void *x, const void *wt, const void *y, int64_t m, int64_t n, int64_t k) {
    if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: ") + what + ": bad shape");
    if (m > 0 && (!x || !wt || !y))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, std::string("Internal error: ") + what + ": NULL pointer");
    if (m > 0 && !(aligned16(x) && aligned16(wt) && aligned16(y)))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             std::string("Internal error: ") + what + ": operands not 16-byte aligned");
    return ZK_OK;
}

}  // namespace

extern "C" {

int zk_linear_rms_norm(const void *x, const void *w, int64_t m, int64_t n, int64_t k, const void *residual,
                       const void *norm_weight, float eps, void *out, void *residual_out, void *stream) {
    return linear_rms_norm(x, w, false, m, n, k, residual, norm_weight, eps, out, residual_out, stream);
}

int zk_linear_rms_norm_tiled(const void *x, const void *wt, int64_t m, int64_t n, int64_t k, const void *residual,
                             const void *norm_weight, float eps, void *out, void *residual_out, void *stream) {
    return linear_rms_norm(x, wt, true, m, n, k, residual, norm_weight, eps, out, residual_out, stream);
}

int zk_weight_tile(const void *w, void *wt, int64_t n, int64_t k, void *stream) {
    return zk::tile_weight(w, wt, n, k, (hipStream_t)stream);
}

int zk_linear_tiled(const void *x, const void *wt, void *y, int64_t m, int64_t n, int64_t k, zk_dtype out_dtype,
                    void *stream) {
    if (out_dtype != ZK_F32 && out_dtype != ZK_BF16)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_tiled: out dtype must be f32 or bf16");
    if (int rc = tiled_args("zk_linear_tiled", x, wt, y, m, n, k)) return rc;
    if (m == 0) return ZK_OK;
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    Scratch *sc;
    if (int rc = scratch_for(*d, (hipStream_t)stream, false, &sc)) return rc;
    Plan *p;
    if (int rc = make_tiled_plan(*d, *sc, m, n, k, out_dtype, x, wt, y, (hipStream_t)stream, g_tune, &p)) return rc;
    return run_plan(*d, sc, p, x, wt, y, m, n, k, out_dtype, (hipStream_t)stream);
}

int zk_linear_silu_mul_tiled(const void *x, const void *wt, void *act, int64_t m, int64_t inter, int64_t k,
                             void *stream) {
    if (inter <= 0 || inter % 64 || 2 * inter > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_silu_mul_tiled: bad shape (inter must be a multiple of 64)");
    if (int rc = tiled_args("zk_linear_silu_mul_tiled", x, wt, act, m, 2 * inter, k)) return rc;
    if (m == 0) return ZK_OK;
    zk::KernelTimer timer("linear", (hipStream_t)stream);
    return zk::skinny_linear_silu(x, wt, act, m, 2 * inter, k, (hipStream_t)stream, /*tiled=*/true);
}

int zk_linear_tiled_choice(int64_t m, int64_t n, int64_t k, zk_dtype out_dtype, int choice[4]) {
    if (!choice) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_tiled_choice: NULL pointer");
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    auto it = d->plans.find(std::make_tuple(m, n, k, (int)ZK_BF16, (int)out_dtype, true));
    if (it == d->plans.end())
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_tiled_choice: no plan for this shape yet");
    choice[0] = it->second.splits;
    choice[1] = it->second.tile_rows;
    choice[2] = it->second.fused_splits;
    choice[3] = it->second.fused_rows;
    return ZK_OK;
}

int zk_linear_skinny(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, zk_dtype out_dtype,
                     int tile_rows, int splits, void *stream) {
    if (out_dtype != ZK_F32 && out_dtype != ZK_BF16)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_skinny: out dtype must be f32 or bf16");
    if (m == 0 && n > 0 && k > 0) return ZK_OK;
    if (!skinny_fits(m, n, k, tile_rows, splits))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_skinny: needs 1 <= m <= 64, tile_rows 64 or 128, "
                             "n % tile_rows == 0, k % (128 * splits) == 0 and splits * m * n * 4 <= 32 MiB");
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    Scratch *sc;
    if (int rc = scratch_for(*d, (hipStream_t)stream, splits > 1, &sc)) return rc;
    zk::KernelTimer timer("linear", (hipStream_t)stream);
    return run_skinny(*sc, Problem{x, w, y, m, n, k, out_dtype == ZK_F32}, tile_rows, splits, (hipStream_t)stream);
}

int zk_linear_silu_mul(const void *x, const void *w, void *act, int64_t m, int64_t inter, int64_t k, void *gu,
                       void *stream) {
    if (m < 0 || inter <= 0 || inter % 16 || k <= 0 || m > 0x7fffffff || 2 * inter > 0x7fffffff || k > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_silu_mul: bad shape (inter must be a multiple of 16)");
    if (m == 0) return ZK_OK;
    if (!x || !w || !act || !gu)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_silu_mul: NULL pointer");
    hipStream_t s = (hipStream_t)stream;
    const int64_t n = 2 * inter;
    {
        std::lock_guard<std::mutex> g(g_mu);
        DeviceState *d;
        if (int rc = device_state(&d)) return rc;
        Scratch *sc;
        if (int rc = scratch_for(*d, s, false, &sc)) return rc;
        Plan *p;
        if (int rc = make_plan(*d, *sc, m, n, k, ZK_BF16, ZK_BF16, x, w, gu, s, g_tune, &p)) return rc;
        if (p->splits == 1 && p->tile_rows == 128 && aligned16(x) && aligned16(w) && aligned16(act)) {
            // each wave holds the gate and up outputs of the same columns: SiLU * up in its epilogue
            zk::KernelTimer timer("linear", s);
            return zk::skinny_linear_silu(x, w, act, m, n, k, s);
        }
        if (int rc = run_plan(*d, sc, p, x, w, gu, m, n, k, ZK_BF16, s)) return rc;
    }
    zk::KernelTimer timer("silu_mul", s);
    return zk::silu_mul_blocked(gu, act, m, inter, s);
}

int zk_linear_choice(int64_t m, int64_t n, int64_t k, zk_dtype in_dtype, zk_dtype out_dtype, int choice[4]) {
    if (!choice) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_choice: NULL pointer");
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    auto it = d->plans.find(std::make_tuple(m, n, k, (int)in_dtype, (int)out_dtype, false));
    if (it == d->plans.end())
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_choice: no plan for this shape yet");
    choice[0] = it->second.splits;
    choice[1] = it->second.tile_rows;
    choice[2] = it->second.fused_splits;
    choice[3] = it->second.fused_rows;
    return ZK_OK;
}

int zk_linear_pin_split(int64_t m, int64_t n, int64_t k, zk_dtype in_dtype, zk_dtype out_dtype, int tiled,
                        int fused_splits, int fused_rows) {
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    auto it = d->plans.find(std::make_tuple(m, n, k, (int)in_dtype, (int)out_dtype, tiled != 0));
    if (it == d->plans.end())
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: zk_linear_pin_split: no plan for this shape yet");
    if (fused_splits != 0 &&
        (in_dtype != ZK_BF16 || fused_splits < 2 || !skinny_fits(m, n, k, fused_rows, fused_splits, tiled != 0)))
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT,
                             "Internal error: zk_linear_pin_split: configuration does not fit the shape");
    it->second.fused_splits = fused_splits;
    it->second.fused_rows = fused_splits ? fused_rows : 0;
    return ZK_OK;
}

int zk_linear_tuning(int on) {
    std::lock_guard<std::mutex> g(g_mu);
    g_tune = on != 0;
    return ZK_OK;
}

}  // extern "C"

int zk::linear_split_sums(const void *x, const void *w, void *y, int64_t m, int64_t n, int64_t k, hipStream_t stream,
                          const SplitSumsConsumer &consume, bool *fused) {
    if (!fused) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: linear_split_sums: NULL");
    *fused = false;
    if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
        return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: linear_split_sums: bad shape");
    if (m == 0) return ZK_OK;
    if (!x || !w || !y) return zk::set_error(ZK_ERR_INVALID_ARGUMENT, "Internal error: linear_split_sums: NULL pointer");
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState *d;
    if (int rc = device_state(&d)) return rc;
    Scratch *sc;
    if (int rc = scratch_for(*d, stream, false, &sc)) return rc;
    Plan *p;
    if (int rc = make_plan(*d, *sc, m, n, k, ZK_BF16, ZK_BF16, x, w, y, stream, g_tune, &p)) return rc;
    if (p->fused_splits > 1 && skinny_fits(m, n, k, p->fused_rows, p->fused_splits) && aligned16(x) && aligned16(w) &&
        aligned16(y) && n % 8 == 0) {
        if (int rc = scratch_for(*d, stream, true, &sc)) return rc;
        {
            zk::KernelTimer timer("linear", stream);
            if (int rc = zk::skinny_linear(x, w, nullptr, m, n, k, false, p->fused_rows, p->fused_splits, sc->partial,
                                           kSkinnyPartial, stream, /*reduce=*/false))
                return rc;
        }
        // the consumer's launch is enqueued before the lock goes: no other
        // call can evict this stream's workspace in between
        if (int rc = consume((const float *)sc->partial, p->fused_splits)) return rc;
        *fused = true;
        return ZK_OK;
    }
    return run_plan(*d, sc, p, x, w, y, m, n, k, ZK_BF16, stream);
}


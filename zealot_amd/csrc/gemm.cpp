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
// (device, m, n, k, dtypes); one workspace per device.  On first use of a
// shape the heuristic's first 16 candidates are timed on the caller's
// operands and the fastest kept (zk_linear_tuning(0) keeps the heuristic's
// first instead, e.g. under graph capture, where nothing may synchronize).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "zk_common.h"

namespace {

constexpr size_t kWorkspace = 64ull << 20;
constexpr int kCandidates = 16;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};

struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    std::map<std::tuple<int64_t, int64_t, int64_t, int, int>, Plan> plans;
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
        ZK_HIP_CHECK(hipMalloc(&d.workspace, kWorkspace), "zk_linear workspace");
    }
    *out = &d;
    return ZK_OK;
}

// Times each candidate (a warm-up call, then kReps calls between events) on
// the stream and returns the fastest that ran.  Runs once per shape; the
// output y is overwritten by every candidate and finally by the real call.
int pick_fastest(DeviceState &d, Plan &p, const hipblasLtMatmulHeuristicResult_t *heur, int found, const void *x,
                 const void *w, void *y, hipStream_t stream, int *best) {
    constexpr int kReps = 5;
    hipEvent_t e0, e1;
    ZK_HIP_CHECK(hipEventCreate(&e0), "zk_linear tuning");
    ZK_HIP_CHECK(hipEventCreate(&e1), "zk_linear tuning");
    const float alpha = 1.0f, beta = 0.0f;
    float best_ms = 1e30f;
    for (int i = 0; i < found; ++i) {
        if (heur[i].state != HIPBLAS_STATUS_SUCCESS || heur[i].workspaceSize > kWorkspace) continue;
        auto run = [&]() {
            return hipblasLtMatmul(d.handle, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.c, y, p.c, &heur[i].algo,
                                   d.workspace, heur[i].workspaceSize, stream);
        };
        if (run() != HIPBLAS_STATUS_SUCCESS) continue;
        (void)hipEventRecord(e0, stream);
        bool ok = true;
        for (int r = 0; r < kReps && ok; ++r) ok = run() == HIPBLAS_STATUS_SUCCESS;
        (void)hipEventRecord(e1, stream);
        if (hipEventSynchronize(e1) != hipSuccess || !ok) continue;
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (ms < best_ms) {
            best_ms = ms;
            *best = i;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return ZK_OK;
}

int make_plan(DeviceState &d, int64_t m, int64_t n, int64_t k, zk_dtype in, zk_dtype out, const void *x,
              const void *w, void *y, hipStream_t stream, bool tune, Plan **res) {
    auto key = std::make_tuple(m, n, k, (int)in, (int)out);
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
    int best = 0;
    if (found > 1 && tune) {
        // the heuristic's order is not the fastest for the skinny (decode)
        // shapes: time every candidate on the caller's operands once
        if (int rc = pick_fastest(d, p, heur, found, x, w, y, stream, &best)) return rc;
    }
    p.algo = heur[best].algo;
    p.ws = heur[best].workspaceSize;
    *res = &(d.plans[key] = p);
    return ZK_OK;
}

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
    Plan *p;
    if (int rc = make_plan(*d, m, n, k, in_dtype, out_dtype, x, w, y, (hipStream_t)stream, g_tune, &p)) return rc;
    const float alpha = 1.0f, beta = 0.0f;
    zk::KernelTimer timer("linear", (hipStream_t)stream);
    hipblasStatus_t st = hipblasLtMatmul(d->handle, p->desc, &alpha, w, p->a, x, p->b, &beta, y, p->c, y, p->c,
                                         &p->algo, d->workspace, p->ws, (hipStream_t)stream);
    if (st != HIPBLAS_STATUS_SUCCESS) return fail("hipblasLtMatmul", st);
    return ZK_OK;
}

int zk_linear_tuning(int on) {
    std::lock_guard<std::mutex> g(g_mu);
    g_tune = on != 0;
    return ZK_OK;
}

}  // extern "C"

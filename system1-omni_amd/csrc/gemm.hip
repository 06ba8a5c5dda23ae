// bfloat16 GEMMs of the decoder's projections through hipBLASLt, float32 accumulation
// (reference interface ops.h:117-124, gemm.cu).
//
// Row-major y [M, N] (row stride ldy >= N) = x [M, K] * w [N, K]^T. hipBLASLt is
// column-major, so the call computes y^T [N, M] = op(A) * B with A = w seen as the
// column-major [K, N] matrix (transposed) and B = x seen as the column-major [K, M]
// matrix; y^T's leading dimension is ldy, so one GEMM can fill a column slice of a wider
// row-major buffer.
//
// Every shape (M, N, K, ldy) gets one plan, built on first use from hipBLASLt's first
// heuristic choice and then reused, so a given shape always runs the same kernel and its
// float32 summation order is fixed from call to call. The plans live in the caller-owned
// handle, which is not safe for concurrent use (one model drives it from one thread, as
// the reference's executor does).
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <tuple>

#include "qwen3_5_ops.h"

namespace {

struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

using Key = std::tuple<int, int, int, int>;  // M, N, K, ldy

struct Gemm {
    hipblasLtHandle_t handle = nullptr;
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    std::map<Key, Plan> plans;
};

// hipBLASLt statuses are reported as 1000 + status, like the reference's cuBLAS codes.
int status(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? 0 : 1000 + (int)s; }

void release(Plan& p) {
    if (p.a) hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b) hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c) hipblasLtMatrixLayoutDestroy(p.c);
    if (p.op) hipblasLtMatmulDescDestroy(p.op);
    p = Plan{};
}

int build_plan(Gemm& g, int M, int N, int K, int ldy, Plan& p) {
    hipblasStatus_t s = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (s != HIPBLAS_STATUS_SUCCESS) return status(s);
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if ((s = hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta))) !=
        HIPBLAS_STATUS_SUCCESS)
        return status(s);
    if ((s = hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb))) !=
        HIPBLAS_STATUS_SUCCESS)
        return status(s);
    if ((s = hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, N, K)) != HIPBLAS_STATUS_SUCCESS) return status(s);
    if ((s = hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, M, K)) != HIPBLAS_STATUS_SUCCESS) return status(s);
    if ((s = hipblasLtMatrixLayoutCreate(&p.c, HIP_R_16BF, N, M, ldy)) != HIPBLAS_STATUS_SUCCESS) return status(s);

    hipblasLtMatmulPreference_t pref = nullptr;
    if ((s = hipblasLtMatmulPreferenceCreate(&pref)) != HIPBLAS_STATUS_SUCCESS) return status(s);
    const uint64_t ws = g.workspace_bytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t r{};
    int found = 0;
    s = hipblasLtMatmulAlgoGetHeuristic(g.handle, p.op, p.a, p.b, p.c, p.c, pref, 1, &r, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS) return status(s);
    if (found == 0 || r.state != HIPBLAS_STATUS_SUCCESS) return status(HIPBLAS_STATUS_NOT_SUPPORTED);
    p.algo = r.algo;
    return 0;
}

int plan_for(Gemm& g, int M, int N, int K, int ldy, Plan*& out) {
    const Key key{M, N, K, ldy};
    auto it = g.plans.find(key);
    if (it != g.plans.end()) {
        out = &it->second;
        return 0;
    }
    Plan p;
    const int rc = build_plan(g, M, N, K, ldy, p);
    if (rc != 0) {
        release(p);
        return rc;
    }
    out = &g.plans.emplace(key, p).first->second;
    return 0;
}

}  // namespace

extern "C" {

void* cs1_gemm_create(size_t workspace_bytes) {
    Gemm* g = new Gemm();
    if (hipblasLtCreate(&g->handle) != HIPBLAS_STATUS_SUCCESS) {
        delete g;
        return nullptr;
    }
    if (workspace_bytes > 0 && hipMalloc(&g->workspace, workspace_bytes) != hipSuccess) {
        hipblasLtDestroy(g->handle);
        delete g;
        return nullptr;
    }
    g->workspace_bytes = workspace_bytes;
    return g;
}

void cs1_gemm_destroy(void* gemm) {
    Gemm* g = static_cast<Gemm*>(gemm);
    if (!g) return;
    for (auto& kv : g->plans) release(kv.second);
    if (g->workspace) (void)hipFree(g->workspace);
    hipblasLtDestroy(g->handle);
    delete g;
}

int cs1_gemm(void* gemm, const void* x, const void* w, void* y, int M, int N, int K, int ldy, void* stream) {
    Gemm* g = static_cast<Gemm*>(gemm);
    if (!g || M < 0 || N <= 0 || K <= 0 || ldy < N) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    Plan* p = nullptr;
    const int rc = plan_for(*g, M, N, K, ldy, p);
    if (rc != 0) return rc;
    const float alpha = 1.f, beta = 0.f;
    return status(hipblasLtMatmul(g->handle, p->op, &alpha, w, p->a, x, p->b, &beta, y, p->c, y, p->c, &p->algo,
                                  g->workspace, g->workspace_bytes, static_cast<hipStream_t>(stream)));
}

}  // extern "C"

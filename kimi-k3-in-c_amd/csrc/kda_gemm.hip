// SPDX-License-Identifier: Apache-2.0
// kda_gemm.hip - the layer's projections as bf16 MFMA GEMMs through hipBLASLt.
//
// Replaces the reference's per-token k3_mmw calls (include/k3/k3.h:290-296 ->
// k3_matmul_bf16, src/core/k3_ops.c:1122-1227; call sites :879-886, :946, :948) for a
// T-token prefill on bf16 weights and bf16 activations:
//   C[M][N] = A[M][K] . W[N][K]^T     A, W row-major bf16; fp32 accumulation; C bf16 or fp32
// These are plain GEMMs (no fusion), so they go to the vendor library: in hipBLASLt's
// column-major terms C^T = W . A^T, i.e. op(A) = T on W (K x N, ld K), op(B) = N on A
// (K x M, ld K), D = C^T (N x M, ld N).
//
// Per device: one handle and one workspace, created on first use. On the first call of a
// shape (M, N, K, C dtype) up to 8 heuristic candidates are timed on that call's buffers and
// the fastest is cached; that first call synchronizes its stream (keep it out of graph
// capture). Later calls are stream-ordered on the caller's stream.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "kda_internal.h"

namespace k3kda {

namespace {

constexpr size_t GEMM_WS = 64ull << 20;   // hipBLASLt workspace per device
constexpr int MAX_DEV = 64;

struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo;
    size_t ws = 0;
};

struct DevGemm {
    hipblasLtHandle_t h = nullptr;
    void *ws = nullptr;
    std::map<std::tuple<int, int, int, int>, Plan> plans;
};

std::mutex g_mu;
DevGemm g_dev[MAX_DEV];

const char *lt_status(hipblasStatus_t s)
{
    switch (s) {
    case HIPBLAS_STATUS_SUCCESS: return "success";
    case HIPBLAS_STATUS_NOT_INITIALIZED: return "not initialized";
    case HIPBLAS_STATUS_ALLOC_FAILED: return "allocation failed";
    case HIPBLAS_STATUS_INVALID_VALUE: return "invalid value";
    case HIPBLAS_STATUS_ARCH_MISMATCH: return "arch mismatch";
    case HIPBLAS_STATUS_EXECUTION_FAILED: return "execution failed";
    case HIPBLAS_STATUS_NOT_SUPPORTED: return "not supported";
    default: return "error";
    }
}

#define K3_LT(call)                                                                      \
    do {                                                                                 \
        hipblasStatus_t s_ = (call);                                                     \
        if (s_ != HIPBLAS_STATUS_SUCCESS)                                                \
            K3_FAIL(K3HIP_EHIP, "%s: hipBLASLt %s (%s:%d)", #call, lt_status(s_), __FILE__, \
                    __LINE__);                                                           \
    } while (0)

// Candidates from the heuristic, each timed on the call's own buffers (first call of a
// shape only; that call synchronizes the stream). The fastest is kept.
constexpr int NCAND = 8;

int make_plan(DevGemm &d, int M, int N, int K, int cdt, Plan &p, const void *A, const void *W,
              void *Cm, hipStream_t st)
{
    const hipDataType ct = cdt == K3HIP_BF16 ? HIP_R_16BF : HIP_R_32F;
    K3_LT(hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    K3_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta));
    K3_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb));
    K3_LT(hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, N, K));
    K3_LT(hipblasLtMatrixLayoutCreate(&p.lb, HIP_R_16BF, K, M, K));
    K3_LT(hipblasLtMatrixLayoutCreate(&p.lc, ct, N, M, N));
    hipblasLtMatmulPreference_t pref = nullptr;
    K3_LT(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wmax = GEMM_WS;
    hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(
        pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wmax, sizeof wmax);
    hipblasLtMatmulHeuristicResult_t res[NCAND];
    int n = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(d.h, p.op, p.la, p.lb, p.lc, p.lc, pref, NCAND, res, &n);
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS || n == 0)
        K3_FAIL(K3HIP_EUNSUPPORTED, "hipBLASLt has no algorithm for %dx%dx%d bf16 GEMM (%s)", M, N,
                K, lt_status(s));
    int best = 0;
    if (n > 1) {
        hipEvent_t e0, e1;
        K3_HIP(hipEventCreate(&e0));
        K3_HIP(hipEventCreate(&e1));
        const float alpha = 1.0f, beta = 0.0f;
        float best_ms = 1e30f;
        for (int i = 0; i < n; i++) {
            if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > GEMM_WS) continue;
            auto run = [&]() {
                return hipblasLtMatmul(d.h, p.op, &alpha, W, p.la, A, p.lb, &beta, Cm, p.lc, Cm, p.lc,
                                       &res[i].algo, res[i].workspaceSize ? d.ws : nullptr,
                                       res[i].workspaceSize, st);
            };
            if (run() != HIPBLAS_STATUS_SUCCESS) continue;   // warm-up; skip what fails
            K3_HIP(hipEventRecord(e0, st));
            for (int r = 0; r < 3; r++) (void)run();
            K3_HIP(hipEventRecord(e1, st));
            K3_HIP(hipEventSynchronize(e1));
            float ms = 0.0f;
            K3_HIP(hipEventElapsedTime(&ms, e0, e1));
            if (ms < best_ms) {
                best_ms = ms;
                best = i;
            }
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    p.algo = res[best].algo;
    p.ws = res[best].workspaceSize;
    return K3HIP_OK;
}

}  // namespace

int gemm_bf16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st)
{
    if (M <= 0 || N <= 0 || K <= 0) return K3HIP_OK;
    if (c_dtype != K3HIP_BF16 && c_dtype != K3HIP_F32)
        K3_FAIL(K3HIP_EINVAL, "gemm_bf16: output dtype %d", c_dtype);
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEV) K3_FAIL(K3HIP_EUNSUPPORTED, "gemm_bf16: device %d", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    DevGemm &d = g_dev[dev];
    if (!d.h) {
        K3_LT(hipblasLtCreate(&d.h));
        K3_HIP(hipMalloc(&d.ws, GEMM_WS));
    }
    const auto key = std::make_tuple(M, N, K, c_dtype);
    auto it = d.plans.find(key);
    if (it == d.plans.end()) {
        Plan p;
        int rc = make_plan(d, M, N, K, c_dtype, p, A, W, C, st);
        if (rc) return rc;
        it = d.plans.emplace(key, p).first;
    }
    const Plan &p = it->second;
    const float alpha = 1.0f, beta = 0.0f;
    K3_LT(hipblasLtMatmul(d.h, p.op, &alpha, W, p.la, A, p.lb, &beta, C, p.lc, C, p.lc, &p.algo,
                          p.ws ? d.ws : nullptr, p.ws, st));
    return K3HIP_OK;
}

}  // namespace k3kda

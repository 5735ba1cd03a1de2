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
// Per device: one handle, created on first use. The algorithm of a shape is hipBLASLt's
// heuristic first choice, never a timing, so two processes run the same kernel and produce
// the same bits. A plan (descriptors + algorithm) is cached per shape; shapes that change
// every call (GemmDesc::cache = false, e.g. a growing decode context) build one, run it and
// destroy it. An algorithm that needs workspace gets it stream-ordered on the caller's
// stream for that call, so calls in flight on different streams never share it.
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "kda_internal.h"

namespace k3kda {

namespace {

constexpr size_t GEMM_WS = 64ull << 20;   // largest workspace an algorithm may ask for
constexpr int MAX_DEV = 64;

struct Plan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo;
    size_t ws = 0;
};

typedef std::tuple<int, int, int, int, int, int, long, long, long, int, long, long, long> Key;

struct DevGemm {
    hipblasLtHandle_t h = nullptr;
    std::map<Key, Plan> plans;
};

void destroy_plan(Plan &p)
{
    if (p.la) (void)hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) (void)hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) (void)hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.op) (void)hipblasLtMatmulDescDestroy(p.op);
    p = Plan();
}

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

int set_batch(hipblasLtMatrixLayout_t l, int batch, long stride)
{
    if (batch <= 1) return K3HIP_OK;
    const int32_t n = batch;
    const int64_t st = stride;
    K3_LT(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &n, sizeof n));
    K3_LT(hipblasLtMatrixLayoutSetAttribute(l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &st, sizeof st));
    return K3HIP_OK;
}

// The heuristic's first algorithm for the shape (deterministic: no timing).
int make_plan(DevGemm &d, const GemmDesc &g, Plan &p)
{
    const hipDataType abt = g.ab_dtype == K3HIP_BF16 ? HIP_R_16BF : g.ab_dtype == K3_DT_F16 ? HIP_R_16F : HIP_R_32F;
    const hipDataType ct = g.c_dtype == K3HIP_BF16 ? HIP_R_16BF : HIP_R_32F;
    K3_LT(hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F));
    // column-major view: C^T (N x M) = op(B') . op(A'), B' = B, A' = A
    const hipblasOperation_t ta = g.b_trans ? HIPBLAS_OP_T : HIPBLAS_OP_N, tb = HIPBLAS_OP_N;
    K3_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta));
    K3_LT(hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb));
    if (g.b_trans) K3_LT(hipblasLtMatrixLayoutCreate(&p.la, abt, g.K, g.N, g.ldb));
    else K3_LT(hipblasLtMatrixLayoutCreate(&p.la, abt, g.N, g.K, g.ldb));
    K3_LT(hipblasLtMatrixLayoutCreate(&p.lb, abt, g.K, g.M, g.lda));
    K3_LT(hipblasLtMatrixLayoutCreate(&p.lc, ct, g.N, g.M, g.ldc));
    int rc;
    if ((rc = set_batch(p.la, g.batch, g.sb)) || (rc = set_batch(p.lb, g.batch, g.sa)) ||
        (rc = set_batch(p.lc, g.batch, g.sc)))
        return rc;
    hipblasLtMatmulPreference_t pref = nullptr;
    K3_LT(hipblasLtMatmulPreferenceCreate(&pref));
    const uint64_t wmax = GEMM_WS;
    hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(
        pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wmax, sizeof wmax);
    hipblasLtMatmulHeuristicResult_t res[1];
    int n = 0;
    if (s == HIPBLAS_STATUS_SUCCESS)
        s = hipblasLtMatmulAlgoGetHeuristic(d.h, p.op, p.la, p.lb, p.lc, p.lc, pref, 1, res, &n);
    (void)hipblasLtMatmulPreferenceDestroy(pref);
    if (s != HIPBLAS_STATUS_SUCCESS || n == 0 || res[0].state != HIPBLAS_STATUS_SUCCESS)
        K3_FAIL(K3HIP_EUNSUPPORTED, "hipBLASLt has no algorithm for a %dx%dx%d (batch %d) GEMM (%s)",
                g.M, g.N, g.K, g.batch, lt_status(s));
    p.algo = res[0].algo;
    p.ws = res[0].workspaceSize;
    return K3HIP_OK;
}

int run_plan(DevGemm &d, const Plan &p, const void *A, const void *B, void *C, hipStream_t st)
{
    StreamBuf ws;
    if (p.ws) {
        int rc = stream_alloc(ws, p.ws, st);
        if (rc) return rc;
    }
    const float alpha = 1.0f, beta = 0.0f;
    K3_LT(hipblasLtMatmul(d.h, p.op, &alpha, B, p.la, A, p.lb, &beta, C, p.lc, C, p.lc, &p.algo, ws.p,
                          p.ws, st));
    return K3HIP_OK;
}

}  // namespace

int gemm(const GemmDesc &g, const void *A, const void *B, void *C, hipStream_t st)
{
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.batch <= 0) return K3HIP_OK;
    if ((g.c_dtype != K3HIP_BF16 && g.c_dtype != K3HIP_F32) ||
        (g.ab_dtype != K3HIP_BF16 && g.ab_dtype != K3HIP_F32 && g.ab_dtype != K3_DT_F16))
        K3_FAIL(K3HIP_EINVAL, "gemm: dtypes %d/%d", g.ab_dtype, g.c_dtype);
    int dev = 0;
    K3_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= MAX_DEV) K3_FAIL(K3HIP_EUNSUPPORTED, "gemm: device %d", dev);
    std::lock_guard<std::mutex> lock(g_mu);
    DevGemm &d = g_dev[dev];
    if (!d.h) K3_LT(hipblasLtCreate(&d.h));
    if (!g.cache) {
        Plan p;
        int rc = make_plan(d, g, p);
        if (rc == K3HIP_OK) rc = run_plan(d, p, A, B, C, st);
        destroy_plan(p);
        return rc;
    }
    const Key key{g.M, g.N, g.K, g.ab_dtype, g.c_dtype, g.b_trans ? 1 : 0, g.lda, g.ldb, g.ldc, g.batch,
                  g.sa, g.sb, g.sc};
    auto it = d.plans.find(key);
    if (it == d.plans.end()) {
        Plan p;
        int rc = make_plan(d, g, p);
        if (rc) {
            destroy_plan(p);
            return rc;
        }
        it = d.plans.emplace(key, p).first;
    }
    return run_plan(d, it->second, A, B, C, st);
}

int gemm_bf16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st)
{
    GemmDesc g;
    g.M = M; g.N = N; g.K = K;
    g.ab_dtype = K3HIP_BF16; g.c_dtype = c_dtype; g.b_trans = true;
    g.lda = K; g.ldb = K; g.ldc = N;
    return gemm(g, A, W, C, st);
}

int gemm_f16(int M, int N, int K, const void *A, const void *W, void *C, int c_dtype, hipStream_t st)
{
    GemmDesc g;
    g.M = M; g.N = N; g.K = K;
    g.ab_dtype = K3_DT_F16; g.c_dtype = c_dtype; g.b_trans = true;
    g.lda = K; g.ldb = K; g.ldc = N;
    return gemm(g, A, W, C, st);
}

}  // namespace k3kda

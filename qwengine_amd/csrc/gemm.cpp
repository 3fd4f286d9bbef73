// FP16 GEMM of the prefill projections on hipBLASLt: Y[b][n] (+)= sum_k X[b][k] W[n][k], fp16 inputs, fp32
// accumulation and output (src/cuda/prefill.cuh:20-29, the reference's cublasGemmEx call at src/cuda/prefill.cu:839-852).
// A plain library GEMM: the reference hands it to cuBLAS, this build to hipBLASLt's gfx950 kernels.
//
// In hipBLASLt's column-major terms: D [N x B] = op(A) [N x K] * B [K x B] with A = W viewed as a K x N column-major
// matrix (lda = K) transposed, B = X viewed as K x B (ldb = ldx), C = D = Y viewed as N x B (ldc = ldy).  A handle
// keeps the caller's stream, the caller's workspace and one algorithm per shape, chosen by hipBLASLt's heuristic on
// first use of the shape (no allocation after qwa_gemm_bind).
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>

#include "launch.hpp"
#include "qwattn.h"

namespace {

struct GemmShape {
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

struct GemmCtx {
    hipblasLtHandle_t lt = nullptr;
    hipblasLtMatmulDesc_t desc = nullptr;  // compute fp32, A transposed
    hipStream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    std::mutex mu;
    std::map<std::tuple<int, int, int, int, int>, GemmShape> shapes;  // (N, K, B, ldx, ldy)
};

}  // namespace

extern "C" {

int qwa_fail_status(int status, const char* what);  // capi.hip

void* qwa_gemm_create(void) {
    GemmCtx* g = new GemmCtx();
    if (hipblasLtCreate(&g->lt) != HIPBLAS_STATUS_SUCCESS) {
        delete g;
        return nullptr;
    }
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&g->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(g->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) !=
            HIPBLAS_STATUS_SUCCESS) {
        if (g->desc) hipblasLtMatmulDescDestroy(g->desc);
        hipblasLtDestroy(g->lt);
        delete g;
        return nullptr;
    }
    return g;
}

int qwa_gemm_bind(void* handle, void* stream, void* workspace, size_t bytes) {
    GemmCtx* g = static_cast<GemmCtx*>(handle);
    if (g == nullptr) return qwa_fail_status(QWA_ERR_INVALID, "gemm_bind: no handle");
    if (bytes > 0 && workspace == nullptr) return qwa_fail_status(QWA_ERR_INVALID, "gemm_bind: workspace missing");
    std::lock_guard<std::mutex> lock(g->mu);
    g->stream = static_cast<hipStream_t>(stream);
    g->ws = workspace;
    g->ws_bytes = bytes;
    for (auto& kv : g->shapes) {  // algorithms were chosen for the previous workspace size
        hipblasLtMatrixLayoutDestroy(kv.second.a);
        hipblasLtMatrixLayoutDestroy(kv.second.b);
        hipblasLtMatrixLayoutDestroy(kv.second.c);
    }
    g->shapes.clear();
    return QWA_OK;
}

void qwa_gemm_destroy(void* handle) {
    GemmCtx* g = static_cast<GemmCtx*>(handle);
    if (g == nullptr) return;
    for (auto& kv : g->shapes) {
        hipblasLtMatrixLayoutDestroy(kv.second.a);
        hipblasLtMatrixLayoutDestroy(kv.second.b);
        hipblasLtMatrixLayoutDestroy(kv.second.c);
    }
    hipblasLtMatmulDescDestroy(g->desc);
    hipblasLtDestroy(g->lt);
    delete g;
}

int qwa_gemm_f16(void* handle, const uint16_t* W, int N, int K, const uint16_t* X, int ldx, int B, float* Y, int ldy,
                 int accumulate, void* stream) {
    GemmCtx* g = static_cast<GemmCtx*>(handle);
    if (g == nullptr) return qwa_fail_status(QWA_ERR_INVALID, "gemm_f16: no handle");
    if (N <= 0 || K <= 0 || B <= 0 || ldx < K || ldy < N)
        return qwa_fail_status(QWA_ERR_RANGE, "gemm_f16: bad shape");
    if (!W || !X || !Y) return qwa_fail_status(QWA_ERR_INVALID, "gemm_f16: missing buffer");
    std::lock_guard<std::mutex> lock(g->mu);
    const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : g->stream;
    const auto key = std::make_tuple(N, K, B, ldx, ldy);
    auto it = g->shapes.find(key);
    if (it == g->shapes.end()) {
        GemmShape s;
        if (hipblasLtMatrixLayoutCreate(&s.a, HIP_R_16F, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
            hipblasLtMatrixLayoutCreate(&s.b, HIP_R_16F, K, B, ldx) != HIPBLAS_STATUS_SUCCESS ||
            hipblasLtMatrixLayoutCreate(&s.c, HIP_R_32F, N, B, ldy) != HIPBLAS_STATUS_SUCCESS)
            return qwa_fail_status(QWA_ERR_HIP, "gemm_f16: matrix layouts");
        hipblasLtMatmulPreference_t pref = nullptr;
        hipblasLtMatmulPreferenceCreate(&pref);
        uint64_t ws = g->ws_bytes;
        hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
        hipblasLtMatmulHeuristicResult_t res[1];
        int found = 0;
        const hipblasStatus_t hs =
            hipblasLtMatmulAlgoGetHeuristic(g->lt, g->desc, s.a, s.b, s.c, s.c, pref, 1, res, &found);
        hipblasLtMatmulPreferenceDestroy(pref);
        if (hs != HIPBLAS_STATUS_SUCCESS || found == 0) {
            hipblasLtMatrixLayoutDestroy(s.a);
            hipblasLtMatrixLayoutDestroy(s.b);
            hipblasLtMatrixLayoutDestroy(s.c);
            return qwa_fail_status(QWA_ERR_HIP, "gemm_f16: no hipBLASLt algorithm for this shape");
        }
        s.algo = res[0].algo;
        it = g->shapes.emplace(key, s).first;
    }
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    const GemmShape& s = it->second;
    const hipblasStatus_t hs = hipblasLtMatmul(g->lt, g->desc, &alpha, W, s.a, X, s.b, &beta, Y, s.c, Y, s.c, &s.algo,
                                               g->ws, g->ws_bytes, st);
    if (hs != HIPBLAS_STATUS_SUCCESS) return qwa_fail_status(QWA_ERR_HIP, "gemm_f16: hipblasLtMatmul failed");
    return QWA_OK;
}

}  // extern "C"

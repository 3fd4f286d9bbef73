// FP16 GEMM of the prefill projections on hipBLASLt: Y[b][n] (+)= sum_k X[b][k] W[n][k], fp16 inputs, fp32
// accumulation and output (src/cuda/prefill.cuh:20-29, the reference's cublasGemmEx call at src/cuda/prefill.cu:839-852).
// A plain library GEMM: the reference hands it to cuBLAS, this build to hipBLASLt's gfx950 kernels.
//
// In hipBLASLt's column-major terms: D [N x B] = op(A) [N x K] * B [K x B] with A = W viewed as a K x N column-major
// matrix (lda = K) transposed, B = X viewed as K x B (ldb = ldx), C = D = Y viewed as N x B (ldc = ldy).  A handle
// keeps the caller's stream, the caller's workspace and one algorithm per shape, chosen by hipBLASLt's heuristic on
// first use of the shape (no allocation after qwa_gemm_bind), or by measurement: qwa_gemm_tune runs the heuristic's
// first candidates on the caller's buffers at set-up and keeps the fastest for the shape.
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

static int gemm_layouts(GemmShape& s, int N, int K, int ldx, int B, int ldy) {
    if (hipblasLtMatrixLayoutCreate(&s.a, HIP_R_16F, K, N, K) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&s.b, HIP_R_16F, K, B, ldx) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&s.c, HIP_R_32F, N, B, ldy) != HIPBLAS_STATUS_SUCCESS)
        return qwa_fail_status(QWA_ERR_HIP, "gemm_f16: matrix layouts");
    return QWA_OK;
}

static void gemm_destroy_layouts(GemmShape& s) {
    if (s.a) hipblasLtMatrixLayoutDestroy(s.a);
    if (s.b) hipblasLtMatrixLayoutDestroy(s.b);
    if (s.c) hipblasLtMatrixLayoutDestroy(s.c);
    s.a = s.b = s.c = nullptr;
}

// Up to n candidate algorithms for the shape, best heuristic first; returns how many were found.
static int gemm_candidates(GemmCtx* g, const GemmShape& s, hipblasLtMatmulHeuristicResult_t* res, int n) {
    hipblasLtMatmulPreference_t pref = nullptr;
    hipblasLtMatmulPreferenceCreate(&pref);
    uint64_t ws = g->ws_bytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    int found = 0;
    const hipblasStatus_t hs = hipblasLtMatmulAlgoGetHeuristic(g->lt, g->desc, s.a, s.b, s.c, s.c, pref, n, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    return hs == HIPBLAS_STATUS_SUCCESS ? found : 0;
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
        if (gemm_layouts(s, N, K, ldx, B, ldy) != QWA_OK) {
            gemm_destroy_layouts(s);
            return QWA_ERR_HIP;
        }
        hipblasLtMatmulHeuristicResult_t res[1];
        if (gemm_candidates(g, s, res, 1) == 0) {
            gemm_destroy_layouts(s);
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

int qwa_gemm_tune(void* handle, const uint16_t* W, int N, int K, const uint16_t* X, int ldx, int B, float* Y, int ldy,
                  int max_candidates, void* stream, float* best_us) {
    GemmCtx* g = static_cast<GemmCtx*>(handle);
    if (g == nullptr) return qwa_fail_status(QWA_ERR_INVALID, "gemm_tune: no handle");
    if (N <= 0 || K <= 0 || B <= 0 || ldx < K || ldy < N)
        return qwa_fail_status(QWA_ERR_RANGE, "gemm_tune: bad shape");
    if (!W || !X || !Y) return qwa_fail_status(QWA_ERR_INVALID, "gemm_tune: missing buffer");
    std::lock_guard<std::mutex> lock(g->mu);
    const hipStream_t st = stream ? static_cast<hipStream_t>(stream) : g->stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return qwa_fail_status(QWA_ERR_INVALID, "gemm_tune: the stream is capturing (tune at set-up)");
    // the candidates run with the handle's workspace, which belongs to its bound stream: work still queued there must
    // finish first (a set-up call, so the wait is cheap)
    if (st != g->stream && g->stream != nullptr && hipStreamSynchronize(g->stream) != hipSuccess)
        return qwa_fail_status(QWA_ERR_HIP, "gemm_tune: synchronising the bound stream");
    constexpr int MAXC = 64;
    const int want = max_candidates < 1 ? 16 : (max_candidates > MAXC ? MAXC : max_candidates);
    GemmShape s;
    if (gemm_layouts(s, N, K, ldx, B, ldy) != QWA_OK) {
        gemm_destroy_layouts(s);
        return QWA_ERR_HIP;
    }
    hipblasLtMatmulHeuristicResult_t res[MAXC];
    const int found = gemm_candidates(g, s, res, want);
    if (found == 0) {
        gemm_destroy_layouts(s);
        return qwa_fail_status(QWA_ERR_HIP, "gemm_tune: no hipBLASLt algorithm for this shape");
    }
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
        if (e0) hipEventDestroy(e0);
        gemm_destroy_layouts(s);
        return qwa_fail_status(QWA_ERR_HIP, "gemm_tune: events");
    }
    const float alpha = 1.0f, beta = 0.0f;
    int best = -1;
    float best_ms = 0.0f;
    for (int i = 0; i < found; i++) {
        // 2 warm-up calls, then 5 timed; an algorithm that fails to run is skipped
        bool ok = true;
        for (int r = 0; r < 7 && ok; r++) {
            if (r == 2) hipEventRecord(e0, st);
            ok = hipblasLtMatmul(g->lt, g->desc, &alpha, W, s.a, X, s.b, &beta, Y, s.c, Y, s.c, &res[i].algo, g->ws,
                                 g->ws_bytes, st) == HIPBLAS_STATUS_SUCCESS;
        }
        if (!ok) continue;
        hipEventRecord(e1, st);
        float ms = 0.0f;
        if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) continue;
        if (best < 0 || ms < best_ms) {
            best = i;
            best_ms = ms;
        }
    }
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (best < 0) {
        gemm_destroy_layouts(s);
        return qwa_fail_status(QWA_ERR_HIP, "gemm_tune: no candidate ran");
    }
    s.algo = res[best].algo;
    const auto key = std::make_tuple(N, K, B, ldx, ldy);
    auto it = g->shapes.find(key);
    if (it != g->shapes.end()) {
        gemm_destroy_layouts(it->second);
        g->shapes.erase(it);
    }
    g->shapes.emplace(key, s);
    if (best_us) *best_us = best_ms * 1000.0f / 5.0f;
    return QWA_OK;
}

}  // extern "C"

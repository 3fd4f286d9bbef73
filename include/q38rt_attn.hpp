// q38rt_attn.hpp -- header-only C++ shim that re-creates the reference runtime's attention / KV-cache and Gated
// DeltaNet operator signatures (namespace q38rt::cuda, src/cuda/ops.cuh:54-140 and src/cuda/prefill.cuh:37-62) on top
// of the C ABI in qwattn.h, so the engine's call sites (src/runtime/engine.cpp:1587-1592, 2457-2479) compile unchanged against the
// MI355X library.  The stream type is hipStream_t; fp16 outputs are uint16_t bits (the reference's __half).
// Like the reference, a rejected call prints the reason and aborts (src/cuda/ops.cu:1002-1008).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "qwattn.h"

namespace q38rt {
namespace cuda {

enum class KVType : int { F16 = QWA_KV_F16, Q8_0 = QWA_KV_Q8_0, Q4_0 = QWA_KV_Q4_0 };

struct KVLayer {
    uint8_t* k = nullptr;
    uint8_t* v = nullptr;
    uint16_t* ks = nullptr;
    uint16_t* vs = nullptr;
    int capacity = 0;
};

struct ActQ8 {
    int8_t* q = nullptr;
    float* d = nullptr;
    float* s = nullptr;
};

struct RowSrc {
    const float* dev = nullptr;
    const float* host = nullptr;
    int split = 0, host_ld = 0;
    static RowSrc device(const float* p, int n) {
        RowSrc s;
        s.dev = p;
        s.split = n;
        return s;
    }
    static RowSrc split_at(const float* dev, int split, const float* host, int host_ld) {
        RowSrc s;
        s.dev = dev;
        s.split = split;
        s.host = host;
        s.host_ld = host_ld;
        return s;
    }
};

// src/cuda/ops.cuh:54-62
struct DeltaNetParams {
    const float* conv_w = nullptr;
    const float* dt_bias = nullptr;
    const float* ssm_a = nullptr;
    const float* ssm_norm = nullptr;
    float* conv_state = nullptr;
    float* ssm_state = nullptr;
};

// src/cuda/ops.cuh:74-91 (same defaults: no host part)
struct DNTokens {
    const float* sqkv = nullptr;
    const float* sbeta = nullptr;
    const float* salpha = nullptr;
    const float* qkv = nullptr;
    const float* z = nullptr;
    const float* beta = nullptr;
    const float* alpha = nullptr;
    float* oqkv = nullptr;
    float* obeta = nullptr;
    float* oalpha = nullptr;
    const float* qkv_host = nullptr;
    int qkv_split = 1 << 30, qkv_ld = 0;
    const float* z_host = nullptr;
    int z_split = 1 << 30, z_ld = 0;
    float* o_host = nullptr;
};

namespace detail {
inline void check(int status, const char* fn) {
    if (status != QWA_OK) {
        std::fprintf(stderr, "%s: %s (%s)\n", fn, qwa_status_string(status), qwa_last_error());
        std::abort();
    }
}
inline qwa_kv_layer c(const KVLayer& kv) { return qwa_kv_layer{kv.k, kv.v, kv.ks, kv.vs, kv.capacity}; }
inline qwa_row_src c(const RowSrc& s) { return qwa_row_src{s.dev, s.host, s.split, s.host_ld}; }
inline qwa_dn_params c(const DeltaNetParams& p) {
    return qwa_dn_params{p.conv_w, p.dt_bias, p.ssm_a, p.ssm_norm, p.conv_state, p.ssm_state};
}
inline qwa_dn_tokens c(const DNTokens& t) {
    return qwa_dn_tokens{t.sqkv, t.sbeta,    t.salpha,    t.qkv,    t.z,       t.beta,   t.alpha, t.oqkv, t.obeta,
                         t.oalpha, t.qkv_host, t.qkv_split, t.qkv_ld, t.z_host, t.z_split, t.z_ld, t.o_host};
}
}  // namespace detail

inline size_t kv_value_bytes(KVType t) { return qwa_kv_value_bytes((int)t); }
inline size_t kv_scale_bytes(KVType t) { return qwa_kv_scale_bytes((int)t); }

inline void attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, int pos,
                      float theta, float eps, KVType kvt, KVLayer& kv, float* q_out, float* gate, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    detail::check(qwa_attn_prep(qg, k, v, q_norm, k_norm, pos, theta, eps, (int)kvt, &l, q_out, gate, st), "attn_prep");
}

inline void attn_prep_multi(const RowSrc& qg, const RowSrc& k, const RowSrc& v, const float* q_norm,
                            const float* k_norm, int pos0, int rope_pos0, int n, float theta, float eps, KVType kvt,
                            KVLayer& kv, float* q_out, float* gate, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    const qwa_row_src a = detail::c(qg), b = detail::c(k), c = detail::c(v);
    detail::check(qwa_attn_prep_multi(&a, &b, &c, q_norm, k_norm, pos0, rope_pos0, n, theta, eps, (int)kvt, &l, q_out,
                                      gate, st),
                  "attn_prep_multi");
}

inline size_t attn_work_bytes(int n_pos) { return qwa_attn_work_bytes(n_pos); }
inline int attn_max_positions() { return qwa_attn_max_positions(); }

inline void attn_decode(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int n_pos, void* work,
                        float* out, const ActQ8* oq, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    const qwa_act_q8 a = oq ? qwa_act_q8{oq->q, oq->d, oq->s} : qwa_act_q8{nullptr, nullptr, nullptr};
    detail::check(qwa_attn_decode(q, gate, &l, (int)kvt, n_pos, work, out, oq ? &a : nullptr, st), "attn_decode");
}

inline void attn_decode_multi(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int pos0, int nq,
                              void* work, float* out, const ActQ8* oq, hipStream_t st, float* out_host = nullptr) {
    const qwa_kv_layer l = detail::c(kv);
    const qwa_act_q8 a = oq ? qwa_act_q8{oq->q, oq->d, oq->s} : qwa_act_q8{nullptr, nullptr, nullptr};
    detail::check(qwa_attn_decode_multi(q, gate, &l, (int)kvt, pos0, nq, work, out, oq ? &a : nullptr, st, out_host),
                  "attn_decode_multi");
}

inline void attn_decode_simple(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int n_pos, void* work,
                               float* out, const ActQ8* oq, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    const qwa_act_q8 a = oq ? qwa_act_q8{oq->q, oq->d, oq->s} : qwa_act_q8{nullptr, nullptr, nullptr};
    detail::check(qwa_attn_decode_simple(q, gate, &l, (int)kvt, n_pos, work, out, oq ? &a : nullptr, st),
                  "attn_decode_simple");
}

inline void rope_table(int p0, int B, float theta, float* rope, hipStream_t st) {
    detail::check(qwa_rope_table(p0, B, theta, rope, st), "rope_table");
}

inline void rope_table_pos(const int* pos, int B, float theta, float* rope, hipStream_t st) {
    detail::check(qwa_rope_table_pos(pos, B, theta, rope, st), "rope_table_pos");
}

inline void attn_prep_rows(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm,
                           int B, int p0, const float* rope, float eps, KVType kvt, KVLayer& kv, float* q, float* gate,
                           hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    detail::check(qwa_attn_prep_rows(qg, k, v, q_norm, k_norm, B, p0, rope, eps, (int)kvt, &l, q, gate, st),
                  "attn_prep_rows");
}

// attn_decode_multi without a work buffer, for callers that cannot allocate (no reference counterpart): the library's
// static per-GPU scratch; calls that overlap on one GPU race
inline void attn_decode_multi_noalloc(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int pos0,
                                      int nq, float* out, const ActQ8* oq, hipStream_t st, float* out_host = nullptr) {
    const qwa_kv_layer l = detail::c(kv);
    qwa_act_q8 q8{};
    if (oq) q8 = qwa_act_q8{oq->q, oq->d, oq->s};
    detail::check(qwa_attn_decode_multi_noalloc(q, gate, &l, (int)kvt, pos0, nq, out, oq ? &q8 : nullptr, st, out_host),
                  "attn_decode_multi_noalloc");
}

inline void attn_prefill(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int B, int p0,
                         uint16_t* out16, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    detail::check(qwa_attn_prefill(q, gate, &l, (int)kvt, B, p0, out16, st), "attn_prefill");
}

// optional set-up of the drop-in attn_prefill (no reference counterpart): the workspace of `st`, reserved where the
// engine reserves attn_work_bytes (src/runtime/engine.cpp:724); without it the first prefill on `st` reserves it
inline void attn_prefill_reserve(int max_B, int max_pos, hipStream_t st) {
    detail::check(qwa_attn_prefill_reserve(max_B, max_pos, st), "attn_prefill_reserve");
}
inline void attn_prefill_release(hipStream_t st) { detail::check(qwa_attn_prefill_release(st), "attn_prefill_release"); }
inline size_t attn_prefill_work_bytes(int B, int n_pos) { return qwa_attn_prefill_work_bytes(B, n_pos); }
inline void attn_prefill(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int B, int p0,
                         uint16_t* out16, void* work, size_t work_bytes, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    detail::check(qwa_attn_prefill_ws(q, gate, &l, (int)kvt, B, p0, out16, work, work_bytes, st), "attn_prefill");
}

inline void attn_prefill_simple(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int B, int p0,
                                uint16_t* out16, hipStream_t st) {
    const qwa_kv_layer l = detail::c(kv);
    detail::check(qwa_attn_prefill_simple(q, gate, &l, (int)kvt, B, p0, out16, st), "attn_prefill_simple");
}

// the engine passes its fp16 output buffer as __half* (src/runtime/engine.cpp:2479)
inline void attn_prefill(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int B, int p0,
                         __half* out16, hipStream_t st) {
    attn_prefill(q, gate, kv, kvt, B, p0, reinterpret_cast<uint16_t*>(out16), st);
}

inline void attn_prefill_simple(const float* q, const float* gate, const KVLayer& kv, KVType kvt, int B, int p0,
                                __half* out16, hipStream_t st) {
    attn_prefill_simple(q, gate, kv, kvt, B, p0, reinterpret_cast<uint16_t*>(out16), st);
}

// ---- Gated DeltaNet: src/cuda/ops.cuh:67-68, 96-97; src/cuda/prefill.cuh:41-44
inline void deltanet_step(const DeltaNetParams& p, const float* qkv, const float* z, const float* beta_raw,
                          const float* alpha_raw, int parity, float eps, float* o, const ActQ8* oq, hipStream_t st) {
    const qwa_dn_params cp = detail::c(p);
    qwa_act_q8 q8{};
    if (oq) q8 = qwa_act_q8{oq->q, oq->d, oq->s};
    detail::check(qwa_deltanet_step(&cp, qkv, z, beta_raw, alpha_raw, parity, eps, o, oq ? &q8 : nullptr, st),
                  "deltanet_step");
}

inline void deltanet_multi(const DeltaNetParams& p, int cin, const DNTokens& in, int n_commit, int n_new,
                           int write_after, float eps, float* o, const ActQ8* oq, hipStream_t st) {
    const qwa_dn_params cp = detail::c(p);
    const qwa_dn_tokens ct = detail::c(in);
    qwa_act_q8 q8{};
    if (oq) q8 = qwa_act_q8{oq->q, oq->d, oq->s};
    detail::check(qwa_deltanet_multi(&cp, cin, &ct, n_commit, n_new, write_after, eps, o, oq ? &q8 : nullptr, st),
                  "deltanet_multi");
}

inline size_t dn_work_bytes(int B) { return qwa_dn_work_bytes(B); }

inline void deltanet_rows(const DeltaNetParams& p, const float* qkv, const float* z, const float* beta_raw,
                          const float* alpha_raw, int B, int cin, float eps, void* work, float* core_out, __half* o16,
                          hipStream_t st) {
    const qwa_dn_params cp = detail::c(p);
    detail::check(qwa_deltanet_rows(&cp, qkv, z, beta_raw, alpha_raw, B, cin, eps, work, core_out,
                                    reinterpret_cast<uint16_t*>(o16), st),
                  "deltanet_rows");
}

// ---- consumers of the attention output (src/cuda/gemv.cuh:20-39, src/cuda/prefill.cuh:16-18).  The format argument
// is the engine's QuantFormat (include/q38rt/q38rt_types.h:36-66), taken as any enum whose values are the format ids.
// Like the reference these return false for a format without a kernel; other rejected arguments abort.
template <class QF>
inline bool gemv_q8_supported(QF type) {
    return qwa_gemv_q8_supported(static_cast<int>(type)) != 0;
}

inline void quantize_act_q8(const float* x, int K, int n_rows, ActQ8 out, hipStream_t st) {
    const qwa_act_q8 q8{out.q, out.d, out.s};
    detail::check(qwa_quantize_act_q8(x, K, n_rows, &q8, st), "quantize_act_q8");
}

template <class QF>
inline bool gemv_q8(QF type, const void* W, size_t row_bytes, int K, int N, const ActQ8& act, float* y, hipStream_t st,
                    bool accumulate = false) {
    if (!gemv_q8_supported(type)) return false;
    const qwa_act_q8 q8{act.q, act.d, act.s};
    detail::check(qwa_gemv_q8(static_cast<int>(type), W, row_bytes, K, N, &q8, y, st, accumulate ? 1 : 0), "gemv_q8");
    return true;
}

template <class QF>
inline bool gemv_q8n(QF type, const void* W, size_t row_bytes, int K, int N, const ActQ8& act, int nb, int act_ld,
                     float* y, int y_ld, hipStream_t st, bool accumulate = false) {
    if (!gemv_q8_supported(type)) return false;
    const qwa_act_q8 q8{act.q, act.d, act.s};
    detail::check(qwa_gemv_q8n(static_cast<int>(type), W, row_bytes, K, N, &q8, nb, act_ld, y, y_ld, st,
                               accumulate ? 1 : 0),
                  "gemv_q8n");
    return true;
}

inline void gemv_bf16(const uint16_t* W, int K, int N, const float* x, float* y, hipStream_t st) {
    detail::check(qwa_gemv_bf16(W, K, N, x, y, st), "gemv_bf16");
}

template <class QF>
inline bool dequant_rows_f16(QF type, const void* W, size_t row_bytes, int K, int rows, __half* out, hipStream_t st) {
    if (qwa_w_row_bytes(static_cast<int>(type), K) == 0) return false;
    detail::check(qwa_dequant_rows_f16(static_cast<int>(type), W, row_bytes, K, rows, reinterpret_cast<uint16_t*>(out),
                                       st),
                  "dequant_rows_f16");
    return true;
}

// src/cuda/prefill.cuh:20-29: the handle is this library's hipBLASLt context (the reference's cuBLAS handle)
inline void* cublas_create() { return qwa_gemm_create(); }
inline bool cublas_bind(void* h, hipStream_t st, void* workspace, size_t bytes) {
    return qwa_gemm_bind(h, st, workspace, bytes) == QWA_OK;
}
inline void cublas_destroy(void* h) { qwa_gemm_destroy(h); }
inline void gemm_f16(void* h, const __half* W, int N, int K, const __half* X, int ldx, int B, float* Y, int ldy,
                     bool accumulate, hipStream_t st) {
    detail::check(qwa_gemm_f16(h, reinterpret_cast<const uint16_t*>(W), N, K, reinterpret_cast<const uint16_t*>(X),
                               ldx, B, Y, ldy, accumulate ? 1 : 0, st),
                  "gemm_f16");
}

}  // namespace cuda
}  // namespace q38rt

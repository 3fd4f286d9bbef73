/*
 * qwo.h -- CPU oracle for the gated-attention hot path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and only as the
 * checker or the timed CPU baseline.  The product path (qwengine_amd/) never links, imports or calls it.
 *
 * It is a from-scratch C restatement of the reference's CPU semantics for this path:
 *   - fp16 conversion          : src/quant/quant_formats.h:29-78 (exact IEEE binary16, round to nearest even)
 *   - Q8_0 / Q4_0 quantizers   : src/quant/quant_ref.cpp:507-538 (ggml semantics, no FMA contraction)
 *   - Q8_0 / Q4_0 dequantizers : src/quant/quant_ref.cpp:302-319
 *   - split KV row layout      : src/cuda/ops.cuh:99-113, src/cuda/common.cuh:54-80
 *   - gated attention          : src/reference/ref_model.cpp:23-40 (dot_f32), :138-163 (softmax / P.V), :48 (sigmoid)
 *   - q/k prep (RMSNorm, RoPE) : src/cuda/ops.cu:309-358, tests/kernels/test_ops.cu:260-272 (double precision)
 *   - RoPE tables              : src/cuda/prefill.cu:385-407
 *   - ActQ8 epilogue           : src/cuda/common.cuh:188-197
 *   - Gated DeltaNet core      : src/reference/ref_model.cpp:169-256 (after the projections), :41-50 (helpers)
 * Each function below names the reference lines it follows.
 */
#ifndef QWO_H
#define QWO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { QWO_F16 = 0, QWO_Q8_0 = 1, QWO_Q4_0 = 2 };
enum { QWO_NH = 24, QWO_NKV = 4, QWO_D = 256, QWO_GROUP = 6, QWO_NROT = 64 };

uint16_t qwo_fp32_to_fp16(float f);
float qwo_fp16_to_fp32(uint16_t h);
void qwo_fp32_to_fp16_n(const float* x, uint16_t* y, int64_t n);
void qwo_fp16_to_fp32_n(const uint16_t* x, float* y, int64_t n);

/* ggml block formats: Q8_0 = {fp16 d; int8 qs[32]} (34 B), Q4_0 = {fp16 d; uint8 qs[16]} (18 B, element j in the
 * low nibble and j+16 in the high nibble of byte j). n must be a multiple of 32. */
void qwo_quantize_q8_0(const float* x, uint8_t* blocks, int64_t n);
void qwo_quantize_q4_0(const float* x, uint8_t* blocks, int64_t n);
void qwo_dequantize_q8_0(const uint8_t* blocks, float* y, int64_t n);
void qwo_dequantize_q4_0(const uint8_t* blocks, float* y, int64_t n);

/* Split KV layout of one 256-value head row: values (F16 512 B, Q8_0 256 B, Q4_0 128 B with element 2i in the low
 * nibble of byte i) and 8 fp16 block scales (absent for F16). */
size_t qwo_kv_value_bytes(int kvt);
size_t qwo_kv_scale_bytes(int kvt);
void qwo_kv_store_rows(int kvt, const float* x, int64_t nrows, uint8_t* vals, uint16_t* scales);
void qwo_kv_load_rows(int kvt, const uint8_t* vals, const uint16_t* scales, int64_t nrows, float* out);

/* Gated GQA attention for nq queries at cache positions pos0..pos0+nq-1 (query t sees keys 0..pos0+t).
 * q, gate: [nq][24][256]; K, V: dequantized cache [4][ld][256] (head-major, row stride ld positions);
 * out: [nq][24][256].  mode 0: dot products in double (exact oracle); mode 1: the reference CPU arithmetic
 * (fp32 8-lane x 4 FMA partial sums reduced in double).  threads <= 0: OpenMP default. */
void qwo_attention(const float* q, const float* gate, const float* K, const float* V, int64_t ld, int pos0, int nq,
                   int mode, int threads, float* out);

/* attn_prep for n tokens (cache/rotary positions rope_pos0 + r): qg [n][24][512] (q | gate per head),
 * k, v [n][4][256], norm weights [256].  Writes q_out, gate [n][24][256] and the normed+roped k_out [n][4][256]
 * (v is stored unmodified).  Double precision throughout. */
void qwo_attn_prep(const float* qg, const float* k, const float* q_norm, const float* k_norm, int n, int rope_pos0,
                   float theta, float eps, float* q_out, float* gate, float* k_out);
/* The same with a precomputed rope table [n][64] (cos[32] | sin[32]) as in attn_prep_rows. */
void qwo_attn_prep_table(const float* qg, const float* k, const float* q_norm, const float* k_norm, int n,
                         const float* rope, float eps, float* q_out, float* gate, float* k_out);

/* rope[t][i] = cos, rope[t][32+i] = sin of (p0+t) * theta^(-2i/64), angle reduced mod 2 pi in double. */
void qwo_rope_table(int p0, int B, float theta, float* rope);
/* M-RoPE: frequency i turns with pos[t*3 + i%3]. */
void qwo_rope_table_pos(const int* pos, int B, float theta, float* rope);

/* ActQ8 epilogue over n values (n multiple of 32): d = amax/127, q = round-half-even(v/d), s = d * sum(q). */
void qwo_act_q8(const float* v, int64_t n, int8_t* q, float* d, float* s);

int qwo_max_threads(void);

/* Gated DeltaNet core of one layer over T tokens (src/reference/ref_model.cpp:169-256, from the projection outputs
 * on; helpers :41-50).  Per token: causal depthwise conv (width 4) + SiLU over the 10240 q|k|v channels, L2
 * normalization of the 16 q and k heads (sums in double, clamp eps), per value head h (key head h % 16):
 * beta = sigmoid(b), decay = exp(softplus(a + dt_bias) * ssm_a), S *= decay, kv = S^T k, delta = (v - kv) * beta,
 * S += k delta^T, o = S^T q / sqrt(128), then the gated RMSNorm rmsnorm(o) * ssm_norm * silu(z).
 * qkv [T][10240], z [T][6144], b / a [T][ld_ba] (the first 48 used), conv_w [10240][4], dt_bias / ssm_a [48],
 * ssm_norm [128].  conv_state [3][10240] (oldest input first) and S [48][128 k index i][128 v index j] are read and
 * updated in place.  o [T][6144]. */
enum { QWO_DN_CH = 10240, QWO_DN_QK = 2048, QWO_DN_V = 6144, QWO_DN_VH = 48, QWO_DN_KH = 16, QWO_DN_HD = 128 };
void qwo_deltanet(const float* qkv, const float* z, const float* b, const float* a, int ld_ba, int T,
                  const float* conv_w, const float* dt_bias, const float* ssm_a, const float* ssm_norm, float eps,
                  float* conv_state, float* S, float* o);

/* Weight formats of the output-projection consumer (decode GEMV over ActQ8 activations, prefill fp16 dequant):
 * ggml block layouts of src/quant/quant_formats.h:92-104, 256 weights per block.  Format ids are the reference's
 * QuantFormat values (include/q38rt/q38rt_types.h:36-66). */
enum {
    QWO_W_Q2_K = 10, QWO_W_Q4_K = 12, QWO_W_Q6_K = 14, QWO_W_IQ2_XXS = 16, QWO_W_IQ2_XS = 17, QWO_W_IQ3_XXS = 18,
    QWO_W_IQ3_S = 21, QWO_W_IQ2_S = 22, QWO_W_IQ4_XS = 23, QWO_W_BF16 = 30
};
/* Entry idx of an i-quant codebook as its little-endian grid bytes (table: 0 IQ2XXS, 1 IQ2XS, 2 IQ2S, 3 IQ3XXS,
 * 4 IQ3S); 0 for an index out of range. */
uint64_t qwo_iq_grid(int table, int idx);
/* bytes of one row of K weights (0 for an unsupported format or K not a multiple of the block) */
size_t qwo_w_row_bytes(int fmt, int64_t K);
/* dequantize one row of K weights to fp32; 0 on success, -1 for an unsupported format */
int qwo_w_dequant_row(int fmt, const uint8_t* row, float* y, int64_t K);
/* y[c][r] = sum_k dequant(W[r])[k] * d_c[k / 32] * q_c[k] in double, for nc activation columns (q [nc][K],
 * d [nc][K / 32]); the decode GEMV's exact target (tests/kernels/test_gemv.cu:69-92) */
int qwo_gemv_ref(int fmt, const uint8_t* W, size_t row_bytes, int K, int N, const int8_t* q, const float* d, int nc,
                 double* y);

#ifdef __cplusplus
}
#endif
#endif

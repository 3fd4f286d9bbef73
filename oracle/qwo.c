/*
 * qwo.c -- CPU oracle for the gated-attention hot path.  TEST INFRASTRUCTURE ONLY: loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker / CPU baseline, never by the product.
 *
 * Compiled with -ffp-contract=off (no FMA contraction) so the quantizers round exactly like the reference's
 * scalar code (the reference builds src/quant/quant_ref.cpp with the same flag, CMakeLists.txt:66-68).
 */
#include "qwo.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#if defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define QWO_HAVE_AVX2 1
#endif

/* ---------------------------------------------------------------------------------------------------------------
 * fp16 <-> fp32, exact IEEE binary16 with round-to-nearest-even.  Semantics of src/quant/quant_formats.h:29-78.
 * ------------------------------------------------------------------------------------------------------------- */
float qwo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int e = (h >> 10) & 31;
    const uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13); /* inf / nan keep their payload */
    } else if (e == 0) {
        /* zero or subnormal: value is m * 2^-24, exactly representable in fp32 */
        float f = (float)m * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else {
        bits = sign | ((uint32_t)(e - 15 + 127) << 23) | (m << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

uint16_t qwo_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u); /* nan -> quiet nan */
    if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
    const int e = (int)(ax >> 23) - 127; /* unbiased exponent of the fp32 value */
    if (e >= 16) return (uint16_t)(sign | 0x7C00u);
    uint32_t mant = (ax & 0x7FFFFFu) | (ax >= 0x00800000u ? 0x800000u : 0u);
    int shift; /* number of low mantissa bits dropped */
    uint32_t base;
    if (e >= -14) {
        /* normal fp16: keep 10 fraction bits */
        shift = 13;
        base = ((uint32_t)(e + 15) << 10);
        mant &= 0x7FFFFFu;
    } else {
        /* subnormal fp16: value = mant * 2^(e-23) expressed in units of 2^-24 */
        shift = 13 + (-14 - e);
        if (ax < 0x00800000u) return sign; /* fp32 subnormals are far below fp16's range */
        if (shift > 24) return sign;
        base = 0;
    }
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    /* a carry out of the fraction correctly bumps the exponent (or turns the max normal into inf) */
    return (uint16_t)(sign | (base + q));
}

void qwo_fp32_to_fp16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = qwo_fp32_to_fp16(x[i]);
}
void qwo_fp16_to_fp32_n(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = qwo_fp16_to_fp32(x[i]);
}

/* ---------------------------------------------------------------------------------------------------------------
 * ggml Q8_0 / Q4_0 block quantizers: src/quant/quant_ref.cpp:507-538.
 * ------------------------------------------------------------------------------------------------------------- */
void qwo_quantize_q8_0(const float* x, uint8_t* blocks, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float* xb = x + 32 * b;
        uint8_t* out = blocks + 34 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = qwo_fp32_to_fp16(d);
        memcpy(out, &dh, 2);
        for (int j = 0; j < 32; j++) {
            const float r = roundf(xb[j] * id); /* half away from zero */
            out[2 + j] = (uint8_t)(int8_t)(int)r;
        }
    }
}

void qwo_quantize_q4_0(const float* x, uint8_t* blocks, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        const float* xb = x + 32 * b;
        uint8_t* out = blocks + 18 * b;
        /* max = signed value of the FIRST element of largest magnitude */
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(xb[j]);
            if (a > amax) {
                amax = a;
                mx = xb[j];
            }
        }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = qwo_fp32_to_fp16(d);
        memcpy(out, &dh, 2);
        for (int j = 0; j < 16; j++) {
            const float t0 = xb[j] * id;
            const float t1 = xb[j + 16] * id;
            /* truncating conversion through int8, then clamp to 15 */
            int c0 = (int)(int8_t)(int)(t0 + 8.5f);
            int c1 = (int)(int8_t)(int)(t1 + 8.5f);
            if (c0 > 15) c0 = 15;
            if (c1 > 15) c1 = 15;
            out[2 + j] = (uint8_t)((c0 & 15) | ((c1 & 15) << 4));
        }
    }
}

void qwo_dequantize_q8_0(const uint8_t* blocks, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        uint16_t dh;
        memcpy(&dh, blocks + 34 * b, 2);
        const float d = qwo_fp16_to_fp32(dh);
        for (int j = 0; j < 32; j++) y[32 * b + j] = (float)(int8_t)blocks[34 * b + 2 + j] * d;
    }
}

void qwo_dequantize_q4_0(const uint8_t* blocks, float* y, int64_t n) {
    for (int64_t b = 0; b < n / 32; b++) {
        uint16_t dh;
        memcpy(&dh, blocks + 18 * b, 2);
        const float d = qwo_fp16_to_fp32(dh);
        for (int j = 0; j < 16; j++) {
            const uint8_t byte = blocks[18 * b + 2 + j];
            y[32 * b + j] = (float)((int)(byte & 15) - 8) * d;
            y[32 * b + j + 16] = (float)((int)(byte >> 4) - 8) * d;
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------------
 * Split KV layout (src/cuda/ops.cuh:99-113, src/cuda/common.cuh:54-80): the same quantizer values as ggml's
 * blocks, regrouped per 256-value row into contiguous values + 8 fp16 scales, Q4_0 codes pairwise (2i low, 2i+1 high).
 * ------------------------------------------------------------------------------------------------------------- */
size_t qwo_kv_value_bytes(int kvt) {
    return kvt == QWO_F16 ? 512u : kvt == QWO_Q8_0 ? 256u : kvt == QWO_Q4_0 ? 128u : 0u;
}
size_t qwo_kv_scale_bytes(int kvt) { return kvt == QWO_Q8_0 || kvt == QWO_Q4_0 ? 16u : 0u; }

void qwo_kv_store_rows(int kvt, const float* x, int64_t nrows, uint8_t* vals, uint16_t* scales) {
    const size_t vb = qwo_kv_value_bytes(kvt);
    for (int64_t r = 0; r < nrows; r++) {
        const float* xr = x + 256 * r;
        uint8_t* vr = vals + vb * r;
        if (kvt == QWO_F16) {
            for (int i = 0; i < 256; i++) {
                const uint16_t h = qwo_fp32_to_fp16(xr[i]);
                memcpy(vr + 2 * i, &h, 2);
            }
            continue;
        }
        uint16_t* sr = scales + 8 * r;
        for (int b = 0; b < 8; b++) {
            uint8_t blk[34];
            if (kvt == QWO_Q8_0) {
                qwo_quantize_q8_0(xr + 32 * b, blk, 32);
                memcpy(&sr[b], blk, 2);
                memcpy(vr + 32 * b, blk + 2, 32);
            } else {
                qwo_quantize_q4_0(xr + 32 * b, blk, 32);
                memcpy(&sr[b], blk, 2);
                uint8_t codes[32];
                for (int j = 0; j < 16; j++) {
                    codes[j] = blk[2 + j] & 15;
                    codes[j + 16] = blk[2 + j] >> 4;
                }
                for (int i = 0; i < 16; i++) vr[16 * b + i] = (uint8_t)(codes[2 * i] | (codes[2 * i + 1] << 4));
            }
        }
    }
}

void qwo_kv_load_rows(int kvt, const uint8_t* vals, const uint16_t* scales, int64_t nrows, float* out) {
    const size_t vb = qwo_kv_value_bytes(kvt);
    for (int64_t r = 0; r < nrows; r++) {
        const uint8_t* vr = vals + vb * r;
        float* o = out + 256 * r;
        if (kvt == QWO_F16) {
            for (int i = 0; i < 256; i++) {
                uint16_t h;
                memcpy(&h, vr + 2 * i, 2);
                o[i] = qwo_fp16_to_fp32(h);
            }
            continue;
        }
        const uint16_t* sr = scales + 8 * r;
        for (int i = 0; i < 256; i++) {
            const float d = qwo_fp16_to_fp32(sr[i / 32]);
            int c;
            if (kvt == QWO_Q8_0) c = (int8_t)vr[i];
            else c = (int)((vr[i / 2] >> (4 * (i & 1))) & 15) - 8;
            o[i] = (float)c * d;
        }
    }
}

/* ---------------------------------------------------------------------------------------------------------------
 * Gated attention: src/reference/ref_model.cpp:138-163 (+ :48 sigmoid).  Scores in double, softmax in double,
 * P.V accumulated in double, normalised, then multiplied by sigmoid(gate).
 * ------------------------------------------------------------------------------------------------------------- */

/* The reference CPU dot product (src/reference/ref_model.cpp:23-40): four 8-lane fp32 FMA accumulators over
 * 32-element steps, lanes summed pairwise in fp32, the 8 lanes then summed in double. */
static float dot_ref(const float* a, const float* b, int n) {
#ifdef QWO_HAVE_AVX2
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int u = 0; u < 4; u++)
            acc[u] = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8 * u), _mm256_loadu_ps(b + i + 8 * u), acc[u]);
    const __m256 s = _mm256_add_ps(_mm256_add_ps(acc[0], acc[1]), _mm256_add_ps(acc[2], acc[3]));
    float lanes[8];
    _mm256_storeu_ps(lanes, s);
    double total = 0.0;
    for (int j = 0; j < 8; j++) total += lanes[j];
    for (; i < n; i++) total += (double)a[i] * b[i];
    return (float)total;
#else
    float lanes[4][8];
    memset(lanes, 0, sizeof lanes);
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int u = 0; u < 4; u++)
            for (int j = 0; j < 8; j++) lanes[u][j] = fmaf(a[i + 8 * u + j], b[i + 8 * u + j], lanes[u][j]);
    double total = 0.0;
    for (int j = 0; j < 8; j++) total += (double)((lanes[0][j] + lanes[1][j]) + (lanes[2][j] + lanes[3][j]));
    for (; i < n; i++) total += (double)a[i] * b[i];
    return (float)total;
#endif
}

/* Products of two floats are exact in double; four interleaved partial sums (n is a multiple of 4 here) let the
 * compiler keep the sum in vector registers. */
static double dot_exact(const float* a, const float* b, int n) {
    double s[4] = {0.0, 0.0, 0.0, 0.0};
    int i = 0;
    for (; i + 4 <= n; i += 4)
        for (int u = 0; u < 4; u++) s[u] += (double)a[i + u] * (double)b[i + u];
    for (; i < n; i++) s[0] += (double)a[i] * (double)b[i];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

void qwo_attention(const float* q, const float* gate, const float* K, const float* V, int64_t ld, int pos0, int nq,
                   int mode, int threads, float* out) {
    const int nthr = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nthr)
    {
        const int64_t maxpos = (int64_t)pos0 + nq;
        double* s = (double*)malloc(sizeof(double) * (size_t)maxpos);
        double* acc = (double*)malloc(sizeof(double) * 256);
#pragma omp for collapse(2) schedule(dynamic)
        for (int t = 0; t < nq; t++) {
            for (int h = 0; h < QWO_NH; h++) {
                const int g = h / QWO_GROUP;
                const int64_t npos = (int64_t)pos0 + t + 1; /* causal: keys 0..pos0+t */
                const float* qh = q + ((int64_t)t * QWO_NH + h) * 256;
                const float* Kg = K + (int64_t)g * ld * 256;
                const float* Vg = V + (int64_t)g * ld * 256;
                double mx = -INFINITY;
                for (int64_t j = 0; j < npos; j++) {
                    const double dot = mode == 0 ? dot_exact(qh, Kg + j * 256, 256) : (double)dot_ref(qh, Kg + j * 256, 256);
                    s[j] = dot * (1.0 / 16.0); /* softmax scale 1/sqrt(256) */
                    if (s[j] > mx) mx = s[j];
                }
                double den = 0.0;
                for (int64_t j = 0; j < npos; j++) {
                    s[j] = exp(s[j] - mx);
                    den += s[j];
                }
                for (int d = 0; d < 256; d++) acc[d] = 0.0;
                for (int64_t j = 0; j < npos; j++) {
                    const float* vr = Vg + j * 256;
                    const double p = s[j];
                    for (int d = 0; d < 256; d++) acc[d] += p * (double)vr[d];
                }
                const float* gh = gate + ((int64_t)t * QWO_NH + h) * 256;
                float* o = out + ((int64_t)t * QWO_NH + h) * 256;
                for (int d = 0; d < 256; d++) {
                    const float a = (float)(acc[d] / den);
                    const float sg = 1.0f / (1.0f + expf(-gh[d]));
                    o[d] = a * sg;
                }
            }
        }
        free(s);
        free(acc);
    }
}

/* ---------------------------------------------------------------------------------------------------------------
 * q/k prep: per-head RMSNorm * weight, NeoX RoPE on dims [0,64) in pairs (i, i+32); the angle theta^(-2i/64)*pos in
 * double.  Follows src/cuda/ops.cu:309-358 with the double-precision arithmetic of tests/kernels/test_ops.cu:260-272.
 * ------------------------------------------------------------------------------------------------------------- */
static void norm_rope_row(const float* src, const float* w, const double* cs, const double* sn, float eps, float* dst) {
    double ss = 0.0;
    for (int d = 0; d < 256; d++) ss += (double)src[d] * (double)src[d];
    const double sc = 1.0 / sqrt(ss / 256.0 + (double)eps);
    double x[256];
    for (int d = 0; d < 256; d++) x[d] = (double)src[d] * sc * (double)w[d];
    for (int i = 0; i < 32; i++) {
        const double x0 = x[i], x1 = x[i + 32];
        x[i] = x0 * cs[i] - x1 * sn[i];
        x[i + 32] = x0 * sn[i] + x1 * cs[i];
    }
    for (int d = 0; d < 256; d++) dst[d] = (float)x[d];
}

static void prep_token(const float* qg, const float* k, const float* q_norm, const float* k_norm, const double* cs,
                       const double* sn, float eps, float* q_out, float* gate, float* k_out) {
    for (int h = 0; h < QWO_NH; h++) {
        norm_rope_row(qg + h * 512, q_norm, cs, sn, eps, q_out + h * 256);
        memcpy(gate + h * 256, qg + h * 512 + 256, 256 * sizeof(float));
    }
    for (int g = 0; g < QWO_NKV; g++) norm_rope_row(k + g * 256, k_norm, cs, sn, eps, k_out + g * 256);
}

static void rope_angles(double pos, double theta, int i, double* c, double* s) {
    const double inv = pow(theta, -2.0 * i / 64.0);
    const double ang = fmod(pos * inv, 6.283185307179586476925286766559);
    *c = cos(ang);
    *s = sin(ang);
}

void qwo_attn_prep(const float* qg, const float* k, const float* q_norm, const float* k_norm, int n, int rope_pos0,
                   float theta, float eps, float* q_out, float* gate, float* k_out) {
    for (int r = 0; r < n; r++) {
        double cs[32], sn[32];
        for (int i = 0; i < 32; i++) rope_angles((double)(rope_pos0 + r), (double)theta, i, &cs[i], &sn[i]);
        prep_token(qg + (int64_t)r * QWO_NH * 512, k + (int64_t)r * 1024, q_norm, k_norm, cs, sn, eps,
                   q_out + (int64_t)r * 6144, gate + (int64_t)r * 6144, k_out + (int64_t)r * 1024);
    }
}

void qwo_attn_prep_table(const float* qg, const float* k, const float* q_norm, const float* k_norm, int n,
                         const float* rope, float eps, float* q_out, float* gate, float* k_out) {
    for (int r = 0; r < n; r++) {
        double cs[32], sn[32];
        for (int i = 0; i < 32; i++) {
            cs[i] = rope[(int64_t)r * 64 + i];
            sn[i] = rope[(int64_t)r * 64 + 32 + i];
        }
        prep_token(qg + (int64_t)r * QWO_NH * 512, k + (int64_t)r * 1024, q_norm, k_norm, cs, sn, eps,
                   q_out + (int64_t)r * 6144, gate + (int64_t)r * 6144, k_out + (int64_t)r * 1024);
    }
}

/* src/cuda/prefill.cu:385-407 */
void qwo_rope_table(int p0, int B, float theta, float* rope) {
    for (int t = 0; t < B; t++)
        for (int i = 0; i < 32; i++) {
            double c, s;
            rope_angles((double)(p0 + t), (double)theta, i, &c, &s);
            rope[(int64_t)t * 64 + i] = (float)c;
            rope[(int64_t)t * 64 + 32 + i] = (float)s;
        }
}

void qwo_rope_table_pos(const int* pos, int B, float theta, float* rope) {
    for (int t = 0; t < B; t++)
        for (int i = 0; i < 32; i++) {
            double c, s;
            rope_angles((double)pos[t * 3 + i % 3], (double)theta, i, &c, &s);
            rope[(int64_t)t * 64 + i] = (float)c;
            rope[(int64_t)t * 64 + 32 + i] = (float)s;
        }
}

/* ActQ8 epilogue, src/cuda/common.cuh:188-197: round half to even (not the KV quantizer's half-away). */
void qwo_act_q8(const float* v, int64_t n, int8_t* q, float* d, float* s) {
    for (int64_t b = 0; b < n / 32; b++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(v[32 * b + j]);
            if (a > amax) amax = a;
        }
        const float db = amax / 127.0f;
        int sum = 0;
        for (int j = 0; j < 32; j++) {
            const int qi = db > 0.0f ? (int)nearbyintf(v[32 * b + j] / db) : 0;
            q[32 * b + j] = (int8_t)qi;
            sum += qi;
        }
        d[b] = db;
        s[b] = db * (float)sum;
    }
}

int qwo_max_threads(void) { return omp_get_max_threads(); }


/* ---- Gated DeltaNet core: src/reference/ref_model.cpp:169-256 (helpers rmsnorm / sigmoidf / siluf / softplusf at
 * :41-50).  Same statement order as the reference's token loop. */
static float dn_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
static float dn_silu(float x) { return x / (1.0f + expf(-x)); }
static float dn_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

static void dn_rmsnorm(const float* x, const float* w, float* y, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float scale = 1.0f / sqrtf((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) y[i] = x[i] * scale * w[i];
}

void qwo_deltanet(const float* qkv, const float* z, const float* b, const float* a, int ld_ba, int T,
                  const float* conv_w, const float* dt_bias, const float* ssm_a, const float* ssm_norm, float eps,
                  float* conv_state, float* S, float* o) {
    enum { CH = QWO_DN_CH, QK = QWO_DN_QK, VD = QWO_DN_V, VH = QWO_DN_VH, KH = QWO_DN_KH, HD = QWO_DN_HD };
    float* conv = (float*)malloc(sizeof(float) * CH);
    float* qn = (float*)malloc(sizeof(float) * QK);
    float* kn = (float*)malloc(sizeof(float) * QK);
    float* cs = conv_state;
    for (int t = 0; t < T; t++) {
        const float* x = qkv + (size_t)t * CH;
        /* causal conv (width 4) + SiLU, the window slides by one input (ref_model.cpp:191-200) */
        for (int c = 0; c < CH; c++) {
            const float* w = conv_w + (size_t)c * 4;
            const float acc = w[0] * cs[0 * CH + c] + w[1] * cs[1 * CH + c] + w[2] * cs[2 * CH + c] + w[3] * x[c];
            conv[c] = dn_silu(acc);
            cs[0 * CH + c] = cs[1 * CH + c];
            cs[1 * CH + c] = cs[2 * CH + c];
            cs[2 * CH + c] = x[c];
        }
        /* L2 normalization of q and k per key head, sums in double (ref_model.cpp:202-215) */
        for (int h = 0; h < KH; h++) {
            double sq = 0, sk = 0;
            for (int d = 0; d < HD; d++) {
                sq += (double)conv[h * HD + d] * conv[h * HD + d];
                sk += (double)conv[QK + h * HD + d] * conv[QK + h * HD + d];
            }
            const float sqf = (float)sqrt(sq), skf = (float)sqrt(sk);
            const float iq = 1.0f / (sqf > eps ? sqf : eps);
            const float ik = 1.0f / (skf > eps ? skf : eps);
            for (int d = 0; d < HD; d++) {
                qn[h * HD + d] = conv[h * HD + d] * iq;
                kn[h * HD + d] = conv[QK + h * HD + d] * ik;
            }
        }
        const float* vv = conv + 2 * QK;
        const float qscale = 1.0f / sqrtf((float)HD);
#pragma omp parallel for
        for (int h = 0; h < VH; h++) {
            const int kh = h % KH;
            const float beta = dn_sigmoid(b[(size_t)t * ld_ba + h]);
            const float g = dn_softplus(a[(size_t)t * ld_ba + h] + dt_bias[h]) * ssm_a[h];
            const float decay = expf(g);
            float* Sh = S + (size_t)h * HD * HD; /* Sh[i * 128 + j]: i = k index, j = v index */
            const float* kk = kn + kh * HD;
            const float* qq = qn + kh * HD;
            const float* vh = vv + h * HD;
            float kv[HD], delta[HD], oh[HD];
            for (int j = 0; j < HD; j++) kv[j] = 0.0f;
            for (int i = 0; i < HD; i++)
                for (int j = 0; j < HD; j++) {
                    Sh[i * HD + j] *= decay;
                    kv[j] += Sh[i * HD + j] * kk[i];
                }
            for (int j = 0; j < HD; j++) delta[j] = (vh[j] - kv[j]) * beta;
            for (int j = 0; j < HD; j++) oh[j] = 0.0f;
            for (int i = 0; i < HD; i++)
                for (int j = 0; j < HD; j++) {
                    Sh[i * HD + j] += kk[i] * delta[j];
                    oh[j] += Sh[i * HD + j] * qq[i];
                }
            /* gated RMSNorm: rmsnorm(o_h / sqrt(128)) * ssm_norm * silu(z_h) (ref_model.cpp:245-252) */
            float* od = o + (size_t)t * VD + h * HD;
            for (int j = 0; j < HD; j++) oh[j] *= qscale;
            dn_rmsnorm(oh, ssm_norm, od, HD, eps);
            const float* zh = z + (size_t)t * VD + h * HD;
            for (int j = 0; j < HD; j++) od[j] *= dn_silu(zh[j]);
        }
    }
    free(conv);
    free(qn);
    free(kn);
}


/* ---- Weight formats (src/quant/quant_ref.cpp:24-33, 35-101, 281-299; ggml's block layouts) ---------------------
 * Every value is formed as in the reference's scalar code (float products and differences in the same order, no FMA
 * contraction), so that a fp16 rounding of it is the reference's prefill dequantizer output bit for bit. */
static float w_h(const uint8_t* p) { return qwo_fp16_to_fp32((uint16_t)(p[0] | (p[1] << 8))); }

size_t qwo_w_row_bytes(int fmt, int64_t K) {
    if (fmt == QWO_W_BF16) return (size_t)K * 2;
    if (K % 256) return 0;
    const int64_t nb = K / 256;
    switch (fmt) {
        case QWO_W_Q2_K: return (size_t)nb * 84;
        case QWO_W_Q4_K: return (size_t)nb * 144;
        case QWO_W_Q6_K: return (size_t)nb * 210;
        case QWO_W_IQ4_XS: return (size_t)nb * 136;
        case QWO_W_IQ2_XXS: return (size_t)nb * 66;
        case QWO_W_IQ2_XS: return (size_t)nb * 74;
        case QWO_W_IQ2_S: return (size_t)nb * 82;
        case QWO_W_IQ3_XXS: return (size_t)nb * 98;
        case QWO_W_IQ3_S: return (size_t)nb * 110;
        default: return 0;
    }
}

/* ---- i-quant grid formats (src/quant/quant_ref.cpp:105-222) -----------------------------------------------------
 * Codebooks from the level-index code words of iq_grids.inc (pinned against the reference's byte tables by their
 * SHA-256).  Sign bytes of IQ2_XXS / IQ2_XS / IQ3_XXS come from a 7-bit index whose 8th bit makes the count of
 * negative signs even (ksigns_iq2xs of ggml, src/quant/iq_tables.inc:8-17). */
#define IQ_TABLE static const
#include "iq_grids.inc"
#undef IQ_TABLE

static uint64_t iq_expand(const uint16_t* codes, const uint8_t* levels, int bits, int nbytes, int idx) {
    uint64_t e = 0;
    for (int j = 0; j < nbytes; j++) e |= (uint64_t)levels[(codes[idx] >> (bits * j)) & ((1 << bits) - 1)] << (8 * j);
    return e;
}

uint64_t qwo_iq_grid(int table, int idx) {
    switch (table) {
        case 0: return idx >= 0 && idx < IQ2XXS_N ? iq_expand(IQ2XXS_CODES, IQ2XXS_LEVELS, IQ2XXS_BITS, 8, idx) : 0;
        case 1: return idx >= 0 && idx < IQ2XS_N ? iq_expand(IQ2XS_CODES, IQ2XS_LEVELS, IQ2XS_BITS, 8, idx) : 0;
        case 2: return idx >= 0 && idx < IQ2S_N ? iq_expand(IQ2S_CODES, IQ2S_LEVELS, IQ2S_BITS, 8, idx) : 0;
        case 3: return idx >= 0 && idx < IQ3XXS_N ? iq_expand(IQ3XXS_CODES, IQ3XXS_LEVELS, IQ3XXS_BITS, 4, idx) : 0;
        case 4: return idx >= 0 && idx < IQ3S_N ? iq_expand(IQ3S_CODES, IQ3S_LEVELS, IQ3S_BITS, 4, idx) : 0;
        default: return 0;
    }
}

static uint8_t iq_signs7(unsigned s7) {
    s7 &= 127;
    return (uint8_t)(s7 | ((unsigned)(__builtin_popcount(s7) & 1) << 7));
}

static uint32_t w_u32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }

/* 8 weights = db * grid byte j * (sign bit j ? -1 : 1) */
static void iq_put8(float* y, float db, uint64_t grid, uint8_t signs) {
    for (int j = 0; j < 8; j++) y[j] = db * (float)((grid >> (8 * j)) & 255) * ((signs >> j) & 1 ? -1.f : 1.f);
}

static void w_dequant_iq(int fmt, const uint8_t* blk, float* out) {
    const float d = w_h(blk);
    if (fmt == QWO_W_IQ2_XXS) { /* d | per 32 weights: 4 grid indices (bytes), then 4 x 7 sign bits | 4-bit scale */
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t* q = blk + 2 + 8 * ib;
            const uint32_t a1 = w_u32(q + 4);
            const float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
            for (int l = 0; l < 4; l++) iq_put8(out + 32 * ib + 8 * l, db, qwo_iq_grid(0, q[l]), iq_signs7(a1 >> (7 * l)));
        }
    } else if (fmt == QWO_W_IQ2_XS) { /* d | qs[32] u16 (9-bit index | 7 sign bits) | scales[8]: two 4-bit per 32 */
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t sc = blk[66 + ib];
            const float db[2] = {d * (0.5f + (float)(sc & 15)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
            for (int l = 0; l < 4; l++) {
                const unsigned q = (unsigned)(blk[2 + 2 * (4 * ib + l)] | (blk[3 + 2 * (4 * ib + l)] << 8));
                iq_put8(out + 32 * ib + 8 * l, db[l / 2], qwo_iq_grid(1, (int)(q & 511)), iq_signs7(q >> 9));
            }
        }
    } else if (fmt == QWO_W_IQ2_S) { /* d | qs[32] index low bits | signs[32] | qh[8] (2 high bits each) | scales[8] */
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t sc = blk[74 + ib], qh = blk[66 + ib];
            const float db[2] = {d * (0.5f + (float)(sc & 15)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
            for (int l = 0; l < 4; l++) {
                const int idx = blk[2 + 4 * ib + l] | (((qh >> (2 * l)) & 3) << 8);
                iq_put8(out + 32 * ib + 8 * l, db[l / 2], qwo_iq_grid(2, idx), blk[34 + 4 * ib + l]);
            }
        }
    } else if (fmt == QWO_W_IQ3_XXS) { /* d | qs[64] grid indices | per 32 weights 4 x 7 sign bits | 4-bit scale */
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t* q = blk + 2 + 8 * ib;
            const uint32_t a = w_u32(blk + 66 + 4 * ib);
            const float db = d * (0.5f + (float)(a >> 28)) * 0.5f;
            for (int l = 0; l < 4; l++) {
                const uint64_t g = qwo_iq_grid(3, q[2 * l]) | (qwo_iq_grid(3, q[2 * l + 1]) << 32);
                iq_put8(out + 32 * ib + 8 * l, db, g, iq_signs7(a >> (7 * l)));
            }
        }
    } else { /* IQ3_S: d | qs[64] index low bytes | qh[8] (9th bits) | signs[32] | scales[4]: 4-bit per 32 */
        for (int ib = 0; ib < 8; ib++) {
            const uint8_t* q = blk + 2 + 8 * ib;
            const uint8_t qh = blk[66 + ib];
            const float db = d * (float)(1 + 2 * ((blk[106 + ib / 2] >> (4 * (ib & 1))) & 15));
            for (int l = 0; l < 4; l++) {
                const int i0 = q[2 * l] | (((qh >> (2 * l)) & 1) << 8), i1 = q[2 * l + 1] | (((qh >> (2 * l + 1)) & 1) << 8);
                const uint64_t g = qwo_iq_grid(4, i0) | (qwo_iq_grid(4, i1) << 32);
                iq_put8(out + 32 * ib + 8 * l, db, g, blk[74 + 4 * ib + l]);
            }
        }
    }
}

/* the 6-bit scale / min pair j of a Q4_K block (12 bytes pack 8 pairs) */
static void w_q4k_scale_min(const uint8_t* sc, int j, int* s, int* m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

static const int8_t w_iq4_levels[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

int qwo_w_dequant_row(int fmt, const uint8_t* row, float* y, int64_t K) {
    if (qwo_w_row_bytes(fmt, K) == 0) return -1;
    if (fmt == QWO_W_BF16) {
        for (int64_t k = 0; k < K; k++) {
            const uint32_t bits = (uint32_t)(row[2 * k] | (row[2 * k + 1] << 8)) << 16;
            memcpy(&y[k], &bits, 4);
        }
        return 0;
    }
    for (int64_t b = 0; b < K / 256; b++) {
        float* out = y + 256 * b;
        if (fmt == QWO_W_Q2_K) { /* scales[16] | qs[64] | d | dmin: 16 groups of 16, 2-bit codes */
            const uint8_t* blk = row + 84 * b;
            const uint8_t* sc = blk;
            const uint8_t* qs = blk + 16;
            const float d = w_h(blk + 80), dmin = w_h(blk + 82);
            for (int g = 0; g < 16; g++) {
                /* group g: weights 16 g .. 16 g + 15 = half (g & 1) of 32-byte column (g >> 3), bit pair (g >> 1) & 3 */
                const int half = g & 1, shift = 2 * ((g >> 1) & 3), col = g >> 3;
                const float dl = d * (float)(sc[g] & 15), ml = dmin * (float)(sc[g] >> 4);
                for (int l = 0; l < 16; l++) {
                    const int code = (qs[32 * col + 16 * half + l] >> shift) & 3;
                    out[16 * g + l] = dl * (float)code - ml;
                }
            }
        } else if (fmt == QWO_W_Q4_K) { /* d | dmin | scales[12] | qs[128]: 8 sub-blocks of 32, 4-bit codes */
            const uint8_t* blk = row + 144 * b;
            const float d = w_h(blk), dmin = w_h(blk + 2);
            const uint8_t* sc = blk + 4;
            const uint8_t* qs = blk + 16;
            for (int j = 0; j < 8; j++) {
                int s6, m6;
                w_q4k_scale_min(sc, j, &s6, &m6);
                const float dl = d * (float)s6, ml = dmin * (float)m6;
                /* sub-block j: bytes 32 (j >> 1) .. + 31, low nibbles for even j, high for odd */
                for (int l = 0; l < 32; l++) {
                    const uint8_t byte = qs[32 * (j >> 1) + l];
                    const int code = (j & 1) ? byte >> 4 : byte & 15;
                    out[32 * j + l] = dl * (float)code - ml;
                }
            }
        } else if (fmt == QWO_W_Q6_K) { /* ql[128] | qh[64] | scales[16] (int8) | d: 16 groups of 16, 6-bit codes */
            const uint8_t* blk = row + 210 * b;
            const uint8_t* ql = blk;
            const uint8_t* qh = blk + 128;
            const int8_t* sc = (const int8_t*)(blk + 192);
            const float d = w_h(blk + 208);
            for (int k = 0; k < 256; k++) {
                /* weight k: half h = k / 128, quarter r = (k % 128) / 32, lane l = k % 32 */
                const int h = k >> 7, r = (k >> 5) & 3, l = k & 31;
                const uint8_t lo = ql[64 * h + 32 * (r & 1) + l];
                const int low4 = (r & 2) ? lo >> 4 : lo & 15;
                const int high2 = (qh[32 * h + l] >> (2 * r)) & 3;
                const int code = (low4 | (high2 << 4)) - 32;
                out[k] = d * (float)sc[8 * h + 2 * r + l / 16] * (float)code;
            }
        } else if (fmt != QWO_W_IQ4_XS) {
            w_dequant_iq(fmt, row + qwo_w_row_bytes(fmt, 256) * b, out);
        } else { /* IQ4_XS: d | scales_h (u16) | scales_l[4] | qs[128]: 8 sub-blocks of 32, 4-bit level indices */
            const uint8_t* blk = row + 136 * b;
            const float d = w_h(blk);
            const unsigned sh = (unsigned)(blk[2] | (blk[3] << 8));
            const uint8_t* sl = blk + 4;
            const uint8_t* qs = blk + 8;
            for (int j = 0; j < 8; j++) {
                const int ls = ((sl[j / 2] >> (4 * (j % 2))) & 15) | (((sh >> (2 * j)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                for (int l = 0; l < 16; l++) {
                    const uint8_t byte = qs[16 * j + l];
                    out[32 * j + l] = dl * (float)w_iq4_levels[byte & 15];
                    out[32 * j + 16 + l] = dl * (float)w_iq4_levels[byte >> 4];
                }
            }
        }
    }
    return 0;
}

int qwo_gemv_ref(int fmt, const uint8_t* W, size_t row_bytes, int K, int N, const int8_t* q, const float* d, int nc,
                 double* y) {
    if (qwo_w_row_bytes(fmt, K) == 0) return -1;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(+ : bad)
    for (int r = 0; r < N; r++) {
        float* w = (float*)malloc((size_t)K * sizeof(float));
        if (!w) { bad++; continue; }
        qwo_w_dequant_row(fmt, W + (size_t)r * row_bytes, w, K);
        for (int c = 0; c < nc; c++) {
            double acc = 0.0;
            for (int k = 0; k < K; k++)
                acc += (double)w[k] * ((double)d[(size_t)c * (K / 32) + k / 32] * (double)q[(size_t)c * K + k]);
            y[(size_t)c * N + r] = acc;
        }
        free(w);
    }
    return bad ? -2 : 0;
}

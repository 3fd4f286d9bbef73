// Attention prep and quantize-on-append (gfx950).
//
// k_prep / k_prep_rows: one workgroup per (head, token): per-head RMSNorm * weight, NeoX RoPE on dims [0, 64) in
// pairs (i, i+32), gate split, and the append of the token's K (normed + roped) and V (raw) rows into the split
// KV layout.  Semantics of src/cuda/ops.cu:309-358 and src/cuda/prefill.cu:344-383; RoPE tables of
// src/cuda/prefill.cu:385-407; the row store follows src/cuda/common.cuh:199-228 (ggml quantizer values of
// src/quant/quant_ref.cpp:507-538, bit for bit).
#include "launch.hpp"
#include "qwattn_common.hpp"

namespace qwa {

// The quantizers must round exactly like the reference's scalar C++ (no FMA contraction anywhere here).
#pragma clang fp contract(off)

// Store one 256-value row: thread t (0..255) holds element t.  Each 32-lane half wave is one quant block.
__device__ __forceinline__ void store_row(uint8_t* vals, uint16_t* scales, int kvt, float v, int t) {
    const int lane = t & 31, blk = t >> 5;
    if (kvt == QWA_KV_F16) {
        reinterpret_cast<uint16_t*>(vals)[t] = f2h_bits(v);
    } else if (kvt == QWA_KV_Q8_0) {
        const float amax = half_max(fabsf(v));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const float r = roundf(v * id);  // half away from zero, like roundf in the reference
        vals[t] = (uint8_t)(int8_t)(int)r;
        if (lane == 0) scales[blk] = f2h_bits(d);
    } else {
        // Q4_0: d = max / -8 with max the signed value of the first element of largest magnitude
        float amax = fabsf(v), mx = v;
        int idx = lane;
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) {
            const float oa = __shfl_xor(amax, o, 32);
            const float om = __shfl_xor(mx, o, 32);
            const int oi = __shfl_xor(idx, o, 32);
            if (oa > amax || (oa == amax && oi < idx)) {
                amax = oa;
                mx = om;
                idx = oi;
            }
        }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const float x = v * id;
        const float y = x + 8.5f;
        int c = (int)(int8_t)(int)y;  // truncation, as the reference's (int8_t) cast
        c = c < 15 ? c : 15;
        const int nxt = __shfl_down(c, 1, 32);
        if ((t & 1) == 0) vals[t >> 1] = (uint8_t)((c & 15) | ((nxt & 15) << 4));
        if (lane == 0) scales[blk] = f2h_bits(d);
    }
}

__device__ __forceinline__ float src_at(const qwa_row_src& s, int r, int n, int i) {
    return i < s.split ? s.dev[(size_t)r * n + i] : s.host[(size_t)r * s.host_ld + (i - s.split)];
}

// block-wide sum over 256 threads (4 waves)
__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ void rope_cs(double pos, float theta, int i, float* c, float* s) {
    const double inv = pow((double)theta, -2.0 * i / NROT);
    // reduce the angle in double before rounding to float: positions reach 262144
    const double ang = fmod(pos * inv, 6.283185307179586476925286766559);
    double sn, cs;
    sincos(ang, &sn, &cs);
    *c = (float)cs;
    *s = (float)sn;
}

// common tail of prep: normalise, rotate, store q / append k,v
__device__ __forceinline__ void prep_head(float x, float vval, bool is_q, int head, const float* qn_w, const float* kn_w,
                                          float eps, const float* s_cos, const float* s_sin, float* sx, float* red,
                                          float* q_out, int kvt, const qwa_kv_layer& kv, int pos) {
    const int t = threadIdx.x;
    const float tot = block_sum256(x * x, red);
    x = x * rsqrtf(tot / (float)HD + eps) * (is_q ? qn_w[t] : kn_w[t]);
    sx[t] = x;
    __syncthreads();
    if (t < NROT / 2) {
        const float x0 = sx[t], x1 = sx[t + NROT / 2];
        sx[t] = x0 * s_cos[t] - x1 * s_sin[t];
        sx[t + NROT / 2] = x0 * s_sin[t] + x1 * s_cos[t];
    }
    __syncthreads();
    x = sx[t];
    if (is_q) {
        q_out[head * HD + t] = x;
    } else {
        const int vb = value_bytes(kvt);
        const size_t row = (size_t)head * kv.capacity + pos;
        store_row(kv.k + row * vb, kv.ks + row * 8, kvt, x, t);
        store_row(kv.v + row * vb, kv.vs + row * 8, kvt, vval, t);
    }
}

// grid (28, n): blockIdx.x < 24 -> query head, else KV head; blockIdx.y = token r at cache position pos0 + r and
// rotary position rpos0 + r.
__global__ void __launch_bounds__(256) k_prep(qwa_row_src qg, qwa_row_src ks, qwa_row_src vs, const float* qn_w,
                                              const float* kn_w, int pos0, int rpos0, float theta, float eps, int kvt,
                                              qwa_kv_layer kv, float* q_out, float* gate) {
    const int hb = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    __shared__ float sx[HD];
    __shared__ float red[4];
    __shared__ float s_cos[NROT / 2], s_sin[NROT / 2];
    if (t < NROT / 2) rope_cs((double)(rpos0 + r), theta, t, &s_cos[t], &s_sin[t]);
    const bool is_q = hb < NH;
    const int head = is_q ? hb : hb - NH;
    q_out += (size_t)r * NH * HD;
    gate += (size_t)r * NH * HD;
    float x, vval = 0.0f;
    if (is_q) {
        x = src_at(qg, r, 2 * NH * HD, head * 2 * HD + t);
        gate[head * HD + t] = src_at(qg, r, 2 * NH * HD, head * 2 * HD + HD + t);
    } else {
        x = src_at(ks, r, NKV * HD, head * HD + t);
        vval = src_at(vs, r, NKV * HD, head * HD + t);
    }
    prep_head(x, vval, is_q, head, qn_w, kn_w, eps, s_cos, s_sin, sx, red, q_out, kvt, kv, pos0 + r);
}

// prefill form: rope table [B][64] precomputed per chunk
__global__ void __launch_bounds__(256) k_prep_rows(const float* qg, const float* k, const float* v, const float* qn_w,
                                                   const float* kn_w, int p0, const float* rope, float eps, int kvt,
                                                   qwa_kv_layer kv, float* q_out, float* gate) {
    const int hb = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    __shared__ float sx[HD];
    __shared__ float red[4];
    __shared__ float s_cos[NROT / 2], s_sin[NROT / 2];
    if (t < NROT / 2) {
        s_cos[t] = rope[(size_t)r * NROT + t];
        s_sin[t] = rope[(size_t)r * NROT + NROT / 2 + t];
    }
    const bool is_q = hb < NH;
    const int head = is_q ? hb : hb - NH;
    q_out += (size_t)r * NH * HD;
    gate += (size_t)r * NH * HD;
    float x, vval = 0.0f;
    if (is_q) {
        const float* qrow = qg + (size_t)r * NH * 2 * HD;
        x = qrow[head * 2 * HD + t];
        gate[head * HD + t] = qrow[head * 2 * HD + HD + t];
    } else {
        x = k[(size_t)r * NKV * HD + head * HD + t];
        vval = v[(size_t)r * NKV * HD + head * HD + t];
    }
    prep_head(x, vval, is_q, head, qn_w, kn_w, eps, s_cos, s_sin, sx, red, q_out, kvt, kv, p0 + r);
}

__global__ void k_rope_table(int p0, float theta, float* rope) {
    const int t = blockIdx.x, i = threadIdx.x;
    float c, s;
    rope_cs((double)(p0 + t), theta, i, &c, &s);
    rope[(size_t)t * NROT + i] = c;
    rope[(size_t)t * NROT + NROT / 2 + i] = s;
}

// M-RoPE: frequency i turns with component i % 3 of the token's (t, h, w) position
__global__ void k_rope_table_pos(const int* pos3, float theta, float* rope) {
    const int t = blockIdx.x, i = threadIdx.x;
    float c, s;
    rope_cs((double)pos3[t * 3 + i % 3], theta, i, &c, &s);
    rope[(size_t)t * NROT + i] = c;
    rope[(size_t)t * NROT + NROT / 2 + i] = s;
}

// raw append: grid (8, n): blockIdx.x = 2 * head + (0: K, 1: V)
__global__ void __launch_bounds__(256) k_kv_append(const float* xk, const float* xv, int pos0, int kvt,
                                                   qwa_kv_layer kv) {
    const int head = blockIdx.x >> 1, is_v = blockIdx.x & 1, r = blockIdx.y, t = threadIdx.x;
    const float* src = is_v ? xv : xk;
    if (src == nullptr) return;  // uniform over the workgroup
    const float x = src[((size_t)r * NKV + head) * HD + t];
    const int vb = value_bytes(kvt);
    const size_t row = (size_t)head * kv.capacity + pos0 + r;
    if (is_v) store_row(kv.v + row * vb, kv.vs + row * 8, kvt, x, t);
    else store_row(kv.k + row * vb, kv.ks + row * 8, kvt, x, t);
}

// grid.y is limited to 65535: long token ranges go in slices
constexpr int MAX_GRID_Y = 32768;

static qwa_row_src advance(qwa_row_src s, int rows, int n) {
    if (s.dev) s.dev += (size_t)rows * n;
    if (s.host) s.host += (size_t)rows * s.host_ld;
    return s;
}

hipError_t launch_prep(const qwa_row_src& qg, const qwa_row_src& k, const qwa_row_src& v, const float* qn,
                       const float* kn, int pos0, int rpos0, int n, float theta, float eps, int kvt,
                       const qwa_kv_layer& kv, float* q_out, float* gate, hipStream_t st) {
    for (int r0 = 0; r0 < n; r0 += MAX_GRID_Y) {
        const int nr = min(MAX_GRID_Y, n - r0);
        hipLaunchKernelGGL(k_prep, dim3(NH + NKV, nr), dim3(256), 0, st, advance(qg, r0, 2 * NH * HD),
                           advance(k, r0, NKV * HD), advance(v, r0, NKV * HD), qn, kn, pos0 + r0, rpos0 + r0, theta,
                           eps, kvt, kv, q_out + (size_t)r0 * NH * HD, gate + (size_t)r0 * NH * HD);
    }
    return hipGetLastError();
}

hipError_t launch_prep_rows(const float* qg, const float* k, const float* v, const float* qn, const float* kn, int B,
                            int p0, const float* rope, float eps, int kvt, const qwa_kv_layer& kv, float* q,
                            float* gate, hipStream_t st) {
    for (int r0 = 0; r0 < B; r0 += MAX_GRID_Y) {
        const int nr = min(MAX_GRID_Y, B - r0);
        hipLaunchKernelGGL(k_prep_rows, dim3(NH + NKV, nr), dim3(256), 0, st, qg + (size_t)r0 * 2 * NH * HD,
                           k + (size_t)r0 * NKV * HD, v + (size_t)r0 * NKV * HD, qn, kn, p0 + r0,
                           rope + (size_t)r0 * NROT, eps, kvt, kv, q + (size_t)r0 * NH * HD,
                           gate + (size_t)r0 * NH * HD);
    }
    return hipGetLastError();
}

hipError_t launch_rope_table(int p0, int B, float theta, float* rope, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_table, dim3(B), dim3(NROT / 2), 0, st, p0, theta, rope);  // grid.x: no slicing
    return hipGetLastError();
}

hipError_t launch_rope_table_pos(const int* pos3, int B, float theta, float* rope, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_table_pos, dim3(B), dim3(NROT / 2), 0, st, pos3, theta, rope);
    return hipGetLastError();
}

hipError_t launch_kv_append(const float* xk, const float* xv, int pos0, int n, int kvt, const qwa_kv_layer& kv,
                            hipStream_t st) {
    for (int r0 = 0; r0 < n; r0 += MAX_GRID_Y) {
        const int nr = min(MAX_GRID_Y, n - r0);
        const size_t off = (size_t)r0 * NKV * HD;
        hipLaunchKernelGGL(k_kv_append, dim3(2 * NKV, nr), dim3(256), 0, st, xk ? xk + off : nullptr,
                           xv ? xv + off : nullptr, pos0 + r0, kvt, kv);
    }
    return hipGetLastError();
}

}  // namespace qwa

// FP32 vector-ALU attention kernels kept for tests (the reference keeps the same pair: attn_decode_simple,
// src/cuda/ops.cu:360-505, and attn_prefill_simple, src/cuda/prefill.cu:409-519).  One workgroup per
// (query, head): keys in chunks of 256 (thread = key) for the scores, online softmax in fp32 with expf, then
// thread = head dim for P.V.  Dequantized values are exact fp32 products d * x.
#include <float.h>

#include "launch.hpp"
#include "qwattn_common.hpp"

namespace qwa {

__device__ __forceinline__ float deq(const uint8_t* row, const uint16_t* sc, int kvt, int d) {
    if (kvt == QWA_KV_F16) return h2f_bits(reinterpret_cast<const uint16_t*>(row)[d]);
    const float s = h2f_bits(sc[d >> 5]);
    if (kvt == QWA_KV_Q8_0) return s * (float)(int8_t)row[d];
    return s * (float)((int)((row[d >> 1] >> (4 * (d & 1))) & 15) - 8);
}

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return is_max ? fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) : (red[0] + red[1]) + (red[2] + red[3]);
}

// returns the normalised attention output for head dim threadIdx.x (before the gate)
__device__ float simple_attend(const float* qrow, const qwa_kv_layer& kv, int kvt, int g, int npos) {
    __shared__ float sq[HD];
    __shared__ float sp[256];
    __shared__ float red[4];
    const int t = threadIdx.x;
    const int vb = value_bytes(kvt);
    sq[t] = qrow[t] * 0.0625f;
    __syncthreads();
    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    const size_t rowbase = (size_t)g * kv.capacity;
    for (int c0 = 0; c0 < npos; c0 += 256) {
        const int np = min(256, npos - c0);
        float s = -INFINITY;
        if (t < np) {
            const size_t row = rowbase + c0 + t;
            const uint8_t* kr = kv.k + row * vb;
            const uint16_t* ks = kv.ks ? kv.ks + row * 8 : nullptr;
            float a = 0.0f;
            for (int d = 0; d < HD; d++) a += sq[d] * deq(kr, ks, kvt, d);
            s = a;
        }
        const float mx = block_reduce(s, red, true);
        const float mn = fmaxf(m, mx);
        const float e = t < np ? expf(s - mn) : 0.0f;
        const float corr = expf(m - mn);
        sp[t] = e;
        const float sum = block_reduce(e, red, false);
        l = l * corr + sum;
        m = mn;
        acc *= corr;
        for (int j = 0; j < np; j++) {
            const size_t row = rowbase + c0 + j;
            acc += sp[j] * deq(kv.v + row * vb, kv.vs ? kv.vs + row * 8 : nullptr, kvt, t);
        }
        __syncthreads();
    }
    return acc / l;
}

__global__ void __launch_bounds__(256) k_dec_simple(const float* q, const float* gate, qwa_kv_layer kv, int kvt,
                                                    int n_pos, float* out, qwa_act_q8 oq, int do_q) {
    const int h = blockIdx.x, t = threadIdx.x;
    const float a = simple_attend(q + (size_t)h * HD, kv, kvt, h / GRP, n_pos);
    const size_t o = (size_t)h * HD + t;
    const float v = a * (1.0f / (1.0f + expf(-gate[o])));
    out[o] = v;
    if (do_q) {
        const float amax = half_max(fabsf(v));
        const float db = amax / 127.0f;
        const int qi = db > 0.0f ? (int)__builtin_rintf(v / db) : 0;
        oq.q[o] = (int8_t)qi;
        const float sum = half_sum((float)qi);
        if ((t & 31) == 0) {
            oq.d[o >> 5] = db;
            oq.s[o >> 5] = db * sum;
        }
    }
}

__global__ void __launch_bounds__(256) k_prefill_simple(const float* q, const float* gate, qwa_kv_layer kv, int kvt,
                                                        int p0, uint16_t* out16) {
    const int h = blockIdx.x, tok = blockIdx.y, t = threadIdx.x;
    const size_t o = ((size_t)tok * NH + h) * HD + t;
    const float a = simple_attend(q + ((size_t)tok * NH + h) * HD, kv, kvt, h / GRP, p0 + tok + 1);
    out16[o] = f2h_bits(a * (1.0f / (1.0f + expf(-gate[o]))));
}

hipError_t launch_decode_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int n_pos,
                                float* out, const qwa_act_q8* oq, hipStream_t st) {
    const qwa_act_q8 a = oq ? *oq : qwa_act_q8{nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_dec_simple, dim3(NH), dim3(256), 0, st, q, gate, kv, kvt, n_pos, out, a, oq ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_prefill_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                                 uint16_t* out16, hipStream_t st) {
    for (int r0 = 0; r0 < B; r0 += 32768) {
        const size_t off = (size_t)r0 * NH * HD;
        hipLaunchKernelGGL(k_prefill_simple, dim3(NH, min(32768, B - r0)), dim3(256), 0, st, q + off, gate + off, kv,
                           kvt, p0 + r0, out16 + off);
    }
    return hipGetLastError();
}

}  // namespace qwa

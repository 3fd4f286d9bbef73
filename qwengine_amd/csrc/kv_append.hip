// Attention prep and quantize-on-append (gfx950).
//
// Work unit: one wave64 per (token, head slot).  A slot covers 512 floats as two 32-lane halves of 8 consecutive
// values per lane:
//   slot s < 24   query head s:  half 0 = the q half of the head's 512-float qg span (RMSNorm * weight, RoPE),
//                                 half 1 = the gate half (copied);
//   slot 24 + h   KV head h:     half 0 = the K row (RMSNorm * weight, RoPE, quantized into the cache),
//                                 half 1 = the V row (quantized as it comes).
// A 32-value quant block is 4 neighbouring lanes, so every block reduction is two xor steps inside the half, the
// RoPE pair (i, i + 32) is lanes l and l + 4 of half 0, and each lane writes its share of the row as one store
// (16 B of F16, 8 B of Q8_0, 4 B of Q4_0 codes; one lane writes the row's 8 fp16 scales as one 16-byte store).
// Four waves share a workgroup and no LDS or barrier, so the tokens' 28 slots spread over 7 workgroups each.
//
// Semantics: attention prep of src/cuda/ops.cu:309-358 (q / k RMSNorm, NeoX RoPE with double angles reduced mod 2 pi)
// and src/cuda/prefill.cu:344-383 (table form; tables of :385-407); the stored bytes are the KV split layout of
// src/cuda/common.cuh:54-80 with the ggml quantizer values of src/quant/quant_ref.cpp:507-538, bit for bit.
#include <math.h>

#include "launch.hpp"
#include "qwattn_common.hpp"

namespace qwa {

// The quantizers must round exactly like the reference's scalar C++ (no FMA contraction anywhere here).
#pragma clang fp contract(off)

constexpr int SLOTS = NH + NKV;  // head slots per token
constexpr int VPL = 8;           // values per lane

__device__ __forceinline__ bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// x[0..7] = elements [i, i + 8) of row r of a split row source (device prefix, mapped-host tail)
__device__ __forceinline__ void fetch8(const qwa_row_src& s, int r, int n, int i, float* x) {
    const float* d = s.dev + (size_t)r * n + i;
    if (i + VPL <= s.split && al16(s.dev) && (n & 3) == 0) {
        const float4 a = reinterpret_cast<const float4*>(d)[0], b = reinterpret_cast<const float4*>(d)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++)
            x[j] = i + j < s.split ? d[j] : s.host[(size_t)r * s.host_ld + (i + j - s.split)];
    }
}

__device__ __forceinline__ void load8(const float* p, float* x) {
    if (al16(p)) {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) x[j] = p[j];
    }
}

__device__ __forceinline__ void put8(float* p, const float* x) {
    if (al16(p)) {
        reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
    } else {
#pragma unroll
        for (int j = 0; j < VPL; j++) p[j] = x[j];
    }
}

// reductions over the 4 lanes of one quant block / the 32 lanes of one half
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 1, 64));
    return fmaxf(v, __shfl_xor(v, 2, 64));
}

// Quantize the 256-value row held by one half (lane l of the half owns elements 8l..8l+7) into the split layout.
__device__ __forceinline__ void quant_row(uint8_t* vals, uint16_t* scales, int kvt, const float* x, int l) {
    if (kvt == QWA_KV_F16) {
        uint32_t w[4];
#pragma unroll
        for (int m = 0; m < 4; m++) w[m] = (uint32_t)f2h_bits(x[2 * m]) | ((uint32_t)f2h_bits(x[2 * m + 1]) << 16);
        uint8_t* p = vals + 16 * l;
        if (al16(vals)) {
            *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            uint16_t* p16 = reinterpret_cast<uint16_t*>(p);
#pragma unroll
            for (int m = 0; m < 4; m++) {
                p16[2 * m] = (uint16_t)w[m];
                p16[2 * m + 1] = (uint16_t)(w[m] >> 16);
            }
        }
        return;
    }
    float d;
    if (kvt == QWA_KV_Q8_0) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < VPL; j++) a = fmaxf(a, fabsf(x[j]));
        const float amax = quad_max(a);
        d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t w[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            const int c = (int)roundf(x[j] * id);  // half away from zero
            w[j >> 2] |= ((uint32_t)c & 0xFFu) << (8 * (j & 3));
        }
        uint8_t* p = vals + 8 * l;
        if (((uintptr_t)vals & 7) == 0) {
            *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
        } else {
#pragma unroll
            for (int j = 0; j < VPL; j++) p[j] = (uint8_t)(w[j >> 2] >> (8 * (j & 3)));
        }
    } else {
        // Q4_0: the scale is max / -8 where max is the signed value of the block's first element of largest
        // magnitude.  Lane-local candidate first (ascending scan, strict >), then the 4 lanes' candidates with the
        // lower element index winning ties.
        float am = fabsf(x[0]), mx = x[0];
        int ix = 0;
#pragma unroll
        for (int j = 1; j < VPL; j++)
            if (fabsf(x[j]) > am) am = fabsf(x[j]), mx = x[j], ix = j;
        ix += VPL * (l & 3);
#pragma unroll
        for (int o = 1; o <= 2; o <<= 1) {
            const float oa = __shfl_xor(am, o, 64), om = __shfl_xor(mx, o, 64);
            const int oi = __shfl_xor(ix, o, 64);
            const bool take = oa > am || (oa == am && oi < ix);
            am = take ? oa : am;
            mx = take ? om : mx;
            ix = take ? oi : ix;
        }
        d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t w = 0u;
#pragma unroll
        for (int j = 0; j < VPL; j++) {
            int c = (int)(x[j] * id + 8.5f);  // truncation toward zero of a value in [0.5, 16.5]
            c = c < 15 ? c : 15;
            w |= (uint32_t)(c & 15) << (4 * j);  // element 2m -> low nibble of byte m, 2m + 1 -> high nibble
        }
        uint8_t* p = vals + 4 * l;
        if (((uintptr_t)vals & 3) == 0) {
            *reinterpret_cast<uint32_t*>(p) = w;
        } else {
#pragma unroll
            for (int m = 0; m < 4; m++) p[m] = (uint8_t)(w >> (8 * m));
        }
    }
    // the row's 8 block scales: lane 4b of the half holds block b's; lane 0 of the half gathers and stores them
    const uint32_t sb = f2h_bits(d);
    const int base = (int)(threadIdx.x & 32);
    uint32_t sw[4];
#pragma unroll
    for (int m = 0; m < 4; m++)
        sw[m] = (uint32_t)__shfl((int)sb, base + 8 * m, 64) | ((uint32_t)__shfl((int)sb, base + 8 * m + 4, 64) << 16);
    if (l == 0) {
        if (al16(scales)) {
            *reinterpret_cast<uint4*>(scales) = make_uint4(sw[0], sw[1], sw[2], sw[3]);
        } else {
#pragma unroll
            for (int m = 0; m < 4; m++) {
                scales[2 * m] = (uint16_t)sw[m];
                scales[2 * m + 1] = (uint16_t)(sw[m] >> 16);
            }
        }
    }
}

// cos / sin of rotary frequency i at position pos: theta^(-2i/64) * pos in double, reduced mod 2 pi before the
// float rounding (positions reach 262144)
__device__ __forceinline__ void rope_cs(double pos, float theta, int i, float* c, float* s) {
    const double ang = fmod(pos * pow((double)theta, -2.0 * i / NROT), 2.0 * M_PI);
    double sn, cs;
    sincos(ang, &sn, &cs);
    *c = (float)cs;
    *s = (float)sn;
}

// per-head RMSNorm over half 0's 256 values (all lanes return; only half 0's result is used)
__device__ __forceinline__ void rms_norm_half(float* x, const float* w, int l, float eps) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < VPL; j++) ss += x[j] * x[j];
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) ss += __shfl_xor(ss, o, 64);
    const float r = rsqrtf(ss / (float)HD + eps);
    float wv[VPL];
    load8(w + VPL * l, wv);
#pragma unroll
    for (int j = 0; j < VPL; j++) x[j] = x[j] * r * wv[j];
}

// NeoX rotation of dims [0, 64) in pairs (i, i + 32): lanes 0-3 hold the first members, lanes 4-7 the second.
// c[j], s[j] belong to frequency 8 (l & 3) + j.
__device__ __forceinline__ void rope_half(float* x, const float* c, const float* s, int l) {
    float y[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) y[j] = __shfl_xor(x[j], 4, 64);
    if (l < 4) {
#pragma unroll
        for (int j = 0; j < VPL; j++) x[j] = x[j] * c[j] - y[j] * s[j];
    } else if (l < 8) {
#pragma unroll
        for (int j = 0; j < VPL; j++) x[j] = y[j] * s[j] + x[j] * c[j];
    }
}

struct Slot {
    int r, s, l, half;
};
__device__ __forceinline__ Slot slot_of() {
    Slot o;
    const int task = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
    o.r = task / SLOTS;
    o.s = task - o.r * SLOTS;
    o.half = (threadIdx.x >> 5) & 1;
    o.l = threadIdx.x & 31;
    return o;
}

// the work of one slot once its 8 values per lane and the rotation's cos / sin are in registers
__device__ __forceinline__ void finish_slot(const Slot& t, float* x, const float* c, const float* sn, const float* qn_w,
                                            const float* kn_w, float eps, int kvt, const qwa_kv_layer& kv, int pos,
                                            float* q_out, float* gate) {
    const bool is_q = t.s < NH;
    float xn[VPL];
#pragma unroll
    for (int j = 0; j < VPL; j++) xn[j] = x[j];
    rms_norm_half(xn, is_q ? qn_w : kn_w, t.l, eps);
    rope_half(xn, c, sn, t.l);
    if (t.half == 0) {
#pragma unroll
        for (int j = 0; j < VPL; j++) x[j] = xn[j];
    }
    if (is_q) {
        float* dst = (t.half ? gate : q_out) + ((size_t)t.r * NH + t.s) * HD + VPL * t.l;
        put8(dst, x);
    } else {
        const int h = t.s - NH, vb = value_bytes(kvt);
        const size_t row = (size_t)h * kv.capacity + pos;
        uint8_t* vals = (t.half ? kv.v : kv.k) + row * vb;
        uint16_t* sc = t.half ? (kv.vs ? kv.vs + row * 8 : nullptr) : (kv.ks ? kv.ks + row * 8 : nullptr);
        quant_row(vals, sc, kvt, x, t.l);
    }
}

// decode form: tokens r = 0..n-1 at cache position pos0 + r and rotary position rpos0 + r
__global__ void __launch_bounds__(256) k_prep(qwa_row_src qg, qwa_row_src ks, qwa_row_src vs, const float* qn_w,
                                              const float* kn_w, int n, int pos0, int rpos0, float theta, float eps,
                                              int kvt, qwa_kv_layer kv, float* q_out, float* gate) {
    const Slot t = slot_of();
    if (t.r >= n) return;  // wave-uniform
    float x[VPL];
    if (t.s < NH) fetch8(qg, t.r, 2 * NH * HD, t.s * 2 * HD + t.half * HD + VPL * t.l, x);
    else fetch8(t.half ? vs : ks, t.r, NKV * HD, (t.s - NH) * HD + VPL * t.l, x);
    float c[VPL] = {}, sn[VPL] = {};
    if (t.half == 0 && t.l < 8) {
#pragma unroll
        for (int j = 0; j < VPL; j++) rope_cs((double)(rpos0 + t.r), theta, VPL * (t.l & 3) + j, &c[j], &sn[j]);
    }
    finish_slot(t, x, c, sn, qn_w, kn_w, eps, kvt, kv, pos0 + t.r, q_out, gate);
}

// prefill form: cos / sin from a per-chunk table rope [B][64] (cos of the 32 frequencies, then sin)
__global__ void __launch_bounds__(256) k_prep_rows(const float* qg, const float* k, const float* v, const float* qn_w,
                                                   const float* kn_w, int B, int p0, const float* rope, float eps,
                                                   int kvt, qwa_kv_layer kv, float* q_out, float* gate) {
    const Slot t = slot_of();
    if (t.r >= B) return;
    float x[VPL];
    if (t.s < NH) load8(qg + ((size_t)t.r * NH + t.s) * 2 * HD + t.half * HD + VPL * t.l, x);
    else load8((t.half ? v : k) + ((size_t)t.r * NKV + (t.s - NH)) * HD + VPL * t.l, x);
    float c[VPL] = {}, sn[VPL] = {};
    if (t.half == 0 && t.l < 8) {
        const float* rr = rope + (size_t)t.r * NROT + VPL * (t.l & 3);
        load8(rr, c);
        load8(rr + NROT / 2, sn);
    }
    finish_slot(t, x, c, sn, qn_w, kn_w, eps, kvt, kv, p0 + t.r, q_out, gate);
}

// one thread per (token, frequency); pos3 != nullptr selects M-RoPE, where frequency i turns with component i % 3
// of the token's (t, h, w) position
__global__ void __launch_bounds__(256) k_rope_table(int B, int p0, const int* pos3, float theta, float* rope) {
    const int g = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (g >= B * (NROT / 2)) return;
    const int t = g / (NROT / 2), i = g % (NROT / 2);
    const double pos = pos3 ? (double)pos3[3 * t + i % 3] : (double)(p0 + t);
    float c, s;
    rope_cs(pos, theta, i, &c, &s);
    rope[(size_t)t * NROT + i] = c;
    rope[(size_t)t * NROT + NROT / 2 + i] = s;
}

// raw append: one wave per (token, KV head), K in half 0 and V in half 1; a null source leaves its rows alone
__global__ void __launch_bounds__(256) k_kv_append(const float* xk, const float* xv, int n, int pos0, int kvt,
                                                   qwa_kv_layer kv) {
    const int task = (int)(blockIdx.x * 4 + (threadIdx.x >> 6));
    const int r = task / NKV, h = task % NKV, half = (threadIdx.x >> 5) & 1, l = threadIdx.x & 31;
    const float* src = half ? xv : xk;
    if (r >= n || src == nullptr) return;  // uniform over the half, which is all the block reductions span
    float x[VPL];
    load8(src + ((size_t)r * NKV + h) * HD + VPL * l, x);
    const size_t row = (size_t)h * kv.capacity + pos0 + r;
    const int vb = value_bytes(kvt);
    uint8_t* vals = (half ? kv.v : kv.k) + row * vb;
    uint16_t* sc = half ? (kv.vs ? kv.vs + row * 8 : nullptr) : (kv.ks ? kv.ks + row * 8 : nullptr);
    quant_row(vals, sc, kvt, x, l);
}

static unsigned blocks_for(long long waves) { return (unsigned)((waves + 3) / 4); }

hipError_t launch_prep(const qwa_row_src& qg, const qwa_row_src& k, const qwa_row_src& v, const float* qn,
                       const float* kn, int pos0, int rpos0, int n, float theta, float eps, int kvt,
                       const qwa_kv_layer& kv, float* q_out, float* gate, hipStream_t st) {
    hipLaunchKernelGGL(k_prep, dim3(blocks_for((long long)n * SLOTS)), dim3(256), 0, st, qg, k, v, qn, kn, n, pos0,
                       rpos0, theta, eps, kvt, kv, q_out, gate);
    return hipGetLastError();
}

hipError_t launch_prep_rows(const float* qg, const float* k, const float* v, const float* qn, const float* kn, int B,
                            int p0, const float* rope, float eps, int kvt, const qwa_kv_layer& kv, float* q,
                            float* gate, hipStream_t st) {
    hipLaunchKernelGGL(k_prep_rows, dim3(blocks_for((long long)B * SLOTS)), dim3(256), 0, st, qg, k, v, qn, kn, B, p0,
                       rope, eps, kvt, kv, q, gate);
    return hipGetLastError();
}

hipError_t launch_rope_table(int p0, int B, float theta, float* rope, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_table, dim3((B * (NROT / 2) + 255) / 256), dim3(256), 0, st, B, p0, nullptr, theta,
                       rope);
    return hipGetLastError();
}

hipError_t launch_rope_table_pos(const int* pos3, int B, float theta, float* rope, hipStream_t st) {
    hipLaunchKernelGGL(k_rope_table, dim3((B * (NROT / 2) + 255) / 256), dim3(256), 0, st, B, 0, pos3, theta, rope);
    return hipGetLastError();
}

hipError_t launch_kv_append(const float* xk, const float* xv, int pos0, int n, int kvt, const qwa_kv_layer& kv,
                            hipStream_t st) {
    hipLaunchKernelGGL(k_kv_append, dim3(blocks_for((long long)n * NKV)), dim3(256), 0, st, xk, xv, n, pos0, kvt, kv);
    return hipGetLastError();
}

}  // namespace qwa

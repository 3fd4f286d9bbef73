// Quantized KV bytes -> fp16 MFMA operands (gfx950, v_mfma_f32_16x16x32_f16).
//
// Operand conventions used by the decode and prefill kernels (lane l: column/row index l % 16, k-group l / 16):
//  * K operand (A of S^T = K Q^T): a lane holds 8 head dims of one key.  For k-step s (32 dims per MFMA) lane
//    group g holds the dims 64g + 8s + perm(j), j = 0..7, where perm is the identity for F16 / Q8_0 and
//    [0,4,1,5,2,6,3,7] for Q4_0 (the order in which a packed Q4_0 word unpacks).  Q, the B operand, is loaded in
//    the same dim order, so the contraction is unchanged.
//  * V operand (A of O^T = V^T P^T): a lane holds one head dim of 8 keys; keys come in pairs (a, b) packed as
//    half2 {V_a[d], V_b[d]}.
// All conversions are exact up to one fp16 rounding of d * x, the value the reference's GPU kernels use.
#pragma once

#include "qwattn_common.hpp"

namespace qwa {

template <int KVT> struct KRaw;  // 64 dims of one key row (a lane group's quarter of the row) + block scales
template <> struct KRaw<QWA_KV_Q4_0> { uint32_t w[8]; uint32_t sc; };
template <> struct KRaw<QWA_KV_Q8_0> { uint32_t w[16]; uint32_t sc; };
template <> struct KRaw<QWA_KV_F16> { uint32_t w[32]; uint32_t sc; };

template <int KVT> struct VRaw;  // 16 dims of one value row + its block scale
template <> struct VRaw<QWA_KV_Q4_0> { uint32_t w[2]; uint32_t sc; };
template <> struct VRaw<QWA_KV_Q8_0> { uint32_t w[4]; uint32_t sc; };
template <> struct VRaw<QWA_KV_F16> { uint32_t w[8]; uint32_t sc; };

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld8(const uint8_t* p) { return *reinterpret_cast<const uint2*>(p); }

// Load dims [64 g, 64 g + 64) of key row `row` (g = lane group).  Dead keys (beyond the window) read as zeros.
template <int KVT>
__device__ __forceinline__ void load_k(KRaw<KVT>& r, const qwa_kv_layer& kv, size_t row, int g, bool live) {
    constexpr int VB = value_bytes(KVT);
    constexpr int NW = sizeof(r.w) / 4;
    if (live) {
        const uint8_t* p = kv.k + row * VB + (VB / 4) * g;
#pragma unroll
        for (int i = 0; i < NW / 4; i++) {
            const uint4 u = ld16(p + 16 * i);
            r.w[4 * i] = u.x; r.w[4 * i + 1] = u.y; r.w[4 * i + 2] = u.z; r.w[4 * i + 3] = u.w;
        }
        if (KVT != QWA_KV_F16) r.sc = reinterpret_cast<const uint32_t*>(kv.ks + row * 8)[g];
        else r.sc = 0;
    } else {
#pragma unroll
        for (int i = 0; i < NW; i++) r.w[i] = 0;
        r.sc = 0;
    }
}

// Load dims [16 c, 16 c + 16) of value row `row`.
template <int KVT>
__device__ __forceinline__ void load_v(VRaw<KVT>& r, const qwa_kv_layer& kv, size_t row, int c, bool live) {
    constexpr int VB = value_bytes(KVT);
    if (live) {
        const uint8_t* p = kv.v + row * VB + (VB / 16) * c;
        if constexpr (KVT == QWA_KV_Q4_0) {
            const uint2 u = ld8(p);
            r.w[0] = u.x; r.w[1] = u.y;
        } else if constexpr (KVT == QWA_KV_Q8_0) {
            const uint4 u = ld16(p);
            r.w[0] = u.x; r.w[1] = u.y; r.w[2] = u.z; r.w[3] = u.w;
        } else {
            const uint4 u0 = ld16(p), u1 = ld16(p + 16);
            r.w[0] = u0.x; r.w[1] = u0.y; r.w[2] = u0.z; r.w[3] = u0.w;
            r.w[4] = u1.x; r.w[5] = u1.y; r.w[6] = u1.z; r.w[7] = u1.w;
        }
        if (KVT != QWA_KV_F16) r.sc = kv.vs[row * 8 + (c >> 1)];
        else r.sc = 0;
    } else {
#pragma unroll
        for (int i = 0; i < (int)(sizeof(r.w) / 4); i++) r.w[i] = 0;
        r.sc = 0;
    }
}

// K operand for k-step s (0..7): 8 dims 64g + 8s + perm(j) as fp16.
template <int KVT>
__device__ __forceinline__ h8 k_operand(const KRaw<KVT>& r, int s) {
    if constexpr (KVT == QWA_KV_F16) {
        return make_h8(r.w[4 * s], r.w[4 * s + 1], r.w[4 * s + 2], r.w[4 * s + 3]);
    } else {
        const uint16_t sb = (uint16_t)(r.sc >> (16 * (s >> 2)));
        const h2 d = scale_pair(sb, sb);
        uint32_t o[4];
        if constexpr (KVT == QWA_KV_Q4_0) {
            q4_word_to_h8(r.w[s], d, o);
        } else {
            q8_word_to_h4(r.w[2 * s], d, o);
            q8_word_to_h4(r.w[2 * s + 1], d, o + 2);
        }
        return make_h8(o[0], o[1], o[2], o[3]);
    }
}

// Exact small integers as fp16 (no scale): the codes c - 8 of a Q4_0 word in the k_operand order, or the int8
// values of a Q8_0 word.
// (the low nibbles of the 4 bytes go to bytes {0, 2} / {1, 3} of two perm results: {e0,e4}, {e2,e6}; the high
// nibbles likewise give {e1,e5}, {e3,e7})
__device__ __forceinline__ void q4_word_int(uint32_t w, uint32_t* out) {
    const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    out[0] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04020400u)) - bias);  // e0, e4
    out[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04020400u)) - bias);  // e1, e5
    out[2] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030401u)) - bias);  // e2, e6
    out[3] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030401u)) - bias);  // e3, e7
}
__device__ __forceinline__ void q8_word_int(uint32_t w, uint32_t* out) {
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t u = w ^ 0x80808080u;
    out[0] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05010400u)) - bias);
    out[1] = h2_bits(bits_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x05030402u)) - bias);
}

// Position of dim j inside the 8-dim group a K operand lane holds (see k_operand).
template <int KVT>
__device__ __forceinline__ constexpr int k_perm(int j) {
    return KVT == QWA_KV_Q4_0 ? ((j & 1) ? 4 + (j >> 1) : (j >> 1)) : j;
}

// V pair (keys a, b): NW raw words of each key's row piece (Q4_0: 8 dims / word, Q8_0: 4, F16: 2) ->
// out[d] = half2 {V_a[d], V_b[d]} for every dim d of the piece (sa, sb: the two keys' fp16 block scales).
template <int KVT, int NW>
__device__ __forceinline__ void v_pair_words(const uint32_t* aw, const uint32_t* bw, uint32_t sa, uint32_t sb,
                                             uint32_t* out) {
    if constexpr (KVT == QWA_KV_F16) {
#pragma unroll
        for (int i = 0; i < NW; i++) {
            out[2 * i] = __builtin_amdgcn_perm(bw[i], aw[i], 0x05040100u);      // {a lo, b lo}
            out[2 * i + 1] = __builtin_amdgcn_perm(bw[i], aw[i], 0x07060302u);  // {a hi, b hi}
        }
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const h2 d = scale_pair((uint16_t)sa, (uint16_t)sb);
        const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const uint32_t xa = aw[i] ^ 0x80808080u, xb = bw[i] ^ 0x80808080u;
            const uint32_t y0 = __builtin_amdgcn_perm(xb, xa, 0x05010400u);  // bytes {a0, b0, a1, b1}
            const uint32_t y1 = __builtin_amdgcn_perm(xb, xa, 0x07030602u);  // bytes {a2, b2, a3, b3}
            const uint32_t w0 = __builtin_amdgcn_perm(0x64646464u, y0, 0x04010400u);
            const uint32_t w1 = __builtin_amdgcn_perm(0x64646464u, y0, 0x04030402u);
            const uint32_t w2 = __builtin_amdgcn_perm(0x64646464u, y1, 0x04010400u);
            const uint32_t w3 = __builtin_amdgcn_perm(0x64646464u, y1, 0x04030402u);
            out[4 * i] = h2_bits((bits_h2(w0) - bias) * d);
            out[4 * i + 1] = h2_bits((bits_h2(w1) - bias) * d);
            out[4 * i + 2] = h2_bits((bits_h2(w2) - bias) * d);
            out[4 * i + 3] = h2_bits((bits_h2(w3) - bias) * d);
        }
    } else {
        const h2 d = scale_pair((uint16_t)sa, (uint16_t)sb);
        const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const uint32_t x0 = __builtin_amdgcn_perm(bw[i], aw[i], 0x05040100u);  // bytes {a0, a1, b0, b1}
            const uint32_t x1 = __builtin_amdgcn_perm(bw[i], aw[i], 0x07060302u);  // bytes {a2, a3, b2, b3}
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t u0 = ((x0 >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
                const uint32_t u1 = ((x1 >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
                out[8 * i + k] = h2_bits((bits_h2(u0) - bias) * d);
                out[8 * i + 4 + k] = h2_bits((bits_h2(u1) - bias) * d);
            }
        }
    }
}

template <int KVT>
__device__ __forceinline__ void v_pair(const VRaw<KVT>& a, const VRaw<KVT>& b, uint32_t* out) {
    v_pair_words<KVT, (int)(sizeof(a.w) / 4)>(a.w, b.w, a.sc, b.sc, out);
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// ---- direct-to-LDS loads
typedef __attribute__((address_space(3))) void lds_void;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Direct-to-LDS loads written as inline asm: the compiler's wait-count pass would otherwise treat every later LDS
// read as possibly reading the in-flight DMA data and wait for all outstanding loads (vmcnt(0)), which serialises the
// chunk ring.  The kernel orders them itself: s_waitcnt vmcnt before reading a slot, lgkmcnt(0) before refilling it.
// LDS destination = m0 + lane * size; source = scalar base + per-lane 32-bit offset (or a per-lane 64-bit address).
// An SALU write of m0 needs one wait state before an LDS DMA reads it (the s_nop).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <int SIZE>
__device__ __forceinline__ void dma_sv(uint32_t lds, const void* sbase, uint32_t voff) {
    if constexpr (SIZE == 16)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(voff), "s"(sbase) : "memory", "m0");
    else if constexpr (SIZE == 4)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(voff), "s"(sbase) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_ushort %1, %2" ::"s"(lds), "v"(voff), "s"(sbase) : "memory", "m0");
}
template <int SIZE>
__device__ __forceinline__ void dma_v(uint32_t lds, const void* addr) {
    if constexpr (SIZE == 16)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(addr) : "memory", "m0");
    else if constexpr (SIZE == 4)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds), "v"(addr) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_ushort %1, off" ::"s"(lds), "v"(addr) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }

}  // namespace qwa

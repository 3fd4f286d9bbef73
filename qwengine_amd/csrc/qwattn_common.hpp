// Device-side helpers shared by the gated-attention kernels (gfx950 only).
//
// Model shape constants, fp16 packing, the quantized-row unpackers that turn Q8_0 / Q4_0 / F16 KV bytes into fp16
// MFMA operands, and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qwattn.h"

namespace qwa {

constexpr int NH = 24;     // query heads
constexpr int NKV = 4;     // KV heads
constexpr int HD = 256;    // head dim
constexpr int GRP = 6;     // query heads per KV head
constexpr int NROT = 64;   // rotary dims
constexpr int MAXQ = 8;    // queries per decode call
constexpr int MAX_POS = 262144;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__host__ __device__ constexpr int value_bytes(int kvt) {
    return kvt == QWA_KV_F16 ? 512 : kvt == QWA_KV_Q8_0 ? 256 : kvt == QWA_KV_Q4_0 ? 128 : 0;
}

__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }
__device__ __forceinline__ h2 bits_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint16_t f2h_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
__device__ __forceinline__ float h2f_bits(uint16_t u) { return (float)__builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ h2 scale_pair(uint16_t a, uint16_t b) { return bits_h2((uint32_t)a | ((uint32_t)b << 16)); }

__device__ __forceinline__ h4 make_h4(uint32_t w0, uint32_t w1) {
    typedef uint32_t u2v __attribute__((ext_vector_type(2)));
    u2v u = {w0, w1};
    return __builtin_bit_cast(h4, u);
}
__device__ __forceinline__ h8 make_h8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    u4v u = {w0, w1, w2, w3};
    return __builtin_bit_cast(h8, u);
}

// ---- fp16 from small integers by the exponent trick: the half 0x6400 | x is 1024 + x for x < 1024, so one packed
// subtraction recovers x exactly; one packed multiply by the fp16 block scale then rounds once (the same value as
// fp16(d * x) computed in fp32).

// Q4_0 word (8 codes, element 2i in the low nibble of byte i) -> 4 half2 {(c - 8) * d} in the order
// [e0,e4], [e1,e5], [e2,e6], [e3,e7].
__device__ __forceinline__ void q4_word_to_h8(uint32_t w, h2 d, uint32_t* out) {
    const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t x = ((w >> (4 * k)) & 0x000F000Fu) | 0x64006400u;
        out[k] = h2_bits((bits_h2(x) - bias) * d);
    }
}

// Q8_0: 4 int8 (one word) -> 2 half2 {x0, x1} * d, {x2, x3} * d.
__device__ __forceinline__ void q8_word_to_h4(uint32_t w, h2 d, uint32_t* out) {
    const h2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 128
    const uint32_t u = w ^ 0x80808080u;                       // biased bytes x + 128
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u);  // bytes {u0, 0x64, u1, 0x64}
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u);  // bytes {u2, 0x64, u3, 0x64}
    out[0] = h2_bits((bits_h2(lo) - bias) * d);
    out[1] = h2_bits((bits_h2(hi) - bias) * d);
}

// ---- wave64 reductions (all 64 lanes)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
// reductions over the 32-lane half of a wave that holds one quant block
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
    return v;
}
__device__ __forceinline__ float half_max(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
    return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

}  // namespace qwa

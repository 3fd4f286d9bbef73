// The consumers of the attention output (gfx950): the decode GEMV over ActQ8 activations, the activation quantizer,
// the BF16 GEMV of the small projections and the prefill dequantizer of weight rows to fp16.
//
// Decode GEMV: y[c][r] (+)= W[r, :] . x_c for up to 4 activation columns x_c = d_c * q_c (int8 per 32 values,
// src/cuda/gemv.cuh:12-36).  One wave per weight row (grid-stride); lane u takes the 32-weight sub-blocks u, u + 64,
// ... of the row.  A sub-block is decoded once into 8 dwords of int8 codes plus its group scales / mins, dotted with
// every column by v_dot4_i32_i8, and scaled in fp32:
//     sum_k W x = d_x (g0 . i0 + g1 . i1) - (m0 . q0 + m1 . q1) d_x
// (i = integer dot of the codes with the activation bytes over a 16-weight group, q = sum of the activation bytes
// of the group, g / m = the group's scale / min).  Weight bytes stream once through HBM; the activations (a few KB)
// stay in L1 / L2.  A column's result does not depend on how many columns share the call.
//
// Formats (ggml layouts of src/quant/quant_formats.h:92-104): Q2_K, Q4_K, Q6_K, IQ4_XS and the grid formats IQ2_XXS,
// IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S; BF16 through gemv_bf16 and the dequantizer.  A grid format's codebook is expanded
// from its code words (iq_grids.inc) into LDS by every workgroup, then each lane looks its grid entries up there; the
// signs are applied to the int8 codes (through a table of byte masks, also in LDS, for all but IQ3_S), so the dot
// products stay exact v_dot4 integer sums.  IQ1_S / IQ1_M are not built.
//
// What bounds it: a graph-replayed launch costs ~2.6 us even when empty, and beyond that the kernel is VALU-bound
// (the decode of a sub-block costs more issue cycles than its bytes take to arrive).  The decode therefore avoids
// runtime-indexed byte arrays (compare / select chains), branches between loads (a second round trip) and integer
// multiplies where a table or a shift does.
#include "launch.hpp"
#include "qwattn_common.hpp"

namespace qwa {

#define IQ_TABLE static constexpr
#include "iq_grids.inc"
#undef IQ_TABLE

constexpr int GV_WAVES = 8;  // rows (waves) per workgroup

__device__ __forceinline__ float gv_h(const uint8_t* p) {
    return h2f_bits((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}
__device__ __forceinline__ uint32_t gv_u32(const uint8_t* p) {  // 4-byte aligned
    return *reinterpret_cast<const uint32_t*>(p);
}
__device__ __forceinline__ uint32_t gv_u32_a2(const uint8_t* p) {  // 2-byte aligned (Q6_K blocks are 210 bytes)
    const uint16_t* h = reinterpret_cast<const uint16_t*>(p);
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// A decoded 32-weight sub-block: int8 codes (natural order) and per-16-weight scale / min.  Weight k of group h
// (k = 16 h + l) is g_h * code_k - m_h, with code_k = c[k / 4] byte k % 4 minus `bias`.
struct WSub {
    uint32_t c[8];
    float g0, g1, m0, m1;
};

template <int FMT> struct WFmt;

// Formats without a codebook
struct NoGrid {
    static constexpr int GRID_DWORDS = 0;
    __device__ static void fill(uint32_t*, int, int) {}
};

template <> struct WFmt<QWA_W_Q4_K> : NoGrid {  // d | dmin | scales[12] | qs[128]
    static constexpr int BYTES = 144, BIAS = 0;
    static constexpr bool HALVES = false, MINS = true;
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t*) {
        const float d = gv_h(b), dmin = gv_h(b + 2);
        // 6-bit scale / min of sub-block j from the 12 scale bytes, by shifts (a byte array indexed by the lane's j
        // would compile to compare / select chains): j < 4 takes the low 6 bits of bytes j and j + 4; j >= 4 the
        // nibbles of byte j + 4 and the top 2 bits of bytes j - 4 and j
        const uint32_t s0 = gv_u32(b + 4), s1 = gv_u32(b + 8), s2 = gv_u32(b + 12);
        const uint32_t sh8 = 8 * (j & 3), b0 = s0 >> sh8, b1 = s1 >> sh8, b2 = s2 >> sh8;
        const uint32_t lo = 0u - (uint32_t)(j < 4);  // all ones for j < 4: a mask select, no branch between loads
        const int s6 = (int)(((b0 & 63u) & lo) | (((b2 & 15u) | ((b0 >> 2) & 0x30u)) & ~lo));
        const int m6 = (int)(((b1 & 63u) & lo) | ((((b2 >> 4) & 15u) | ((b1 >> 2) & 0x30u)) & ~lo));
        const uint4* q = reinterpret_cast<const uint4*>(b + 16 + 32 * (j >> 1));
        const uint4 a = q[0], bb = q[1];
        const uint32_t raw[8] = {a.x, a.y, a.z, a.w, bb.x, bb.y, bb.z, bb.w};
        const int sh = 4 * (j & 1);
#pragma unroll
        for (int i = 0; i < 8; i++) w.c[i] = (raw[i] >> sh) & 0x0F0F0F0Fu;
        w.g0 = w.g1 = d * (float)s6;
        w.m0 = w.m1 = dmin * (float)m6;
    }
};

template <> struct WFmt<QWA_W_Q2_K> : NoGrid {  // scales[16] | qs[64] | d | dmin
    static constexpr int BYTES = 84, BIAS = 0;
    static constexpr bool HALVES = true, MINS = true;
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t*) {
        const uint32_t dd = gv_u32(b + 80);
        const float d = h2f_bits((uint16_t)dd), dmin = h2f_bits((uint16_t)(dd >> 16));
        const uint32_t scw = gv_u32(b + 4 * (j >> 1));
        const uint32_t sa = (scw >> (16 * (j & 1))) & 0xFF, sb = (scw >> (16 * (j & 1) + 8)) & 0xFF;
        const uint8_t* q = b + 16 + 32 * (j >> 2);
        const int sh = 2 * (j & 3);
#pragma unroll
        for (int i = 0; i < 8; i++) w.c[i] = (gv_u32(q + 4 * i) >> sh) & 0x03030303u;
        w.g0 = d * (float)(sa & 15);
        w.m0 = dmin * (float)(sa >> 4);
        w.g1 = d * (float)(sb & 15);
        w.m1 = dmin * (float)(sb >> 4);
    }
};

template <> struct WFmt<QWA_W_Q6_K> : NoGrid {  // ql[128] | qh[64] | scales[16] (int8) | d
    static constexpr int BYTES = 210, BIAS = 32;
    static constexpr bool HALVES = true, MINS = false;
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t*) {
        const int h = j >> 2, r = j & 3;
        const float d = gv_h(b + 208);
        const uint8_t* ql = b + 64 * h + 32 * (r & 1);
        const uint8_t* qh = b + 128 + 32 * h;
        const int sl = 4 * (r >> 1), sh = 2 * r;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t lo = (gv_u32_a2(ql + 4 * i) >> sl) & 0x0F0F0F0Fu;
            const uint32_t hi = ((gv_u32_a2(qh + 4 * i) >> sh) & 0x03030303u) << 4;
            w.c[i] = lo | hi;  // 0 .. 63; the bias 32 is taken off through the activation sums
        }
        const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + 8 * h + 2 * r);
        w.g0 = d * (float)sc[0];
        w.g1 = d * (float)sc[1];
        w.m0 = w.m1 = 0.0f;
    }
};

template <> struct WFmt<QWA_W_IQ4_XS> : NoGrid {  // d | scales_h (u16) | scales_l[4] | qs[128]
    static constexpr int BYTES = 136, BIAS = 0;
    static constexpr bool HALVES = false, MINS = false;
    // the 16 non-uniform levels as four little-endian dwords (ggml's kvalues_iq4nl, src/quant/iq_tables.inc:373-375)
    static constexpr uint32_t T0 = 0xBFAD9881u, T1 = 0xF6EADDCFu, T2 = 0x26190D01u, T3 = 0x71594535u;
    __device__ static uint32_t levels(uint32_t nib) {  // four nibble indices (one per byte) -> four int8 levels
        const uint32_t sel = nib & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(T1, T0, sel), hi = __builtin_amdgcn_perm(T3, T2, sel);
        const uint32_t m = ((nib >> 3) & 0x01010101u) * 0xFFu;
        return (hi & m) | (lo & ~m);
    }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t*) {
        const uint32_t hdr = gv_u32(b), sl = gv_u32(b + 4);
        const float d = h2f_bits((uint16_t)hdr);
        const uint32_t shi = hdr >> 16;
        const int ls = (int)(((sl >> (8 * (j >> 1) + 4 * (j & 1))) & 15) | (((shi >> (2 * j)) & 3) << 4));
        const uint4 q = *reinterpret_cast<const uint4*>(b + 8 + 16 * j);
        const uint32_t raw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w.c[i] = levels(raw[i] & 0x0F0F0F0Fu);
            w.c[4 + i] = levels((raw[i] >> 4) & 0x0F0F0F0Fu);
        }
        w.g0 = w.g1 = d * (float)(ls - 32);
        w.m0 = w.m1 = 0.0f;
    }
};

// ---- i-quant grid formats (src/quant/quant_ref.cpp:105-222) ----------------------------------------------------
// Expands a codebook (entries of NB bytes, each byte LEVELS[index of BITS bits]) into LDS as NB / 4 dwords per entry.
// The (at most 8) levels travel as two packed dwords, so a byte is one v_perm lookup, not a dependent memory read.
constexpr uint32_t iq_pack(const uint8_t* lv, int n, int o) {
    uint32_t v = 0;
    for (int j = 0; j < 4; j++) v |= o + j < n ? (uint32_t)lv[o + j] << (8 * j) : 0u;
    return v;
}
template <int N, int NB, int BITS, uint32_t LV_LO, uint32_t LV_HI>
__device__ __forceinline__ void iq_fill(uint32_t* lds, const uint16_t* codes, int t, int nt) {
    for (int e = t; e < N; e += nt) {
        const uint32_t c = codes[e];
#pragma unroll
        for (int w = 0; w < NB / 4; w++) {
            uint32_t sel = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) sel |= ((c >> (BITS * (4 * w + j))) & ((1u << BITS) - 1)) << (8 * j);
            lds[e * (NB / 4) + w] = __builtin_amdgcn_perm(LV_HI, LV_LO, sel);
        }
    }
}
#define QWA_IQ_FILL(P, NB) \
    iq_fill<P##_N, NB, P##_BITS, iq_pack(P##_LEVELS, sizeof(P##_LEVELS), 0), iq_pack(P##_LEVELS, sizeof(P##_LEVELS), 4)>( \
        lds, P##_CODES, t, nt)

// the bytes of g whose sign bit (4 bits, bit j for byte j) is set, negated (g's bytes are 1..127, so no borrow)
__device__ __forceinline__ uint32_t iq_neg(uint32_t g, uint32_t s4) {
    const uint32_t one = ((s4 & 15u) * 0x00204081u) & 0x01010101u;
    return (g ^ (one * 0xFFu)) + one;
}
// ggml's ksigns: a 7-bit index plus the parity bit that makes the number of negative signs even
__device__ __forceinline__ uint32_t iq_signs7(uint32_t s7) {
    s7 &= 127u;
    return s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
}

// Sign masks in LDS, after each grid format's codebook: entry e < 256 holds, for the sign byte e, two dwords whose
// byte k is 0xFF where bit k of e is set; entry 256 + i the same for ggml's ksigns of the 7-bit index i.  Applying
// one is an xor and an add per 4 weights (iq_apply), instead of spreading the bits with integer multiplies.
constexpr int IQ_SIGN_DWORDS = 2 * (256 + 128);
__device__ __forceinline__ void iq_fill_signs(uint32_t* t, int tid, int nt) {
    for (int e = tid; e < 256 + 128; e += nt) {
        const uint32_t sg = e < 256 ? (uint32_t)e : iq_signs7((uint32_t)(e - 256));
        uint32_t m0 = 0, m1 = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            m0 |= ((sg >> k) & 1u) * (0xFFu << (8 * k));
            m1 |= ((sg >> (k + 4)) & 1u) * (0xFFu << (8 * k));
        }
        t[2 * e] = m0;
        t[2 * e + 1] = m1;
    }
}
// the bytes of g under the 0xFF bytes of mask m, negated (g's bytes are 1..127, so no borrow crosses a byte)
__device__ __forceinline__ uint32_t iq_apply(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }

template <> struct WFmt<QWA_W_IQ2_XXS> {  // d | per 32 weights: 4 grid indices, then 4 x 7 sign bits | 4-bit scale
    static constexpr int BYTES = 66, BIAS = 0, CODE_DWORDS = 2 * IQ2XXS_N, GRID_DWORDS = CODE_DWORDS + IQ_SIGN_DWORDS;
    static constexpr bool HALVES = false, MINS = false;
    __device__ static void fill(uint32_t* lds, int t, int nt) {
        QWA_IQ_FILL(IQ2XXS, 8);
        iq_fill_signs(lds + CODE_DWORDS, t, nt);
    }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t* grid) {
        const float d = gv_h(b);
        const uint32_t a0 = gv_u32_a2(b + 2 + 8 * j), a1 = gv_u32_a2(b + 6 + 8 * j);
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t* g = grid + 2 * ((a0 >> (8 * l)) & 255);
            const uint32_t* m = grid + CODE_DWORDS + 2 * (256 + ((a1 >> (7 * l)) & 127));
            w.c[2 * l] = iq_apply(g[0], m[0]);
            w.c[2 * l + 1] = iq_apply(g[1], m[1]);
        }
        w.g0 = w.g1 = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
        w.m0 = w.m1 = 0.0f;
    }
};

template <> struct WFmt<QWA_W_IQ2_XS> {  // d | qs[32] u16 (9-bit index | 7 sign bits) | scales[8] (two 4-bit per 32)
    static constexpr int BYTES = 74, BIAS = 0, CODE_DWORDS = 2 * IQ2XS_N, GRID_DWORDS = CODE_DWORDS + IQ_SIGN_DWORDS;
    static constexpr bool HALVES = true, MINS = false;
    __device__ static void fill(uint32_t* lds, int t, int nt) {
        QWA_IQ_FILL(IQ2XS, 8);
        iq_fill_signs(lds + CODE_DWORDS, t, nt);
    }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t* grid) {
        const float d = gv_h(b);
        const uint32_t q01 = gv_u32_a2(b + 2 + 8 * j), q23 = gv_u32_a2(b + 6 + 8 * j);
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t q = ((l < 2 ? q01 : q23) >> (16 * (l & 1))) & 0xFFFFu;
            const uint32_t* g = grid + 2 * (q & 511u);
            const uint32_t* m = grid + CODE_DWORDS + 2 * (256 + (q >> 9));
            w.c[2 * l] = iq_apply(g[0], m[0]);
            w.c[2 * l + 1] = iq_apply(g[1], m[1]);
        }
        const uint32_t sc = b[66 + j];
        w.g0 = d * (0.5f + (float)(sc & 15u)) * 0.25f;
        w.g1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        w.m0 = w.m1 = 0.0f;
    }
};

template <> struct WFmt<QWA_W_IQ2_S> {  // d | qs[32] index low bytes | signs[32] | qh[8] (2 high bits each) | scales[8]
    static constexpr int BYTES = 82, BIAS = 0, CODE_DWORDS = 2 * IQ2S_N, GRID_DWORDS = CODE_DWORDS + IQ_SIGN_DWORDS;
    static constexpr bool HALVES = true, MINS = false;
    __device__ static void fill(uint32_t* lds, int t, int nt) {
        QWA_IQ_FILL(IQ2S, 8);
        iq_fill_signs(lds + CODE_DWORDS, t, nt);
    }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t* grid) {
        const float d = gv_h(b);
        const uint32_t lo = gv_u32_a2(b + 2 + 4 * j), sg4 = gv_u32_a2(b + 34 + 4 * j), qh = b[66 + j];
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t idx = ((lo >> (8 * l)) & 255u) | (((qh >> (2 * l)) & 3u) << 8);
            const uint32_t* g = grid + 2 * idx;
            const uint32_t* m = grid + CODE_DWORDS + 2 * ((sg4 >> (8 * l)) & 255u);
            w.c[2 * l] = iq_apply(g[0], m[0]);
            w.c[2 * l + 1] = iq_apply(g[1], m[1]);
        }
        const uint32_t sc = b[74 + j];
        w.g0 = d * (0.5f + (float)(sc & 15u)) * 0.25f;
        w.g1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        w.m0 = w.m1 = 0.0f;
    }
};

template <> struct WFmt<QWA_W_IQ3_XXS> {  // d | qs[64] grid indices | per 32 weights 4 x 7 sign bits | 4-bit scale
    static constexpr int BYTES = 98, BIAS = 0, CODE_DWORDS = IQ3XXS_N, GRID_DWORDS = CODE_DWORDS + IQ_SIGN_DWORDS;
    static constexpr bool HALVES = false, MINS = false;
    __device__ static void fill(uint32_t* lds, int t, int nt) {
        QWA_IQ_FILL(IQ3XXS, 4);
        iq_fill_signs(lds + CODE_DWORDS, t, nt);
    }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t* grid) {
        const float d = gv_h(b);
        const uint32_t i0 = gv_u32_a2(b + 2 + 8 * j), i1 = gv_u32_a2(b + 6 + 8 * j), a = gv_u32_a2(b + 66 + 4 * j);
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t q = (l < 2 ? i0 : i1) >> (16 * (l & 1));
            const uint32_t* m = grid + CODE_DWORDS + 2 * (256 + ((a >> (7 * l)) & 127u));
            w.c[2 * l] = iq_apply(grid[q & 255u], m[0]);
            w.c[2 * l + 1] = iq_apply(grid[(q >> 8) & 255u], m[1]);
        }
        w.g0 = w.g1 = d * (0.5f + (float)(a >> 28)) * 0.5f;
        w.m0 = w.m1 = 0.0f;
    }
};

template <> struct WFmt<QWA_W_IQ3_S> {  // d | qs[64] index low bytes | qh[8] (9th bits) | signs[32] | scales[4]
    // signs spread by multiplies here: with 12 LDS reads per sub-block (8 codebook dwords + 4 mask pairs) the mask
    // table measured slower than the arithmetic for this format
    static constexpr int BYTES = 110, BIAS = 0, GRID_DWORDS = IQ3S_N;
    static constexpr bool HALVES = false, MINS = false;
    __device__ static void fill(uint32_t* lds, int t, int nt) { QWA_IQ_FILL(IQ3S, 4); }
    __device__ static void sub(const uint8_t* b, int j, WSub& w, const uint32_t* grid) {
        const float d = gv_h(b);
        const uint32_t i0 = gv_u32_a2(b + 2 + 8 * j), i1 = gv_u32_a2(b + 6 + 8 * j), qh = b[66 + j];
        const uint32_t sg4 = gv_u32_a2(b + 74 + 4 * j);
#pragma unroll
        for (int l = 0; l < 4; l++) {
            const uint32_t q = (l < 2 ? i0 : i1) >> (16 * (l & 1));
            const uint32_t ia = (q & 255u) | (((qh >> (2 * l)) & 1u) << 8);
            const uint32_t ib = ((q >> 8) & 255u) | (((qh >> (2 * l + 1)) & 1u) << 8);
            const uint32_t sg = sg4 >> (8 * l);
            w.c[2 * l] = iq_neg(grid[ia], sg);
            w.c[2 * l + 1] = iq_neg(grid[ib], sg >> 4);
        }
        w.g0 = w.g1 = d * (float)(1 + 2 * (int)((b[106 + j / 2] >> (4 * (j & 1))) & 15));
        w.m0 = w.m1 = 0.0f;
    }
};

#ifndef QWA_GV_BATCH
#define QWA_GV_BATCH -1  // -1: per format as below; 0 / 1: never / always (tuning builds)
#endif
template <int FMT> struct GvBatched {
    static constexpr bool value =
        QWA_GV_BATCH >= 0 ? QWA_GV_BATCH == 1 : FMT != QWA_W_IQ4_XS && FMT != QWA_W_Q2_K && FMT != QWA_W_Q6_K;
};

// One wave per row; NB activation columns at aq + c * act_ld (d / s at + c * act_ld / 32)
template <int FMT, int NB, int U>
__global__ void __launch_bounds__(GV_WAVES * 64) k_gemv_q8(const uint8_t* __restrict__ W, size_t row_bytes, int K,
                                                           int N, const int8_t* __restrict__ aq,
                                                           const float* __restrict__ ad, const float* __restrict__ as,
                                                           int act_ld, float* __restrict__ y, int y_ld,
                                                           int accumulate) {
    using F = WFmt<FMT>;
    const int lane = threadIdx.x & 63;
    const int nsub = K / 32;
    const uint32_t ones = 0x01010101u;
    __shared__ uint32_t s_grid[F::GRID_DWORDS > 0 ? F::GRID_DWORDS : 1];
    if constexpr (F::GRID_DWORDS > 0) {
        F::fill(s_grid, threadIdx.x, GV_WAVES * 64);
        __syncthreads();
    }
    for (int row = blockIdx.x * GV_WAVES + (int)(threadIdx.x >> 6); row < N; row += gridDim.x * GV_WAVES) {
        const uint8_t* wr = W + (size_t)row * row_bytes;
        float acc[NB];
#pragma unroll
        for (int c = 0; c < NB; c++) acc[c] = 0.0f;
        // U sub-blocks per lane at a time: every weight and activation load of the batch (and, for the grid formats,
        // the codebook reads that depend on them) is issued before any of them is used.  Indices past the row are
        // clamped so that the batch stays one basic block, and their products are dropped by a select.  Sub-blocks
        // are accumulated in the order u = lane, lane + 64, ... whatever U is.
        for (int u0 = lane; u0 < nsub; u0 += 64 * U) {
            WSub w[U];
            uint4 x0[U][NB], x1[U][NB];
            float dx[U][NB], sx[U][NB];
#pragma unroll
            for (int k = 0; k < U; k++) {
                const int u = min(u0 + 64 * k, nsub - 1);
                F::sub(wr + (size_t)(u >> 3) * F::BYTES, u & 7, w[k], s_grid);
#pragma unroll
                for (int c = 0; c < NB; c++) {
                    const uint4* xp = reinterpret_cast<const uint4*>(aq + (size_t)c * act_ld + 32 * u);
                    x0[k][c] = xp[0];
                    x1[k][c] = xp[1];
                    dx[k][c] = ad[(size_t)c * (act_ld / 32) + u];
                    sx[k][c] = (!F::HALVES && F::MINS) ? as[(size_t)c * (act_ld / 32) + u] : 0.0f;
                }
            }
#pragma unroll
            for (int k = 0; k < U; k++) {
                const bool valid = u0 + 64 * k < nsub;
#pragma unroll
                for (int c = 0; c < NB; c++) {
                    const float acc_in = acc[c];
                    const uint4 xa = x0[k][c], xb = x1[k][c];
                    int i0 = dot4(w[k].c[0], xa.x, dot4(w[k].c[1], xa.y, dot4(w[k].c[2], xa.z, dot4(w[k].c[3], xa.w, 0))));
                    int i1 = dot4(w[k].c[4], xb.x, dot4(w[k].c[5], xb.y, dot4(w[k].c[6], xb.z, dot4(w[k].c[7], xb.w, 0))));
                    if constexpr (F::HALVES) {
                        if constexpr (F::BIAS != 0 || F::MINS) {
                            const int q0 = dot4(ones, xa.x, dot4(ones, xa.y, dot4(ones, xa.z, dot4(ones, xa.w, 0))));
                            const int q1 = dot4(ones, xb.x, dot4(ones, xb.y, dot4(ones, xb.z, dot4(ones, xb.w, 0))));
                            if constexpr (F::BIAS != 0) {
                                i0 -= F::BIAS * q0;
                                i1 -= F::BIAS * q1;
                            }
                            float v = w[k].g0 * (float)i0 + w[k].g1 * (float)i1;
                            if constexpr (F::MINS) v -= w[k].m0 * (float)q0 + w[k].m1 * (float)q1;
                            acc[c] = fmaf(dx[k][c], v, acc[c]);
                        } else {
                            acc[c] = fmaf(dx[k][c], w[k].g0 * (float)i0 + w[k].g1 * (float)i1, acc[c]);
                        }
                    } else {
                        acc[c] = fmaf(dx[k][c] * w[k].g0, (float)(i0 + i1), acc[c]);
                        if constexpr (F::MINS) acc[c] = fmaf(-w[k].m0, sx[k][c], acc[c]);
                    }
                    acc[c] = valid ? acc[c] : acc_in;
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NB; c++) {
            const float v = wave_sum(acc[c]);
            if (lane == 0) {
                float* yo = y + (size_t)c * y_ld + row;
                *yo = accumulate ? *yo + v : v;
            }
        }
    }
}

// The one-column instantiations of IQ4_XS and IQ2_S are compiled in gemv_mc.hip, with LLVM's max-memory-clause
// machine scheduler (one-column GEMV at 6144 -> 5120: IQ4_XS 6.6 -> 6.15 us, IQ2_S 6.3 -> 6.1 us; the other formats
// measured the same or slower with it).  The schedule moves no arithmetic.
#define QWA_GV_KPARAMS                                                                                                \
    const uint8_t* __restrict__, size_t, int, int, const int8_t* __restrict__, const float* __restrict__,            \
        const float* __restrict__, int, float* __restrict__, int, int
#define QWA_GV_ONE_COLUMN(PRE, FMT)                     \
    PRE __global__ void k_gemv_q8<FMT, 1, 1>(QWA_GV_KPARAMS); \
    PRE __global__ void k_gemv_q8<FMT, 1, 2>(QWA_GV_KPARAMS); \
    PRE __global__ void k_gemv_q8<FMT, 1, 3>(QWA_GV_KPARAMS); \
    PRE __global__ void k_gemv_q8<FMT, 1, 4>(QWA_GV_KPARAMS);
#ifndef QWA_GV_KERNELS_ONLY
QWA_GV_ONE_COLUMN(extern template, QWA_W_IQ4_XS)
QWA_GV_ONE_COLUMN(extern template, QWA_W_IQ2_S)

// ActQ8 of n_rows rows of K values (stride K): one 32-lane half-wave per 32-value block (src/cuda/gemv.cu:30-46)
__global__ void __launch_bounds__(256) k_act_q8_rows(const float* __restrict__ x, int n_blocks, int8_t* __restrict__ q,
                                                     float* __restrict__ d, float* __restrict__ s) {
    const int blk = blockIdx.x * 8 + (int)(threadIdx.x >> 5), l = threadIdx.x & 31;
    const bool on = blk < n_blocks;
    const float v = on ? x[(size_t)blk * 32 + l] : 0.0f;
    const float amax = half_max(fabsf(v));
    const float db = amax / 127.0f;
    const int qi = db > 0.0f ? (int)__builtin_rintf(v / db) : 0;
    const float sum = half_sum((float)qi);
    if (on) {
        q[(size_t)blk * 32 + l] = (int8_t)qi;
        if (l == 0) {
            d[blk] = db;
            s[blk] = db * sum;
        }
    }
}

// y[r] = W[r, :] . x for BF16 weights: one wave per row, 8 weights per lane and step (src/cuda/gemv.cu:125-143)
__global__ void __launch_bounds__(256) k_gemv_bf16(const uint16_t* __restrict__ W, int K, int N,
                                                   const float* __restrict__ x, float* __restrict__ y) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (row >= N) return;
    const uint16_t* w = W + (size_t)row * K;
    float acc = 0.0f;
    for (int k = 8 * lane; k < K; k += 512) {
        const uint4 p = *reinterpret_cast<const uint4*>(w + k);
        const uint32_t u[4] = {p.x, p.y, p.z, p.w};
        const float4 xa = *reinterpret_cast<const float4*>(x + k), xb = *reinterpret_cast<const float4*>(x + k + 4);
        const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            acc = fmaf(__uint_as_float(u[i] << 16), xv[2 * i], acc);
            acc = fmaf(__uint_as_float(u[i] & 0xFFFF0000u), xv[2 * i + 1], acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

// ---- prefill: weight rows to fp16, bit-exact with fp16(RNE) of the reference dequantizer's fp32 value
// (src/cuda/prefill.cuh:16-18).  One thread per 32-weight sub-block; values formed as the reference forms them, with
// no FMA contraction.
#pragma clang fp contract(off)
template <int FMT>
__device__ __forceinline__ void dq_sub(const uint8_t* b, int j, float* v, const uint32_t* grid) {
    if constexpr (FMT == QWA_W_Q4_K) {
        WSub w;
        WFmt<FMT>::sub(b, j, w, grid);
        // w.g0 = d * s6, w.m0 = dmin * m6, as the reference's d1 / m1
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = w.g0 * (float)((w.c[i / 4] >> (8 * (i % 4))) & 0xFF) - w.m0;
    } else if constexpr (FMT == QWA_W_Q2_K) {
        WSub w;
        WFmt<FMT>::sub(b, j, w, grid);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float code = (float)((w.c[i / 4] >> (8 * (i % 4))) & 0xFF);
            v[i] = i < 16 ? w.g0 * code - w.m0 : w.g1 * code - w.m1;
        }
    } else if constexpr (FMT == QWA_W_Q6_K) {
        WSub w;
        WFmt<FMT>::sub(b, j, w, grid);
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const float code = (float)((int)((w.c[i / 4] >> (8 * (i % 4))) & 0xFF) - 32);
            v[i] = (i < 16 ? w.g0 : w.g1) * code;
        }
    } else {  // IQ4_XS and the grid formats: signed int8 codes times the sub-block's (half) scale
        WSub w;
        WFmt<FMT>::sub(b, j, w, grid);
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = (i < 16 ? w.g0 : w.g1) * (float)(int8_t)((w.c[i / 4] >> (8 * (i % 4))) & 0xFF);
    }
}

template <int FMT>
__global__ void __launch_bounds__(256) k_dequant_f16(const uint8_t* __restrict__ W, size_t row_bytes, int K, int rows,
                                                     uint16_t* __restrict__ out) {
    const int nsub = K / 32;
    __shared__ uint32_t s_grid[WFmt<FMT>::GRID_DWORDS > 0 ? WFmt<FMT>::GRID_DWORDS : 1];
    if constexpr (WFmt<FMT>::GRID_DWORDS > 0) {
        WFmt<FMT>::fill(s_grid, threadIdx.x, 256);
        __syncthreads();
    }
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)rows * nsub) return;
    const int r = (int)(i / nsub), u = (int)(i % nsub);
    float v[32];
    dq_sub<FMT>(W + (size_t)r * row_bytes + (size_t)(u >> 3) * WFmt<FMT>::BYTES, u & 7, v, s_grid);
    // the fp32 values stay opaque to the conversion: otherwise a product and its fp16 rounding fold into one
    // mixed-precision fma with a +0 addend, which turns -0 into +0
#pragma unroll
    for (int k = 0; k < 32; k++) asm volatile("" : "+v"(v[k]));
    uint32_t h[16];
#pragma unroll
    for (int k = 0; k < 16; k++) h[k] = (uint32_t)f2h_bits(v[2 * k]) | ((uint32_t)f2h_bits(v[2 * k + 1]) << 16);
    uint4* dst = reinterpret_cast<uint4*>(out + (size_t)r * K + 32 * u);
#pragma unroll
    for (int k = 0; k < 4; k++) dst[k] = make_uint4(h[4 * k], h[4 * k + 1], h[4 * k + 2], h[4 * k + 3]);
}

__global__ void __launch_bounds__(256) k_bf16_to_f16(const uint16_t* __restrict__ W, long long n,
                                                     uint16_t* __restrict__ out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f2h_bits(__uint_as_float((uint32_t)W[i] << 16));
}
#pragma clang fp contract(on)

// ------------------------------------------------------------------------------------------------------ launchers
size_t w_row_bytes(int fmt, long long K) {
    if (fmt == QWA_W_BF16) return (size_t)K * 2;
    if (K <= 0 || K % 256) return 0;
    switch (fmt) {
        case QWA_W_Q2_K: return (size_t)(K / 256) * WFmt<QWA_W_Q2_K>::BYTES;
        case QWA_W_Q4_K: return (size_t)(K / 256) * WFmt<QWA_W_Q4_K>::BYTES;
        case QWA_W_Q6_K: return (size_t)(K / 256) * WFmt<QWA_W_Q6_K>::BYTES;
        case QWA_W_IQ4_XS: return (size_t)(K / 256) * WFmt<QWA_W_IQ4_XS>::BYTES;
        case QWA_W_IQ2_XXS: return (size_t)(K / 256) * WFmt<QWA_W_IQ2_XXS>::BYTES;
        case QWA_W_IQ2_XS: return (size_t)(K / 256) * WFmt<QWA_W_IQ2_XS>::BYTES;
        case QWA_W_IQ2_S: return (size_t)(K / 256) * WFmt<QWA_W_IQ2_S>::BYTES;
        case QWA_W_IQ3_XXS: return (size_t)(K / 256) * WFmt<QWA_W_IQ3_XXS>::BYTES;
        case QWA_W_IQ3_S: return (size_t)(K / 256) * WFmt<QWA_W_IQ3_S>::BYTES;
        default: return 0;
    }
}

bool gemv_q8_supported(int fmt) {
    return fmt == QWA_W_Q2_K || fmt == QWA_W_Q4_K || fmt == QWA_W_Q6_K || fmt == QWA_W_IQ4_XS || fmt == QWA_W_IQ2_XXS ||
           fmt == QWA_W_IQ2_XS || fmt == QWA_W_IQ2_S || fmt == QWA_W_IQ3_XXS || fmt == QWA_W_IQ3_S;
}

template <int FMT>
static hipError_t gemv_fmt(const void* W, size_t rb, int K, int N, const qwa_act_q8& a, int nb, int act_ld, float* y,
                           int y_ld, int acc, hipStream_t st) {
    const dim3 grid((unsigned)min((N + GV_WAVES - 1) / GV_WAVES, 65535)), block(GV_WAVES * 64);
    const uint8_t* w = static_cast<const uint8_t*>(W);
    // one column: a lane's sub-block rounds (K / 2048 of them, up to 4) loaded as one batch, for the formats whose
    // decode chain is long enough to gain from it (measured: Q4_K and the grid formats; IQ4_XS, Q2_K, Q6_K run
    // faster one sub-block at a time).  Several columns keep one sub-block per batch (registers).
    const int rounds = (K / 32 + 63) / 64;
    const int ub = (nb == 1 && GvBatched<FMT>::value) ? min(rounds, 4) : 1;
#define QWA_GV_LAUNCH(NB, U) \
    hipLaunchKernelGGL((k_gemv_q8<FMT, NB, U>), grid, block, 0, st, w, rb, K, N, a.q, a.d, a.s, act_ld, y, y_ld, acc)
    switch (nb) {
        case 1:
            switch (ub) {
                case 1: QWA_GV_LAUNCH(1, 1); break;
                case 2: QWA_GV_LAUNCH(1, 2); break;
                case 3: QWA_GV_LAUNCH(1, 3); break;
                default: QWA_GV_LAUNCH(1, 4); break;
            }
            break;
        case 2: QWA_GV_LAUNCH(2, 1); break;
        case 3: QWA_GV_LAUNCH(3, 1); break;
        default: QWA_GV_LAUNCH(4, 1); break;
    }
#undef QWA_GV_LAUNCH
    return hipGetLastError();
}

hipError_t launch_gemv_q8(int fmt, const void* W, size_t rb, int K, int N, const qwa_act_q8& a, int nb, int act_ld,
                          float* y, int y_ld, int accumulate, hipStream_t st) {
    switch (fmt) {
        case QWA_W_Q2_K: return gemv_fmt<QWA_W_Q2_K>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_Q4_K: return gemv_fmt<QWA_W_Q4_K>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_Q6_K: return gemv_fmt<QWA_W_Q6_K>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ4_XS: return gemv_fmt<QWA_W_IQ4_XS>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ2_XXS: return gemv_fmt<QWA_W_IQ2_XXS>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ2_XS: return gemv_fmt<QWA_W_IQ2_XS>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ2_S: return gemv_fmt<QWA_W_IQ2_S>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ3_XXS: return gemv_fmt<QWA_W_IQ3_XXS>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        case QWA_W_IQ3_S: return gemv_fmt<QWA_W_IQ3_S>(W, rb, K, N, a, nb, act_ld, y, y_ld, accumulate, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_act_q8(const float* x, long long n, const qwa_act_q8& out, hipStream_t st) {
    const long long nblk = n / 32;
    hipLaunchKernelGGL(k_act_q8_rows, dim3((unsigned)((nblk + 7) / 8)), dim3(256), 0, st, x, (int)nblk, out.q, out.d,
                       out.s);
    return hipGetLastError();
}

hipError_t launch_gemv_bf16(const uint16_t* W, int K, int N, const float* x, float* y, hipStream_t st) {
    hipLaunchKernelGGL(k_gemv_bf16, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, W, K, N, x, y);
    return hipGetLastError();
}

hipError_t launch_dequant_f16(int fmt, const void* W, size_t rb, int K, int rows, uint16_t* out, hipStream_t st) {
    const uint8_t* w = static_cast<const uint8_t*>(W);
    if (fmt == QWA_W_BF16) {
        const long long n = (long long)rows * K;
        hipLaunchKernelGGL(k_bf16_to_f16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                           reinterpret_cast<const uint16_t*>(W), n, out);
        return hipGetLastError();
    }
    const long long n = (long long)rows * (K / 32);
    const dim3 grid((unsigned)((n + 255) / 256)), block(256);
    switch (fmt) {
        case QWA_W_Q2_K: hipLaunchKernelGGL(k_dequant_f16<QWA_W_Q2_K>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_Q4_K: hipLaunchKernelGGL(k_dequant_f16<QWA_W_Q4_K>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_Q6_K: hipLaunchKernelGGL(k_dequant_f16<QWA_W_Q6_K>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ4_XS: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ4_XS>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ2_XXS: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ2_XXS>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ2_XS: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ2_XS>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ2_S: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ2_S>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ3_XXS: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ3_XXS>, grid, block, 0, st, w, rb, K, rows, out); break;
        case QWA_W_IQ3_S: hipLaunchKernelGGL(k_dequant_f16<QWA_W_IQ3_S>, grid, block, 0, st, w, rb, K, rows, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

#endif  // QWA_GV_KERNELS_ONLY

}  // namespace qwa

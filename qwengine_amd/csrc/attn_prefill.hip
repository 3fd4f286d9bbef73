// Causal prefill attention over the quantized KV cache on fp16 MFMA (gfx950).
//
// FlashAttention-2 structure (the reference's k_attn_prefill_mma, src/cuda/prefill.cu:522-794, re-designed for
// wave64 / MFMA / 160 KB LDS):
//  * a workgroup owns 128 consecutive (query, head) rows of one KV head (row r = 6 * token + head) and walks the
//    causal key range in 32-key tiles; 4 consumer waves own 32 rows each (two 16-row MFMA tiles);
//  * 4 producer waves (one per SIMD) stage the tiles: the raw quantized K/V bytes of tile kt + 2 sit in their
//    registers while tile kt + 1 is dequantized to fp16 into the other half of a double buffer in LDS -- K as
//    [key][dim], V transposed as [dim][key] so both MFMA A-operands are single 16-byte LDS reads; one barrier per
//    tile.  The role branch keeps the two register sets apart, so the consumers keep Q, S, P and O in registers;
//  * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_f16 (fp32 accumulation); each K / V fragment read from
//    LDS feeds both row tiles of the wave;  P^T comes out of the S^T accumulator already in B-operand layout;
//  * online softmax in fp32 (exp2 with log2 e folded in), lazy rescale, deferred 1/l, fused sigmoid gate, fp16 out.
//  32-key tiles keep the consumer at 256 VGPRs (two waves per SIMD); 64-key tiles spill.
#include <float.h>

#include "kv_operands.hpp"
#include "launch.hpp"

namespace qwa {

#ifndef QWA_PF_CW
#define QWA_PF_CW 4
#endif
constexpr int PF_CWAVES = QWA_PF_CW;             // consumer (MFMA) waves
constexpr int PF_PWAVES = 4;                     // producer (staging) waves, one per SIMD
constexpr int PF_PT = PF_PWAVES * 64;            // producer threads
constexpr int PF_THREADS = (PF_CWAVES + PF_PWAVES) * 64;
constexpr int PF_RT = 8 / PF_CWAVES;             // 16-row MFMA tiles per consumer wave
constexpr int PF_ROWS = PF_CWAVES * PF_RT * 16;  // 128 rows per workgroup
#ifndef QWA_PF_TILE
#define QWA_PF_TILE 32
#endif
constexpr int PF_TILE = QWA_PF_TILE;             // keys per tile
constexpr int PF_KT = PF_TILE / 16;              // 16-key MFMA tiles per tile
constexpr int PF_KS = PF_TILE / 32;              // 32-key P.V steps per tile
constexpr int PF_CB = PF_TILE / 8;               // V column blocks (8 key positions each)
constexpr int KS_LD = HD + 8;                    // K tile row stride (halves): conflict-free 16-byte reads
constexpr int VT_LD = PF_TILE + 8;               // V^T tile row stride (halves)
constexpr float PF_LOG2E = 1.4426950408889634f;
constexpr float PF_RESCALE_T = 8.0f;  // lazy-rescale threshold on the running maximum (natural-log units)

// raw bytes of one tile held by one thread between the global load and the LDS store
template <int KVT> struct PfRaw {
    static constexpr int VB = value_bytes(KVT);
    static constexpr int KP = PF_TILE * (VB / 16) / PF_PT;   // 16-byte K pieces per producer thread
    static constexpr int VR = PF_TILE / 32;                  // V (8 keys x 4 dims) groups per producer thread
    static constexpr int VW = KVT == QWA_KV_F16 ? 2 : 1;     // V words per key for 4 dims
    uint4 k[KP];
    uint16_t ks[KP];
    uint32_t v[VR][8][VW];
    uint16_t vs[VR][8];
};

// producer thread t (of 256): K pieces idx = t + 256 c (key idx / P, piece idx % P); V: for each rep the position
// tt = t + 256 rep gives column block cb = tt % PF_CB (keys of the 32-key step cb / 4, lane group cb % 4) and dims
// 4 (tt / PF_CB) .. + 4.  Keys past kmax re-read row kmax: their scores are masked (p = 0) and the row holds finite
// values, so the loads need no branches.
template <int KVT>
__device__ __forceinline__ void pf_load(PfRaw<KVT>& r, const qwa_kv_layer& kv, size_t rowbase, int k0, int kmax,
                                        int t) {
    constexpr int VB = value_bytes(KVT);
    constexpr int P = VB / 16;
#pragma unroll
    for (int c = 0; c < PfRaw<KVT>::KP; c++) {
        const int idx = t + PF_PT * c, key = min(k0 + idx / P, kmax), pc = idx % P;
        const size_t row = rowbase + key;
        r.k[c] = ld16(kv.k + row * VB + 16 * pc);
        if (KVT == QWA_KV_Q4_0) r.ks[c] = kv.ks[row * 8 + pc];
        else if (KVT == QWA_KV_Q8_0) r.ks[c] = kv.ks[row * 8 + (pc >> 1)];
        else r.ks[c] = 0;
    }
#pragma unroll
    for (int rep = 0; rep < PfRaw<KVT>::VR; rep++) {
        const int tt = t + PF_PT * rep, cb = tt % PF_CB, dc = tt / PF_CB, h32 = cb >> 2, gq = cb & 3;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int key = min(k0 + 32 * h32 + (j < 4 ? 4 * gq + j : 16 + 4 * gq + (j - 4)), kmax);
            const size_t row = rowbase + key;
            if constexpr (KVT == QWA_KV_Q4_0) {
                r.v[rep][j][0] = *reinterpret_cast<const uint16_t*>(kv.v + row * VB + 2 * dc);  // 4 dims = 2 bytes
            } else if constexpr (KVT == QWA_KV_Q8_0) {
                r.v[rep][j][0] = *reinterpret_cast<const uint32_t*>(kv.v + row * VB + 4 * dc);
            } else {
                const uint2 u = ld8(kv.v + row * VB + 8 * dc);
                r.v[rep][j][0] = u.x;
                r.v[rep][j][1] = u.y;
            }
            r.vs[rep][j] = KVT == QWA_KV_F16 ? 0 : kv.vs[row * 8 + (dc >> 3)];
        }
    }
}

// 4 dims of one V key as two half2 {d0, d1}, {d2, d3}, scaled by the key's block scale (one fp16 rounding)
template <int KVT>
__device__ __forceinline__ void pf_v4(const uint32_t* w, uint32_t sc, uint32_t* out) {
    if constexpr (KVT == QWA_KV_F16) {
        out[0] = w[0];
        out[1] = w[1];
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const h2 d = scale_pair((uint16_t)sc, (uint16_t)sc);
        q8_word_to_h4(w[0], d, out);
    } else {
        const h2 d = scale_pair((uint16_t)sc, (uint16_t)sc);
        const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
        const uint32_t x = w[0];
        // byte 0 -> dims 0 (low nibble), 1 (high nibble); byte 1 -> dims 2, 3
        const uint32_t p01 = ((x & 0x0Fu) | ((x & 0xF0u) << 12)) | 0x64006400u;
        const uint32_t p23 = (((x >> 8) & 0x0Fu) | (((x >> 8) & 0xF0u) << 12)) | 0x64006400u;
        out[0] = h2_bits((bits_h2(p01) - bias) * d);
        out[1] = h2_bits((bits_h2(p23) - bias) * d);
    }
}

template <int KVT>
__device__ __forceinline__ void pf_store(const PfRaw<KVT>& r, _Float16* Ks, _Float16* Vt, int t) {
    constexpr int VB = value_bytes(KVT);
    constexpr int P = VB / 16;
#pragma unroll
    for (int c = 0; c < PfRaw<KVT>::KP; c++) {
        const int idx = t + PF_PT * c, key = idx / P, pc = idx % P;
        const uint4 u = r.k[c];
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        if constexpr (KVT == QWA_KV_F16) {
            *reinterpret_cast<uint4*>(Ks + key * KS_LD + 8 * pc) = u;
        } else if constexpr (KVT == QWA_KV_Q8_0) {
            const h2 d = scale_pair(r.ks[c], r.ks[c]);
            uint32_t o[8];
#pragma unroll
            for (int i = 0; i < 4; i++) q8_word_to_h4(w[i], d, o + 2 * i);
            *reinterpret_cast<uint4*>(Ks + key * KS_LD + 16 * pc) = make_uint4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<uint4*>(Ks + key * KS_LD + 16 * pc + 8) = make_uint4(o[4], o[5], o[6], o[7]);
        } else {
            const h2 d = scale_pair(r.ks[c], r.ks[c]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t o[4];
                q4_word_to_h8(w[i], d, o);
                *reinterpret_cast<uint4*>(Ks + key * KS_LD + 32 * pc + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    // V^T: row (dim) 4 dc + d, positions 8 cb .. 8 cb + 7
#pragma unroll
    for (int rep = 0; rep < PfRaw<KVT>::VR; rep++) {
        const int tt = t + PF_PT * rep, cb = tt % PF_CB, dc = tt / PF_CB;
        uint32_t hv[8][2];  // [key position][dim pair]
#pragma unroll
        for (int j = 0; j < 8; j++) pf_v4<KVT>(r.v[rep][j], r.vs[rep][j], hv[j]);
#pragma unroll
        for (int d = 0; d < 4; d++) {
            uint32_t w[4];
            const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;  // high / low half of both words
#pragma unroll
            for (int jp = 0; jp < 4; jp++)
                w[jp] = __builtin_amdgcn_perm(hv[2 * jp + 1][d >> 1], hv[2 * jp][d >> 1], sel);
            *reinterpret_cast<uint4*>(Vt + (4 * dc + d) * VT_LD + 8 * cb) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

__device__ __forceinline__ h8 lds_h8(const _Float16* p) { return *reinterpret_cast<const h8*>(p); }

template <int KVT>
__global__ void __launch_bounds__(PF_THREADS)
__attribute__((amdgpu_waves_per_eu(PF_THREADS / 256, PF_THREADS / 256)))
k_prefill(const float* __restrict__ q, const float* __restrict__ gate, qwa_kv_layer kv, int B, int p0,
          uint16_t* __restrict__ out16) {
    __shared__ __attribute__((aligned(16))) _Float16 s_k[2][PF_TILE * KS_LD];
    __shared__ __attribute__((aligned(16))) _Float16 s_vt[2][HD * VT_LD];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const bool producer = wave >= PF_CWAVES;
    const int pt = threadIdx.x - PF_CWAVES * 64;  // producer thread index
    const int i16 = lane & 15, lg = lane >> 4;
    const int g = blockIdx.y;
    const int row0 = blockIdx.x * PF_ROWS;
    const int nrows = GRP * B;
    // last key any row of the workgroup sees; tiles past it are never needed
    const int last_row = min(row0 + PF_ROWS, nrows) - 1;
    const int kmax = p0 + last_row / GRP;
    const int n_tiles = kmax / PF_TILE + 1;
    const size_t rowbase = (size_t)g * kv.capacity;

    if (producer) {
        // staging waves: the raw bytes of tile kt + 2 are in registers while the consumers compute tile kt; tile
        // kt + 1 is dequantised into the other buffer meanwhile (the last iteration writes a copy that is never read).
        // The role branch encloses each role's whole state, so the two register sets never overlap.
        PfRaw<KVT> raw;
        pf_load<KVT>(raw, kv, rowbase, 0, kmax, pt);
        pf_store<KVT>(raw, s_k[0], s_vt[0], pt);
        pf_load<KVT>(raw, kv, rowbase, min(1, n_tiles - 1) * PF_TILE, kmax, pt);
        __syncthreads();
        for (int kt = 0; kt < n_tiles; kt++) {
            const int buf = kt & 1;
            pf_store<KVT>(raw, s_k[buf ^ 1], s_vt[buf ^ 1], pt);
            pf_load<KVT>(raw, kv, rowbase, min(kt + 2, n_tiles - 1) * PF_TILE, kmax, pt);
            __syncthreads();
        }
        return;
    }

    // ---- consumer (MFMA) waves
    // this lane's rows: token tq, head hh, last visible key qpos
    int tq[PF_RT], hh[PF_RT], qpos[PF_RT];
    h8 qb[PF_RT][8];
    const int wrow0 = row0 + 16 * PF_RT * wave;
#pragma unroll
    for (int rt = 0; rt < PF_RT; rt++) {
        const int r = wrow0 + 16 * rt + i16;
        tq[rt] = r / GRP;
        hh[rt] = r % GRP;
        const bool valid = tq[rt] < B;
        qpos[rt] = valid ? p0 + tq[rt] : -1;
        const float* qrow = q + ((size_t)(valid ? tq[rt] : 0) * NH + g * GRP + hh[rt]) * HD;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            // LDS position 32 s + 8 lg + j of a K row holds dim 32 s + 8 lg + perm(j)
            const float* src = qrow + 32 * s + 8 * lg;
            const float4 a = *reinterpret_cast<const float4*>(src);
            const float4 b = *reinterpret_cast<const float4*>(src + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            h8 v;
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = valid ? (_Float16)(x[k_perm<KVT>(j)] * 0.0625f) : (_Float16)0.0f;
            qb[rt][s] = v;
        }
    }
    // first query of the wave: tiles entirely at or before it need no causal mask
    const int wave_qmin = p0 + wrow0 / GRP;

    f4 o[PF_RT][16];
    float m[PF_RT], l[PF_RT], msl[PF_RT], mthr[PF_RT];
#pragma unroll
    for (int rt = 0; rt < PF_RT; rt++) {
        m[rt] = -INFINITY;
        l[rt] = 0.0f;
        msl[rt] = 0.0f;
        mthr[rt] = -INFINITY;
#pragma unroll
        for (int dt = 0; dt < 16; dt++) o[rt][dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    __syncthreads();  // tile 0 staged

    for (int kt = 0; kt < n_tiles; kt++) {
        const int k0 = kt * PF_TILE, buf = kt & 1;
        const _Float16* Ks = s_k[buf];
        const _Float16* Vt = s_vt[buf];

        // ---- S^T = K Q^T for PF_KT key tiles of 16
        f4 sc[PF_RT][PF_KT];
#pragma unroll
        for (int k4 = 0; k4 < PF_KT; k4++)
#pragma unroll
            for (int rt = 0; rt < PF_RT; rt++) sc[rt][k4] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 8; s++) {
#pragma unroll
            for (int k4 = 0; k4 < PF_KT; k4++) {
                const h8 a = lds_h8(Ks + (16 * k4 + i16) * KS_LD + 8 * lg + 32 * s);
#pragma unroll
                for (int rt = 0; rt < PF_RT; rt++) sc[rt][k4] = mfma16(a, qb[rt][s], sc[rt][k4]);
            }
        }

        // ---- mask + online softmax (lane: row (rt, i16), keys k0 + 16 k4 + 4 lg + i).  The reference maximum m
        // moves only when a score exceeds it by more than PF_RESCALE_T (probabilities stay <= e^PF_RESCALE_T, far
        // inside fp16), so the accumulators are rarely rescaled.
        const bool need_mask = k0 + PF_TILE - 1 > wave_qmin;
        h8 pb[PF_RT][PF_KS];
        float cr[PF_RT];
#pragma unroll
        for (int rt = 0; rt < PF_RT; rt++) {
            if (need_mask) {
#pragma unroll
                for (int k4 = 0; k4 < PF_KT; k4++)
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int key = k0 + 16 * k4 + 4 * lg + i;
                        sc[rt][k4][i] = key > qpos[rt] ? -INFINITY : sc[rt][k4][i];
                    }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int k4 = 0; k4 < PF_KT; k4++)
                mx = fmaxf(mx, fmaxf(fmaxf(sc[rt][k4][0], sc[rt][k4][1]), fmaxf(sc[rt][k4][2], sc[rt][k4][3])));
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = mx > mthr[rt] ? mx : m[rt];
            cr[rt] = mn == m[rt] ? 1.0f : fast_exp2((m[rt] - mn) * PF_LOG2E);  // m = -inf: c = 0
            m[rt] = mn;
            msl[rt] = mn == -INFINITY ? 0.0f : mn * PF_LOG2E;
            mthr[rt] = mn + PF_RESCALE_T;
            float rs = 0.0f;
#pragma unroll
            for (int ks = 0; ks < PF_KS; ks++) {
                h8 p;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float e = fast_exp2(fmaf(sc[rt][2 * ks + (j >> 2)][j & 3], PF_LOG2E, -msl[rt]));
                    rs += e;
                    p[j] = (_Float16)e;
                }
                pb[rt][ks] = p;
            }
            l[rt] = l[rt] * cr[rt] + rs;
        }
        if (__any(cr[0] != 1.0f || cr[PF_RT - 1] != 1.0f)) {
#pragma unroll
            for (int rt = 0; rt < PF_RT; rt++)
#pragma unroll
                for (int dt = 0; dt < 16; dt++) o[rt][dt] *= cr[rt];
        }

        // ---- O^T += V^T P^T: 16 dim tiles x PF_KS key steps of 32; dim tile dt + 1's fragments are read while dt
        // multiplies
        {
            h8 cur[PF_KS], nxt[PF_KS];
#pragma unroll
            for (int ks = 0; ks < PF_KS; ks++) nxt[ks] = lds_h8(Vt + i16 * VT_LD + 8 * lg + 32 * ks);
#pragma unroll
            for (int dt = 0; dt < 16; dt++) {
#pragma unroll
                for (int ks = 0; ks < PF_KS; ks++) cur[ks] = nxt[ks];
                if (dt < 15) {
#pragma unroll
                    for (int ks = 0; ks < PF_KS; ks++) nxt[ks] = lds_h8(Vt + (16 * (dt + 1) + i16) * VT_LD + 8 * lg + 32 * ks);
                }
#pragma unroll
                for (int ks = 0; ks < PF_KS; ks++)
#pragma unroll
                    for (int rt = 0; rt < PF_RT; rt++) o[rt][dt] = mfma16(cur[ks], pb[rt][ks], o[rt][dt]);
            }
        }

        __syncthreads();
    }

    // ---- normalise, gate, fp16 out: lane holds dims 16 dt + 4 lg + i of row (rt, i16)
#pragma unroll
    for (int rt = 0; rt < PF_RT; rt++) {
        float lt = l[rt];
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        if (qpos[rt] < 0) continue;
        const float il = 1.0f / lt;
        const size_t base = ((size_t)tq[rt] * NH + g * GRP + hh[rt]) * HD;
#pragma unroll
        for (int dt = 0; dt < 16; dt++) {
            const int d = 16 * dt + 4 * lg;
            const float4 gv = *reinterpret_cast<const float4*>(gate + base + d);
            const float gg[4] = {gv.x, gv.y, gv.z, gv.w};
            uint16_t hv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) hv[i] = f2h_bits(o[rt][dt][i] * il * sigmoid(gg[i]));
            *reinterpret_cast<uint2*>(out16 + base + d) =
                make_uint2((uint32_t)hv[0] | ((uint32_t)hv[1] << 16), (uint32_t)hv[2] | ((uint32_t)hv[3] << 16));
        }
    }
}

hipError_t launch_prefill(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                          uint16_t* out16, hipStream_t st) {
    const dim3 grid((GRP * B + PF_ROWS - 1) / PF_ROWS, NKV);
    profile_mark_begin(st);
    if (kvt == QWA_KV_F16) hipLaunchKernelGGL(k_prefill<QWA_KV_F16>, grid, dim3(PF_THREADS), 0, st, q, gate, kv, B, p0, out16);
    else if (kvt == QWA_KV_Q8_0) hipLaunchKernelGGL(k_prefill<QWA_KV_Q8_0>, grid, dim3(PF_THREADS), 0, st, q, gate, kv, B, p0, out16);
    else hipLaunchKernelGGL(k_prefill<QWA_KV_Q4_0>, grid, dim3(PF_THREADS), 0, st, q, gate, kv, B, p0, out16);
    profile_mark_end(st);
    return hipGetLastError();
}

}  // namespace qwa

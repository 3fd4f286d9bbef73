// Decode / speculative-verify attention over the quantized KV cache (gfx950).
//
// Split-K flash-decoding (the reference's structure, src/cuda/ops.cu:507-815, re-designed for wave64 + MFMA):
//  * rows are (query, head) pairs of one KV head, row r = 6 * query + head, in 16-row MFMA tiles
//    (RT = ceil(6 nq / 16) tiles); a wave owns one fixed 256-key split x one row tile, and the RT waves of a split
//    sit in the same workgroup so their K/V reads share L1 / L2;
//  * 16-key chunks: S = Q K^T on v_mfma_f32_16x16x32_f16 (one MFMA per 32-dim quant block, exact integer K codes,
//    fp32 block-scale applied to the partial dots, Q / 16 as fp16 hi + lo) and O^T = V^T P^T on
//    v_mfma_f32_16x16x16_f16 (V dequantized to fp16 in registers), fp32 accumulation; K and V are read straight
//    from HBM; the 16 x 16 score tile is transposed through LDS so that a lane holds 4 keys of ONE row: the online
//    softmax is lane-local up to a 4-lane max / sum, and P^T is already the B operand of the P.V product;
//  * a ring of NBUF chunks per wave keeps loads in flight while the current chunk is computed;
//  * each split writes a partial record (m, l, O[256]); k_dec_combine merges them in a fixed order, normalises,
//    applies the sigmoid gate and the optional ActQ8 epilogue.
// Split boundaries are fixed multiples of 256 keys and masked keys contribute exact zeros, so a query's output does
// not depend on how many queries share the call (the reference's decode == decode_batch contract,
// src/cuda/ops.cuh:134-135).
#include <float.h>

#include "kv_operands.hpp"
#include "launch.hpp"

namespace qwa {

constexpr int REC = 260;   // partial record: m, l, 2 pad, O[256] (16-byte aligned O)
constexpr int CGRP = 32;   // combine: splits per fixed summation group
constexpr float LOG2E = 1.4426950408889634f;

size_t dec_work_bytes(int n_pos) {
    const size_t nsplit = (size_t)dec_nsplit(n_pos + MAXQ);
    const size_t mma = nsplit * NKV * MAXQ * GRP * REC * sizeof(float);
    return mma;
}

// Raw bytes of one 16-key chunk held by one lane.
//  K (B operand of S = Q K^T, one MFMA per 32-dim quant block): key kb + (lane % 16), for every block b the 8 dims
//    32 b + 8 g + perm(j) as raw bytes (Q4_0: 1 word per block, Q8_0: 2, F16: 4), plus that key's 8 block scales.
//  V (A operand of O^T = V^T P^T): keys kb + 4 g + j, j = 0..3, dims 16 (lane % 16) .. + 15, with their scales.
template <int KVT> struct KChunk;
template <> struct KChunk<QWA_KV_Q4_0> { uint32_t w[8]; uint32_t sc[4]; };
template <> struct KChunk<QWA_KV_Q8_0> { uint32_t w[16]; uint32_t sc[4]; };
template <> struct KChunk<QWA_KV_F16> { uint32_t w[32]; uint32_t sc[4]; };

template <int KVT>
struct Chunk {
    KChunk<KVT> k;
    VRaw<KVT> v[4];
};

template <int KVT>
__device__ __forceinline__ void load_chunk(Chunk<KVT>& c, const qwa_kv_layer& kv, size_t rowbase, int kb, int kmax,
                                           int i16, int lg) {
    constexpr int VB = value_bytes(KVT);
    constexpr int WPB = sizeof(c.k.w) / 4 / 8;  // raw words per block per lane
    const int key = kb + i16;
    if (key <= kmax) {
        const size_t row = rowbase + key;
        const uint8_t* p = kv.k + row * VB + 4 * WPB * lg;
#pragma unroll
        for (int b = 0; b < 8; b++) {
            const uint8_t* pb = p + (VB / 8) * b;
            if constexpr (WPB == 1) {
                c.k.w[b] = *reinterpret_cast<const uint32_t*>(pb);
            } else if constexpr (WPB == 2) {
                const uint2 u = ld8(pb);
                c.k.w[2 * b] = u.x; c.k.w[2 * b + 1] = u.y;
            } else {
                const uint4 u = ld16(pb);
                c.k.w[4 * b] = u.x; c.k.w[4 * b + 1] = u.y; c.k.w[4 * b + 2] = u.z; c.k.w[4 * b + 3] = u.w;
            }
        }
        if constexpr (KVT != QWA_KV_F16) {
            const uint4 u = *reinterpret_cast<const uint4*>(kv.ks + row * 8);
            c.k.sc[0] = u.x; c.k.sc[1] = u.y; c.k.sc[2] = u.z; c.k.sc[3] = u.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8 * WPB; i++) c.k.w[i] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) c.k.sc[i] = 0;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int vk = kb + 4 * lg + j;
        load_v<KVT>(c.v[j], kv, rowbase + vk, i16, vk <= kmax);
    }
}

// B operand of block b: exact integers (no scale), dims 32 b + 8 g + perm(j)
template <int KVT>
__device__ __forceinline__ h8 k_block_int(const KChunk<KVT>& k, int b) {
    if constexpr (KVT == QWA_KV_F16) {
        return make_h8(k.w[4 * b], k.w[4 * b + 1], k.w[4 * b + 2], k.w[4 * b + 3]);
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        uint32_t o[4];
        q8_word_int(k.w[2 * b], o);
        q8_word_int(k.w[2 * b + 1], o + 2);
        return make_h8(o[0], o[1], o[2], o[3]);
    } else {
        uint32_t o[4];
        q4_word_int(k.w[b], o);
        return make_h8(o[0], o[1], o[2], o[3]);
    }
}

__device__ __forceinline__ f4 mfma16k16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// One wave = one 256-key split x one 16-row tile.  Workgroup = SPW splits x RT row tiles (waves of the same split
// share the K/V lines through L1 / L2).  NBUF chunks are in flight per wave (register ring).
//
// Scores are exact up to fp32 accumulation: K enters the MFMA as the exact integer codes and its fp16 block scale is
// applied to each block's fp32 partial dot (one MFMA per 32-dim block); Q / 16 is split into fp16 hi + lo parts
// (two MFMAs), i.e. ~22 significant bits.  This keeps large (outlier) logits within tolerance where fp16(Q) and
// fp16(d * x) would not.
template <int KVT, int RT, int SPW, int NBUF>
__global__ void __launch_bounds__(64 * RT * SPW) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_dec(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int nsplit, float* __restrict__ work) {
    // Q / 16 hi and lo parts in A-operand order: [rt][block][hi, lo][lane] x 8 halves (16 KB per row tile)
    __shared__ h8 s_q[RT][8][2][64];
    __shared__ float s_t[RT * SPW][16][20];  // per-wave transpose of the 16 x 16 score tile
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i16 = lane & 15, lg = lane >> 4;
    const int g = blockIdx.y;
    const int kmax = pos0 + nq - 1;

    for (int e = threadIdx.x; e < RT * 8 * 64; e += 64 * RT * SPW) {
        const int rt = e >> 9, b = (e >> 6) & 7, ln = e & 63;
        const int r = 16 * rt + (ln & 15);
        const int qt = r / GRP, hh = r % GRP;
        h8 hi, lo;
        if (qt < nq) {
            const float* src = q + ((size_t)qt * NH + g * GRP + hh) * HD + 32 * b + 8 * (ln >> 4);
            const float4 a = *reinterpret_cast<const float4*>(src);
            const float4 c = *reinterpret_cast<const float4*>(src + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float v = x[k_perm<KVT>(j)] * 0.0625f;
                hi[j] = (_Float16)v;
                lo[j] = (_Float16)(v - (float)hi[j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) hi[j] = lo[j] = (_Float16)0.0f;
        }
        s_q[rt][b][0][ln] = hi;
        s_q[rt][b][1][ln] = lo;
    }
    __syncthreads();

    const int split = blockIdx.x * SPW + wave / RT;
    const int rt = wave % RT;
    if (split >= nsplit) return;
    // this lane's row in the S^T layout: query qt, head hh, last visible key qpos (-1: padding row)
    const int r = 16 * rt + i16;
    const int qt = r / GRP, hh = r % GRP;
    const int qpos = qt < nq ? pos0 + qt : -1;
    float (*tr)[20] = s_t[wave];

    f4 o[16];
#pragma unroll
    for (int dt = 0; dt < 16; dt++) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -INFINITY, l = 0.0f;

    const int k_begin = split * DEC_SPLIT;
    const int k_end = min(k_begin + DEC_SPLIT, kmax + 1);
    const size_t rowbase = (size_t)g * kv.capacity;
    Chunk<KVT> buf[NBUF];
#pragma unroll
    for (int b = 0; b < NBUF; b++)
        if (k_begin + 16 * b < k_end) load_chunk<KVT>(buf[b], kv, rowbase, k_begin + 16 * b, kmax, i16, lg);

    for (int kb0 = k_begin; kb0 < k_end; kb0 += 16 * NBUF) {
#pragma unroll
        for (int bi = 0; bi < NBUF; bi++) {
            const int kb = kb0 + 16 * bi;
            if (kb >= k_end) break;
            const Chunk<KVT>& c = buf[bi];

            // ---- S = Q K^T (16 rows x 16 keys): per block, (Q_hi + Q_lo) . K_int, scaled by the key's block scale
            f4 S = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const h8 kb8 = k_block_int<KVT>(c.k, b);
                f4 a = mfma16(s_q[rt][b][0][lane], kb8, f4{0.0f, 0.0f, 0.0f, 0.0f});
                a = mfma16(s_q[rt][b][1][lane], kb8, a);
                if constexpr (KVT == QWA_KV_F16) {
                    S += a;
                } else {
                    const float d = h2f_bits((uint16_t)(c.k.sc[b >> 1] >> (16 * (b & 1))));
#pragma unroll
                    for (int i = 0; i < 4; i++) S[i] = fmaf(d, a[i], S[i]);
                }
            }
            // lane (key i16, g) holds rows 4 g + i -> transpose through LDS to lane (row i16, g) holding keys 4 g + i
#pragma unroll
            for (int i = 0; i < 4; i++) tr[4 * lg + i][i16] = S[i];
            __builtin_amdgcn_wave_barrier();
            const float4 st = *reinterpret_cast<const float4*>(&tr[i16][4 * lg]);
            __builtin_amdgcn_wave_barrier();

            // ---- causal mask + online softmax: lane holds keys kb + 4 lg + i of its row
            const float sc4[4] = {st.x, st.y, st.z, st.w};
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[i] = kb + 4 * lg + i <= qpos ? sc4[i] : -INFINITY;
                mx = fmaxf(mx, sv[i]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m, mx);
            const float msl = (mn == -INFINITY ? 0.0f : mn) * LOG2E;  // a row that saw nothing keeps l = 0, O = 0
            const float cr = fast_exp2(m * LOG2E - msl);
            h4 p;
            float rs = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = fast_exp2(fmaf(sv[i], LOG2E, -msl));
                rs += e;
                p[i] = (_Float16)e;
            }
            l = l * cr + rs;
            m = mn;
            // rescale only when some row's max moved (multiplying by exactly 1 is the identity)
            if (__any(cr != 1.0f)) {
#pragma unroll
                for (int dt = 0; dt < 16; dt++) o[dt] *= cr;
            }

            // ---- O^T += V^T P^T: 16 dim tiles (lane dim 16 i16 + dt), keys 4 lg .. 4 lg + 3
            constexpr int NW = sizeof(c.v[0].w) / 4;  // raw words per 16 dims
            constexpr int DPW = 16 / NW;              // dims per raw word
#pragma unroll
            for (int wi = 0; wi < NW; wi++) {
                uint32_t w01[DPW], w23[DPW];
                v_pair_words<KVT, 1>(&c.v[0].w[wi], &c.v[1].w[wi], c.v[0].sc, c.v[1].sc, w01);
                v_pair_words<KVT, 1>(&c.v[2].w[wi], &c.v[3].w[wi], c.v[2].sc, c.v[3].sc, w23);
#pragma unroll
                for (int d = 0; d < DPW; d++) {
                    const int dt = wi * DPW + d;
                    o[dt] = mfma16k16(make_h4(w01[d], w23[d]), p, o[dt]);
                }
            }

            // ---- refill this slot with the chunk NBUF ahead
            const int kn = kb + 16 * NBUF;
            if (kn < k_end) load_chunk<KVT>(buf[bi], kv, rowbase, kn, kmax, i16, lg);
        }
    }

    // ---- partial record of the row: m, l (summed over the 4 lanes of the row), O at dims 64 lg + 16 i + dt
    float lt = l;
    lt += __shfl_xor(lt, 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    if (qpos < 0) return;
    float* rec = work + ((((size_t)split * NKV + g) * MAXQ + qt) * GRP + hh) * REC;
    if (lg == 0) {
        rec[0] = m;
        rec[1] = lt;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float* dst = rec + 4 + 64 * lg + 16 * i;
#pragma unroll
        for (int d4 = 0; d4 < 4; d4++)
            *reinterpret_cast<float4*>(dst + 4 * d4) =
                make_float4(o[4 * d4][i], o[4 * d4 + 1][i], o[4 * d4 + 2][i], o[4 * d4 + 3][i]);
    }
}

// Combine: one workgroup per (query t, head h, quarter of the head dims).  256 threads = 64 dims x 4 slices.
// Sums run over fixed groups of CGRP consecutive splits, in split order inside a group and in group order across
// groups: the summation tree depends only on split indices, never on nq (splits past a query's window hold l = 0
// and add exact zeros).
__global__ void __launch_bounds__(256) k_dec_combine(const float* __restrict__ work, int nsplit,
                                                     const float* __restrict__ gate, float* __restrict__ out,
                                                     float* __restrict__ out_host, qwa_act_q8 oq, int do_q) {
    constexpr int MAXSPLIT = MAX_POS / DEC_SPLIT + 1;
    constexpr int MAXGRP = (MAXSPLIT + CGRP - 1) / CGRP;
    __shared__ float s_f[MAXSPLIT];
    __shared__ float s_l[MAXSPLIT];
    __shared__ float s_red[8];
    __shared__ float s_gl[MAXGRP];
    __shared__ float s_ga[MAXGRP][64];
    const int t = blockIdx.x / NH, h = blockIdx.x % NH, g = h / GRP, hh = h % GRP;
    const int quarter = blockIdx.y;
    const int tid = threadIdx.x, dim = tid & 63, slice = tid >> 6;
    const size_t sstride = (size_t)NKV * MAXQ * GRP * REC;
    const float* base = work + (((size_t)g * MAXQ + t) * GRP + hh) * REC;

    // global max over splits that saw keys
    float mx = -INFINITY;
    for (int s = tid; s < nsplit; s += 256) {
        const float ls = base[s * sstride + 1];
        const float ms = base[s * sstride];
        s_l[s] = ls;
        s_f[s] = ms;
        if (ls > 0.0f) mx = fmaxf(mx, ms);
    }
    mx = wave_max(mx);
    if ((tid & 63) == 0) s_red[tid >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    for (int s = tid; s < nsplit; s += 256) s_f[s] = s_l[s] > 0.0f ? __expf(s_f[s] - M) : 0.0f;
    __syncthreads();

    const int ngrp = (nsplit + CGRP - 1) / CGRP;
    // group partial sums of l * f (one thread per group) and of O * f (slice per group, round robin)
    if (tid < ngrp) {
        float L = 0.0f;
        const int s1 = min(nsplit, (tid + 1) * CGRP);
        for (int s = tid * CGRP; s < s1; s++) L += s_l[s] * s_f[s];
        s_gl[tid] = L;
    }
    const int d = 64 * quarter + dim;
    for (int gr = slice; gr < ngrp; gr += 4) {
        float A = 0.0f;
        const int s1 = min(nsplit, (gr + 1) * CGRP);
#pragma unroll 8
        for (int s = gr * CGRP; s < s1; s++) A += base[s * sstride + 4 + d] * s_f[s];
        s_ga[gr][dim] = A;
    }
    __syncthreads();
    if (slice != 0) return;
    float L = 0.0f, A = 0.0f;
    for (int gr = 0; gr < ngrp; gr++) {
        L += s_gl[gr];
        A += s_ga[gr][dim];
    }
    const size_t o = ((size_t)t * NH + h) * HD + d;
    const float v = (A / L) * sigmoid(gate[o]);
    out[o] = v;
    if (out_host) {
        out_host[o] = v;
        __threadfence_system();
    }
    if (do_q) {
        // ActQ8 (src/cuda/common.cuh:188-197): d = amax/127, q = round-half-even(v/d), s = d * sum(q)
        const float amax = half_max(fabsf(v));
        const float db = amax / 127.0f;
        const int qi = db > 0.0f ? (int)__builtin_rintf(v / db) : 0;
        const size_t blk = ((size_t)t * NH * HD + (size_t)h * HD + d) >> 5;
        oq.q[o] = (int8_t)qi;
        const float sum = half_sum((float)qi);
        if ((dim & 31) == 0) {
            oq.d[blk] = db;
            oq.s[blk] = db * sum;
        }
    }
}

template <int KVT>
static void launch_dec_kvt(const float* q, const qwa_kv_layer& kv, int pos0, int nq, int nsplit, float* work,
                           hipStream_t st) {
    const int rt = (GRP * nq + 15) / 16;
    constexpr int NB = KVT == QWA_KV_Q4_0 ? 4 : KVT == QWA_KV_Q8_0 ? 2 : 1;
    if (rt == 1) {
        hipLaunchKernelGGL((k_dec<KVT, 1, 4, NB>), dim3((nsplit + 3) / 4, NKV), dim3(256), 0, st, q, kv, pos0, nq,
                           nsplit, work);
    } else if (rt == 2) {
        hipLaunchKernelGGL((k_dec<KVT, 2, 2, NB>), dim3((nsplit + 1) / 2, NKV), dim3(256), 0, st, q, kv, pos0, nq,
                           nsplit, work);
    } else {
        hipLaunchKernelGGL((k_dec<KVT, 3, 2, NB>), dim3((nsplit + 1) / 2, NKV), dim3(384), 0, st, q, kv, pos0, nq,
                           nsplit, work);
    }
}

hipError_t launch_decode(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int pos0, int nq,
                         void* work, float* out, const qwa_act_q8* oq, float* out_host, hipStream_t st) {
    const int nsplit = dec_nsplit(pos0 + nq - 1);
    float* w = static_cast<float*>(work);
    if (kvt == QWA_KV_F16) launch_dec_kvt<QWA_KV_F16>(q, kv, pos0, nq, nsplit, w, st);
    else if (kvt == QWA_KV_Q8_0) launch_dec_kvt<QWA_KV_Q8_0>(q, kv, pos0, nq, nsplit, w, st);
    else launch_dec_kvt<QWA_KV_Q4_0>(q, kv, pos0, nq, nsplit, w, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const qwa_act_q8 a = oq ? *oq : qwa_act_q8{nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_dec_combine, dim3(nq * NH, 4), dim3(256), 0, st, w, nsplit, gate, out, out_host, a,
                       oq != nullptr ? 1 : 0);
    return hipGetLastError();
}

}  // namespace qwa

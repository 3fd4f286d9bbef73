// Decode / speculative-verify attention over the quantized KV cache (gfx950).
//
// Split-K flash-decoding (the reference's structure, src/cuda/ops.cu:507-815, re-designed for wave64 + MFMA):
//  * rows are (query, head) pairs of one KV head, row r = 6 * query + head, in 16-row MFMA tiles
//    (RT = ceil(6 nq / 16) tiles); a wave owns one fixed 256-key split x one row tile, and the RT waves of a split
//    sit in the same workgroup so their K/V reads share L1 / L2;
//  * 16-key chunks: S^T = K Q^T on v_mfma_f32_16x16x32_f16 and O^T = V^T P^T on v_mfma_f32_16x16x16_f16, fp32
//    accumulation, Q pre-scaled by 1/16 (exact in fp16); K and V are read straight from HBM with 8/16-byte loads
//    and dequantized in registers; with S^T in the accumulator a lane holds 4 keys of ONE row, so the online
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

// Raw bytes of one 16-key chunk held by one lane: K of key kb + (lane % 16) (dims 64 g .. 64 g + 63) and V of keys
// kb + 4 g + j, j = 0..3 (dims 16 (lane % 16) .. + 15).
template <int KVT>
struct Chunk {
    KRaw<KVT> k;
    VRaw<KVT> v[4];
};

template <int KVT>
__device__ __forceinline__ void load_chunk(Chunk<KVT>& c, const qwa_kv_layer& kv, size_t rowbase, int kb, int kmax,
                                           int i16, int lg) {
    const int key = kb + i16;
    load_k<KVT>(c.k, kv, rowbase + key, lg, key <= kmax);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int vk = kb + 4 * lg + j;
        load_v<KVT>(c.v[j], kv, rowbase + vk, i16, vk <= kmax);
    }
}

__device__ __forceinline__ f4 mfma16k16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// One wave = one 256-key split x one 16-row tile.  Workgroup = SPW splits x RT row tiles (waves of the same split
// share the K/V lines through L1 / L2).  NBUF chunks are in flight per wave (register ring).
template <int KVT, int RT, int SPW, int NBUF>
__global__ void __launch_bounds__(64 * RT * SPW) __attribute__((amdgpu_waves_per_eu(2, 2))) k_dec(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq,
                                                       int nsplit, float* __restrict__ work) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int split = blockIdx.x * SPW + wave / RT;
    const int rt = wave % RT;
    if (split >= nsplit) return;
    const int g = blockIdx.y;
    const int i16 = lane & 15, lg = lane >> 4;
    const int kmax = pos0 + nq - 1;

    // this lane's row: query qt, head hh, last visible key qpos (-1: padding row)
    const int r = 16 * rt + i16;
    const int qt = r / GRP, hh = r % GRP;
    const bool valid = qt < nq;
    const int qpos = valid ? pos0 + qt : -1;
    h8 qb[8];
    {
        const float* qrow = q + ((size_t)(valid ? qt : 0) * NH + g * GRP + hh) * HD + 64 * lg;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float4 a = *reinterpret_cast<const float4*>(qrow + 8 * s);
            const float4 b = *reinterpret_cast<const float4*>(qrow + 8 * s + 4);
            const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            h8 v;
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = valid ? (_Float16)(x[k_perm<KVT>(j)] * 0.0625f) : (_Float16)0.0f;
            qb[s] = v;
        }
    }

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
        for (int b = 0; b < NBUF; b++) {
            const int kb = kb0 + 16 * b;
            if (kb >= k_end) break;
            const Chunk<KVT>& c = buf[b];

            // ---- S^T = K Q^T (16 keys x 16 rows), two accumulation chains
            f4 s0 = f4{0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0;
#pragma unroll
            for (int s = 0; s < 8; s += 2) {
                s0 = mfma16(k_operand<KVT>(c.k, s), qb[s], s0);
                s1 = mfma16(k_operand<KVT>(c.k, s + 1), qb[s + 1], s1);
            }
            const f4 sc = s0 + s1;

            // ---- causal mask + online softmax: lane holds keys kb + 4 lg + i of its row
            float sv[4];
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sv[i] = kb + 4 * lg + i <= qpos ? sc[i] : -INFINITY;
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
            if (kn < k_end) load_chunk<KVT>(buf[b], kv, rowbase, kn, kmax, i16, lg);
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

// Gated DeltaNet token mixer (gfx950): the recurrent layers that sit between the gated-attention layers.
//
// Per token and value head h (key head h % 16): causal depthwise conv (width 4) + SiLU over the q | k | v channels,
// L2-normalised q and k, beta = sigmoid(b), decay = exp(softplus(a + dt_bias) * A), then the gated delta rule on the
// 128 x 128 state S (column j = value dim, row i = key dim):
//     S <- decay S;  kv = S^T k;  S <- S + k ((v - kv) beta)^T;  o = S^T q / sqrt(128)
// and the gated RMSNorm rmsnorm(o) * ssm_norm * silu(z).  Semantics: src/reference/ref_model.cpp:169-256 (CPU, FP32);
// entry points and state conventions: src/cuda/ops.cuh:54-97 (decode, lazy commit), src/cuda/prefill.cuh:37-44
// (prefill rows).
//
// Decode / verify (k_dn_head): one workgroup of 16 waves per value head holds the head's 64 KB state in registers
// (8 lanes per column), loaded and stored with 128 contiguous bytes per column per instruction.  All of a chunk's
// inputs are loaded up front in one round trip; the conv and the per-token scalars (norms, q.k, beta, decay) are
// computed before the sequential delta rule, which then runs without barriers; the gated RMSNorm, ActQ8 and the
// mapped-host copy finish inside the same kernel.  Tokens are applied one after the other with the same code, so a
// token sequence gives the same bits however it is split into calls (the lazy-commit contract,
// src/cuda/ops.cuh:93-95).
//
// Prefill (B tokens): token-parallel conv, conv-window and q/k-normalisation kernels, the sequential recurrence over
// (48 heads x 8 groups of 16 columns) with the tokens' q / k / v staged in LDS, and the gated norm to fp16.
#include <type_traits>

#include "launch.hpp"
#include "qwattn_common.hpp"

namespace qwa {

constexpr int DN_CH = 10240;  // conv channels: q (16 x 128) | k (16 x 128) | v (48 x 128)
constexpr int DN_QK = 2048;
constexpr int DN_HD = 128;
constexpr int DN_KH = 16;
constexpr int DN_VH = 48;
constexpr int DN_VD = DN_VH * DN_HD;  // 6144
constexpr int DN_BA_LD = 64;          // row stride of the decode path's beta / alpha inputs

__device__ __forceinline__ float dn_silu(float x) { return x / (1.0f + __expf(-x)); }
// ------------------------------------------------------------------------------------------------------- decode
constexpr int DN_TC = 8;  // tokens per chunk

// DPP lane moves within a row of 16 lanes (no LDS round trip)
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// sum over the 16 lanes of a DPP row: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror (lane i <-> 7 - i),
// row_mirror (lane i <-> 15 - i).  Every lane gets the same bits (each step adds the same two values, swapped).
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_mov<0xB1>(x);
    x += dpp_mov<0x4E>(x);
    x += dpp_mov<0x141>(x);
    return x + dpp_mov<0x140>(x);
}

// a0 . b0 + a1 . b1 over 8 values, as two interleaved fma chains
__device__ __forceinline__ float dot8(float4 a0, float4 a1, float4 b0, float4 b1) {
    float x = a0.x * b0.x, y = a0.y * b0.y;
    x = fmaf(a0.z, b0.z, x);
    y = fmaf(a0.w, b0.w, y);
    x = fmaf(a1.x, b1.x, x);
    y = fmaf(a1.y, b1.y, y);
    x = fmaf(a1.z, b1.z, x);
    y = fmaf(a1.w, b1.w, y);
    return x + y;
}

// k_dn_head: one workgroup of 16 waves per value head (48 workgroups), the whole call in one kernel.  Lane
// (column j = t / 8, r8 = t % 8) holds the row quads r8, r8 + 8, r8 + 16, r8 + 24 of its column; the dot products
// reduce over 8 lanes.  Per chunk of DN_TC tokens: (1) the chunk's inputs (branch-free addresses, one round trip) and the conv
// over the 384 channels of the head, beta / decay, the gate inputs z; (2) |q|^2, |k|^2, q.k; (3) the delta rule;
// (4) the gated RMSNorm of the chunk's new tokens over the head's 128 outputs, ActQ8 and the mapped-host copy.
constexpr int DN_HT = 1024;          // threads of k_dn_head

// sum over 8 aligned lanes (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror); same bits in every lane
__device__ __forceinline__ float oct_sum(float x) {
    x += dpp_mov<0xB1>(x);
    x += dpp_mov<0x4E>(x);
    return x + dpp_mov<0x141>(x);
}

__global__ void __launch_bounds__(DN_HT) k_dn_head(qwa_dn_params p, int cin, qwa_dn_tokens in, int n_commit,
                                                   int n_new, int write_after, float eps, float* __restrict__ o,
                                                   qwa_act_q8 oq, int do_q) {
    const int h = blockIdx.x, kh = h % DN_KH, t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    __shared__ __attribute__((aligned(16))) float s_q[DN_TC][DN_HD], s_k[DN_TC][DN_HD];
    __shared__ __attribute__((aligned(16))) float s_sc[DN_TC][8];
    __shared__ float s_v[DN_TC][DN_HD], s_o[DN_TC][DN_HD], s_beta[DN_TC], s_decay[DN_TC], s_red[DN_TC][2];
    const float* cs_in = p.conv_state + (size_t)cin * 3 * DN_CH;
    float* cs_out = p.conv_state + (size_t)(cin ^ 1) * 3 * DN_CH;
    constexpr int NCONV = 3 * DN_HD;  // conv threads: q, k of key head kh, v of head h

    // conv channel of threads < 384 (the others hold a valid copy of channel t % 384 and never use it)
    const int tc = t % NCONV;
    const int c = tc < DN_HD ? kh * DN_HD + tc : tc < 2 * DN_HD ? DN_QK + kh * DN_HD + (tc - DN_HD)
                                                              : 2 * DN_QK + h * DN_HD + (tc - 2 * DN_HD);
    const bool conv_thread = t < NCONV;
    // the q / k channels are shared by value heads kh, kh + 16, kh + 32: only the first writes them back
    const bool owner = conv_thread && (tc >= 2 * DN_HD || h < DN_KH);
    float x0 = 0.0f, x1 = 0.0f, x2 = 0.0f;
    float4 w = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (conv_thread) {
        x0 = cs_in[c];
        x1 = cs_in[DN_CH + c];
        x2 = cs_in[2 * DN_CH + c];
        w = *reinterpret_cast<const float4*>(p.conv_w + (size_t)c * 4);
    }
    const float dtb = p.dt_bias[h], sa = p.ssm_a[h];
    const int jn = t & (DN_HD - 1);  // output column of the gated norm
    const float nw = p.ssm_norm[jn];

    // this lane's 16 state values: column j, the row quads r8, r8 + 8, r8 + 16, r8 + 24 (global layout [h][j][i]),
    // so that each load or store instruction covers 128 contiguous bytes per column
    const int j = t >> 3, r8 = t & 7;
    float* Sh = p.ssm_state + (size_t)h * DN_HD * DN_HD;
    float4* Sq = reinterpret_cast<float4*>(Sh + (size_t)j * DN_HD) + r8;
    float s[16];
    {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float4 v = Sq[8 * r];
            s[4 * r] = v.x; s[4 * r + 1] = v.y; s[4 * r + 2] = v.z; s[4 * r + 3] = v.w;
        }
    }
    const float oscale = 1.0f / sqrtf((float)DN_HD);
    const int ntot = n_commit + n_new;

    for (int t0 = 0; t0 < ntot; t0 += DN_TC) {
        const int nt = min(DN_TC, ntot - t0);
        // 1) inputs.  Conv threads: the chunk's qkv channel values (pending tokens from the save buffer, new ones
        //    from qkv or, for channels >= qkv_split, mapped host memory), addresses selected rather than branched on
        //    so that all loads are in flight together.  Every thread: z of (token t / 128, column t % 128).
        float zv;
        {
            const int tt = t >> 7, i = t0 + tt, ni = i - n_commit, zi = h * DN_HD + jn;
            const bool use = tt < nt && i >= n_commit;
            const float* pz = zi >= in.z_split ? in.z_host + (size_t)ni * in.z_ld + (zi - in.z_split)
                                               : in.z + (size_t)ni * DN_VD + zi;
            zv = *(use ? pz : p.ssm_norm + jn);
        }
        if (conv_thread) {
            float xa[DN_TC];
#pragma unroll
            for (int tt = 0; tt < DN_TC; tt++) {
                const int i = t0 + tt, ni = i - n_commit;
                const float* pa = i < n_commit ? in.sqkv + (size_t)i * DN_CH + c
                                  : c >= in.qkv_split ? in.qkv_host + (size_t)ni * in.qkv_ld + (c - in.qkv_split)
                                                      : in.qkv + (size_t)ni * DN_CH + c;
                xa[tt] = *(tt < nt ? pa : cs_in + c);
            }
            // causal conv + SiLU, the window sliding per thread; saves and the window at the commit point
#pragma unroll
            for (int tt = 0; tt < DN_TC; tt++) {
                if (tt < nt) {
                    const int i = t0 + tt;
                    const float val = dn_silu(fmaf(w.w, xa[tt], fmaf(w.z, x2, fmaf(w.y, x1, w.x * x0))));
                    x0 = x1; x1 = x2; x2 = xa[tt];
                    if (tc < DN_HD) s_q[tt][tc] = val;
                    else if (tc < 2 * DN_HD) s_k[tt][tc - DN_HD] = val;
                    else s_v[tt][tc - 2 * DN_HD] = val;
                    if (owner) {
                        if (i >= n_commit && in.oqkv) in.oqkv[(size_t)(i - n_commit) * DN_CH + c] = xa[tt];
                        if (i == write_after - 1) {
                            cs_out[c] = x0;
                            cs_out[DN_CH + c] = x1;
                            cs_out[2 * DN_CH + c] = x2;
                        }
                    }
                }
            }
        } else if (wave == DN_HT / 64 - 1 && lane < nt) {  // beta and decay of token t0 + lane
            const int i = t0 + lane;
            const bool is_new = i >= n_commit;
            const float* brow = is_new ? in.beta + (i - n_commit) * DN_BA_LD : in.sbeta + i * DN_BA_LD;
            const float* arow = is_new ? in.alpha + (i - n_commit) * DN_BA_LD : in.salpha + i * DN_BA_LD;
            const float br = brow[h], ar = arow[h];
            const float x = ar + dtb;
            const float sp = x > 20.0f ? x : logf(1.0f + expf(x));
            s_beta[lane] = 1.0f / (1.0f + expf(-br));
            s_decay[lane] = expf(sp * sa);
            if (is_new && in.obeta) {
                in.obeta[(i - n_commit) * DN_BA_LD + h] = br;
                in.oalpha[(i - n_commit) * DN_BA_LD + h] = ar;
            }
        }
        __syncthreads();
        // 2) per token: |q|^2, |k|^2 and q.k (16 lanes, 8 elements each), folded into the scalars of step 3
        if (t < 16 * DN_TC) {
            const int tt = t >> 4, r16 = t & 15;
            if (tt < nt) {
                const int e = 8 * r16;
                const float4 q0 = *reinterpret_cast<const float4*>(&s_q[tt][e]);
                const float4 q1 = *reinterpret_cast<const float4*>(&s_q[tt][e + 4]);
                const float4 k0 = *reinterpret_cast<const float4*>(&s_k[tt][e]);
                const float4 k1 = *reinterpret_cast<const float4*>(&s_k[tt][e + 4]);
                const float qq = row16_sum(dot8(q0, q1, q0, q1));
                const float kk = row16_sum(dot8(k0, k1, k0, k1));
                const float kq = row16_sum(dot8(k0, k1, q0, q1));
                if (r16 == 0) {
                    const float qs = 1.0f / fmaxf(sqrtf(qq), eps), ks = 1.0f / fmaxf(sqrtf(kk), eps);
                    const float decay = s_decay[tt], beta = s_beta[tt];
                    *reinterpret_cast<float4*>(&s_sc[tt][0]) =
                        make_float4(decay, decay * ks, beta * ks, qs * oscale * decay);
                    s_sc[tt][4] = qs * oscale * kq;
                }
            }
        }
        __syncthreads();
        // 3) the gated delta rule, token after token, on this lane's 16 state values, in the form
        //      sk = S^T k_raw, sq = S^T q_raw (old state; both reductions run interleaved)
        //      dk = (v - decay ks sk) beta ks,  o = qs / sqrt(128) (decay sq + (q.k) dk),  S = decay S + k_raw dk
        //    which equals S <- decay S; S += k ((v - S^T k) beta)^T; o = S^T q / sqrt(128) with unit q, k.
        for (int tt = 0; tt < nt; tt++) {
            const float4* kp = reinterpret_cast<const float4*>(&s_k[tt][0]) + r8;  // quad r8 + 8 r at kp[8 r]
            const float4* qp = reinterpret_cast<const float4*>(&s_q[tt][0]) + r8;
            const float4 cc = *reinterpret_cast<const float4*>(&s_sc[tt][0]);
            const float c2 = s_sc[tt][4], v = s_v[tt][j];
            float ka = 0.0f, kb = 0.0f, qa = 0.0f, qb = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float4 k4 = kp[8 * r], q4 = qp[8 * r];
                ka = fmaf(s[4 * r], k4.x, ka);
                kb = fmaf(s[4 * r + 1], k4.y, kb);
                qa = fmaf(s[4 * r], q4.x, qa);
                qb = fmaf(s[4 * r + 1], q4.y, qb);
                ka = fmaf(s[4 * r + 2], k4.z, ka);
                kb = fmaf(s[4 * r + 3], k4.w, kb);
                qa = fmaf(s[4 * r + 2], q4.z, qa);
                qb = fmaf(s[4 * r + 3], q4.w, qb);
            }
            const float sk = oct_sum(ka + kb), sq = oct_sum(qa + qb);
            const float dk = fmaf(-cc.y, sk, v) * cc.z;
            const float oj = fmaf(cc.w, sq, c2 * dk);
#pragma unroll
            for (int r = 0; r < 4; r++) {  // k read again from LDS rather than held in 16 more registers
                const float4 k4 = kp[8 * r];
                s[4 * r] = fmaf(k4.x, dk, s[4 * r] * cc.x);
                s[4 * r + 1] = fmaf(k4.y, dk, s[4 * r + 1] * cc.x);
                s[4 * r + 2] = fmaf(k4.z, dk, s[4 * r + 2] * cc.x);
                s[4 * r + 3] = fmaf(k4.w, dk, s[4 * r + 3] * cc.x);
            }
            if (r8 == 0) s_o[tt][j] = oj;
            if (t0 + tt == write_after - 1) {  // the state at the commit point, in place
#pragma unroll
                for (int r = 0; r < 4; r++) Sq[8 * r] = make_float4(s[4 * r], s[4 * r + 1], s[4 * r + 2], s[4 * r + 3]);
            }
        }
        __syncthreads();
        // 4) gated RMSNorm of the chunk's new tokens: thread (token t / 128, column t % 128)
        const int tt = t >> 7, i = t0 + tt;
        const bool emit = tt < nt && i >= n_commit;
        const float y0 = s_o[tt][jn];
        const float ss = wave_sum(y0 * y0);
        if (lane == 0) s_red[tt][wave & 1] = ss;
        __syncthreads();
        if (emit) {
            const float rs = 1.0f / sqrtf((s_red[tt][0] + s_red[tt][1]) / DN_HD + eps);
            const float y = y0 * rs * nw * dn_silu(zv);
            const size_t oi = (size_t)(i - n_commit) * DN_VD + h * DN_HD + jn;
            o[oi] = y;
            if (in.o_host) in.o_host[oi] = y;
            if (do_q) {
                // ActQ8 (src/cuda/common.cuh:188-197) per 32 outputs: d = amax / 127, q = rint(y / d), s = d sum(q)
                const float amax = half_max(fabsf(y));
                const float db = amax / 127.0f;
                const int qi = db > 0.0f ? (int)__builtin_rintf(y / db) : 0;
                oq.q[oi] = (int8_t)qi;
                const float qsum = half_sum((float)qi);
                if ((lane & 31) == 0) {
                    oq.d[oi / 32] = db;
                    oq.s[oi / 32] = db * qsum;
                }
            }
        }
        // the next chunk rewrites s_q .. s_o only after every thread has passed this point
        __syncthreads();
    }
    if (in.o_host) __threadfence_system();
}

// ------------------------------------------------------------------------------------------------------ prefill
constexpr int DN_CT = 16;      // tokens per chunk of the chunked recurrence
#ifndef QWA_DN_CW
#define QWA_DN_CW 4
#endif
constexpr int DN_CW = QWA_DN_CW;        // waves per workgroup of the chunked recurrence (key dims split over them)
constexpr int DN_TPW = 8 / DN_CW;       // 16-row key-dim tiles of the state per wave
constexpr int DN_CP = 20;      // padded row (floats) of the transposed chunk tiles in LDS
constexpr int DN_NCOEF = 704;  // per (chunk, head): T^T [16][20] | P^T [16][20] | gamma | E | c1 | c2
struct DnRows {
    float* conv;   // [B][10240] after SiLU (only the v channels, 4096 .. 10239, are written)
    float* qn;     // [B][2048] L2-normalised q
    float* kn;     // [B][2048] L2-normalised k
    float* beta;   // [B][48]
    float* decay;  // [B][48]
    float* coef;   // [ceil(B / 16)][48][DN_NCOEF] per-chunk coefficients (k_dn_chunk_prep)
};

__host__ __device__ inline DnRows dn_rows_split(void* work, int B) {
    float* f = static_cast<float*>(work);
    DnRows r;
    r.conv = f;
    f += (size_t)B * DN_CH;
    r.qn = f;
    f += (size_t)B * DN_QK;
    r.kn = f;
    f += (size_t)B * DN_QK;
    r.beta = f;
    f += (size_t)B * DN_VH;
    r.decay = f;
    f += (size_t)B * DN_VH;
    r.coef = f;
    return r;
}

size_t dn_work_bytes(int B) {
    return ((size_t)B * (DN_CH + 2 * DN_QK + 2 * DN_VH) + (size_t)((B + DN_CT - 1) / DN_CT) * DN_VH * DN_NCOEF) *
           sizeof(float);
}

// Per channel c and run of DN_CR consecutive tokens (grid (DN_CH / 256, ceil(B / DN_CR))): conv[t][c] =
// silu(sum_k w[c][k] in(t - 3 + k)), in(i) = qkv[i][c] for i >= 0, else row 3 + i of the old window.  A thread
// slides the 4-tap window over its run, so each input row is read once per run instead of once per tap.  The q and
// k channels (blocks x < 16, two heads of 128 each) are not written out: the block L2-normalises its heads through
// LDS (wave w: the (token, head) pairs w, w + 4, ..., lane holding dims lane and lane + 64) into qn / kn.  Blocks
// x = 0 also write beta and the decay of their tokens, and the run holding token B - 1 writes the window after the
// chunk (rows k = input B - 3 + k) into the other buffer.  Only the v channels reach r.conv.
constexpr int DN_CR = 8;  // tokens per thread of k_dn_conv_rows
__global__ void __launch_bounds__(256) k_dn_conv_rows(const float* __restrict__ qkv, const float* __restrict__ cs_old,
                                                      const float* __restrict__ conv_w, DnRows r,
                                                      const float* __restrict__ beta_raw,
                                                      const float* __restrict__ alpha_raw,
                                                      const float* __restrict__ dt_bias,
                                                      const float* __restrict__ ssm_a, float eps, int B,
                                                      float* __restrict__ cs_new) {
    __shared__ float sx[DN_CR][256];
    const int t0 = blockIdx.y * DN_CR, c = blockIdx.x * 256 + threadIdx.x;
    const int nt = min(DN_CR, B - t0);
    const float4 w = *reinterpret_cast<const float4*>(conv_w + (size_t)c * 4);
    float x[DN_CR + 3];
#pragma unroll
    for (int k = 0; k < DN_CR + 3; k++) {
        const int i = t0 - 3 + k;
        x[k] = i < 0 ? cs_old[(size_t)(3 + i) * DN_CH + c] : i < B ? qkv[(size_t)i * DN_CH + c] : 0.0f;
    }
    if (t0 + DN_CR >= B) {
        // the window after the chunk: inputs B - 3 .. B - 1 (x[B - t0 .. B - t0 + 2])
#pragma unroll
        for (int k = 0; k < DN_CR + 3; k++) {
            const int i = t0 - 3 + k, kk = i - (B - 3);
            if (kk >= 0 && kk < 3) cs_new[(size_t)kk * DN_CH + c] = x[k];
        }
    }
    float y[DN_CR];
#pragma unroll
    for (int u = 0; u < DN_CR; u++) y[u] = dn_silu(w.x * x[u] + w.y * x[u + 1] + w.z * x[u + 2] + w.w * x[u + 3]);
    if (c >= 2 * DN_QK) {
#pragma unroll
        for (int u = 0; u < DN_CR; u++)
            if (u < nt) r.conv[(size_t)(t0 + u) * DN_CH + c] = y[u];
        return;
    }
#pragma unroll
    for (int u = 0; u < DN_CR; u++) sx[u][threadIdx.x] = y[u];
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int pr = wave; pr < 2 * nt; pr += 4) {
        const int u = pr >> 1, hw = pr & 1;
        const int hc = 2 * blockIdx.x + hw;  // head of the q | k channels: q heads 0 .. 15, then k heads 0 .. 15
        const float v0 = sx[u][128 * hw + lane], v1 = sx[u][128 * hw + lane + 64];
        const float iv = 1.0f / fmaxf(sqrtf(wave_sum(v0 * v0 + v1 * v1)), eps);
        float* d = (hc < DN_KH ? r.qn + hc * DN_HD : r.kn + (hc - DN_KH) * DN_HD) + (size_t)(t0 + u) * DN_QK;
        d[lane] = v0 * iv;
        d[lane + 64] = v1 * iv;
    }
    if (blockIdx.x == 0) {
        for (int e = threadIdx.x; e < nt * DN_VH; e += 256) {
            const int t = t0 + e / DN_VH, h = e % DN_VH;
            const float a = alpha_raw[(size_t)t * DN_VH + h] + dt_bias[h];
            const float sp = a > 20.0f ? a : logf(1.0f + expf(a));
            r.beta[(size_t)t * DN_VH + h] = 1.0f / (1.0f + expf(-beta_raw[(size_t)t * DN_VH + h]));
            r.decay[(size_t)t * DN_VH + h] = expf(sp * ssm_a[h]);
        }
    }
}

constexpr int DN_RG = 8;               // workgroups (column groups) per head of the chunked recurrence
constexpr int DN_RC = DN_HD / DN_RG;   // 16 value columns per workgroup

// ---- the chunked recurrence (prefill).  For a chunk of 16 tokens with S the state before it, decays g, write
// strengths beta, G(s, t) = g_{s+1} ... g_t and gamma_t = g_0 ... g_t, the per-token rule
//     S <- g S;  u = beta (v - S^T k);  S += k u^T;  o = S^T q
// unrolls to
//     a_t = S^T k_t, b_t = S^T q_t
//     (I + L) U = W,  L[t][s] = beta_t G(s, t) k_s.k_t (s < t),  W_t = beta_t v_t - beta_t gamma_t a_t
//     o_t = gamma_t b_t + sum_{s<=t} G(s, t) (k_s.q_t) u_s
//     S'  = gamma_15 S + sum_s G(s, 15) k_s u_s^T.
// The value dims are independent columns, so a workgroup owns 16 of them.  k_dn_chunk_prep computes, per (head,
// chunk), T = (I + L)^-1, P = M' T with M'[t][s] = G(s, t) k_s.q_t, and the token scalars, so that U = T W and
// O = gamma b + P W are independent; k_dn_chunk_rows keeps its 128 x 16 slice of
// S in fp32 MFMA accumulators and applies a chunk as matrix products on v_mfma_f32_16x16x4_f32: K S and Q S (split over
// the waves by key dims, summed through LDS), U = T W, O = gamma b + P W and the rank-16 state update.  Tokens past
// B are padded with k = q = v = 0, beta = 0, g = 1, which change nothing.
__device__ __forceinline__ f4 mfma4f32(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ void __launch_bounds__(256) k_dn_chunk_prep(DnRows r, int B) {
    const int h = blockIdx.x, c = blockIdx.y, kh = h % DN_KH, t = threadIdx.x;
    __shared__ float sk[DN_CT][DN_HD + 4], sq[DN_CT][DN_HD + 4];
    __shared__ float sg[DN_CT], sb[DN_CT], sL[DN_CT][DN_CT + 1], sM[DN_CT][DN_CT + 1], sT[DN_CT][DN_CT + 1];
    for (int e = t; e < DN_CT * (DN_HD / 4); e += 256) {
        const int tok = e >> 5, f = e & 31, i = c * DN_CT + tok, ii = min(i, B - 1);
        const float4 kv = *reinterpret_cast<const float4*>(r.kn + (size_t)ii * DN_QK + kh * DN_HD + 4 * f);
        const float4 qv = *reinterpret_cast<const float4*>(r.qn + (size_t)ii * DN_QK + kh * DN_HD + 4 * f);
        const bool in = i < B;
        sk[tok][4 * f] = in ? kv.x : 0.0f; sk[tok][4 * f + 1] = in ? kv.y : 0.0f;
        sk[tok][4 * f + 2] = in ? kv.z : 0.0f; sk[tok][4 * f + 3] = in ? kv.w : 0.0f;
        sq[tok][4 * f] = in ? qv.x : 0.0f; sq[tok][4 * f + 1] = in ? qv.y : 0.0f;
        sq[tok][4 * f + 2] = in ? qv.z : 0.0f; sq[tok][4 * f + 3] = in ? qv.w : 0.0f;
    }
    if (t < DN_CT) {
        const int i = c * DN_CT + t, ii = min(i, B - 1);
        const float gd = r.decay[(size_t)ii * DN_VH + h], bt = r.beta[(size_t)ii * DN_VH + h];
        sg[t] = i < B ? gd : 1.0f;
        sb[t] = i < B ? bt : 0.0f;
    }
    __syncthreads();
    float* cf = r.coef + ((size_t)c * DN_VH + h) * DN_NCOEF;
    {
        // thread (s, u): the Gram entries k_s.k_u and k_s.q_u, L[u][s] and M'[u][s]
        const int s = t >> 4, u = t & 15;
        float kk0 = 0.0f, kk1 = 0.0f, kq0 = 0.0f, kq1 = 0.0f;
#pragma unroll 8
        for (int i = 0; i < DN_HD; i += 2) {
            kk0 = fmaf(sk[s][i], sk[u][i], kk0);
            kk1 = fmaf(sk[s][i + 1], sk[u][i + 1], kk1);
            kq0 = fmaf(sk[s][i], sq[u][i], kq0);
            kq1 = fmaf(sk[s][i + 1], sq[u][i + 1], kq1);
        }
        float G = 1.0f;
        for (int e = s + 1; e <= u; e++) G *= sg[e];
        sL[u][s] = s < u ? sb[u] * G * (kk0 + kk1) : 0.0f;
        sM[u][s] = s <= u ? G * (kq0 + kq1) : 0.0f;
    }
    __syncthreads();
    if (t < DN_CT) {
        // column s = t of T = (I + L)^-1 by forward substitution: T[u][s] = [u == s] - sum_{r<u} L[u][r] T[r][s]
        const int s = t;
        float x[DN_CT];
#pragma unroll
        for (int u = 0; u < DN_CT; u++) {
            float acc = u == s ? 1.0f : 0.0f;
#pragma unroll
            for (int q = 0; q < u; q++) acc = fmaf(-sL[u][q], x[q], acc);
            x[u] = u < s ? 0.0f : acc;
        }
#pragma unroll
        for (int u = 0; u < DN_CT; u++) {
            cf[s * DN_CP + u] = x[u];  // T^T[s][u] = T[u][s]
            sT[u][s] = x[u];
        }
        float gam = 1.0f, E = 1.0f;
        for (int e = 0; e <= t; e++) gam *= sg[e];
        for (int e = t + 1; e < DN_CT; e++) E *= sg[e];
        cf[640 + t] = gam;
        cf[656 + t] = E;
        cf[672 + t] = sb[t];
        cf[688 + t] = sb[t] * gam;
    }
    __syncthreads();
    {
        // P = M' T (so that O = gamma b + P W needs no U): P^T[s][u] = sum_{s<=x<=u} M'[u][x] T[x][s]
        const int s = t >> 4, u = t & 15;
        float acc = 0.0f;
        for (int x = s; x <= u; x++) acc = fmaf(sM[u][x], sT[x][s], acc);
        cf[320 + s * DN_CP + u] = acc;
    }
}

// One chunk of k_dn_chunk_rows on its staged operands (see above).  st: this lane's 8 state values, updated.
__device__ __forceinline__ void dn_chunk_step(float (*KT)[DN_CP], float (*QT)[DN_CP], float (*V)[DN_RC],
                                              const float* C, float (*Red)[2][DN_CT][DN_CP], f4* st, int w, int l16,
                                              int g4, int c, int B, int h, int grp, float oscale,
                                              float* __restrict__ core_out) {
    // 1) partial a = K S and b = Q S over this wave's key dims: A[t][i] = K[t][i], B[i][j] = S[i][j]
    f4 pa = f4{0.0f, 0.0f, 0.0f, 0.0f}, pb = pa;
#pragma unroll
    for (int m = 0; m < DN_TPW; m++)
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const int i = 16 * (DN_TPW * w + m) + 4 * g4 + rr;
            pa = mfma4f32(KT[i][l16], st[m][rr], pa);
            pb = mfma4f32(QT[i][l16], st[m][rr], pb);
        }
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        Red[w][0][4 * g4 + rr][l16] = pa[rr];
        Red[w][1][4 * g4 + rr][l16] = pb[rr];
    }
    __syncthreads();
    float a[4], b[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
        const int tt = 4 * g4 + rr;
        float x = Red[0][0][tt][l16], y = Red[0][1][tt][l16];
#pragma unroll
        for (int v = 1; v < DN_CW; v++) {
            x += Red[v][0][tt][l16];
            y += Red[v][1][tt][l16];
        }
        a[rr] = x;
        b[rr] = y;
    }
    // 2) U = T W and O = gamma b + P W with W[s][j] = c1_s v_s - c2_s a_s (this lane: s = 4 g4 + q; A operands
    //    T[t][s] = T^T[s][t], P[t][s] = P^T[s][t] with t = l16)
    f4 U = f4{0.0f, 0.0f, 0.0f, 0.0f}, O;
#pragma unroll
    for (int rr = 0; rr < 4; rr++) O[rr] = C[640 + 4 * g4 + rr] * b[rr];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int s = 4 * g4 + q;
        const float Wv = fmaf(C[672 + s], V[s][l16], -C[688 + s] * a[q]);
        U = mfma4f32(C[s * DN_CP + l16], Wv, U);
        O = mfma4f32(C[320 + s * DN_CP + l16], Wv, O);
    }
    if (w == 0) {
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const int tok = c * DN_CT + 4 * g4 + rr;
            if (tok < B) core_out[(size_t)tok * DN_VD + h * DN_HD + grp * DN_RC + l16] = O[rr] * oscale;
        }
    }
    // 4) S = gamma_15 S + K^T (E U): A[i][s] = K[s][i], B[s][j] = E_s U[s][j]
    const float g15 = C[640 + DN_CT - 1];
#pragma unroll
    for (int m = 0; m < DN_TPW; m++) {
        f4 acc = st[m] * g15;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int s = 4 * g4 + q;
            acc = mfma4f32(KT[16 * (DN_TPW * w + m) + l16][s], C[656 + s] * U[q], acc);
        }
        st[m] = acc;
    }
}

__global__ void __launch_bounds__(DN_CW * 64) __attribute__((amdgpu_waves_per_eu(DN_CW / 2, DN_CW / 2)))
k_dn_chunk_rows(DnRows r, float* __restrict__ state, int B,
                                                       float* __restrict__ core_out) {
    const int h = blockIdx.x, grp = blockIdx.y, kh = h % DN_KH, t = threadIdx.x;
    const int w = t >> 6, l = t & 63, g4 = l >> 4, l16 = l & 15;
    __shared__ __attribute__((aligned(16))) float sKT[2][DN_HD][DN_CP], sQT[2][DN_HD][DN_CP];
    __shared__ float sV[2][DN_CT][DN_RC];
    __shared__ __attribute__((aligned(16))) float sC[2][DN_NCOEF];
    // the waves' partial K S / Q S; one buffer: the next chunk writes it only after the barrier that ends this one
    __shared__ float sRed[DN_CW][2][DN_CT][DN_CP];
    // this lane's state: key-dim tiles m = DN_TPW w .. DN_TPW w + DN_TPW - 1, S[16 m + 4 g4 + rr][grp * 16 + l16]
    const int j = grp * DN_RC + l16;
    float* Sj = state + (size_t)h * DN_HD * DN_HD + (size_t)j * DN_HD;
    f4 st[DN_TPW];
#pragma unroll
    for (int m = 0; m < DN_TPW; m++) {
        const float4 v = *reinterpret_cast<const float4*>(Sj + 16 * (DN_TPW * w + m) + 4 * g4);
        st[m] = f4{v.x, v.y, v.z, v.w};
    }
    const float oscale = 1.0f / sqrtf((float)DN_HD);
    const int nch = (B + DN_CT - 1) / DN_CT;
    // staging: thread (token t % 16, f = t / 16) moves k / q dims DN_SD f .. DN_SD f + DN_SD - 1 (transposed; tokens
    // past B as zero), thread t < 256 (token t / 16, column t % 16) one v, threads < 176 one float4 of the coefficients.  Two register sets
    // hold chunks c + 1 and c + 2 (set A odd chunks, set B even ones), so a chunk's loads have two chunks of compute
    // to arrive.
    constexpr int DN_SD = DN_HD * DN_CT / (64 * DN_CW);  // k / q dims staged per thread
    constexpr int DN_SNF = DN_SD / 4;
    const int s_tok = t & 15, s_f = t >> 4, v_tok = (t >> 4) & 15, v_col = t & 15;
#define DN_CDECL(X)                                                                                               \
    float4 X##k[DN_SNF], X##q[DN_SNF], X##c;                                                                     \
    float X##v;                                                                                                   \
    bool X##in, X##vin
#define DN_CFETCH(X, C)                                                                                           \
    do {                                                                                                          \
        const int i_ = (C) * DN_CT + s_tok, ii_ = min(i_, B - 1);                                                \
        X##in = i_ < B;                                                                                           \
        const float4* kr_ = reinterpret_cast<const float4*>(r.kn + (size_t)ii_ * DN_QK + kh * DN_HD + DN_SD * s_f); \
        const float4* qr_ = reinterpret_cast<const float4*>(r.qn + (size_t)ii_ * DN_QK + kh * DN_HD + DN_SD * s_f); \
        _Pragma("unroll") for (int e_ = 0; e_ < DN_SNF; e_++) {                                                   \
            X##k[e_] = kr_[e_];                                                                                   \
            X##q[e_] = qr_[e_];                                                                                   \
        }                                                                                                         \
        const int iv_ = (C) * DN_CT + v_tok;                                                                      \
        X##vin = iv_ < B && t < DN_CT * DN_RC;                                                                    \
        X##v = r.conv[(size_t)min(iv_, B - 1) * DN_CH + 2 * DN_QK + h * DN_HD + grp * DN_RC + v_col];            \
        if (t < DN_NCOEF / 4)                                                                                     \
            X##c = *reinterpret_cast<const float4*>(r.coef + ((size_t)(C) * DN_VH + h) * DN_NCOEF + 4 * t);      \
    } while (0)
#define DN_CSTAGE(X, BUF)                                                                                         \
    do {                                                                                                          \
        _Pragma("unroll") for (int e_ = 0; e_ < DN_SNF; e_++) {                                                   \
            const float kx_[4] = {X##k[e_].x, X##k[e_].y, X##k[e_].z, X##k[e_].w};                                \
            const float qx_[4] = {X##q[e_].x, X##q[e_].y, X##q[e_].z, X##q[e_].w};                                \
            _Pragma("unroll") for (int d_ = 0; d_ < 4; d_++) {                                                    \
                sKT[BUF][DN_SD * s_f + 4 * e_ + d_][s_tok] = X##in ? kx_[d_] : 0.0f;                              \
                sQT[BUF][DN_SD * s_f + 4 * e_ + d_][s_tok] = X##in ? qx_[d_] : 0.0f;                              \
            }                                                                                                     \
        }                                                                                                         \
        if (t < DN_CT * DN_RC) sV[BUF][v_tok][v_col] = X##vin ? X##v : 0.0f;                                      \
        if (t < DN_NCOEF / 4) *reinterpret_cast<float4*>(&sC[BUF][4 * t]) = X##c;                                 \
    } while (0)
    DN_CDECL(ra_);
    DN_CDECL(rb_);
    DN_CFETCH(ra_, 0);
    DN_CSTAGE(ra_, 0);
    if (1 < nch) DN_CFETCH(ra_, 1);
    if (2 < nch) DN_CFETCH(rb_, 2);
    __syncthreads();
    // one chunk on LDS buffer BUF; then chunk C + 1 (register set X) is staged into the other buffer and chunk C + 3
    // fetched into X
#define DN_CHUNK(C, BUF, X)                                                                                       \
    do {                                                                                                          \
        dn_chunk_step(sKT[BUF], sQT[BUF], sV[BUF], sC[BUF], sRed, st, w, l16, g4, (C), B, h, grp, oscale,       \
                      core_out);                                                                                  \
        if ((C) + 1 < nch) {                                                                                      \
            DN_CSTAGE(X, (BUF) ^ 1);                                                                              \
            if ((C) + 3 < nch) DN_CFETCH(X, (C) + 3);                                          \
        }                                                                                                         \
        __syncthreads();                                                                                          \
    } while (0)
    for (int c = 0; c < nch; c += 2) {
        DN_CHUNK(c, 0, ra_);
        if (c + 1 < nch) DN_CHUNK(c + 1, 1, rb_);
    }
#undef DN_CHUNK
#undef DN_CDECL
#undef DN_CFETCH
#undef DN_CSTAGE
#pragma unroll
    for (int m = 0; m < DN_TPW; m++)
        *reinterpret_cast<float4*>(Sj + 16 * (DN_TPW * w + m) + 4 * g4) =
            make_float4(st[m][0], st[m][1], st[m][2], st[m][3]);
}

// gated RMSNorm per (token, value head), fp16 out: grid (B), 256 threads; wave w normalises value heads w, w + 4,
// ..., lane holding dims 2 lane, 2 lane + 1 (all loads of the token issued before the first reduction)
__global__ void __launch_bounds__(256) k_dn_gnorm_rows(const float* __restrict__ core, const float* __restrict__ z,
                                                       const float* __restrict__ nw, float eps,
                                                       uint16_t* __restrict__ o16) {
    constexpr int NHW = DN_VH / 4;  // heads per wave
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float2 w = *reinterpret_cast<const float2*>(nw + 2 * lane);
    float2 v[NHW], zz[NHW];
#pragma unroll
    for (int i = 0; i < NHW; i++) {
        const size_t idx = (size_t)t * DN_VD + (wave + 4 * i) * DN_HD + 2 * lane;
        v[i] = *reinterpret_cast<const float2*>(core + idx);
        zz[i] = *reinterpret_cast<const float2*>(z + idx);
    }
#pragma unroll
    for (int i = 0; i < NHW; i++) {
        const float rs = 1.0f / sqrtf(wave_sum(v[i].x * v[i].x + v[i].y * v[i].y) / DN_HD + eps);
        const uint32_t lo = f2h_bits(v[i].x * rs * w.x * dn_silu(zz[i].x));
        const uint32_t hi = f2h_bits(v[i].y * rs * w.y * dn_silu(zz[i].y));
        *reinterpret_cast<uint32_t*>(o16 + (size_t)t * DN_VD + (wave + 4 * i) * DN_HD + 2 * lane) = lo | (hi << 16);
    }
}

// ------------------------------------------------------------------------------------------------------ launchers
hipError_t launch_dn_multi(const qwa_dn_params& p, int cin, const qwa_dn_tokens& in, int n_commit, int n_new,
                           int write_after, float eps, float* o, const qwa_act_q8* oq, hipStream_t st) {
    const qwa_act_q8 a = oq ? *oq : qwa_act_q8{nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_dn_head, dim3(DN_VH), dim3(DN_HT), 0, st, p, cin, in, n_commit, n_new, write_after, eps, o,
                       a, oq != nullptr ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_dn_rows(const qwa_dn_params& p, const float* qkv, const float* z, const float* beta_raw,
                          const float* alpha_raw, int B, int cin, float eps, void* work, float* core_out,
                          uint16_t* o16, hipStream_t st) {
    const DnRows r = dn_rows_split(work, B);
    const float* cs_old = p.conv_state + (size_t)cin * 3 * DN_CH;
    float* cs_new = p.conv_state + (size_t)(cin ^ 1) * 3 * DN_CH;
    hipLaunchKernelGGL(k_dn_conv_rows, dim3(DN_CH / 256, (B + DN_CR - 1) / DN_CR), dim3(256), 0, st, qkv, cs_old,
                       p.conv_w, r, beta_raw, alpha_raw, p.dt_bias, p.ssm_a, eps, B, cs_new);
    const int nch = (B + DN_CT - 1) / DN_CT;
    hipLaunchKernelGGL(k_dn_chunk_prep, dim3(DN_VH, nch), dim3(256), 0, st, r, B);
    hipLaunchKernelGGL(k_dn_chunk_rows, dim3(DN_VH, DN_RG), dim3(DN_CW * 64), 0, st, r, p.ssm_state, B, core_out);
    hipLaunchKernelGGL(k_dn_gnorm_rows, dim3(B), dim3(256), 0, st, core_out, z, p.ssm_norm, eps, o16);
    return hipGetLastError();
}

}  // namespace qwa

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
struct DnRows {
    float* conv;   // [B][10240] after SiLU
    float* qn;     // [B][2048] L2-normalised q
    float* kn;     // [B][2048] L2-normalised k
    float* beta;   // [B][48]
    float* decay;  // [B][48]
    float* kq;     // [B][16] qn . kn per key head
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
    r.kq = f;
    return r;
}

size_t dn_work_bytes(int B) { return (size_t)B * (DN_CH + 2 * DN_QK + 2 * DN_VH + DN_KH) * sizeof(float); }

// out[t][c] = silu(sum_k w[c][k] in(t - 3 + k)), in(i) = qkv[i][c] for i >= 0, else row 3 + i of the old window
__global__ void __launch_bounds__(256) k_dn_conv_rows(const float* __restrict__ qkv, const float* __restrict__ cs_old,
                                                      const float* __restrict__ conv_w, float* __restrict__ out) {
    const int t = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
    if (c >= DN_CH) return;
    const float4 w = *reinterpret_cast<const float4*>(conv_w + (size_t)c * 4);
    float x[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = t - 3 + k;
        x[k] = i >= 0 ? qkv[(size_t)i * DN_CH + c] : cs_old[(size_t)(3 + i) * DN_CH + c];
    }
    out[(size_t)t * DN_CH + c] = dn_silu(w.x * x[0] + w.y * x[1] + w.z * x[2] + w.w * x[3]);
}

// the window after the B tokens (rows k = input B - 3 + k), into the other buffer
__global__ void __launch_bounds__(256) k_dn_conv_state(const float* __restrict__ qkv, const float* __restrict__ cs_old,
                                                       int B, float* __restrict__ cs_new) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= DN_CH) return;
#pragma unroll
    for (int k = 0; k < 3; k++) {
        const int i = B - 3 + k;
        cs_new[(size_t)k * DN_CH + c] = i >= 0 ? qkv[(size_t)i * DN_CH + c] : cs_old[(size_t)(3 + i) * DN_CH + c];
    }
}

// per token: L2-normalised q and k of the 16 key heads and their dot product (wave w: key heads w, w + 4, ...),
// beta and decay
__global__ void __launch_bounds__(256) k_dn_prep_rows(DnRows r, const float* __restrict__ beta_raw,
                                                      const float* __restrict__ alpha_raw,
                                                      const float* __restrict__ dt_bias,
                                                      const float* __restrict__ ssm_a, float eps) {
    const int t = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int kh = wave; kh < DN_KH; kh += 4) {
        const float* qs = r.conv + (size_t)t * DN_CH + kh * DN_HD;
        const float* ks = qs + DN_QK;
        const float q0 = qs[lane], q1 = qs[lane + 64], k0 = ks[lane], k1 = ks[lane + 64];
        const float iq = 1.0f / fmaxf(sqrtf(wave_sum(q0 * q0 + q1 * q1)), eps);
        const float ik = 1.0f / fmaxf(sqrtf(wave_sum(k0 * k0 + k1 * k1)), eps);
        const float qa = q0 * iq, qb = q1 * iq, ka = k0 * ik, kb = k1 * ik;
        float* qd = r.qn + (size_t)t * DN_QK + kh * DN_HD;
        float* kd = r.kn + (size_t)t * DN_QK + kh * DN_HD;
        qd[lane] = qa;
        qd[lane + 64] = qb;
        kd[lane] = ka;
        kd[lane + 64] = kb;
        const float kq = wave_sum(qa * ka + qb * kb);
        if (lane == 0) r.kq[(size_t)t * DN_KH + kh] = kq;
    }
    if (threadIdx.x < DN_VH) {
        const int h = threadIdx.x;
        const float a = alpha_raw[(size_t)t * DN_VH + h] + dt_bias[h];
        const float sp = a > 20.0f ? a : logf(1.0f + expf(a));
        r.beta[(size_t)t * DN_VH + h] = 1.0f / (1.0f + expf(-beta_raw[(size_t)t * DN_VH + h]));
        r.decay[(size_t)t * DN_VH + h] = expf(sp * ssm_a[h]);
    }
}

// The recurrence over B tokens: grid (48 heads, 8 groups of 16 columns), 4 waves.  Lane (column jc = t / 16 of the
// group, r16 = t % 16) holds the row quads r16 and r16 + 16 of its column for the whole call (each load / store
// instruction covers 256 contiguous bytes per column).  Per token, with unit q, k and kq = q.k:
//     sk = S^T k, sq = S^T q;  dk = (v - decay sk) beta;  o = decay sq + kq dk;  S = decay S + k dk^T
// (the reference's S <- decay S; S += k ((v - S^T k) beta)^T; o = S^T q).  Blocks of DN_RT tokens are staged in LDS
// double buffers; the next block's global loads are in flight while the current block computes.  core_out may alias
// qkv: it is written only after the conv kernel has read qkv.
constexpr int DN_RT = 16;                 // tokens per staged block
constexpr int DN_RG = 8;                  // workgroups (column groups) per head
constexpr int DN_RC = DN_HD / DN_RG;      // 16 columns per workgroup
__global__ void __launch_bounds__(256) k_dn_recur_rows(DnRows r, float* __restrict__ state, int B,
                                                       float* __restrict__ core_out) {
    const int h = blockIdx.x, grp = blockIdx.y, kh = h % DN_KH, t = threadIdx.x;
    const int jc = t >> 4, r16 = t & 15, j = grp * DN_RC + jc;
    __shared__ float4 sk[2][DN_RT][DN_HD / 4], sq[2][DN_RT][DN_HD / 4];
    __shared__ float4 sc[2][DN_RT];  // decay, beta, kq
    __shared__ float sv[2][DN_RT][DN_RC], so[DN_RT][DN_RC];
    float4* Sq = reinterpret_cast<float4*>(state + (size_t)h * DN_HD * DN_HD + (size_t)j * DN_HD) + r16;
    const float4 s0 = Sq[0], s1 = Sq[16];
    float s[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const float oscale = 1.0f / sqrtf((float)DN_HD);

    // staging: thread (token tt = t / 16, f = t % 16) moves float4 f and f + 16 of q and k, v column f, and (t < 16)
    // the scalars of token t; slots past B read token 0 and are not used
    const int st_tt = t >> 4, st_f = t & 15;
    float4 pk0, pk1, pq0, pq1, pc;
    float pv;
    auto fetch = [&](int b0) {
        const int i = min(b0 + st_tt, B - 1);
        const float4* kr = reinterpret_cast<const float4*>(r.kn + (size_t)i * DN_QK + kh * DN_HD);
        const float4* qr = reinterpret_cast<const float4*>(r.qn + (size_t)i * DN_QK + kh * DN_HD);
        pk0 = kr[st_f];
        pk1 = kr[st_f + 16];
        pq0 = qr[st_f];
        pq1 = qr[st_f + 16];
        pv = r.conv[(size_t)i * DN_CH + 2 * DN_QK + h * DN_HD + grp * DN_RC + st_f];
        const int ic = min(b0 + t, B - 1);
        if (t < DN_RT)
            pc = make_float4(r.decay[(size_t)ic * DN_VH + h], r.beta[(size_t)ic * DN_VH + h],
                             r.kq[(size_t)ic * DN_KH + kh], 0.0f);
    };
    auto stage = [&](int buf) {
        sk[buf][st_tt][st_f] = pk0;
        sk[buf][st_tt][st_f + 16] = pk1;
        sq[buf][st_tt][st_f] = pq0;
        sq[buf][st_tt][st_f + 16] = pq1;
        sv[buf][st_tt][st_f] = pv;
        if (t < DN_RT) sc[buf][t] = pc;
    };
    fetch(0);
    stage(0);
    __syncthreads();
    for (int b0 = 0, buf = 0; b0 < B; b0 += DN_RT, buf ^= 1) {
        const int nt = min(DN_RT, B - b0);
        if (b0 + DN_RT < B) fetch(b0 + DN_RT);
        // two operand sets alternate so that the next token's LDS reads overlap the current token's arithmetic
        struct Op {
            float4 ka, kb, qa, qb, c;
            float v;
        };
        auto load = [&](Op& op, int tt) {
            op.ka = sk[buf][tt][r16];
            op.kb = sk[buf][tt][r16 + 16];
            op.qa = sq[buf][tt][r16];
            op.qb = sq[buf][tt][r16 + 16];
            op.c = sc[buf][tt];
            op.v = sv[buf][tt][jc];
        };
        auto apply = [&](const Op& op, int tt) {
            const float kr[8] = {op.ka.x, op.ka.y, op.ka.z, op.ka.w, op.kb.x, op.kb.y, op.kb.z, op.kb.w};
            const float qr[8] = {op.qa.x, op.qa.y, op.qa.z, op.qa.w, op.qb.x, op.qb.y, op.qb.z, op.qb.w};
            float k0 = 0.0f, k1 = 0.0f, q0 = 0.0f, q1 = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                k0 = fmaf(s[2 * e], kr[2 * e], k0);
                k1 = fmaf(s[2 * e + 1], kr[2 * e + 1], k1);
                q0 = fmaf(s[2 * e], qr[2 * e], q0);
                q1 = fmaf(s[2 * e + 1], qr[2 * e + 1], q1);
            }
            const float skv = row16_sum(k0 + k1), sqv = row16_sum(q0 + q1);
            const float dk = fmaf(-op.c.x, skv, op.v) * op.c.y;
            const float oj = fmaf(op.c.x, sqv, op.c.z * dk);
#pragma unroll
            for (int e = 0; e < 8; e++) s[e] = fmaf(kr[e], dk, s[e] * op.c.x);
            if (r16 == 0) so[tt][jc] = oj * oscale;
        };
        Op opa, opb;
        load(opa, 0);
        for (int tt = 0; tt < nt; tt += 2) {
            if (tt + 1 < nt) load(opb, tt + 1);
            apply(opa, tt);
            if (tt + 1 >= nt) break;
            if (tt + 2 < nt) load(opa, tt + 2);
            apply(opb, tt + 1);
        }
        __syncthreads();  // outputs complete; every read of buffer buf done
        {
            const int tt = t >> 4, e = t & 15;
            if (tt < nt) core_out[(size_t)(b0 + tt) * DN_VD + h * DN_HD + grp * DN_RC + e] = so[tt][e];
        }
        if (b0 + DN_RT < B) stage(buf ^ 1);
        __syncthreads();
    }
    Sq[0] = make_float4(s[0], s[1], s[2], s[3]);
    Sq[16] = make_float4(s[4], s[5], s[6], s[7]);
}

// gated RMSNorm per (token, value head), fp16 out: grid (B, 48), 128 threads
__global__ void __launch_bounds__(128) k_dn_gnorm_rows(const float* __restrict__ core, const float* __restrict__ z,
                                                       const float* __restrict__ nw, float eps,
                                                       uint16_t* __restrict__ o16) {
    __shared__ float red[2];
    const int t = blockIdx.x, h = blockIdx.y, j = threadIdx.x, wave = j >> 6;
    const size_t idx = (size_t)t * DN_VD + h * DN_HD + j;
    const float v = core[idx];
    const float sum = wave_sum(v * v);
    if ((j & 63) == 0) red[wave] = sum;
    __syncthreads();
    const float rs = 1.0f / sqrtf((red[0] + red[1]) / DN_HD + eps);
    o16[idx] = f2h_bits(v * rs * nw[j] * dn_silu(z[idx]));
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
    hipLaunchKernelGGL(k_dn_conv_rows, dim3(DN_CH / 256, B), dim3(256), 0, st, qkv, cs_old, p.conv_w, r.conv);
    hipLaunchKernelGGL(k_dn_conv_state, dim3(DN_CH / 256), dim3(256), 0, st, qkv, cs_old, B, cs_new);
    hipLaunchKernelGGL(k_dn_prep_rows, dim3(B), dim3(256), 0, st, r, beta_raw, alpha_raw, p.dt_bias, p.ssm_a, eps);
    hipLaunchKernelGGL(k_dn_recur_rows, dim3(DN_VH, DN_RG), dim3(256), 0, st, r, p.ssm_state, B, core_out);
    hipLaunchKernelGGL(k_dn_gnorm_rows, dim3(B, DN_VH), dim3(128), 0, st, core_out, z, p.ssm_norm, eps, o16);
    return hipGetLastError();
}

}  // namespace qwa

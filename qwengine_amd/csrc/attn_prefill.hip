// Causal prefill attention over the quantized KV cache on fp16 MFMA (gfx950).
//
// FlashAttention-2 structure (the reference's k_attn_prefill_mma, src/cuda/prefill.cu:522-794), laid out for how
// gfx950 issues work: a wave's VALU instructions do not overlap its own MFMAs, and every 16-byte LDS operand read
// costs matrix-pipe issue time, so
//  * each SIMD runs two MFMA waves (8 waves, 512 threads per workgroup): one wave's softmax / dequantisation VALU work
//    issues while the other's MFMAs run; a wave owns 32 (query, head) rows (two 16-row MFMA tiles), so every K / V
//    fragment read from LDS feeds two MFMAs; a workgroup owns 256 consecutive rows of one KV head
//    (row r = 6 * token + head);
//  * keys are walked in 32-key tiles.  k_pf_image first dequantises every tile of the call's KV range once into an
//    fp16 image (K as [key][dim], V transposed as [dim][key], XOR-swizzled 16-byte units), so both MFMA A-operands
//    are single conflict-free 16-byte LDS reads; k_prefill copies the images HBM -> LDS by direct-to-LDS loads (no
//    registers) two tiles ahead, one barrier per tile.  Built with QWA_PF_IMAGE=0, the raw quantized bytes go to
//    LDS instead and all threads dequantise the next tile cooperatively inside the loop;
//  * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_16x16x32_f16 (fp32 accumulation); P^T comes out of the S^T
//    accumulator already in B-operand layout; online softmax in fp32 with a lazy rescale;
//  * the causal key range of a row block is cut into fixed splits (pf_splits) so that the 24 row blocks x 4 KV
//    heads of a 1024-token chunk fill the chip; the (row block, KV head, split) units run one per workgroup, or, for
//    a 1024-token pass, three consecutive ones per workgroup in a single round (pf_units_per_wg), a run of splits of
//    one row block being walked as one key range.  Each run leaves a partial state (m, l, O / l) in the caller's
//    workspace and k_pf_combine merges them in a fixed order, applies the sigmoid gate and writes fp16.  Chunks
//    longer than PF_MAXB tokens run as several passes.  Nothing here allocates: the images and partial states live
//    in a workspace of prefill_work_bytes(B, p0 + B) bytes.
#include <float.h>

#include "kv_operands.hpp"
#include "launch.hpp"

namespace qwa {

#ifndef QWA_PF_XCD
#define QWA_PF_XCD 1
#endif
#ifndef QWA_PF_WAVES
#define QWA_PF_WAVES 8
#endif
constexpr int PF_WAVES = QWA_PF_WAVES;           // MFMA waves per workgroup
constexpr int PF_THREADS = PF_WAVES * 64;
constexpr int PF_WPE = PF_WAVES / 4;             // waves per SIMD
#ifndef QWA_PF_RT
#define QWA_PF_RT (16 / PF_WAVES > 0 ? 16 / PF_WAVES : 1)
#endif
constexpr int PF_RT = QWA_PF_RT;                 // 16-row MFMA tiles per wave
constexpr int PF_ROWS = PF_WAVES * PF_RT * 16;   // rows per workgroup
constexpr int PF_TILE = 32;                      // keys per tile
constexpr int PF_KT = PF_TILE / 16;              // 16-key MFMA tiles per tile
constexpr int PF_NS = PF_ROWS == 192 ? 6 : 8;    // key-range splits per row block (3 rounds of the chip for B = 1024)
constexpr int PF_MAXB = 1024;                    // tokens per pass
#ifndef QWA_PF_FILL
#define QWA_PF_FILL 1
#endif
// splits of a pass of nb tokens (at most PF_NS): the count that fills the chip's 256 CUs in whole rounds best, i.e.
// the fewest rounds per split, ceil(workgroups / 256) / splits (1024 tokens: 8 splits, 3 rounds; 512 tokens: 5
// splits, one round of 240 workgroups, where 8 would make 1.5 rounds)
inline int pf_splits(int nb) {
    if (!QWA_PF_FILL) return PF_NS;
    const int groups = (GRP * nb + PF_ROWS - 1) / PF_ROWS * NKV;
    int best = PF_NS;
    for (int ns = PF_NS - 1; ns >= 5; ns--)  // 5 .. PF_NS: the instantiated kernels
        if ((long)((groups * ns + 255) / 256) * best < (long)((groups * best + 255) / 256) * ns) best = ns;
    return best;
}
#ifndef QWA_PF_UPW
#define QWA_PF_UPW 1
#endif
#ifndef QWA_PF_SEG_MAXPOS
#define QWA_PF_SEG_MAXPOS 81920
#endif
// (row block, KV head, split) units per workgroup of a pass of nb tokens whose keys end at npos: as many as make the
// units one round of the chip's 256 CUs, when the split count is 8 (so the workgroups of one XCD walk the splits in
// step, see k_prefill) and the pass's keys end within QWA_PF_SEG_MAXPOS; otherwise 1, the units running in rounds.
// Measured, whole call, 1024 tokens (in-process A/B against rounds): Q8_0 -31 us at p0 = 0, -30 at 8192, -43 at
// 32768, -43 at 49152, -23 at 65536, +19 at 100000 (Q4_0 -48 at 32768, -12 at 100000; F16 -41 at 32768).  Past
// ~80000 positions a workgroup's three splits are long enough for the row blocks sharing an XCD's L2 to drift apart.
// (QWA_PF_UPW = 0: always rounds.)
inline int pf_units_per_wg(int nb, int npos) {
    const int ns = pf_splits(nb);
    if (!QWA_PF_UPW || ns != 8 || npos > QWA_PF_SEG_MAXPOS) return 1;
    const int units = (GRP * nb + PF_ROWS - 1) / PF_ROWS * NKV * ns;
    return (units + 255) / 256;
}
constexpr int KS_LD = HD + 8;                    // K tile row stride (halves)
constexpr int VT_LD = PF_TILE + 8;               // V^T tile row stride (halves)
#ifndef QWA_PF_VD
#define QWA_PF_VD 3
#endif
constexpr int PF_VD = QWA_PF_VD;                 // V fragments in flight
#ifndef QWA_PF_KPF
#define QWA_PF_KPF 1
#endif
constexpr int PF_KPF = QWA_PF_KPF;               // score steps of K fragments read ahead (0: compiler's schedule)
#ifndef QWA_PF_GROUP_BIT
#define QWA_PF_GROUP_BIT 4
#endif
constexpr int PF_GROUP_BIT = QWA_PF_GROUP_BIT;   // wave bit that tells the two waves of a SIMD apart
constexpr float PF_LOG2E = 1.4426950408889634f;
constexpr float PF_RESCALE_T = 8.0f;  // lazy-rescale threshold on the running maximum (natural-log units)

// Partial softmax states of one pass live in the caller's workspace: per split and output row
// (row = token * NH + head, ps rows per split) O / l as 16-bit fixed point [split][row][HD] against the row's largest
// |O / l| (pack16x4; absolute error <= that maximum * 2^-16) and (m, l, scale) as fp32 [split][row]; the combine
// reweights them by l * exp(m - M).  (fp16 partials would add a third fp16 rounding, up to 2^-12 |O|, on top of the
// fp16 P and output of the reference's own MMA kernel: measured above the tolerance.)

// raw bytes of one tile in LDS, in the cache's own layout: K rows, V rows, K scales, V scales (8 fp16 per row)
template <int KVT> struct PfRaw {
    static constexpr int VB = value_bytes(KVT);
    static constexpr int K = 0, V = PF_TILE * VB;
    static constexpr int SC = KVT == QWA_KV_F16 ? 0 : PF_TILE * 16;
    static constexpr int KS = 2 * PF_TILE * VB, VS = KS + SC;
    static constexpr int BYTES = 2 * PF_TILE * VB + 2 * SC;
    static constexpr int NKV = PF_TILE * VB / 1024;          // 1 KB load instructions for K (and for V)
    static constexpr int NBUF = KVT == QWA_KV_F16 ? 2 : 3;   // raw tiles in flight (F16 tiles are 32 KB)
    static constexpr int AHEAD = NBUF - 1;                    // tiles loaded ahead of the one being computed
    // load instructions of wave w per tile: K instruction i on wave i % W, V instruction i on wave (i + W / 2) % W,
    // K scales (two 256-byte instructions) on waves W - 2, W - 1, V scales on waves W / 2 - 2, W / 2 - 1
    __device__ static constexpr int count(int w) {
        int n = 0;
        for (int i = 0; i < NKV; i++) n += (i % PF_WAVES == w) + ((i + PF_WAVES / 2) % PF_WAVES == w);
        if (SC) n += (w >= PF_WAVES - 2) + (w >= PF_WAVES / 2 - 2 && w < PF_WAVES / 2);
        return n;
    }
};

// Issues this wave's direct-to-LDS loads of the tile starting at key k0: K instructions wave, wave + 8, ..., V
// instructions (wave + 4) % 8, + 8, ..., scales on waves 2, 3 (V) and 6, 7 (K).  Keys past kmax re-read row kmax
// (they are masked, and no read leaves the window).  wave is wave-uniform.
template <int KVT>
__device__ __forceinline__ void pf_issue(uint32_t raw, const qwa_kv_layer& kv, size_t rowbase, int k0, int kmax,
                                         int wave, int lane) {
    using L = PfRaw<KVT>;
    constexpr int VB = L::VB;
    const int kn = kmax - k0;  // last valid key of the tile, relative
    const uint8_t* kb = kv.k + (rowbase + k0) * VB;
    const uint8_t* vb = kv.v + (rowbase + k0) * VB;
#pragma unroll
    for (int c = 0; c < (L::NKV + PF_WAVES - 1) / PF_WAVES; c++) {
        const int ik = wave + PF_WAVES * c, iv = (wave + PF_WAVES / 2) % PF_WAVES + PF_WAVES * c;
        if (ik < L::NKV) {
            const int p = 1024 * ik + 16 * lane;
            dma_sv<16>(raw + L::K + 1024 * ik, kb, (uint32_t)(min(p / VB, kn) * VB + p % VB));
        }
        if (iv < L::NKV) {
            const int p = 1024 * iv + 16 * lane;
            dma_sv<16>(raw + L::V + 1024 * iv, vb, (uint32_t)(min(p / VB, kn) * VB + p % VB));
        }
    }
    if constexpr (L::SC != 0) {
        // lane l: dword l % 4 of the 8 scales of key 16 j + l / 4
        const int j = wave & 1;
        const uint32_t off = (uint32_t)(min(16 * j + lane / 4, kn) * 16 + 4 * (lane & 3));
        if (wave >= PF_WAVES - 2) dma_sv<4>(raw + L::KS + 256 * j, kv.ks + (rowbase + k0) * 8, off);
        if (wave >= PF_WAVES / 2 - 2 && wave < PF_WAVES / 2)
            dma_sv<4>(raw + L::VS + 256 * j, kv.vs + (rowbase + k0) * 8, off);
    }
}

// waits until at most n of this wave's direct-to-LDS loads are outstanding (n is wave-uniform)
__device__ __forceinline__ void wait_vm(int n) {
    switch (n) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<1>(); break;
        case 2: wait_vmcnt<2>(); break;
        case 3: wait_vmcnt<3>(); break;
        case 4: wait_vmcnt<4>(); break;
        case 5: wait_vmcnt<5>(); break;
        case 6: wait_vmcnt<6>(); break;
        case 7: wait_vmcnt<7>(); break;
        case 8: wait_vmcnt<8>(); break;
        case 9: wait_vmcnt<9>(); break;
        case 10: wait_vmcnt<10>(); break;
        case 11: wait_vmcnt<11>(); break;
        case 12: wait_vmcnt<12>(); break;
        default: wait_vmcnt<0>(); break;
    }
}

// 4 dims of one V key as two half2 {d0, d1}, {d2, d3}, scaled by the key's block scale (one fp16 rounding)
template <int KVT>
__device__ __forceinline__ void pf_v4(const uint8_t* vrow, int dc, uint32_t sc, uint32_t* out) {
    if constexpr (KVT == QWA_KV_F16) {
        const uint2 u = *reinterpret_cast<const uint2*>(vrow + 8 * dc);
        out[0] = u.x;
        out[1] = u.y;
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const h2 d = scale_pair((uint16_t)sc, (uint16_t)sc);
        q8_word_to_h4(*reinterpret_cast<const uint32_t*>(vrow + 4 * dc), d, out);
    } else {
        const h2 d = scale_pair((uint16_t)sc, (uint16_t)sc);
        const h2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};
        const uint32_t x = *reinterpret_cast<const uint16_t*>(vrow + 2 * dc);
        // byte 0 -> dims 0 (low nibble), 1 (high nibble); byte 1 -> dims 2, 3
        const uint32_t p01 = ((x & 0x0Fu) | ((x & 0xF0u) << 12)) | 0x64006400u;
        const uint32_t p23 = (((x >> 8) & 0x0Fu) | (((x >> 8) & 0xF0u) << 12)) | 0x64006400u;
        out[0] = h2_bits((bits_h2(p01) - bias) * d);
        out[1] = h2_bits((bits_h2(p23) - bias) * d);
    }
}

// Dequantises one raw tile into the fp16 tiles (thread t of 512).  K: LDS position 32 s + 8 g + j of a row holds dim
// 32 s + 8 g + perm(j) (the Q operand is loaded with the same permutation).  V^T: row d, position 8 cb + j holds key
// 16 (j / 4) + 4 cb + j % 4, the key order of the P^T operand (lane group g of a 16-key MFMA tile holds keys
// 4 g .. 4 g + 3).
template <int KVT>
__device__ __forceinline__ void pf_convert_kv(const uint8_t* raw, _Float16* Ks, _Float16* Vt, int t, bool do_k,
                                              bool do_v) {
    using L = PfRaw<KVT>;
    constexpr int VB = L::VB;
    const uint16_t* kss = reinterpret_cast<const uint16_t*>(raw + L::KS);
    const uint16_t* vss = reinterpret_cast<const uint16_t*>(raw + L::VS);
    if (!do_k) {
    } else if constexpr (KVT == QWA_KV_F16) {
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int idx = t + 512 * c, key = idx >> 5, pc = idx & 31;
            *reinterpret_cast<uint4*>(Ks + key * KS_LD + 8 * pc) =
                *reinterpret_cast<const uint4*>(raw + L::K + key * VB + 16 * pc);
        }
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const int key = t >> 4, pc = t & 15;
        const uint4 u = *reinterpret_cast<const uint4*>(raw + L::K + key * VB + 16 * pc);
        const uint16_t sc = kss[key * 8 + (pc >> 1)];
        const h2 d = scale_pair(sc, sc);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 4; i++) q8_word_to_h4(w[i], d, o + 2 * i);
        *reinterpret_cast<uint4*>(Ks + key * KS_LD + 16 * pc) = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(Ks + key * KS_LD + 16 * pc + 8) = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
        if (t < PF_TILE * 8) {
            const int key = t >> 3, pc = t & 7;
            const uint4 u = *reinterpret_cast<const uint4*>(raw + L::K + key * VB + 16 * pc);
            const uint16_t sc = kss[key * 8 + pc];
            const h2 d = scale_pair(sc, sc);
            const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t o[4];
                q4_word_to_h8(w[i], d, o);
                *reinterpret_cast<uint4*>(Ks + key * KS_LD + 32 * pc + 8 * i) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    if (!do_v) return;
    // V^T: thread (cb, dc, h) converts keys 16 h + 4 cb + jj (jj < 4), dims 4 dc .. 4 dc + 3
    const int cb = t & 3, dc = (t >> 2) & 63, h = t >> 8;
    uint32_t hv[4][2];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) {
        const int key = 16 * h + 4 * cb + jj;
        const uint32_t sc = KVT == QWA_KV_F16 ? 0u : (uint32_t)vss[key * 8 + (dc >> 3)];
        pf_v4<KVT>(raw + L::V + key * VB, dc, sc, hv[jj]);
    }
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;  // high / low half of both words
        const uint32_t w0 = __builtin_amdgcn_perm(hv[1][d >> 1], hv[0][d >> 1], sel);
        const uint32_t w1 = __builtin_amdgcn_perm(hv[3][d >> 1], hv[2][d >> 1], sel);
        *reinterpret_cast<uint2*>(Vt + (4 * dc + d) * VT_LD + 8 * cb + 4 * h) = make_uint2(w0, w1);
    }
}

// The conversion is cut into 512 K units and 512 V units, spread over the workgroup's threads
template <int KVT>
__device__ __forceinline__ void pf_convert(const uint8_t* raw, _Float16* Ks, _Float16* Vt, int t) {
    if constexpr (PF_THREADS == 512) {
        pf_convert_kv<KVT>(raw, Ks, Vt, t, true, true);
    } else {
#pragma unroll
        for (int u = t; u < 1024; u += PF_THREADS) pf_convert_kv<KVT>(raw, Ks, Vt, u & 511, u < 512, u >= 512);
    }
}

#ifndef QWA_PF_IMAGE
#define QWA_PF_IMAGE 1
#endif
// fp16 tile images: the KV range is dequantised once per call (k_pf_image), not once per row block inside the loop
constexpr bool PF_IMAGE = QWA_PF_IMAGE != 0;
constexpr int PF_IMG_K = PF_TILE * HD * 2;      // bytes of the K part of an image: [32 keys][256 dims] fp16
constexpr int PF_IMG_BYTES = 2 * PF_IMG_K;      // K part, then V^T part [256 dims][32 keys] fp16
constexpr int PF_IMG_NBUF = 3;   // images in LDS: the one computed on and two in flight
constexpr int PF_IMG_AHEAD = 2;

// Image layout (unpadded, so that a direct-to-LDS copy of 1 KB per instruction reproduces it in LDS, and XOR-swizzled
// in 16-byte units so that the MFMA operand reads stay conflict-free without padding):
//  * K: key r, 16-byte unit c (dims 8c .. 8c + 7, in the permuted order of pf_convert_kv) at byte 512 r + 16 (c ^ (r & 7));
//  * V^T: dim d, unit c (keys 8c .. 8c + 7 in P^T operand order) at byte PF_IMG_K + 64 d + 16 (c ^ ((d >> 1) & 3)).
__device__ __forceinline__ int pf_img_k_off(int r, int c) { return 512 * r + 16 * (c ^ (r & 7)); }
__device__ __forceinline__ int pf_img_v_off(int d, int c) { return PF_IMG_K + 64 * d + 16 * (c ^ ((d >> 1) & 3)); }

// One 32-key tile of one KV head per workgroup (grid (tiles, NKV), PF_THREADS threads): the same direct-to-LDS load
// and the same conversion as the in-loop path (so the fp16 values are identical), then a swizzled copy to the image.
// Keys past kmax re-read key kmax, as in the loop.
template <int KVT>
__global__ void __launch_bounds__(PF_THREADS) k_pf_image(qwa_kv_layer kv, int kmax, int ntiles, uint8_t* __restrict__ img) {
    using L = PfRaw<KVT>;
    __shared__ __attribute__((aligned(16))) uint8_t s_raw[L::BYTES];
    __shared__ __attribute__((aligned(16))) _Float16 s_k[PF_TILE * KS_LD];
    __shared__ __attribute__((aligned(16))) _Float16 s_vt[HD * VT_LD];
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(t >> 6));
    const int tile = blockIdx.x, g = blockIdx.y;
    pf_issue<KVT>(lds_addr(s_raw), kv, (size_t)g * kv.capacity, tile * PF_TILE, kmax, wave, lane);
    wait_vmcnt<0>();
    __syncthreads();
    pf_convert<KVT>(s_raw, s_k, s_vt, t);
    __syncthreads();
    uint8_t* dst = img + ((size_t)g * ntiles + tile) * PF_IMG_BYTES;
    for (int u = t; u < PF_IMG_K / 16; u += PF_THREADS) {
        const int r = u >> 5, c = u & 31;
        *reinterpret_cast<uint4*>(dst + pf_img_k_off(r, c)) = *reinterpret_cast<const uint4*>(s_k + r * KS_LD + 8 * c);
    }
    for (int u = t; u < PF_IMG_K / 16; u += PF_THREADS) {
        const int d = u >> 2, c = u & 3;
        *reinterpret_cast<uint4*>(dst + pf_img_v_off(d, c)) = *reinterpret_cast<const uint4*>(s_vt + d * VT_LD + 8 * c);
    }
}

// this wave's share of the direct-to-LDS copy of one image: 1 KB instructions wave, wave + 8, ...
__device__ __forceinline__ void pf_issue_img(uint32_t lds, const uint8_t* src, int wave, int lane) {
#pragma unroll
    for (int c = 0; c < PF_IMG_BYTES / 1024 / PF_WAVES; c++) {
        const int i = wave + PF_WAVES * c;
        dma_sv<16>(lds + 1024 * i, src, (uint32_t)(1024 * i + 16 * lane));
    }
}

__device__ __forceinline__ h8 lds_h8(const _Float16* p) { return *reinterpret_cast<const h8*>(p); }

// max of three floats in one instruction (fmaxf would first canonicalize each MFMA result; scores are never sNaN)
__device__ __forceinline__ float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// max / sum over the four 16-lane rows of the wave (lanes l, l ^ 16, l ^ 32, l ^ 48) with the gfx950 lane swaps:
// permlane16_swap(x, x) leaves row pairs {r0, r0, r2, r2} / {r1, r1, r3, r3}, permlane32_swap {lo, lo} / {hi, hi}
__device__ __forceinline__ float rows_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    float y;
    asm("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(__uint_as_float(a[0])), "v"(__uint_as_float(a[1])));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    asm("v_max_f32 %0, %1, %2" : "=v"(y) : "v"(__uint_as_float(b[0])), "v"(__uint_as_float(b[1])));
    return y;
}
__device__ __forceinline__ float rows_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 16-bit partials: O / l of a (split, row) as signed 16-bit fixed point against the row's largest |O / l| (the scale
// s = max / 32767 goes with (m, l)): absolute error <= s / 2 = max |O / l| * 2^-16 per value.
__device__ __forceinline__ int pf_q16(float v) { return (int)fminf(fmaxf(__builtin_rintf(v), -32767.0f), 32767.0f); }
__device__ __forceinline__ uint2 pack16x4(float a, float b, float c, float d) {
    return make_uint2(((uint32_t)pf_q16(a) & 0xFFFFu) | ((uint32_t)pf_q16(b) << 16),
                      ((uint32_t)pf_q16(c) & 0xFFFFu) | ((uint32_t)pf_q16(d) << 16));
}
__device__ __forceinline__ float4 unpack16x4(uint2 w) {
    return make_float4((float)(int16_t)(w.x & 0xFFFFu), (float)(int16_t)(w.x >> 16), (float)(int16_t)(w.y & 0xFFFFu),
                       (float)(int16_t)(w.y >> 16));
}
using PfPartO = uint2;    // four 16-bit values
using PfPartMl = float4;  // (m, l, scale, unused)

// One split of one row block: grid (row blocks, NKV, NS splits).  Tokens 0 .. B-1 of this pass sit at cache positions
// p0 .. p0 + B - 1.
// IMG: tiles come as fp16 images (k_pf_image) of img_tiles tiles per KV head, copied straight into LDS; otherwise as
// raw quantized bytes dequantised in the loop.
template <int KVT, bool IMG, int NS>
__global__ void __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(PF_WPE, PF_WPE)))
k_prefill(const float* __restrict__ q, qwa_kv_layer kv, int B, int p0, const uint8_t* __restrict__ img, int img_tiles,
          PfPartO* __restrict__ part_o, PfPartMl* __restrict__ part_ml, int ps, int upw, unsigned long long* prof) {
    prof_start(prof);
    using L = PfRaw<KVT>;
    constexpr int NBUF = IMG ? PF_IMG_NBUF : L::NBUF;
    constexpr int AHEAD = IMG ? PF_IMG_AHEAD : NBUF - 1;
    __shared__ __attribute__((aligned(16))) uint8_t s_raw[NBUF][IMG ? PF_IMG_BYTES : L::BYTES];
    __shared__ __attribute__((aligned(16))) _Float16 s_k[IMG ? 1 : 2][IMG ? 8 : PF_TILE * KS_LD];
    __shared__ __attribute__((aligned(16))) _Float16 s_vt[IMG ? 1 : 2][IMG ? 8 : HD * VT_LD];
    const int t = threadIdx.x, lane = t & 63, i16 = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((int)(t >> 6));
    // Work units: (KV head g, row block bx, split) triples.  upw = 1: one unit per workgroup, grid (row blocks, NKV,
    // NS).  upw > 1: grid (units / upw), workgroup w takes units upw w .. upw w + upw - 1 of the list ordered by
    // (g, bx, split); a run of consecutive splits of one (g, bx) is one key range, walked as one segment (one online
    // softmax) that leaves one partial state, in the slot of its first split (k_pf_combine merges only those).  The
    // workgroups that one XCD runs (w = x mod 8) then all start at split (upw x) mod NS and move through the splits in
    // step, so they read the same image tiles at the same time, as the XCD-aware numbering of upw = 1 arranges.
    const int nrb = (GRP * B + PF_ROWS - 1) / PF_ROWS;
    const int units = nrb * NKV * NS;
    int unit = upw == 1 ? 0 : (int)blockIdx.x * upw;
    const int unit_end = upw == 1 ? 1 : min(unit + upw, units);
    for (int seg = 0; unit < unit_end; seg++) {
        int bx, g, sp, sp_last;
        if (upw == 1) {
#if QWA_PF_XCD
            // XCD-aware numbering: workgroup lin is dispatched to XCD lin % 8; give each XCD whole (KV head, split)
            // pairs, so the row blocks that read the same image tiles share one L2
            // (a split count with NKV x NS not a multiple of 8 keeps the plain numbering)
            bx = blockIdx.x;
            g = blockIdx.y;
            sp = blockIdx.z;
            if constexpr ((NKV * NS) % 8 == 0) {
                const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
                const int xcd = lin & 7, slot = lin >> 3;
                const int pair = NKV * NS / 8 * xcd + slot / nrb;
                bx = slot % nrb;
                g = pair % NKV;
                sp = pair / NKV;
            }
#else
            bx = blockIdx.x;
            g = blockIdx.y;
            sp = blockIdx.z;
#endif
            sp_last = sp;
            unit = 1;
        } else {
            const int pr = unit / NS;
            sp = unit % NS;
            sp_last = min(NS - 1, sp + (unit_end - unit) - 1);
            g = pr / nrb;
            bx = pr % nrb;
            unit += sp_last - sp + 1;
            if (seg > 0) __syncthreads();  // every wave is done with the previous segment's images
        }
        const int row0 = bx * PF_ROWS;
        const int nrows = GRP * B;
        // last key any row of the workgroup sees, and this split's tiles [tb, tb + nt) of the row block's range
        const int last_row = min(row0 + PF_ROWS, nrows) - 1;
        const int kmax = p0 + last_row / GRP;
        const int n_tiles = kmax / PF_TILE + 1;
        const int tb = sp * n_tiles / NS, nt = (sp_last + 1) * n_tiles / NS - tb;
        const size_t rowbase = (size_t)g * kv.capacity;
        const int nvm = IMG ? PF_IMG_BYTES / 1024 / PF_WAVES : L::count(wave);
        uint32_t raw_lds[NBUF];
#pragma unroll
        for (int b = 0; b < NBUF; b++) raw_lds[b] = lds_addr(s_raw[b]);
        const uint8_t* isrc = IMG ? img + (size_t)g * img_tiles * PF_IMG_BYTES : nullptr;

        // this lane's rows (token r / 6, head r % 6) and last visible key qpos; Q / 16 as the fp16 B operand
        int qpos[PF_RT];
        h8 qb[PF_RT][8];
        const int wrow0 = row0 + 16 * PF_RT * wave;
#pragma unroll
        for (int rt = 0; rt < PF_RT; rt++) {
            const int r = wrow0 + 16 * rt + i16, tq = r / GRP, hh = r % GRP;
            const bool valid = tq < B;
            qpos[rt] = valid ? p0 + tq : -1;
            const float* qrow = q + ((size_t)(valid ? tq : 0) * NH + g * GRP + hh) * HD;
#pragma unroll
            for (int s = 0; s < 8; s++) {
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
        float m[PF_RT], l[PF_RT];
#pragma unroll
        for (int rt = 0; rt < PF_RT; rt++) {
            m[rt] = -INFINITY;
            l[rt] = 0.0f;
#pragma unroll
            for (int dt = 0; dt < 16; dt++) o[rt][dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        }

        if (IMG && nt > 0) {
            // prologue: images 0 .. AHEAD - 1 in flight, image 0 landed
            wait_vmcnt<0>();  // the Q loads; from here on vmcnt counts only the tile loads
#pragma unroll
            for (int i = 0; i < AHEAD; i++)
                pf_issue_img(raw_lds[i], isrc + (size_t)(tb + min(i, nt - 1)) * PF_IMG_BYTES, wave, lane);
            wait_vm(nvm * (AHEAD - 1));
            __syncthreads();
        } else if (nt > 0) {
            // prologue: raw tiles 0 .. AHEAD - 1 in flight, tile 0 dequantised (and, with AHEAD >= 2, tile 1 landed)
            wait_vmcnt<0>();  // the Q loads; from here on vmcnt counts only the tile loads
#pragma unroll
            for (int i = 0; i < L::AHEAD; i++)
                pf_issue<KVT>(raw_lds[i], kv, rowbase, (tb + min(i, nt - 1)) * PF_TILE, kmax, wave, lane);
            wait_vm(nvm * (L::AHEAD - 1));
            __syncthreads();
            pf_convert<KVT>(s_raw[0], s_k[0], s_vt[0], t);
            if constexpr (L::AHEAD >= 2) wait_vm(nvm * (L::AHEAD - 2));
            __syncthreads();
        }

        // The two waves of a SIMD (w and w + 4) run the phases of a tile in different orders so that one issues VALU /
        // LDS work (dequantisation, softmax) while the other's MFMAs run:
        //   waves 0-3: convert | S       | softmax | PV
        //   waves 4-7: S       | softmax | PV      | convert
        // With images there is no conversion and every wave runs S | softmax | PV.
        const bool lead = (wave & PF_GROUP_BIT) == 0;
        h8 pb[PF_RT];
        auto pv = [&](const _Float16* Vt) {
            h8 vf[PF_VD];
            const _Float16* vrow = IMG ? Vt + i16 * PF_TILE + 8 * (lg ^ ((i16 >> 1) & 3)) : Vt + i16 * VT_LD + 8 * lg;
            constexpr int vstep = IMG ? 16 * PF_TILE : 16 * VT_LD;
#pragma unroll
            for (int dt = 0; dt < PF_VD - 1; dt++) vf[dt] = lds_h8(vrow + vstep * dt);
#pragma unroll
            for (int dt = 0; dt < 16; dt++) {
                if (dt + PF_VD - 1 < 16) vf[(dt + PF_VD - 1) % PF_VD] = lds_h8(vrow + vstep * (dt + PF_VD - 1));
#pragma unroll
                for (int rt = 0; rt < PF_RT; rt++) o[rt][dt] = mfma16(vf[dt % PF_VD], pb[rt], o[rt][dt]);
            }
        };
        for (int i = 0; i < nt; i++) {
            const int k0 = (tb + i) * PF_TILE, cur = i & 1;
            // tile i + AHEAD (the last tile again near the end: a harmless re-read) into the raw buffer freed last
            // iteration
            if constexpr (IMG)
                pf_issue_img(raw_lds[(i + AHEAD) % NBUF], isrc + (size_t)(tb + min(i + AHEAD, nt - 1)) * PF_IMG_BYTES,
                             wave, lane);
            else
                pf_issue<KVT>(raw_lds[(i + AHEAD) % NBUF], kv, rowbase, (tb + min(i + AHEAD, nt - 1)) * PF_TILE, kmax,
                              wave, lane);
            const _Float16* Ks = IMG ? reinterpret_cast<const _Float16*>(s_raw[i % NBUF]) : s_k[cur];
            const _Float16* Vt = IMG ? Ks + PF_IMG_K / 2 : s_vt[cur];

            // the next tile's raw bytes landed before the last barrier: dequantise them into the other fp16 tile
            auto convert = [&]() {
                if constexpr (!IMG && AHEAD >= 2)
                    pf_convert<KVT>(s_raw[(i + 1) % NBUF], s_k[cur ^ 1], s_vt[cur ^ 1], t);
            };

            f4 sc[PF_RT][PF_KT];
            // image K operand bases: row i16, unit lg ^ (i16 & 3), s shifted by +-1 when bit 2 of i16 is set
            const _Float16* kimg_e = Ks + i16 * HD + 8 * (lg ^ (i16 & 3)) + 32 * ((i16 >> 2) & 1);
            const _Float16* kimg_o = kimg_e - 64 * ((i16 >> 2) & 1);
            // ---- S^T = K Q^T for PF_KT key tiles of 16 (lane: key k0 + 16 k4 + 4 lg + i, row (rt, i16))
            auto scores = [&]() {
#pragma unroll
                for (int k4 = 0; k4 < PF_KT; k4++)
#pragma unroll
                    for (int rt = 0; rt < PF_RT; rt++) sc[rt][k4] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                // swizzled unit (4 s + lg) ^ x = 4 (s ^ (x >> 2)) + (lg ^ (x & 3)): two lane bases, even / odd s
                auto kfrag = [&](int s, int k4) {
                    return IMG ? lds_h8((s & 1 ? kimg_o : kimg_e) + (16 * k4) * HD + 32 * s)
                               : lds_h8(Ks + (16 * k4 + i16) * KS_LD + 8 * lg + 32 * s);
                };
                if constexpr (PF_KPF > 0) {
                    // the K fragments of step s + PF_KPF are read while step s multiplies (scheduling barriers keep the
                    // compiler from sinking the reads next to their MFMAs)
                    h8 kf[PF_KPF + 1][PF_KT];
#pragma unroll
                    for (int s = 0; s < PF_KPF; s++)
#pragma unroll
                        for (int k4 = 0; k4 < PF_KT; k4++) kf[s][k4] = kfrag(s, k4);
#pragma unroll
                    for (int s = 0; s < 8; s++) {
                        if (s + PF_KPF < 8) {
#pragma unroll
                            for (int k4 = 0; k4 < PF_KT; k4++)
                                kf[(s + PF_KPF) % (PF_KPF + 1)][k4] = kfrag(s + PF_KPF, k4);
                        }
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int k4 = 0; k4 < PF_KT; k4++)
#pragma unroll
                            for (int rt = 0; rt < PF_RT; rt++)
                                sc[rt][k4] = mfma16(kf[s % (PF_KPF + 1)][k4], qb[rt][s], sc[rt][k4]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
#pragma unroll
                    for (int s = 0; s < 8; s++) {
#pragma unroll
                        for (int k4 = 0; k4 < PF_KT; k4++) {
                            const h8 a = kfrag(s, k4);
#pragma unroll
                            for (int rt = 0; rt < PF_RT; rt++) sc[rt][k4] = mfma16(a, qb[rt][s], sc[rt][k4]);
                        }
                    }
                }
            };

            // ---- mask + online softmax.  The reference maximum m moves only when a score exceeds it by more than
            // PF_RESCALE_T (probabilities stay <= e^PF_RESCALE_T, far inside fp16), so the accumulators are rarely
            // rescaled.
            auto softmax = [&]() {
                const bool need_mask = k0 + PF_TILE - 1 > wave_qmin;
                float cr[PF_RT];
#pragma unroll
                for (int rt = 0; rt < PF_RT; rt++) {
                    if (need_mask) {
#pragma unroll
                        for (int k4 = 0; k4 < PF_KT; k4++)
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const int key = k0 + 16 * k4 + 4 * lg + j;
                                sc[rt][k4][j] = key > qpos[rt] ? -INFINITY : sc[rt][k4][j];
                            }
                    }
                    float mx = -INFINITY;
#pragma unroll
                    for (int k4 = 0; k4 < PF_KT; k4++)
                        mx = max3f(max3f(mx, sc[rt][k4][0], sc[rt][k4][1]), sc[rt][k4][2], sc[rt][k4][3]);
                    mx = rows_max(mx);
                    const float mn = mx > m[rt] + PF_RESCALE_T ? mx : m[rt];
                    cr[rt] = mn == m[rt] ? 1.0f : fast_exp2((m[rt] - mn) * PF_LOG2E);  // m = -inf: c = 0
                    m[rt] = mn;
                    const float msl = mn == -INFINITY ? 0.0f : mn * PF_LOG2E;
                    // the row's lane sum of the fp16 probabilities themselves (the weights P.V applies), two per dot2
                    h8 p;
#pragma unroll
                    for (int j = 0; j < 8; j++) p[j] = (_Float16)fast_exp2(fmaf(sc[rt][j >> 2][j & 3], PF_LOG2E, -msl));
                    const h2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
                    float rs = __builtin_amdgcn_fdot2(h2{p[0], p[1]}, one2, 0.0f, false);
                    rs = __builtin_amdgcn_fdot2(h2{p[2], p[3]}, one2, rs, false);
                    rs = __builtin_amdgcn_fdot2(h2{p[4], p[5]}, one2, rs, false);
                    rs = __builtin_amdgcn_fdot2(h2{p[6], p[7]}, one2, rs, false);
                    pb[rt] = p;
                    l[rt] = l[rt] * cr[rt] + rs;
                }
                if (__any(cr[0] != 1.0f || cr[PF_RT - 1] != 1.0f)) {
#pragma unroll
                    for (int rt = 0; rt < PF_RT; rt++)
#pragma unroll
                        for (int dt = 0; dt < 16; dt++) o[rt][dt] *= cr[rt];
                }
            };

            if (!IMG && lead) convert();
            scores();
            softmax();
            pv(Vt);
            if (!IMG && !lead) convert();

            if constexpr (IMG) {
                // image i + 1 must have landed before the next iteration reads it; image i + 2 may stay in flight
                wait_vm(nvm * (AHEAD - 1));
                __syncthreads();
            } else if constexpr (AHEAD >= 2) {
                // tile i + 2 must have landed before the next iteration dequantises it; later tiles may stay in flight
                wait_vm(nvm * (AHEAD - 2));
                __syncthreads();
            } else {
                wait_vm(0);
                __syncthreads();
                if (i + 1 < nt) pf_convert<KVT>(s_raw[(i + 1) % L::NBUF], s_k[cur ^ 1], s_vt[cur ^ 1], t);
                __syncthreads();
            }
        }
        wait_vmcnt<0>();  // no direct-to-LDS load outlives the workgroup

        // ---- partial state of this split: (m, l) and O / l; lane holds dims 16 dt + 4 lg + i of row (rt, i16)
#pragma unroll
        for (int rt = 0; rt < PF_RT; rt++) {
            const float lt = rows_sum(l[rt]);
            if (qpos[rt] < 0) continue;
            const int r = wrow0 + 16 * rt + i16, rr = (r / GRP) * NH + g * GRP + r % GRP;
            const size_t prow = (size_t)sp * ps + rr;
            const float il = lt > 0.0f ? 1.0f / lt : 0.0f;  // a split that saw no key leaves l = 0 and O = 0
            float amax = 0.0f;
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
#pragma unroll
                for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(o[rt][dt][i]));
            amax = rows_max(amax) * il;
            const float qs = amax > 1e-30f ? 32767.0f / amax : 0.0f;  // (a row this small stores zeros: no inf scale)
            const float f = il * qs;
            if (lg == 0) part_ml[prow] = make_float4(m[rt], lt, qs > 0.0f ? amax * (1.0f / 32767.0f) : 0.0f, 0.0f);
            PfPartO* dst = part_o + prow * (HD / 4) + lg;
#pragma unroll
            for (int dt = 0; dt < 16; dt++)
                dst[4 * dt] = pack16x4(o[rt][dt][0] * f, o[rt][dt][1] * f, o[rt][dt][2] * f, o[rt][dt][3] * f);
        }
    }  // segments
    prof_end(prof);
}

// Merges the partial states of the ns splits of each output row in split order (the slots that start a segment, see
// k_prefill), applies the sigmoid gate and writes fp16: one wave per row (token * NH + head), 4 dims per lane.
// Split s weighs w_s = l_s exp(m_s - M); the row's output is sum_s w_s (O_s / l_s) / sum_s w_s.
template <int NS>
__global__ void __launch_bounds__(256) k_pf_combine(const float* __restrict__ gate, int nrows,
                                                    const PfPartO* __restrict__ part_o,
                                                    const PfPartMl* __restrict__ part_ml, int ps, int upw,
                                                    uint16_t* __restrict__ out16) {
    const int rr = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (rr >= nrows) return;
    // the row's (KV head, row block) and, with upw > 1 units per workgroup, which of its split slots start a segment
    // (k_prefill): split s does when s = 0 or its unit index is a multiple of upw
    const int head = rr % NH, grow = (rr / NH) * GRP + head % GRP;
    const int pr = (head / GRP) * ((GRP * (nrows / NH) + PF_ROWS - 1) / PF_ROWS) + grow / PF_ROWS;
    PfPartMl ml[NS];
    float4 ov[NS];
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const bool on = s == 0 || (pr * NS + s) % upw == 0;
        ml[s] = on ? part_ml[(size_t)s * ps + rr] : make_float4(-INFINITY, 0.0f, 0.0f, 0.0f);
        ov[s] = on ? unpack16x4(part_o[((size_t)s * ps + rr) * (HD / 4) + lane]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        mx = fmaxf(mx, ml[s].x);
    }
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float wsum = 0.0f;
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const float w = ml[s].x == -INFINITY ? 0.0f : fast_exp2((ml[s].x - mx) * PF_LOG2E) * ml[s].y;
        const float wq = w * ml[s].z;  // the split's weight times its fixed-point scale
        acc.x += wq * ov[s].x;
        acc.y += wq * ov[s].y;
        acc.z += wq * ov[s].z;
        acc.w += wq * ov[s].w;
        wsum += w;
    }
    const float iw = 1.0f / wsum;
    const float4 gv = *reinterpret_cast<const float4*>(gate + (size_t)rr * HD + 4 * lane);
    const uint16_t h0 = f2h_bits(acc.x * iw * sigmoid(gv.x)), h1 = f2h_bits(acc.y * iw * sigmoid(gv.y));
    const uint16_t h2v = f2h_bits(acc.z * iw * sigmoid(gv.z)), h3 = f2h_bits(acc.w * iw * sigmoid(gv.w));
    *reinterpret_cast<uint2*>(out16 + (size_t)rr * HD + 4 * lane) =
        make_uint2((uint32_t)h0 | ((uint32_t)h1 << 16), (uint32_t)h2v | ((uint32_t)h3 << 16));
}

// Workspace layout of one call: the fp16 images of the KV range [0, p0 + B) (NKV x tiles x 32 KB; none when built
// without images), then the (m, l) pairs and the partial O of one pass (up to PF_NS x ps rows, ps = NH x min(B,
// PF_MAXB)).
struct PfWork {
    uint8_t* img;
    PfPartMl* ml;
    PfPartO* o;  // 4 values per element
    int tiles, ps;
    size_t bytes;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static PfWork pf_work_layout(uint8_t* base, int B, int n_pos) {
    PfWork w;
    w.tiles = (n_pos - 1) / PF_TILE + 1;
    w.ps = NH * min(B, PF_MAXB);
    const size_t img = PF_IMAGE ? align256((size_t)NKV * w.tiles * PF_IMG_BYTES) : 0;
    const size_t ml = align256((size_t)PF_NS * w.ps * sizeof(PfPartMl));
    const size_t o = (size_t)PF_NS * w.ps * (HD / 4) * sizeof(PfPartO);
    w.img = base;
    w.ml = reinterpret_cast<PfPartMl*>(base + img);
    w.o = reinterpret_cast<PfPartO*>(base + img + ml);
    w.bytes = img + ml + o;
    return w;
}

size_t prefill_work_bytes(int B, int n_pos) { return pf_work_layout(nullptr, B, n_pos).bytes; }

template <int KVT>
static void launch_prefill_pass(const float* qp, const qwa_kv_layer& kv, int nb, int p0, const PfWork& w,
                                hipStream_t st) {
    const int ns = pf_splits(nb);
    const int upw = pf_units_per_wg(nb, p0 + nb);
    const int nrb = (GRP * nb + PF_ROWS - 1) / PF_ROWS, units = nrb * NKV * ns;
    const dim3 grid = upw == 1 ? dim3(nrb, NKV, ns) : dim3((units + upw - 1) / upw);
    const ProfSlot ps = profile_slot(grid.x * grid.y * grid.z, st);
#define QWA_PF_LAUNCH(N)                                                                                              \
    QWA_LAUNCH_MAIN(ps, (k_prefill<KVT, PF_IMAGE, N>), grid, dim3(PF_THREADS), st, qp, kv, nb, p0, w.img, w.tiles, \
                    w.o, w.ml, w.ps, upw)
    if (ns == 5) QWA_PF_LAUNCH(5);
    else if (ns == 6) QWA_PF_LAUNCH(6);
    else if (ns == 7) QWA_PF_LAUNCH(7);
    else QWA_PF_LAUNCH(PF_NS);
#undef QWA_PF_LAUNCH
}

hipError_t launch_prefill(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                          uint16_t* out16, void* work, hipStream_t st) {
    const PfWork w = pf_work_layout(static_cast<uint8_t*>(work), B, p0 + B);
    if (PF_IMAGE) {
        const dim3 grid(w.tiles, NKV);
        if (kvt == QWA_KV_F16)
            hipLaunchKernelGGL(k_pf_image<QWA_KV_F16>, grid, dim3(PF_THREADS), 0, st, kv, p0 + B - 1, w.tiles, w.img);
        else if (kvt == QWA_KV_Q8_0)
            hipLaunchKernelGGL(k_pf_image<QWA_KV_Q8_0>, grid, dim3(PF_THREADS), 0, st, kv, p0 + B - 1, w.tiles, w.img);
        else
            hipLaunchKernelGGL(k_pf_image<QWA_KV_Q4_0>, grid, dim3(PF_THREADS), 0, st, kv, p0 + B - 1, w.tiles, w.img);
    }
    for (int t0 = 0; t0 < B; t0 += PF_MAXB) {
        const int nb = min(PF_MAXB, B - t0);
        const float* qp = q + (size_t)t0 * NH * HD;
        if (kvt == QWA_KV_F16) launch_prefill_pass<QWA_KV_F16>(qp, kv, nb, p0 + t0, w, st);
        else if (kvt == QWA_KV_Q8_0) launch_prefill_pass<QWA_KV_Q8_0>(qp, kv, nb, p0 + t0, w, st);
        else launch_prefill_pass<QWA_KV_Q4_0>(qp, kv, nb, p0 + t0, w, st);
        const int nrows = nb * NH;
        const float* gp = gate + (size_t)t0 * NH * HD;
        uint16_t* op = out16 + (size_t)t0 * NH * HD;
        const dim3 cg((nrows + 3) / 4), cb(256);
        const int upw = pf_units_per_wg(nb, p0 + t0 + nb);
        switch (pf_splits(nb)) {
#define QWA_PF_COMBINE(N) \
    case N: hipLaunchKernelGGL(k_pf_combine<N>, cg, cb, 0, st, gp, nrows, w.o, w.ml, w.ps, upw, op); break
            QWA_PF_COMBINE(5); QWA_PF_COMBINE(6); QWA_PF_COMBINE(7);
            default: hipLaunchKernelGGL(k_pf_combine<PF_NS>, cg, cb, 0, st, gp, nrows, w.o, w.ml, w.ps, upw, op); break;
#undef QWA_PF_COMBINE
        }
    }
    return hipGetLastError();
}

}  // namespace qwa

// Decode / speculative-verify attention over the quantized KV cache (gfx950).
//
// Split-K flash-decoding (the reference's structure, src/cuda/ops.cu:507-815, re-designed for wave64 + MFMA and for
// streaming HBM at full rate):
//  * the keys of a KV head are cut into 16-key chunks; chunk c belongs to class c mod DEC_CLASSES (512 classes per
//    head, a fixed function of the chunk index); a wave owns one class and walks its chunks in increasing order, so
//    at any moment all waves of the chip stream neighbouring chunks (grid-stride locality) and a 150000-position
//    head gives every wave ~18 chunks (2048 waves = 2 per SIMD);
//  * chunks are fetched with direct-to-LDS loads (global_load_lds, 16 B per lane) into an NST-stage per-wave ring;
//    each lane's source piece is rotated per row so the MFMA operand reads from LDS are (nearly) bank-conflict free;
//  * rows are (query, head) pairs of one KV head, row r = 6 * query + head, in RT 16-row MFMA tiles;
//    S^T = K Q^T on v_mfma_f32_16x16x32_f16, one MFMA per 32-dim quant block with the exact integer K codes and
//    Q / 16 as fp16 hi + lo parts, the key's fp16 block scale applied to each block's fp32 partial dot (scores exact
//    up to fp32 accumulation, so outlier logits stay within tolerance); a lane then holds 4 keys of ONE row: the
//    online softmax is lane-local up to a 4-lane max / sum, and P^T is directly the B operand of
//    O^T += V^T P^T (v_mfma_f32_16x16x16_f16, fp32 accumulation; for Q4_0 the V operand holds the exact codes and
//    the keys' block scales multiply the P operand, one product per block instead of one per V element);
//  * the 8 classes of a workgroup are merged along a fixed pairwise tree into one partial record (m, l, O[256]) per
//    row; k_dec_combine merges the records in a fixed order, normalises, applies the sigmoid gate and the optional
//    ActQ8 epilogue;
//  * a call with several row tiles (verify) streams the cache once per pair of tiles.
// Every reduction runs over a partition of the keys that depends only on key indices, and masked keys contribute
// exact zeros, so a query's output does not depend on how many queries share the call (the reference's
// decode == decode_batch contract, src/cuda/ops.cuh:134-135).
#include <float.h>

#include <mutex>

#include "kv_operands.hpp"
#include "launch.hpp"

namespace qwa {

#ifdef QWA_TRACE
// experimental phase stamps (trace builds only): [workgroup][8] realtime-clock values written by wave 0, lane 0
static __device__ unsigned long long dec_trace[4096][8];
// per-wave stamps: [workgroup][wave] first chunk landed, [workgroup][8 + wave] loop end
static __device__ unsigned long long dec_wtrace[4096][16];
#define WTRACE(k)                                                                                        \
    do {                                                                                                 \
        if ((threadIdx.x & 63) == 0)                                                                     \
            dec_wtrace[blockIdx.x + gridDim.x * blockIdx.y][(k) + (threadIdx.x >> 6)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define TRACE(k)                                                                                         \
    do {                                                                                                 \
        if (threadIdx.x == 0) dec_trace[prof_wg() + trace_base][k] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define TRACE(k) \
    do {         \
    } while (0)
#define WTRACE(k) \
    do {          \
    } while (0)
#endif

constexpr int REC = 260;    // partial record: m, l, 2 pad, O[256] (16-byte aligned O)
constexpr int CGRP = 16;    // combine: records per fixed summation group
#ifndef QWA_DEC3H
#define QWA_DEC3H 1
#endif
#ifndef QWA_DEC3H_CHAIN
#define QWA_DEC3H_CHAIN 1
#endif
#ifndef QWA_Q4_CHAIN_FROM
#define QWA_Q4_CHAIN_FROM 24576
#endif
#ifndef QWA_Q8_CHAIN_FROM
#define QWA_Q8_CHAIN_FROM 12288
#endif
#ifndef QWA_DEC_INTERLEAVE
#define QWA_DEC_INTERLEAVE 1
#endif
constexpr bool DEC_INTERLEAVE = QWA_DEC_INTERLEAVE != 0;  // classes spread over the records (see dec_body)
constexpr int CHUNK = 16;   // keys per chunk
constexpr int WG_CLASSES = 8;                   // classes (waves) per decode workgroup, every format
constexpr int NREC = DEC_CLASSES / WG_CLASSES;  // records (workgroups) per KV head
// record slots per KV head in the work buffer: a record, or (three-tile verify) its two halves, each the merge of 4
// classes written by a 4-wave workgroup, that k_dec_combine folds into the record
constexpr int NSLOT = 2 * NREC;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float RESCALE_T = 8.0f;  // lazy-rescale threshold on the running maximum (natural-log units)

// the record slots of every valid call (up to MAXQ queries, any context up to MAX_POS): the size does not depend on
// the context length
constexpr size_t DEC_WORK_BYTES = (size_t)NSLOT * NKV * MAXQ * GRP * REC * sizeof(float);
#ifndef QWA_DEC_KERNELS_ONLY
size_t dec_work_bytes(int n_pos) {
    (void)n_pos;
    return DEC_WORK_BYTES;
}
#endif

// One 16-key chunk in LDS.  K: piece-major, 16-byte piece p of row n at (16 p + n) * 16 (an MFMA operand read of one
// quant block is then a conflict-free read at a fixed offset); V: row-major; then the K and V block scales
// ([row][8] fp16 each).
template <int KVT>
struct ChunkLds {
    static constexpr int VB = value_bytes(KVT);
    static constexpr int KBYTES = CHUNK * VB;
    static constexpr int NI = KBYTES / 1024;  // 1 KB load instructions per K (and per V) region
    static constexpr int SC = KVT == QWA_KV_F16 ? 0 : CHUNK * 16;
    static constexpr int BYTES = 2 * KBYTES + 2 * SC;
    static constexpr int NLOAD = 2 * NI + (SC ? 2 : 0);  // load instructions per chunk
};

// LDS offset of byte `byte` (< VB) of K row `row` in the piece-major layout
template <int KVT>
__host__ __device__ constexpr int kpos(int row, int byte) {
    return ((byte >> 4) * CHUNK + row) * 16 + (byte & 15);
}


// Direct-to-LDS loads of one chunk (16 B per lane per instruction: K piece-major, V row-major, then the scales).
// A full chunk (every row inside the window) loads from wave-uniform bases (scalar registers) with per-lane offsets
// fixed for the whole kernel: K piece 4 i + lane / 16 of row lane % 16 at koff + 64 i, V bytes 1024 i + 16 lane,
// scales 4 lane.  The chunk holding key kmax takes per-lane addresses: rows past kmax re-read row kmax (no read
// outside the window; their scores are masked and their probabilities are exact zeros).
template <int KVT>
__device__ __forceinline__ uint32_t chunk_koff(int lane) {
    return (uint32_t)((lane & 15) * ChunkLds<KVT>::VB + 16 * (lane >> 4));
}

template <int KVT>
__device__ __forceinline__ void issue_chunk(uint8_t* dst, const qwa_kv_layer& kv, size_t rowbase, int kb, int kmax,
                                            int lane, uint32_t koff) {
    using C = ChunkLds<KVT>;
    constexpr int VB = C::VB;
    const uint32_t d = lds_addr(dst);
    if (kb + CHUNK - 1 <= kmax) {
        const size_t row0 = rowbase + kb;
        const uint8_t* kp = kv.k + row0 * VB;
        const uint8_t* vp = kv.v + row0 * VB;
#pragma unroll
        for (int i = 0; i < C::NI; i++) {
            dma_sv<16>(d + 1024 * i, kp + 64 * i, koff);
            dma_sv<16>(d + C::KBYTES + 1024 * i, vp + 1024 * i, 16 * lane);
        }
        if constexpr (C::SC) {
            dma_sv<4>(d + 2 * C::KBYTES, kv.ks + row0 * 8, 4 * lane);
            dma_sv<4>(d + 2 * C::KBYTES + C::SC, kv.vs + row0 * 8, 4 * lane);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < C::NI; i++) {
        const int kn = lane & 15, kpc = 4 * i + (lane >> 4);               // K slot: piece kpc of row kn
        const int vn = (1024 * i + 16 * lane) / VB, vbyte = (1024 * i + 16 * lane) % VB;  // V: row-major
        dma_v<16>(d + 1024 * i, kv.k + (rowbase + min(kb + kn, kmax)) * VB + 16 * kpc);
        dma_v<16>(d + C::KBYTES + 1024 * i, kv.v + (rowbase + min(kb + vn, kmax)) * VB + vbyte);
    }
    if constexpr (C::SC) {
        const size_t row = rowbase + min(kb + lane / 4, kmax);
        dma_v<4>(d + 2 * C::KBYTES, reinterpret_cast<const uint8_t*>(kv.ks + row * 8) + 4 * (lane & 3));
        dma_v<4>(d + 2 * C::KBYTES + C::SC, reinterpret_cast<const uint8_t*>(kv.vs + row * 8) + 4 * (lane & 3));
    }
}


// A operand of block b for lane (key n, group g): exact integers (no scale), dims 32 b + 8 g + perm(j)
template <int KVT>
__device__ __forceinline__ h8 k_block_int(const uint8_t* kst, int n, int g, int b) {
    constexpr int VB = ChunkLds<KVT>::VB;
    const uint8_t* p = kst + kpos<KVT>(n, (VB / 8) * b + (VB / 32) * g);
    if constexpr (KVT == QWA_KV_F16) {
        return *reinterpret_cast<const h8*>(p);
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        uint32_t o[4];
        q8_word_int(u.x, o);
        q8_word_int(u.y, o + 2);
        return make_h8(o[0], o[1], o[2], o[3]);
    } else {
        uint32_t o[4];
        q4_word_int(*reinterpret_cast<const uint32_t*>(p), o);
        return make_h8(o[0], o[1], o[2], o[3]);
    }
}

// V of chunk row `key`, dims 16 c .. 16 c + 15, with its block scale
template <int KVT>
__device__ __forceinline__ void v_raw(VRaw<KVT>& r, const uint8_t* vst, const uint16_t* vsc, int key, int c) {
    constexpr int VB = ChunkLds<KVT>::VB;
    const uint8_t* p = vst + key * VB + (VB / 16) * c;
    if constexpr (KVT == QWA_KV_Q4_0) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        r.w[0] = u.x; r.w[1] = u.y;
    } else if constexpr (KVT == QWA_KV_Q8_0) {
        const uint4 u = *reinterpret_cast<const uint4*>(p);
        r.w[0] = u.x; r.w[1] = u.y; r.w[2] = u.z; r.w[3] = u.w;
    } else {
        const uint4 u0 = *reinterpret_cast<const uint4*>(p), u1 = *reinterpret_cast<const uint4*>(p + 16);
        r.w[0] = u0.x; r.w[1] = u0.y; r.w[2] = u0.z; r.w[3] = u0.w;
        r.w[4] = u1.x; r.w[5] = u1.y; r.w[6] = u1.z; r.w[7] = u1.w;
    }
    r.sc = KVT == QWA_KV_F16 ? 0u : vsc[key * 8 + (c >> 1)];
}

// max over the 4 lanes l % 16 + 16 k (the 4 lanes that hold one row of S^T): two cross-row swaps, no LDS
__device__ __forceinline__ float row_max4(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ f4 mfma16k16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }

// Merge of two partial softmax states (fold step); the same arithmetic for every record and every nq.
template <int NT = 16>
__device__ __forceinline__ void fold(float& m, float& l, f4* o, float m2, float l2, const f4* o2) {
    const float M = fmaxf(m, m2);
    const float Ms = M == -INFINITY ? 0.0f : M;
    const float fa = fast_exp2((m - Ms) * LOG2E), fb = fast_exp2((m2 - Ms) * LOG2E);
    // explicit fused forms: every kernel that merges rounds the same way (the nq-independence contract)
    l = fmaf(l, fa, l2 * fb);
#pragma unroll
    for (int dt = 0; dt < NT; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[dt][i] = fmaf(o[dt][i], fa, o2[dt][i] * fb);
    m = M;
}

// sum over the 4 lanes l % 16 + 16 k that hold one row
__device__ __forceinline__ float half4_sum(float x) {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
}

// Merge of the partial states of the WGW waves of a workgroup, split across the waves by head dims: every wave puts
// its state in LDS, then wave w folds the WGW states of the output tiles TPW w .. TPW w + TPW - 1 (TPW = 16 / WGW)
// in the fixed tree fold(fold(c0, c1), fold(c2, c3)) (and fold(that, the same over c4..c7) for 8 waves).  Every
// wave folds (m, l) along the same tree, so all of them hold the merged m and l.
// The two waves of a SIMD (w and w + WGW / 2 of a workgroup) stream classes of equal length, but the SIMD's
// arbiter favours the older one, and the younger one then finishes its last chunks alone.  Each wave publishes its
// chunk index; the one that is behind takes issue priority until it has caught up.  (Priority only orders issue
// between the two waves; the arithmetic is unchanged.)
template <int WGW>
__device__ __forceinline__ void pair_priority(int* s_prog, int wave, int lane, int j) {
    if (lane == 0) s_prog[wave] = j;
    const int other = s_prog[wave ^ (WGW / 2)];
    // ties go to the younger wave (w >= WGW / 2), which the arbiter would otherwise hold back: with ties to the
    // older one, the younger wave of a pair ended its loop ~1.5 us (one chunk) after it at 150000 positions
    const bool behind = wave >= WGW / 2 ? j <= other : j < other;
    if (behind) __builtin_amdgcn_s_setprio(2);
    else __builtin_amdgcn_s_setprio(0);
}

template <int WGW>
struct MergeLdsN {
    f4 o[WGW][16][64];
    float ml[WGW][2][64];
};

template <int WGW>
__device__ __forceinline__ void merge_split(MergeLdsN<WGW>& s, int wave, int lane, float& m, float& l, const f4* o,
                                            f4* om) {
    constexpr int TPW = 16 / WGW;
    // a row's l is the sum of its 4 lanes' partial sums: reduced before any fold, so that the folds see the same
    // values wherever they run (here, or in k_dec_combine for half records)
    l = half4_sum(l);
    __syncthreads();  // every wave is done with the ring (or with the previous tile's merge)
#pragma unroll
    for (int dt = 0; dt < 16; dt++) s.o[wave][dt][lane] = o[dt];
    s.ml[wave][0][lane] = m;
    s.ml[wave][1][lane] = l;
    __syncthreads();
    float mm[WGW], ll[WGW];
    f4 oo[WGW][TPW];
#pragma unroll
    for (int w = 0; w < WGW; w++) {
        mm[w] = s.ml[w][0][lane];
        ll[w] = s.ml[w][1][lane];
#pragma unroll
        for (int t = 0; t < TPW; t++) oo[w][t] = s.o[w][TPW * wave + t][lane];
    }
    // pairwise tree: level k folds state i with state i + 2^k into state i
#pragma unroll
    for (int step = 1; step < WGW; step *= 2)
#pragma unroll
        for (int w = 0; w < WGW; w += 2 * step) fold<TPW>(mm[w], ll[w], oo[w], mm[w + step], ll[w + step], oo[w + step]);
    m = mm[0];
    l = ll[0];
#pragma unroll
    for (int t = 0; t < TPW; t++) om[t] = oo[0][t];
}

// merge_split in two rounds of 8 dimension tiles, for workgroups whose LDS holds only half of MergeLdsN: round h
// exchanges tiles 8 h .. 8 h + 7, which the waves of half h of the workgroup own (wave w still owns tiles TPW w ..
// TPW w + TPW - 1).  Every fold is merge_split's, on the same values in the same order, so the results are
// bit-identical.
template <int WGW>
struct MergeLdsH {
    f4 o[WGW][8][64];
    float ml[WGW][2][64];
};

template <int WGW>
__device__ __forceinline__ void merge_split_half(MergeLdsH<WGW>& s, int wave, int lane, float& m, float& l,
                                                 const f4* o, f4* om) {
    static_assert(WGW == 8 || WGW == 4, "two rounds of 8 tiles, owned by half of the waves each");
    constexpr int TPW = 16 / WGW;
    constexpr int OWN = WGW / 2;  // owner waves per round
    l = half4_sum(l);
    const float m_in = m, l_in = l;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        __syncthreads();  // every wave is done with the previous round's (or the previous merge's) reads
#pragma unroll
        for (int dt = 0; dt < 8; dt++) s.o[wave][dt][lane] = o[8 * h + dt];
        if (h == 0) {
            s.ml[wave][0][lane] = m_in;
            s.ml[wave][1][lane] = l_in;
        }
        __syncthreads();
        if (wave / OWN == h) {
            float mm[WGW], ll[WGW];
            f4 oo[WGW][TPW];
#pragma unroll
            for (int w = 0; w < WGW; w++) {
                mm[w] = s.ml[w][0][lane];
                ll[w] = s.ml[w][1][lane];
#pragma unroll
                for (int t = 0; t < TPW; t++) oo[w][t] = s.o[w][TPW * (wave - OWN * h) + t][lane];
            }
#pragma unroll
            for (int step = 1; step < WGW; step *= 2)
#pragma unroll
                for (int w = 0; w < WGW; w += 2 * step)
                    fold<TPW>(mm[w], ll[w], oo[w], mm[w + step], ll[w + step], oo[w + step]);
            m = mm[0];
            l = ll[0];
#pragma unroll
            for (int t = 0; t < TPW; t++) om[t] = oo[0][t];
        }
    }
}

// Q / 16 as fp16 hi + lo MFMA B-operand fragments of RT row tiles, written to LDS by the whole workgroup:
// s_q[((rt * 8 + b) * 2 + part) * 64 + lane] holds, for lane (row i16, group lg) of tile rt0 + rt, the dims
// 32 b + 8 lg + k_perm(j) (part 0: hi = fp16(Q / 16), part 1: lo = fp16(Q / 16 - hi)); padding rows are zero.
// Every fragment is loaded once per workgroup: loading the rows per wave sends several times the bytes through the
// few L2 channels that hold Q, and at kernel start that load sits on every wave's critical path.  The caller
// synchronises the workgroup before reading the fragments.
template <int KVT, int RT>
__device__ __forceinline__ void q_frags_to_lds(const float* __restrict__ q, int nq, int g, int rt0, h8* s_q) {
    for (int f = threadIdx.x; f < RT * 8 * 64; f += blockDim.x) {
        const int rt = f >> 9, b = (f >> 6) & 7, ln = f & 63;
        const int r = 16 * (rt0 + rt) + (ln & 15);
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
        s_q[((rt * 8 + b) * 2 + 0) * 64 + ln] = hi;
        s_q[((rt * 8 + b) * 2 + 1) * 64 + ln] = lo;
    }
}

// ring depth (chunks in flight per wave), sized so that one 8-wave workgroup fits a CU's 160 KB of LDS
template <int KVT, int RT> struct DecCfg {
    static constexpr int NST = KVT == QWA_KV_Q4_0 ? (RT == 1 ? 3 : 2) : 1;
};

// RT row tiles starting at tile rt0 (calls with more tiles launch several passes; a row's arithmetic is the same
// in every pass and every grouping), WGW waves (classes) per workgroup.  RT = 1 keeps Q in registers; RT = 2 reads
// the Q fragments of both tiles from LDS at use (two tiles of Q and O would not fit two waves per SIMD), so each
// chunk is streamed and unpacked once for both tiles.
// WPE waves per SIMD: 2, or 1 for the three-tile verify kernel (k_dec<KVT, 3, 4, 1>: O of three tiles takes 192
// registers), whose 4-wave workgroups each write half a record (classes 8 r .. 8 r + 3 or 8 r + 4 .. 8 r + 7 of
// record r, merged along the first two levels of the 8-class tree) into record slot 2 r or 2 r + 1.
template <int KVT, int RT, int WGW, int WPE>
struct DecLds {
    using C = ChunkLds<KVT>;
    static constexpr int NST = DecCfg<KVT, RT>::NST;
    // pair_priority wherever two waves share a SIMD and its 32 bytes fit (not the F16 two-tile kernel, at 160 KB)
    static constexpr bool PRIO = WPE == 2 && RT * 8 * 2 * 64 * 16 + WGW * NST * C::BYTES + 4 * WGW <= 163840;
    // the Q fragments and the chunk ring of every wave while streaming; the partial states while merging
    union {
        struct {
            h8 q[RT * 8 * 2 * 64];  // [rt][block][hi, lo][lane]
            uint8_t ring[WGW][NST][C::BYTES];
            int prog[PRIO ? WGW : 0];  // chunk index of each wave (pair_priority)
        } a;
        MergeLdsN<WGW> merge;
    } u;
    __device__ h8* qf() { return u.a.q; }
    __device__ h8* qf_next() { return nullptr; }
    __device__ uint8_t (*rings(int w))[C::BYTES] { return u.a.ring[w]; }
    __device__ int* progs() { return u.a.prog; }
    __device__ MergeLdsN<WGW>& mg() { return u.merge; }
    __device__ MergeLdsH<WGW>& mg_half() { return *reinterpret_cast<MergeLdsH<WGW>*>(&u.merge); }
};

// LDS of the two chained passes of a Q8_0 three-tile verify (k_dec_3<Q8_0, ., true>), as Dec4ChainLds: the rings
// and the one-tile pass's Q fragments lie outside the two-tile pass's merge area (two merge rounds), and the one-tile
// pass merges over the whole area.  (F16 chunks are twice as large: its rings leave no room for it.)
template <int KVT, int WGW>
struct DecChainLds {
    using C = ChunkLds<KVT>;
    static_assert(DecCfg<KVT, 1>::NST == 1 && DecCfg<KVT, 2>::NST == 1, "one ring slot in both passes");
    union {
        struct {
            uint8_t ring[WGW][1][C::BYTES];
            h8 q1[8 * 2 * 64];  // the one-tile pass's fragments
            union {
                h8 q2[2 * 8 * 2 * 64];  // the two-tile pass's fragments
                MergeLdsH<WGW> merge;   // the two-tile pass's merge (the rings are in use)
            } u;
        } a;
        MergeLdsN<WGW> merge;  // the one-tile pass's merge
    } v;
    int prog[WGW];
};
// LDS of the one-round three-tile verify (k_dec3h): the Q fragments of the three tiles, kept for both half records,
// and the rings and half of the merge exchange beside them, so the second half's first chunks load while the first
// half merges (in two rounds); the second half merges over rings and exchange together.
template <int KVT>
struct DecHalvesLds {
    using C = ChunkLds<KVT>;
    static_assert(DecCfg<KVT, 3>::NST == 1, "one ring slot");
    h8 q[3 * 8 * 2 * 64];
    union {
        struct {
            uint8_t ring[4][1][C::BYTES];
            MergeLdsH<4> merge;
        } a;
        MergeLdsN<4> merge;
    } u;
    __device__ h8* qf() { return q; }
    __device__ h8* qf_next() { return nullptr; }
    __device__ uint8_t (*rings(int w))[C::BYTES] { return u.a.ring[w]; }
    __device__ int* progs() { return nullptr; }
    __device__ MergeLdsN<4>& mg() { return u.merge; }
    __device__ MergeLdsH<4>& mg_half() { return u.a.merge; }
};

template <int KVT, int RT, int WGW>
struct DecChainView {
    using C = ChunkLds<KVT>;
    DecChainLds<KVT, WGW>& c;
    __device__ explicit DecChainView(DecChainLds<KVT, WGW>& s) : c(s) {}
    __device__ h8* qf() { return RT == 2 ? c.v.a.u.q2 : c.v.a.q1; }
    __device__ h8* qf_next() { return RT == 2 ? c.v.a.q1 : nullptr; }
    __device__ uint8_t (*rings(int w))[C::BYTES] { return c.v.a.ring[w]; }
    __device__ int* progs() { return c.prog; }
    __device__ MergeLdsN<WGW>& mg() { return c.v.merge; }
    __device__ MergeLdsH<WGW>& mg_half() { return c.v.a.u.merge; }
};

// One workgroup (record rec of KV head g) of the F16 / Q8_0 decode; its LDS is s.  CHAIN as in dec4_body: 1 for the
// first of two chained passes (it stages the second's Q fragments, issues the second's first chunk once its own loop
// is done, and merges in two rounds), 2 for the second; 3 and 4 the same for the two half records rec, rec + 1 of
// k_dec3h (the same row tiles, so the Q fragments stay; the second half's classes are the next ones).  The arithmetic
// of a row is that of CHAIN = 0.
template <int KVT, int RT, int WGW, int WPE, int CHAIN = 0, class LDS = DecLds<KVT, RT, WGW, WPE>>
__device__ __forceinline__ void dec_body(LDS& s, const float* __restrict__ q, const qwa_kv_layer& kv, int pos0,
                                         int nq, int rt0, float* __restrict__ work, int rec, int g,
                                         unsigned long long* prof) {
    prof_start(prof);
    using C = ChunkLds<KVT>;
    constexpr int NST = DecCfg<KVT, RT>::NST;
    constexpr bool QLDS = RT > 1;
    constexpr bool PRIO = CHAIN == 1 || CHAIN == 2 || (CHAIN == 0 && DecLds<KVT, RT, WGW, WPE>::PRIO);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
    const int i16 = lane & 15, lg = lane >> 4;
    const int kmax = pos0 + nq - 1;
    const int nchunk = kmax / CHUNK + 1;
    // record r holds classes r, r + R, ..., r + 7 R (R = DEC_CLASSES / WG_CLASSES records), so the classes with one
    // chunk more than the others are spread over the records; a 4-wave workgroup (half records) takes classes
    // r + R (4 h + w) of half h = rec & 1 of record r = rec >> 1
    constexpr int R = DEC_CLASSES / WG_CLASSES;
    const int cls = !DEC_INTERLEAVE ? rec * WGW + wave
                    : WGW == WG_CLASSES ? rec + R * wave : (rec >> 1) + R * (WGW * (rec & 1) + wave);
    const int nmine = cls < nchunk ? (nchunk - 1 - cls) / DEC_CLASSES + 1 : 0;  // chunks of this wave
    const size_t rowbase = (size_t)g * kv.capacity;

#ifdef QWA_TRACE
    // the one-tile pass of a three-tile verify stamps rows 2048 + workgroup (the two-tile pass rows 0 + workgroup)
    const int trace_base = RT == 1 && rt0 >= 2 ? 2048 : 0;
#endif
    TRACE(0);
    uint8_t(*ring)[C::BYTES] = s.rings(wave);
    auto chunk_key = [&](int j) { return CHUNK * (cls + DEC_CLASSES * min(j, nmine - 1)); };
    const uint32_t koff = chunk_koff<KVT>(lane);
    auto issue = [&](uint8_t* dst, int kb) { issue_chunk<KVT>(dst, kv, rowbase, kb, kmax, lane, koff); };
    // the ring's loads go out before the Q set-up, so their HBM latency overlaps it
    if (CHAIN != 2 && CHAIN != 4 && nmine > 0) {
#pragma unroll
        for (int st = 0; st < NST; st++) issue(ring[st], chunk_key(st));
    }

    // Q / 16 as fp16 hi + lo parts, B operand of block b: lane (row i16, group lg) holds dims 32 b + 8 lg + perm(j);
    // the fragments are loaded once per workgroup through LDS
    h8* s_q = s.qf();
    if constexpr (CHAIN != 2 && CHAIN != 4) q_frags_to_lds<KVT, RT>(q, nq, g, rt0, s_q);
    if constexpr (CHAIN == 1) q_frags_to_lds<KVT, 1>(q, nq, g, rt0 + RT, s.qf_next());
    __syncthreads();
    TRACE(1);
    h8 qh[QLDS ? 1 : RT][8], ql[QLDS ? 1 : RT][8];
    if constexpr (!QLDS) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            qh[0][b] = s_q[(b * 2 + 0) * 64 + lane];
            ql[0][b] = s_q[(b * 2 + 1) * 64 + lane];
        }
    }

    // rows of this lane (S^T layout, column i16): query qt, head hh, last visible key qpos (-1: padding row)
    int qpos[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = 16 * (rt0 + rt) + i16;
        qpos[rt] = r / GRP < nq ? pos0 + r / GRP : -1;
    }
    f4 o[RT][16];
    float m[RT], l[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        m[rt] = -INFINITY;
        l[rt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 16; dt++) o[rt][dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    if (nmine > 0) {
        for (int j = 0; j < nmine; j++) {
            if constexpr (PRIO) pair_priority<WGW>(s.progs(), wave, lane, DEC_INTERLEAVE ? j - nmine : j);
            const int slot = j % NST;
            const int kb = chunk_key(j);
            wait_vmcnt<C::NLOAD * (NST - 1)>();  // this slot has landed; the later ones may still fly
            __builtin_amdgcn_wave_barrier();
            if (j == 0) TRACE(2);
            const uint8_t* kst = ring[slot];
            const uint8_t* vst = kst + C::KBYTES;
            const uint16_t* ksc = reinterpret_cast<const uint16_t*>(kst + 2 * C::KBYTES);
            const uint16_t* vsc = reinterpret_cast<const uint16_t*>(kst + 2 * C::KBYTES + C::SC);

            // ---- S^T = K Q^T (16 keys x 16 rows per tile): per block K_int . (Q_hi + Q_lo), times the key's scale
            uint32_t kd[4][4];  // block scales of this lane's 4 keys 4 lg + i
            if constexpr (KVT != QWA_KV_F16) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint4 u = *reinterpret_cast<const uint4*>(ksc + (4 * lg + i) * 8);
                    kd[i][0] = u.x; kd[i][1] = u.y; kd[i][2] = u.z; kd[i][3] = u.w;
                }
            }
            f4 S[RT];
#pragma unroll
            for (int rt = 0; rt < RT; rt++) S[rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            uint32_t dcp[RT][4];  // per-tile copies of the scale dwords (as in the Q4_0 kernel's scores)
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const h8 ka = k_block_int<KVT>(kst, i16, lg, b);
                if (KVT != QWA_KV_F16 && (b & 1) == 0) {
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            dcp[rt][i] = kd[i][b >> 1];
                            // measured: the copy gains with two tiles, not with three (one wave per SIMD)
                            if (RT == 2 && rt == 0) asm("; tile scale copy" : "+v"(dcp[rt][i]));
                        }
                }
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const h8 bh = QLDS ? s_q[((rt * 8 + b) * 2 + 0) * 64 + lane] : qh[QLDS ? 0 : rt][b];
                    const h8 bl = QLDS ? s_q[((rt * 8 + b) * 2 + 1) * 64 + lane] : ql[QLDS ? 0 : rt][b];
                    if constexpr (KVT == QWA_KV_F16) {
                        // no block scale: the blocks accumulate in the MFMA accumulator (no VALU adds, and the
                        // three-tile kernel no longer spills)
                        S[rt] = mfma16(ka, bl, mfma16(ka, bh, S[rt]));
                    } else {
                        f4 a = mfma16(ka, bh, f4{0.0f, 0.0f, 0.0f, 0.0f});
                        a = mfma16(ka, bl, a);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float d = h2f_bits((uint16_t)(dcp[rt][i] >> (16 * (b & 1))));
                            S[rt][i] = fmaf(d, a[i], S[rt][i]);
                        }
                    }
                }
            }

            // ---- online softmax, lane holding keys kb + 4 lg + i of its row.  Causal masking only in chunks that
            // reach past the first query's position.  The reference maximum m moves only when a score exceeds it by
            // more than RESCALE_T (probabilities stay <= e^RESCALE_T, far inside fp16), so O is rarely rescaled.
            const bool tail = kb + CHUNK - 1 > pos0;
            h4 p[RT];
            float cr[RT];
            bool moved = false;
#pragma unroll
            for (int rt = 0; rt < RT; rt++) {
                float sv[4];
#pragma unroll
                for (int i = 0; i < 4; i++) sv[i] = S[rt][i];
                if (tail) {
#pragma unroll
                    for (int i = 0; i < 4; i++) sv[i] = kb + 4 * lg + i <= qpos[rt] ? sv[i] : -INFINITY;
                }
                const float mx = row_max4(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
                const float mn = mx > m[rt] + RESCALE_T ? mx : m[rt];
                const float msl = (mn == -INFINITY ? 0.0f : mn) * LOG2E;  // a row that saw nothing keeps l = 0, O = 0
                cr[rt] = mn == m[rt] ? 1.0f : fast_exp2(m[rt] * LOG2E - msl);
                float rs = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float e = fast_exp2(fmaf(sv[i], LOG2E, -msl));
                    rs += e;
                    p[rt][i] = (_Float16)e;
                }
                l[rt] = l[rt] * cr[rt] + rs;
                m[rt] = mn;
                moved |= cr[rt] != 1.0f;
            }
            if (__any(moved)) {  // multiplying by exactly 1 is the identity
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
#pragma unroll
                    for (int dt = 0; dt < 16; dt++) o[rt][dt] *= cr[rt];
            }

            // ---- O^T += V^T P^T: 16 dim tiles (lane dim 16 i16 + dt), keys 4 lg .. 4 lg + 3
            VRaw<KVT> vr[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) v_raw<KVT>(vr[jj], vst, vsc, 4 * lg + jj, i16);
            // the slot is consumed once these reads have returned: the refill's direct-to-LDS writes must not land
            // before them (a refill served from L2 returns within a few hundred cycles)
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            // refill the slot with the class's next chunk, if it has one (with one slot every iteration waits for
            // vmcnt 0, so a skipped refill needs no other wait; a clamped re-read of the last chunk would put one
            // more memory round trip before the wave's merge)
            static_assert(NST == 1, "the F16 / Q8_0 ring has one slot");
            if (j + NST < nmine) issue(ring[slot], chunk_key(j + NST));
            constexpr int NW = sizeof(vr[0].w) / 4;  // raw words per 16 dims
            constexpr int DPW = 16 / NW;             // dims per raw word
#pragma unroll
            for (int wi = 0; wi < NW; wi++) {
                uint32_t w01[DPW], w23[DPW];
                v_pair_words<KVT, 1>(&vr[0].w[wi], &vr[1].w[wi], vr[0].sc, vr[1].sc, w01);
                v_pair_words<KVT, 1>(&vr[2].w[wi], &vr[3].w[wi], vr[2].sc, vr[3].sc, w23);
#pragma unroll
                for (int d = 0; d < DPW; d++) {
                    const h4 a = make_h4(w01[d], w23[d]);
#pragma unroll
                    for (int rt = 0; rt < RT; rt++) o[rt][wi * DPW + d] = mfma16k16(a, p[rt], o[rt][wi * DPW + d]);
                }
            }
        }
        wait_vmcnt<0>();  // nothing may still fly when the ring is reused or the wave exits
        // the wave's ring is read out: the chained second pass's first chunk loads while this pass merges
        if constexpr (CHAIN == 1) {
#pragma unroll
            for (int st = 0; st < NST; st++) issue(ring[st], chunk_key(st));
        }
    }
    if constexpr (CHAIN == 3) {
        // the next half record's class of this wave (as cls above, for rec + 1), whose first chunk loads while this
        // half merges
        const int cn = (rec + 1) >> 1 == rec >> 1 ? (rec >> 1) + R * (WGW * ((rec + 1) & 1) + wave) : -1;
        if (cn >= 0 && cn < nchunk) issue(ring[0], CHUNK * cn);
    }
    if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    TRACE(3);

    // ---- merge the WGW classes of each row tile, split across the waves by head dims (the fixed pairwise tree of
    // merge_split); every wave writes its dims of the records.  Lane (row i16, lg), tile dt, element i holds dim
    // 16 (4 lg + i) + dt.
    constexpr int TPW = 16 / WGW;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        f4 om[TPW];
        if constexpr (CHAIN == 1 || CHAIN == 3) merge_split_half<WGW>(s.mg_half(), wave, lane, m[rt], l[rt], o[rt], om);
        else merge_split<WGW>(s.mg(), wave, lane, m[rt], l[rt], o[rt], om);
        const int r = 16 * (rt0 + rt) + i16;
        const int qt = r / GRP, hh = r % GRP;
        const float lt = l[rt];  // already summed over the row's lanes by merge_split
        if (qpos[rt] >= 0) {
            float* recp = work + ((((size_t)rec * NKV + g) * MAXQ + qt) * GRP + hh) * REC;
            if (wave == 0 && lg == 0) {
                recp[0] = m[rt];
                recp[1] = lt;
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float* dst = recp + 4 + 16 * (4 * lg + i) + TPW * wave;
                if constexpr (TPW == 2) {
                    *reinterpret_cast<float2*>(dst) = make_float2(om[0][i], om[1][i]);
                } else {
#pragma unroll
                    for (int t = 0; t < TPW; t++) dst[t] = om[t][i];
                }
            }
        }
    }
    TRACE(4);
    prof_end(prof);
}

template <int KVT, int RT, int WGW, int WPE = 2>
__global__ void __launch_bounds__(64 * WGW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
k_dec(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int rt0, float* __restrict__ work,
      unsigned long long* prof) {
    __shared__ __attribute__((aligned(16))) DecLds<KVT, RT, WGW, WPE> s;
    dec_body<KVT, RT, WGW, WPE>(s, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, prof);
}

// The one-pass three-tile verify with both half records of record blockIdx.x in one workgroup, one after the other
// (grid (records, NKV): one round of the chip instead of two; each half is exactly k_dec<KVT, 3, 4, 1>'s code)
template <int KVT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_dec3h(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int rt0, float* __restrict__ work,
        unsigned long long* prof) {
#if QWA_DEC3H_CHAIN
    // the second half's first chunks load while the first half merges; the Q fragments serve both halves
    __shared__ __attribute__((aligned(16))) DecHalvesLds<KVT> s;
    prof_start(prof);
    dec_body<KVT, 3, 4, 1, 3>(s, q, kv, pos0, nq, rt0, work, 2 * blockIdx.x, blockIdx.y, nullptr);
    dec_body<KVT, 3, 4, 1, 4>(s, q, kv, pos0, nq, rt0, work, 2 * blockIdx.x + 1, blockIdx.y, nullptr);
    prof_end(prof);
#else
    __shared__ __attribute__((aligned(16))) DecLds<KVT, 3, 4, 1> s;
    prof_start(prof);
    dec_body<KVT, 3, 4, 1>(s, q, kv, pos0, nq, rt0, work, 2 * blockIdx.x, blockIdx.y, nullptr);
    __syncthreads();  // the first half's merge reads are done before the second half's chunks land in LDS
    dec_body<KVT, 3, 4, 1>(s, q, kv, pos0, nq, rt0, work, 2 * blockIdx.x + 1, blockIdx.y, nullptr);
    prof_end(prof);
#endif
}

// The two passes of a three-tile verify in one launch, grid (records, NKV): every workgroup runs the pass of row
// tiles rt0 and rt0 + 1 over its classes, then the pass of tile rt0 + 2 (as k_dec4_3; CHAIN: chained as there, Q8_0
// only).
template <int KVT, int WGW, bool CHAIN>
__global__ void __launch_bounds__(64 * WGW) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_dec_3(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int rt0, float* __restrict__ work,
        unsigned long long* prof) {
    if constexpr (CHAIN) {
        static_assert(KVT == QWA_KV_Q8_0, "chained passes: Q8_0 (F16 rings are too large)");
        __shared__ __attribute__((aligned(16))) DecChainLds<KVT, WGW> s;
        prof_start(prof);
        DecChainView<KVT, 2, WGW> first(s);
        dec_body<KVT, 2, WGW, 2, 1>(first, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, nullptr);
        DecChainView<KVT, 1, WGW> second(s);
        dec_body<KVT, 1, WGW, 2, 2>(second, q, kv, pos0, nq, rt0 + 2, work, blockIdx.x, blockIdx.y, nullptr);
        prof_end(prof);
    } else {
        __shared__ __attribute__((aligned(16))) union {
            DecLds<KVT, 2, WGW, 2> two;
            DecLds<KVT, 1, WGW, 2> one;
        } s;
        prof_start(prof);
        dec_body<KVT, 2, WGW, 2>(s.two, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, nullptr);
        __syncthreads();  // the first pass's merge reads are done before the second pass's chunk loads land in LDS
        dec_body<KVT, 1, WGW, 2>(s.one, q, kv, pos0, nq, rt0 + 2, work, blockIdx.x, blockIdx.y, nullptr);
        prof_end(prof);
    }
}

// ---------------------------------------------------------------------------------------------- Q4_0 decode
// The same split-K structure as k_dec, with an inner loop laid out for Q4_0 to keep the vector ALU work per KV byte
// low (the kernel has to issue ~4.6 KB of dequantisation and softmax per 16-key chunk at HBM rate):
//  * K and V both sit piece-major in LDS (16-byte piece = one 32-value block of one key): the S^T operand read is one
//    dword per block, and the P.V operand gathers byte m of a block for 4 keys from dwords that 4 lanes read together
//    (broadcast) plus one per-lane byte select per key pair;
//  * fp16 codes come from one and-or per pair (exponent trick: 0x6400 | n is 1024 + n, 0x5400 | (n << 4) is 64 + n)
//    and one exact packed subtraction; V is scaled by its fp16 block scale with one rounding (= fp16(d * (n - 8)));
//  * P.V runs as two 16-dim tiles per block (even and odd dims) that share the lane's 4 keys' block scales;
//  * full chunks load from uniform base addresses with per-lane constant offsets; only the chunk holding the
//    window's last key takes the clamped path;
//  * the softmax only rescales when some score of the chunk exceeds the running maximum by more than RESCALE_T
//    (one compare and a wave vote in the common case).
// Chunk image in LDS (bytes):
//   [0, 2048)    K values: block b of key n at (16 b + n) * 16
//   [2048, 4096) V values, same layout
//   [4096, 4352) K block scales, [key][8] fp16
//   [4352, 4608) V block scales, [key][8] fp16
struct Q4Chunk {
    static constexpr int K = 0, V = 2048, KS = 4096, VS = 4352, BYTES = 4608;
    static constexpr int NLOAD = 6;  // load instructions per chunk
};

// per-lane source offsets (bytes from the chunk's first row) of the K / V piece loads of a full chunk: instruction i,
// lane l fills slot 64 i + l = piece 4 i + l / 16 of row l % 16
struct Q4Offsets {
    uint32_t piece[2];
};

__device__ __forceinline__ Q4Offsets q4_offsets(int lane) {
    Q4Offsets o;
#pragma unroll
    for (int i = 0; i < 2; i++) o.piece[i] = (lane & 15) * 128 + 16 * (4 * i + (lane >> 4));
    return o;
}


__device__ __forceinline__ void q4_issue_full(uint32_t dst, const qwa_kv_layer& kv, size_t row0, const Q4Offsets& off,
                                              int lane) {
    const uint8_t* kb = kv.k + row0 * 128;
    const uint8_t* vb = kv.v + row0 * 128;
    const uint16_t* ksb = kv.ks + row0 * 8;
    const uint16_t* vsb = kv.vs + row0 * 8;
    dma_sv<16>(dst + Q4Chunk::K, kb, off.piece[0]);
    dma_sv<16>(dst + Q4Chunk::K + 1024, kb, off.piece[1]);
    dma_sv<16>(dst + Q4Chunk::V, vb, off.piece[0]);
    dma_sv<16>(dst + Q4Chunk::V + 1024, vb, off.piece[1]);
    dma_sv<4>(dst + Q4Chunk::KS, ksb, 4 * lane);
    dma_sv<4>(dst + Q4Chunk::VS, vsb, 4 * lane);
}

// the chunk holding key kmax: rows past kmax re-read row kmax (their scores are masked, their probabilities are 0)
__device__ __forceinline__ void q4_issue_tail(uint32_t dst, const qwa_kv_layer& kv, size_t rowbase, int kb, int kmax,
                                              int lane) {
    const size_t rk = rowbase + min(kb + (lane & 15), kmax);
    const int pc = 16 * (lane >> 4);
    dma_v<16>(dst + Q4Chunk::K, kv.k + rk * 128 + pc);
    dma_v<16>(dst + Q4Chunk::K + 1024, kv.k + rk * 128 + pc + 64);
    dma_v<16>(dst + Q4Chunk::V, kv.v + rk * 128 + pc);
    dma_v<16>(dst + Q4Chunk::V + 1024, kv.v + rk * 128 + pc + 64);
    const size_t rs = rowbase + min(kb + (lane >> 2), kmax);
    dma_v<4>(dst + Q4Chunk::KS, reinterpret_cast<const uint8_t*>(kv.ks + rs * 8) + 4 * (lane & 3));
    dma_v<4>(dst + Q4Chunk::VS, reinterpret_cast<const uint8_t*>(kv.vs + rs * 8) + 4 * (lane & 3));
}

// Bit masks / fp16 exponent patterns of the code unpacking, held in VGPRs so that each (x & mask) | pattern is one
// v_and_or_b32 (VOP3 encodings take no 32-bit literals on this target).
struct Q4Masks {
    uint32_t lo, hi, e_lo, e_hi;
};
__device__ __forceinline__ Q4Masks q4_masks() {
    Q4Masks k;
    asm volatile("v_mov_b32 %0, 0x000f000f" : "=v"(k.lo));
    asm volatile("v_mov_b32 %0, 0x00f000f0" : "=v"(k.hi));
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(k.e_lo));
    asm volatile("v_mov_b32 %0, 0x54005400" : "=v"(k.e_hi));
    return k;
}

// 8 Q4_0 codes (one dword: block elements 8 g .. 8 g + 7, element 2 j in the low nibble of byte j) as exact fp16
// integers n - 8 in the order [e0, e4, e1, e5, e2, e6, e3, e7] (k_perm<Q4_0>)
__device__ __forceinline__ h8 q4_codes(uint32_t w, const Q4Masks& k) {
    const h2 b_lo = {(_Float16)1032.0f, (_Float16)1032.0f}, b_hi = {(_Float16)72.0f, (_Float16)72.0f};
    const uint32_t w8 = w >> 8;
    const uint32_t e04 = h2_bits(bits_h2((w & k.lo) | k.e_lo) - b_lo);
    const uint32_t e15 = h2_bits(bits_h2((w & k.hi) | k.e_hi) - b_hi);
    const uint32_t e26 = h2_bits(bits_h2((w8 & k.lo) | k.e_lo) - b_lo);
    const uint32_t e37 = h2_bits(bits_h2((w8 & k.hi) | k.e_hi) - b_hi);
    return make_h8(e04, e15, e26, e37);
}

// RT row tiles per wave, WGW waves per workgroup (WGW classes, one record).  RT = 1 keeps Q in registers; RT = 2
// (verify) keeps the Q fragments of both tiles in LDS (shared by the waves), so each chunk's K codes and V operands
// are unpacked once for both tiles while the wave still fits two per SIMD.  A row's arithmetic is the same whatever
// RT is.
template <int NST, int RT, int WGW>
struct Dec4Lds {
    union {
        struct {
            h8 q[RT * 8 * 2 * 64];  // [rt][block][hi, lo][lane]
            uint8_t ring[WGW][NST][Q4Chunk::BYTES];
        } a;
        MergeLdsN<WGW> merge;
    } u;
    int prog[WGW];  // chunk index of each wave (pair_priority)
    __device__ h8* qf() { return u.a.q; }
    __device__ h8* qf_next() { return nullptr; }
    __device__ uint8_t (*rings(int w))[Q4Chunk::BYTES] { return u.a.ring[w]; }
    __device__ MergeLdsN<WGW>& mg() { return u.merge; }
    __device__ MergeLdsH<WGW>& mg_half() { return *reinterpret_cast<MergeLdsH<WGW>*>(&u.merge); }
};

// LDS of the two chained passes of a three-tile verify (k_dec4_3<., true>): while the two-tile pass merges, the
// rings (then holding the one-tile pass's first chunks) and the one-tile pass's Q fragments lie outside its merge
// area, which therefore holds half of MergeLdsN (two merge rounds); the one-tile pass merges over the whole area.
template <int WGW>
struct Dec4ChainLds {
    union {
        struct {
            uint8_t ring[WGW][2][Q4Chunk::BYTES];
            h8 q1[8 * 2 * 64];  // the one-tile pass's fragments
            union {
                h8 q2[2 * 8 * 2 * 64];  // the two-tile pass's fragments
                MergeLdsH<WGW> merge;   // the two-tile pass's merge (the rings are in use)
            } u;
        } a;
        MergeLdsN<WGW> merge;  // the one-tile pass's merge (nothing else is in use any more)
    } v;
    int prog[WGW];
};
// the view of Dec4ChainLds that one of its passes works on (RT = 2: the first pass, RT = 1: the second)
template <int RT, int WGW>
struct Dec4ChainView {
    Dec4ChainLds<WGW>& c;
    int* prog;
    __device__ explicit Dec4ChainView(Dec4ChainLds<WGW>& s) : c(s), prog(s.prog) {}
    __device__ h8* qf() { return RT == 2 ? c.v.a.u.q2 : c.v.a.q1; }
    __device__ h8* qf_next() { return RT == 2 ? c.v.a.q1 : nullptr; }
    __device__ uint8_t (*rings(int w))[Q4Chunk::BYTES] { return c.v.a.ring[w]; }
    __device__ MergeLdsH<WGW>& mg_half() { return c.v.a.u.merge; }
    __device__ MergeLdsN<WGW>& mg() { return c.v.merge; }
};

// One workgroup (record rec of KV head g) of the Q4_0 decode; its LDS is s.  CHAIN = 1: the first of two chained
// passes (it also stages the second pass's Q fragments, issues the second pass's first chunks once its own loop is
// done, and merges in two rounds); CHAIN = 2: the second (its first chunks are in flight and its Q fragments in
// LDS).  Both passes read the same chunks into the same ring slots, and the arithmetic of a row is that of CHAIN = 0.
template <int NST, int RT, int WGW, int CHAIN = 0, class LDS = Dec4Lds<NST, RT, WGW>>
__device__ __forceinline__ void dec4_body(LDS& s, const float* __restrict__ q, const qwa_kv_layer& kv, int pos0,
                                          int nq, int rt0, float* __restrict__ work, int rec, int g,
                                          unsigned long long* prof) {
    static_assert(CHAIN == 0 || NST == 2, "chained passes share one ring layout");
    prof_start(prof);
    constexpr bool QLDS = RT > 1;
    int* s_prog = s.prog;
    h8* s_q = s.qf();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, lg = lane >> 4;
    const int kmax = pos0 + nq - 1;
    const int nchunk = kmax / CHUNK + 1;
    // record rec holds classes rec, rec + R, ..., rec + 7 R (as dec_body)
    const int cls = DEC_INTERLEAVE ? rec + (DEC_CLASSES / WGW) * wave : rec * WGW + wave;
    const int nmine = cls < nchunk ? (nchunk - 1 - cls) / DEC_CLASSES + 1 : 0;
    const size_t rowbase = (size_t)g * kv.capacity;

    uint8_t(*ring)[Q4Chunk::BYTES] = s.rings(wave);
    const Q4Offsets off = q4_offsets(lane);
    auto chunk_key = [&](int j) { return CHUNK * (cls + DEC_CLASSES * j); };
    auto issue = [&](int j) {
        const int kb = chunk_key(j);
        const uint32_t dst = lds_addr(ring[j % NST]);
        if (kb + CHUNK - 1 <= kmax) q4_issue_full(dst, kv, rowbase + kb, off, lane);
        else q4_issue_tail(dst, kv, rowbase, kb, kmax, lane);
    };
#ifdef QWA_TRACE
    // the one-tile pass of a three-tile verify stamps rows 2048 + workgroup (the two-tile pass rows 0 + workgroup)
    const int trace_base = RT == 1 && rt0 >= 2 ? 2048 : 0;
#endif
    TRACE(0);
    // the first chunk's loads go out before the Q set-up, so their latency overlaps it; the rest of the ring follows
    // the set-up, so the first iteration waits for chunk 0 only
    if (CHAIN != 2 && nmine > 0) issue(0);

    // Q / 16 as fp16 hi + lo fragments, loaded once per workgroup
    if constexpr (CHAIN != 2) q_frags_to_lds<QWA_KV_Q4_0, RT>(q, nq, g, rt0, s_q);
    if constexpr (CHAIN == 1) q_frags_to_lds<QWA_KV_Q4_0, 1>(q, nq, g, rt0 + RT, s.qf_next());
    int qt[RT], hh[RT], qpos[RT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const int r = 16 * (rt0 + rt) + i16;
        qt[rt] = r / GRP;
        hh[rt] = r % GRP;
        qpos[rt] = qt[rt] < nq ? pos0 + qt[rt] : -1;  // last visible key of this lane's row (-1: padding row)
    }
    __syncthreads();
    h8 qh[QLDS ? 1 : RT][8], ql[QLDS ? 1 : RT][8];
    if constexpr (!QLDS) {
#pragma unroll
        for (int b = 0; b < 8; b++) {
            qh[0][b] = s_q[(b * 2 + 0) * 64 + lane];
            ql[0][b] = s_q[(b * 2 + 1) * 64 + lane];
        }
    }
    f4 o[RT][16];
    float m[RT], l[RT], msl[RT], mthr[RT];  // msl = m * log2(e) (0 while m = -inf), mthr = m + RESCALE_T
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
#pragma unroll
        for (int t = 0; t < 16; t++) o[rt][t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        m[rt] = -INFINITY;
        l[rt] = 0.0f;
        msl[rt] = 0.0f;
        mthr[rt] = -INFINITY;
    }

    if (nmine > 0) {
        if constexpr (CHAIN != 2) {
#pragma unroll
            for (int st = 1; st < NST; st++)
                if (st < nmine) issue(st);
        }
        const Q4Masks km = q4_masks();
        const uint32_t bsel = (uint32_t)(i16 & 3) | 0x0c000c00u | ((uint32_t)(4 + (i16 & 3)) << 16);
        // K of chunk j from LDS: the 8 code dwords of this lane and the block scales of its 4 keys
        struct KRegs {
            uint32_t w[8];
            uint32_t d[4][4];
        };
        auto read_k = [&](int j, KRegs& r) {
            const uint8_t* cst = ring[j % NST];
#pragma unroll
            for (int b = 0; b < 8; b++)
                r.w[b] = *reinterpret_cast<const uint32_t*>(cst + Q4Chunk::K + (16 * b + i16) * 16 + 4 * lg);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 u = *reinterpret_cast<const uint4*>(cst + Q4Chunk::KS + (4 * lg + i) * 16);
                r.d[i][0] = u.x; r.d[i][1] = u.y; r.d[i][2] = u.z; r.d[i][3] = u.w;
            }
        };
        // V of chunk j: byte i16 of block b for keys 4 lg + {0, 2} / {1, 3} as {byte, 0, byte, 0} (the 4 lanes of a
        // dword read it together, a per-lane byte select picks each lane's byte), and the keys' block scales
        struct VRegs {
            uint32_t x02[8], x13[8];
            uint32_t d[4][4];
        };
        auto read_v = [&](int j, VRegs& r) {
            const uint8_t* cst = ring[j % NST];
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t* vp =
                    reinterpret_cast<const uint32_t*>(cst + Q4Chunk::V + (16 * b + 4 * lg) * 16 + (i16 & 12));
                r.x02[b] = __builtin_amdgcn_perm(vp[8], vp[0], bsel);
                r.x13[b] = __builtin_amdgcn_perm(vp[12], vp[4], bsel);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 u = *reinterpret_cast<const uint4*>(cst + Q4Chunk::VS + (4 * lg + i) * 16);
                r.d[i][0] = u.x; r.d[i][1] = u.y; r.d[i][2] = u.z; r.d[i][3] = u.w;
            }
        };
        // S^T of one chunk for every row tile: per block the exact integer codes (unpacked once) times Q_hi + Q_lo,
        // times the key's block scale
        auto scores = [&](const KRegs& r, f4* S) {
#pragma unroll
            for (int rt = 0; rt < RT; rt++) S[rt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            // each row tile scales its block products from its own copy of the scale dwords (an empty asm makes the
            // copy): with one shared fp16 -> fp32 conversion the compiler issues a conversion plus an FMA per product
            // for every tile after the first, instead of one mixed-precision FMA that reads the fp16 half directly
            uint32_t dcp[RT][4];
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const h8 ka = q4_codes(r.w[b], km);
                if ((b & 1) == 0) {
#pragma unroll
                    for (int rt = 0; rt < RT; rt++)
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            dcp[rt][i] = r.d[i][b >> 1];
                            if (rt + 1 < RT) asm("; tile scale copy" : "+v"(dcp[rt][i]));
                        }
                }
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const h8 bh = QLDS ? s_q[((rt * 8 + b) * 2 + 0) * 64 + lane] : qh[QLDS ? 0 : rt][b];
                    const h8 bl = QLDS ? s_q[((rt * 8 + b) * 2 + 1) * 64 + lane] : ql[QLDS ? 0 : rt][b];
                    f4 a = mfma16(ka, bh, f4{0.0f, 0.0f, 0.0f, 0.0f});
                    a = mfma16(ka, bl, a);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        S[rt][i] = fmaf(h2f_bits((uint16_t)(dcp[rt][i] >> (16 * (b & 1)))), a[i], S[rt][i]);
                }
            }
        };
        // online softmax of chunk j (lane: keys kb + 4 lg + i of row i16) -> P^T operand, keys {0, 2}, {1, 3}
        auto softmax = [&](int j, f4 S, int rt) {
            const int kb = chunk_key(j);
            float sv[4] = {S[0], S[1], S[2], S[3]};
            if (kb + CHUNK - 1 > pos0) {
#pragma unroll
                for (int i = 0; i < 4; i++) sv[i] = kb + 4 * lg + i <= qpos[rt] ? sv[i] : -INFINITY;
            }
            const float mx4 = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            if (__any(mx4 > mthr[rt])) {
                const float mx = row_max4(mx4);
                const float mn = mx > mthr[rt] ? mx : m[rt];
                const float cr = mn == m[rt] ? 1.0f : fast_exp2((m[rt] - mn) * LOG2E);  // m = -inf: cr = 0
                if (__any(cr != 1.0f)) {
#pragma unroll
                    for (int t = 0; t < 16; t++) o[rt][t] *= cr;
                    l[rt] *= cr;
                }
                m[rt] = mn;
                msl[rt] = mn == -INFINITY ? 0.0f : mn * LOG2E;
                mthr[rt] = mn + RESCALE_T;
            }
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = fast_exp2(fmaf(sv[i], LOG2E, -msl[rt]));
            const h2 p02 = {(_Float16)p[0], (_Float16)p[2]}, p13 = {(_Float16)p[1], (_Float16)p[3]};
            const h2 one2 = {(_Float16)1.0f, (_Float16)1.0f};
            l[rt] = __builtin_amdgcn_fdot2(p13, one2, __builtin_amdgcn_fdot2(p02, one2, l[rt], false), false);
            return make_h4(h2_bits(p02), h2_bits(p13));
        };
        // O^T += V^T P^T: block b as two 16-dim tiles, even dims (tile 2 b) and odd dims (tile 2 b + 1); the lane
        // (dim pair i16, group lg) holds keys in the order {4 lg, 4 lg + 2, 4 lg + 1, 4 lg + 3}
        auto pv = [&](const VRegs& r, const h4* P) {
            const h2 b_lo = {(_Float16)1032.0f, (_Float16)1032.0f}, b_hi = {(_Float16)72.0f, (_Float16)72.0f};
#pragma unroll
            for (int b = 0; b < 8; b++) {
                const uint32_t sel = (b & 1) ? 0x07060302u : 0x05040100u;  // halfword b & 1 of both words
                const h2 d02 = bits_h2(__builtin_amdgcn_perm(r.d[2][b >> 1], r.d[0][b >> 1], sel));
                const h2 d13 = bits_h2(__builtin_amdgcn_perm(r.d[3][b >> 1], r.d[1][b >> 1], sel));
                // the V operand holds the exact codes; the keys' block scales multiply the P operand instead (the
                // lane's P keys are the keys of its V operand)
                const uint32_t e02 = h2_bits(bits_h2((r.x02[b] & km.lo) | km.e_lo) - b_lo);
                const uint32_t e13 = h2_bits(bits_h2((r.x13[b] & km.lo) | km.e_lo) - b_lo);
                const uint32_t f02 = h2_bits(bits_h2((r.x02[b] & km.hi) | km.e_hi) - b_hi);
                const uint32_t f13 = h2_bits(bits_h2((r.x13[b] & km.hi) | km.e_hi) - b_hi);
#pragma unroll
                for (int rt = 0; rt < RT; rt++) {
                    const uint2 pw = __builtin_bit_cast(uint2, P[rt]);
                    const h4 Pb = make_h4(h2_bits(bits_h2(pw.x) * d02), h2_bits(bits_h2(pw.y) * d13));
                    o[rt][2 * b] = mfma16k16(make_h4(e02, e13), Pb, o[rt][2 * b]);
                    o[rt][2 * b + 1] = mfma16k16(make_h4(f02, f13), Pb, o[rt][2 * b + 1]);
                }
            }
        };

        if constexpr (RT == 1) {
            // software-pipelined: iteration j multiplies chunk j's V while it scores chunk j + 1, so the two chunks'
            // MFMA and VALU chains interleave within the wave.  Per row the operations and their order are those of
            // one chunk after the other: the P.V of chunk j, then the softmax of chunk j + 1, whose rescale covers it.
#ifdef QWA_TRACE
            unsigned long long wsum = 0, tw = __builtin_amdgcn_s_memtime();
            const unsigned long long tloop = tw;
#endif
            TRACE(1);
            if (NST <= nmine) wait_vmcnt<Q4Chunk::NLOAD * (NST - 1)>();  // later chunks may still fly
            else wait_vmcnt<0>();
            TRACE(2);
            WTRACE(0);
            h4 P[1];
            VRegs vr;
            {
                KRegs kr;
                read_k(0, kr);
                f4 S[1];
                scores(kr, S);
                P[0] = softmax(0, S[0], 0);
                read_v(0, vr);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot 0 is read out: refill it
                if (NST < nmine) issue(NST);
            }
            for (int j = 0; j + 1 < nmine; j++) {
                pair_priority<WGW>(s_prog, wave, lane, DEC_INTERLEAVE ? j - nmine : j);
#ifdef QWA_TRACE
                tw = __builtin_amdgcn_s_memtime();
#endif
                if (j + 1 + NST <= nmine) wait_vmcnt<Q4Chunk::NLOAD * (NST - 1)>();
                else wait_vmcnt<0>();
#ifdef QWA_TRACE
                __builtin_amdgcn_s_waitcnt(0);
                wsum += __builtin_amdgcn_s_memtime() - tw;
#endif
                KRegs kr;
                read_k(j + 1, kr);
                f4 S[1];
                pv(vr, P);
                scores(kr, S);
                const h4 Pn = softmax(j + 1, S[0], 0);
                read_v(j + 1, vr);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot j + 1 is read out: refill it
                if (j + 1 + NST < nmine) issue(j + 1 + NST);
                P[0] = Pn;
            }
            pv(vr, P);
            TRACE(3);
            WTRACE(8);
#ifdef QWA_TRACE
            if (threadIdx.x == 0) dec_trace[prof_wg()][5] = wsum;
            if (threadIdx.x == 0) dec_trace[prof_wg()][6] = nmine;
            if (threadIdx.x == 0) dec_trace[prof_wg()][7] = __builtin_amdgcn_s_memtime() - tloop;
#endif
        } else {
            TRACE(1);
            for (int j = 0; j < nmine; j++) {
                pair_priority<WGW>(s_prog, wave, lane, DEC_INTERLEAVE ? j - nmine : j);
                if (j + NST <= nmine) wait_vmcnt<Q4Chunk::NLOAD * (NST - 1)>();  // later chunks may still fly
                else wait_vmcnt<0>();
                if (j == 0) TRACE(2);
                // two row tiles: V is read after the softmax, so K and V registers are never live together
                f4 S[RT];
                {
                    KRegs kr;
                    read_k(j, kr);
                    scores(kr, S);
                }
                h4 P[RT];
#pragma unroll
                for (int rt = 0; rt < RT; rt++) P[rt] = softmax(j, S[rt], rt);
                VRegs vr;
                read_v(j, vr);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // slot j is read out: refill it
                if (j + NST < nmine) issue(j + NST);
                pv(vr, P);
            }
            TRACE(3);
        }
        // the wave's ring is read out: the chained second pass's first chunks load while this pass merges
        if constexpr (CHAIN == 1) {
#pragma unroll
            for (int st = 0; st < NST; st++)
                if (st < nmine) issue(st);
        }
    }

    __builtin_amdgcn_s_setprio(0);
    // ---- merge the WGW classes of each row tile, split across the waves by head dims; every wave writes its dims of
    // the records.  Lane (row i16, lg), tile 2 b + par, element i holds dim 32 b + 8 lg + 2 i + par.
    constexpr int TPW = 16 / WGW;
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        f4 om[TPW];
        if constexpr (CHAIN == 1) merge_split_half<WGW>(s.mg_half(), wave, lane, m[rt], l[rt], o[rt], om);
        else merge_split<WGW>(s.mg(), wave, lane, m[rt], l[rt], o[rt], om);
        const float lt = l[rt];  // already summed over the row's lanes by merge_split
        if (qpos[rt] >= 0) {
            float* recp = work + ((((size_t)rec * NKV + g) * MAXQ + qt[rt]) * GRP + hh[rt]) * REC;
            if (wave == 0 && lg == 0) {
                recp[0] = m[rt];
                recp[1] = lt;
            }
#pragma unroll
            for (int t = 0; t < TPW; t += 2) {
                const int b = (TPW * wave + t) >> 1;
                float* dst = recp + 4 + 32 * b + 8 * lg;
                *reinterpret_cast<float4*>(dst) = make_float4(om[t][0], om[t + 1][0], om[t][1], om[t + 1][1]);
                *reinterpret_cast<float4*>(dst + 4) = make_float4(om[t][2], om[t + 1][2], om[t][3], om[t + 1][3]);
            }
        }
    }
    TRACE(4);
    prof_end(prof);
}

template <int NST, int RT, int WGW>
__global__ void __launch_bounds__(WGW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_dec4(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int rt0, float* __restrict__ work,
       unsigned long long* prof) {
    __shared__ __attribute__((aligned(16))) Dec4Lds<NST, RT, WGW> s;
    dec4_body<NST, RT, WGW>(s, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, prof);
}

// The two passes of a three-tile verify in one launch, grid (records, NKV): every workgroup runs the pass of row
// tiles rt0 and rt0 + 1 over its classes and then the pass of tile rt0 + 2 over the same classes, each with exactly
// the code of that pass (so a row's bits are those of any other kernel).  Against one workgroup per pass (a second
// round of workgroups filling the CUs as the first frees them) this saves the second round's dispatch and set-up, and
// the second pass re-reads chunks this CU has just brought through its L2.  CHAIN: the passes are chained
// (Dec4ChainLds), so the second pass's Q set-up and first chunks overlap the first pass's merge, at the price of that
// merge running in two rounds.
template <int WGW, bool CHAIN>
__global__ void __launch_bounds__(WGW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_dec4_3(const float* __restrict__ q, qwa_kv_layer kv, int pos0, int nq, int rt0, float* __restrict__ work,
         unsigned long long* prof) {
    if constexpr (CHAIN) {
        __shared__ __attribute__((aligned(16))) Dec4ChainLds<WGW> s;
        prof_start(prof);
        Dec4ChainView<2, WGW> first(s);
        dec4_body<2, 2, WGW, 1>(first, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, nullptr);
        Dec4ChainView<1, WGW> second(s);
        dec4_body<2, 1, WGW, 2>(second, q, kv, pos0, nq, rt0 + 2, work, blockIdx.x, blockIdx.y, nullptr);
        prof_end(prof);
    } else {
        __shared__ __attribute__((aligned(16))) union {
            Dec4Lds<2, 2, WGW> two;
            Dec4Lds<2, 1, WGW> one;
        } s;
        prof_start(prof);
        dec4_body<2, 2, WGW>(s.two, q, kv, pos0, nq, rt0, work, blockIdx.x, blockIdx.y, nullptr);
        __syncthreads();  // the first pass's merge reads are done before the second pass's chunk loads land in LDS
        dec4_body<2, 1, WGW>(s.one, q, kv, pos0, nq, rt0 + 2, work, blockIdx.x, blockIdx.y, nullptr);
        prof_end(prof);
    }
}


#if !defined(QWA_DEC_KERNELS_ONLY) && !defined(QWA_TRACE)
// Instantiated in attn_decode_ilp.hip, compiled with LLVM's iterative-ILP machine scheduler: the F16 one-pass
// three-tile verify measured 1.5-1.8 us faster per layer that way (24576-150000 positions, 7 queries), while every
// other kernel measured the same or slower (the Q4_0 two-tile pass +2 us at 150000 positions).  The schedule moves no
// arithmetic, so the bits are those of any other build.  (Trace builds instantiate it here.)
extern template __global__ void k_dec<QWA_KV_F16, 3, 4, 1>(const float* __restrict__, qwa_kv_layer, int, int, int,
                                                           float* __restrict__, unsigned long long*);
extern template __global__ void k_dec3h<QWA_KV_F16>(const float* __restrict__, qwa_kv_layer, int, int, int,
                                                    float* __restrict__, unsigned long long*);
#endif

#ifndef QWA_DEC_KERNELS_ONLY
// Combine: one workgroup per (query t, head h, quarter of the head dims).  256 threads = 64 dims x 4 slices.
// Sums run over fixed groups of CGRP consecutive splits, in split order inside a group and in group order across
// groups: the summation tree depends only on split indices, never on nq (splits past a query's window hold l = 0
// and add exact zeros).
// halves = 1: record s is the fold of slots 2 s and 2 s + 1 (the last level of the 8-class tree, the same
// arithmetic as fold()), so a record has the same bits whichever kernel wrote it.
__global__ void __launch_bounds__(256) k_dec_combine(const float* __restrict__ work, int nsplit, int halves,
                                                     const float* __restrict__ gate, float* __restrict__ out,
                                                     float* __restrict__ out_host, qwa_act_q8 oq, int do_q) {
    constexpr int MAXSPLIT = NREC;
    constexpr int MAXGRP = MAXSPLIT / CGRP;
    constexpr int GPS = MAXGRP / 4;  // groups per slice
    __shared__ float s_f[MAXSPLIT];
    __shared__ float s_lf[MAXSPLIT];
    __shared__ float s_gl[MAXGRP];
    __shared__ float s_red[4];
    __shared__ float s_ga[MAXGRP][64];
    const int t = blockIdx.x / NH, h = blockIdx.x % NH, g = h / GRP, hh = h % GRP;
    const int quarter = blockIdx.y;
    const int tid = threadIdx.x, dim = tid & 63, slice = tid >> 6;
    const size_t sstride = (size_t)NKV * MAXQ * GRP * REC;
    const float* base = work + (((size_t)g * MAXQ + t) * GRP + hh) * REC;
    const int d = 64 * quarter + dim;
    const size_t o = ((size_t)t * NH + h) * HD + d;
    // the gate of slice 0's output, loaded with the records (not one memory round trip after them)
    const float gv = slice == 0 ? gate[o] : 0.0f;

    // every load up front: this thread's O values (groups slice, slice + 4, ...) and one record's (m, l)
    float ov[GPS][CGRP], ov2[GPS][CGRP];
    const int ss = halves ? 2 : 1;  // slots per record
#pragma unroll
    for (int k = 0; k < GPS; k++)
#pragma unroll
        for (int i = 0; i < CGRP; i++) {
            const int s = (slice + 4 * k) * CGRP + i;
            ov[k][i] = s < nsplit ? base[(size_t)ss * s * sstride + 4 + d] : 0.0f;
            ov2[k][i] = s < nsplit && halves ? base[(size_t)(2 * s + 1) * sstride + 4 + d] : 0.0f;
        }
    float ms = -INFINITY, ls = 0.0f;
    if (tid < nsplit) {
        ms = base[(size_t)ss * tid * sstride];
        ls = base[(size_t)ss * tid * sstride + 1];
    }
    if (halves) {
        __shared__ float s_fa[MAXSPLIT], s_fb[MAXSPLIT];
        if (tid < nsplit) {
            // fold(): M = max(m, m2), factors exp2((m - M') log2 e) with M' = 0 when M = -inf
            const float m2 = base[(size_t)(2 * tid + 1) * sstride], l2 = base[(size_t)(2 * tid + 1) * sstride + 1];
            const float M = fmaxf(ms, m2);
            const float Ms = M == -INFINITY ? 0.0f : M;
            const float fa = fast_exp2((ms - Ms) * LOG2E), fb = fast_exp2((m2 - Ms) * LOG2E);
            ls = fmaf(ls, fa, l2 * fb);
            ms = M;
            s_fa[tid] = fa;
            s_fb[tid] = fb;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < GPS; k++)
#pragma unroll
            for (int i = 0; i < CGRP; i++) {
                const int s = (slice + 4 * k) * CGRP + i;
                if (s < nsplit) ov[k][i] = fmaf(ov[k][i], s_fa[s], ov2[k][i] * s_fb[s]);
            }
    }
    // global max over records that saw keys, then each record's factor exp(m - M) (0 for empty records)
    float mx = wave_max(ls > 0.0f ? ms : -INFINITY);
    if ((tid & 63) == 0) s_red[tid >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float f = ls > 0.0f ? __expf(ms - M) : 0.0f;
    if (tid < MAXSPLIT) {
        s_f[tid] = f;
        s_lf[tid] = ls * f;
    }
    __syncthreads();
    // L and A: sums over fixed groups of CGRP records, in record order inside a group and group order across groups
    if (tid < MAXGRP) {
        float Lg = 0.0f;
#pragma unroll
        for (int i = 0; i < CGRP; i++) Lg += s_lf[tid * CGRP + i];
        s_gl[tid] = Lg;
    }
#pragma unroll
    for (int k = 0; k < GPS; k++) {
        const int gr = slice + 4 * k;
        float A = 0.0f;
#pragma unroll
        for (int i = 0; i < CGRP; i++) A += ov[k][i] * s_f[gr * CGRP + i];
        s_ga[gr][dim] = A;
    }
    __syncthreads();
    if (slice != 0) return;
    float L = 0.0f, A = 0.0f;
    for (int gr = 0; gr < MAXGRP; gr++) {
        L += s_gl[gr];
        A += s_ga[gr][dim];
    }
    const float v = (A / L) * sigmoid(gv);
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

// Decode workgroups: 8 waves, i.e. one workgroup per CU whose two waves on each SIMD belong to it (with two 4-wave
// workgroups per CU the SIMD arbiter favours the older workgroup's waves for the whole kernel, and the younger
// workgroup finishes alone at one wave per SIMD)
constexpr int Q4_WGW = WG_CLASSES;
constexpr int DEC_WGW = WG_CLASSES;
#ifndef QWA_ONE_LAUNCH
#define QWA_ONE_LAUNCH 1
#endif
// 6..8-query verify in two passes (two tiles, one tile): both as one launch
constexpr bool ONE_LAUNCH = QWA_ONE_LAUNCH != 0;
#ifndef QWA_Q8_ONEPASS
#define QWA_Q8_ONEPASS 147456
#endif
#ifndef QWA_F16_ONEPASS
#define QWA_F16_ONEPASS 12288
#endif
#ifndef QWA_DEC3
#define QWA_DEC3 1
#endif
// Three row tiles (6..8 queries) in one pass at one wave per SIMD (k_dec3h: both half records of a record in one
// workgroup, chained), against the two passes (two tiles, one tile) as one launch; 7 queries, us per layer, one pass /
// two passes, in-process A/B of the current kernels, whole call:
//   F16  (from 12288 positions on):  31.0 / 31.0 at 8192, 34.3 / 35.7 at 12288, 38.2 / 40.6 at 16384,
//                                    42.8 / 48.1 at 24576
//   Q8_0 (from 147456 positions on): 95.5 / 85.5 at 100000, 116.7 / 111.1 at 131072, 130.2 / 130.5 at 150000,
//                                    149.9 / 154.9 at 180000, 162.7 / 167.5 at 200000
// (Q8_0's int8 conversion hides behind the second wave of the two-tile pass.)  Q4_0 keeps two passes.
constexpr bool PF3_VERIFY = QWA_DEC3 != 0;

// The one-pass three-tile verify kernel where it is used (F16 or Q8_0, 6..8 queries); false if the call takes the
// passes of one or two tiles.  The kernel's 4-wave workgroups write half records into 2 nrec slots per KV head.
template <int KVT>
static bool dec3_pass(bool three, const float* q, const qwa_kv_layer& kv, int pos0, int nq, int t, int nrec,
                      float* work, const ProfSlot& ps, hipStream_t st) {
    if constexpr (KVT != QWA_KV_Q4_0) {
        if (three) {
            if (QWA_DEC3H)
                QWA_LAUNCH_MAIN(ps, (k_dec3h<KVT>), dim3(nrec, NKV), dim3(256), st, q, kv, pos0, nq, t, work);
            else
                QWA_LAUNCH_MAIN(ps, (k_dec<KVT, 3, 4, 1>), dim3(2 * nrec, NKV), dim3(256), st, q, kv, pos0, nq, t, work);
            return true;
        }
    }
    return false;
}

template <int KVT>
static void launch_dec_kvt(const float* q, const qwa_kv_layer& kv, int pos0, int nq, int nrec, bool three,
                           float* work, hipStream_t st) {
    const int rt = (GRP * nq + 15) / 16;
    const dim3 grid(nrec, NKV);
    // two row tiles share one pass over the cache; a third tile (6..8 queries) gets a pass of its own, in the same
    // launch, unless the one-pass three-tile kernel takes the call
    if (ONE_LAUNCH && rt == 3 && !three) {
        const ProfSlot ps = profile_slot(nrec * NKV, st);
        // Q4_0: the chained passes from QWA_Q4_CHAIN_FROM positions on (bit-identical either way)
        if constexpr (KVT == QWA_KV_Q4_0) {
            if (pos0 + nq >= QWA_Q4_CHAIN_FROM)
                QWA_LAUNCH_MAIN(ps, (k_dec4_3<Q4_WGW, true>), grid, dim3(64 * Q4_WGW), st, q, kv, pos0, nq, 0, work);
            else
                QWA_LAUNCH_MAIN(ps, (k_dec4_3<Q4_WGW, false>), grid, dim3(64 * Q4_WGW), st, q, kv, pos0, nq, 0, work);
        } else if (KVT == QWA_KV_Q8_0 && pos0 + nq >= QWA_Q8_CHAIN_FROM) {
            // Q8_0: the chained passes from QWA_Q8_CHAIN_FROM positions on (bit-identical either way)
            QWA_LAUNCH_MAIN(ps, (k_dec_3<KVT, DEC_WGW, KVT == QWA_KV_Q8_0>), grid, dim3(64 * DEC_WGW), st, q, kv, pos0,
                            nq, 0, work);
        } else {
            QWA_LAUNCH_MAIN(ps, (k_dec_3<KVT, DEC_WGW, false>), grid, dim3(64 * DEC_WGW), st, q, kv, pos0, nq, 0, work);
        }
        return;
    }
    for (int t = 0; t < rt; t++) {
        const ProfSlot ps = profile_slot((three ? 2 : 1) * nrec * NKV, st);  // three: 2 nrec half records
        if constexpr (KVT == QWA_KV_Q4_0) {
            if (t + 1 < rt) {
                QWA_LAUNCH_MAIN(ps, (k_dec4<2, 2, Q4_WGW>), grid, dim3(64 * Q4_WGW), st, q, kv, pos0, nq, t, work);
                t++;
            } else {
                QWA_LAUNCH_MAIN(ps, (k_dec4<2, 1, Q4_WGW>), grid, dim3(64 * Q4_WGW), st, q, kv, pos0, nq, t, work);
            }
        } else if (dec3_pass<KVT>(three, q, kv, pos0, nq, t, nrec, work, ps, st)) {
            t += 2;
        } else if (t + 1 < rt) {
            QWA_LAUNCH_MAIN(ps, (k_dec<KVT, 2, DEC_WGW>), grid, dim3(64 * DEC_WGW), st, q, kv, pos0, nq, t, work);
            t++;
        } else {
            QWA_LAUNCH_MAIN(ps, (k_dec<KVT, 1, DEC_WGW>), grid, dim3(64 * DEC_WGW), st, q, kv, pos0, nq, t, work);
        }
    }
}

hipError_t launch_decode(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int pos0, int nq,
                         void* work, float* out, const qwa_act_q8* oq, float* out_host, hipStream_t st) {
    // one record per workgroup; workgroups past the last chunk would hold no class with a chunk
    const int nchunk = (pos0 + nq - 1) / CHUNK + 1;
    const int wgw = kvt == QWA_KV_Q4_0 ? Q4_WGW : DEC_WGW;
    // records launched: every class with a chunk must belong to one (interleaved records hold classes r + 64 w)
    const int nsplit =
        DEC_INTERLEAVE ? min(DEC_CLASSES / wgw, nchunk) : min(DEC_CLASSES / wgw, (nchunk + wgw - 1) / wgw);
    float* w = static_cast<float*>(work);
    // 6..8 queries: the one-pass three-tile kernel where it is the faster path (every path gives the same bits)
    const int npos = pos0 + nq;
    const bool three = PF3_VERIFY && (GRP * nq + 15) / 16 == 3 &&
                       ((kvt == QWA_KV_F16 && npos >= QWA_F16_ONEPASS) || (kvt == QWA_KV_Q8_0 && npos >= QWA_Q8_ONEPASS));
    if (kvt == QWA_KV_F16) launch_dec_kvt<QWA_KV_F16>(q, kv, pos0, nq, nsplit, three, w, st);
    else if (kvt == QWA_KV_Q8_0) launch_dec_kvt<QWA_KV_Q8_0>(q, kv, pos0, nq, nsplit, three, w, st);
    else launch_dec_kvt<QWA_KV_Q4_0>(q, kv, pos0, nq, nsplit, false, w, st);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const qwa_act_q8 a = oq ? *oq : qwa_act_q8{nullptr, nullptr, nullptr};
    hipLaunchKernelGGL(k_dec_combine, dim3(nq * NH, 4), dim3(256), 0, st, w, nsplit, three ? 1 : 0, gate, out, out_host, a,
                       oq != nullptr ? 1 : 0);
    return hipGetLastError();
}

#ifdef QWA_TRACE
}  // namespace qwa
extern "C" int qwa_trace_read(unsigned long long* host, int nwg) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qwa::dec_trace), sizeof(unsigned long long) * 8 * nwg);
}
extern "C" int qwa_wtrace_read(unsigned long long* host, int nwg) {
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(qwa::dec_wtrace), sizeof(unsigned long long) * 16 * nwg);
}
namespace qwa {
#endif

// ---- allocation-free decode: the partial records live in a file-scope device array instead of a work argument.
// Its size is dec_work_bytes() (25.6 MB), which covers every valid call (up to 8 queries, any context up to
// MAX_POS).  Every GPU holds its own copy at its own address, fetched once per device with hipGetSymbolAddress; host
// code never passes the array's name itself to a kernel.  All calls on one GPU share the array: calls that overlap
// on that GPU (different streams, or different threads without ordering) race on it.  The records need no clearing:
// every record a combine reads is written by the same call first.
constexpr size_t DEC_SCRATCH_FLOATS = (size_t)NSLOT * NKV * MAXQ * GRP * REC;
static __device__ __align__(256) float scratch[DEC_SCRATCH_FLOATS];
// a change of the record layout must not outgrow the static array (dec_work_bytes covers every valid call)
static_assert(DEC_SCRATCH_FLOATS * sizeof(float) >= DEC_WORK_BYTES, "decode scratch smaller than the work buffer");


static float* scratch_ptr(hipError_t* err) {
    constexpr int MAXDEV = 64;
    static std::mutex mu;
    static float* ptrs[MAXDEV] = {};
    int dev = 0;
    if ((*err = hipGetDevice(&dev)) != hipSuccess) return nullptr;
    if (dev < 0 || dev >= MAXDEV) {
        *err = hipErrorInvalidDevice;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* p = nullptr;
        if ((*err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return nullptr;
        ptrs[dev] = static_cast<float*>(p);
    }
    return ptrs[dev];
}

hipError_t launch_decode_noalloc(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int pos0, int nq,
                                 float* out, const qwa_act_q8* oq, float* out_host, hipStream_t st) {
    hipError_t e = hipSuccess;
    float* w = scratch_ptr(&e);
    if (w == nullptr) return e;
    return launch_decode(q, gate, kv, kvt, pos0, nq, w, out, oq, out_host, st);
}
#endif  // QWA_DEC_KERNELS_ONLY

}  // namespace qwa

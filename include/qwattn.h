/*
 * qwattn.h -- C ABI of the MI355X (gfx950) gated-attention path and of the Gated DeltaNet token mixer.
 *
 * Drop-in replacement for the attention / KV-cache and Gated DeltaNet operators of the reference runtime (namespace
 * q38rt::cuda, src/cuda/ops.cuh and src/cuda/prefill.cuh).  Every entry point below names the reference declaration it
 * replaces.  Conventions:
 *   - all tensors are caller-owned device memory (out_host: host memory mapped for device access);
 *   - `stream` is a hipStream_t (NULL = the default stream); every call is asynchronous and stream-ordered;
 *   - the decode `work` buffer is sized by qwa_attn_work_bytes(); the prefill workspace is held per stream by the
 *     library (reserved at set-up with qwa_attn_prefill_reserve, or on the stream's first prefill it does not
 *     cover) or passed in (qwa_attn_prefill_ws); apart from that first-use growth no operator allocates memory;
 *   - the return value is a status code (QWA_OK = 0).  Invalid arguments are rejected before anything is launched
 *     (the reference aborts in the same situations, src/cuda/ops.cu:1002-1008); the C++ shim in q38rt_attn.hpp
 *     turns a nonzero status into abort() exactly like the reference.
 * Shapes are fixed by the model: attention 24 query heads, 4 KV heads (GQA group 6), head_dim 256, 64 rotary dims;
 * Gated DeltaNet 16 key heads, 48 value heads, head dim 128, 10240 conv channels.
 */
#ifndef QWATTN_H
#define QWATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
    QWA_OK = 0,
    QWA_ERR_INVALID = 1,   /* bad argument (null pointer, unknown KV type, nq out of range, ...) */
    QWA_ERR_RANGE = 2,     /* context or position beyond what the kernels / the cache capacity support */
    QWA_ERR_HIP = 3,       /* a HIP runtime call (launch) failed */
};

/* KV cache element type.  Replaces q38rt::cuda::KVType (src/cuda/ops.cuh:99). */
enum { QWA_KV_F16 = 0, QWA_KV_Q8_0 = 1, QWA_KV_Q4_0 = 2 };

/* Per-layer KV cache, split layout.  Replaces q38rt::cuda::KVLayer (src/cuda/ops.cuh:106-113).
 * values k, v: [4 kv heads][capacity positions][qwa_kv_value_bytes] (16-byte aligned rows);
 * scales ks, vs: [4][capacity][8] fp16 bits (Q8_0 / Q4_0 only; may be NULL for F16). */
typedef struct {
    uint8_t* k;
    uint8_t* v;
    uint16_t* ks;
    uint16_t* vs;
    int capacity;
} qwa_kv_layer;

/* int8 activations with per-32 scale d and s = d * sum(q).  Replaces q38rt::cuda::ActQ8 (src/cuda/gemv.cuh:14-18). */
typedef struct {
    int8_t* q;
    float* d;
    float* s;
} qwa_act_q8;

/* Row source: element i of row r is dev[r*n + i] for i < split, else host[r*host_ld + i - split] (mapped host
 * memory).  Replaces q38rt::cuda::RowSrc (src/cuda/ops.cuh:24-34). */
typedef struct {
    const float* dev;
    const float* host;
    int split;
    int host_ld;
} qwa_row_src;

/* Bytes of one 256-value head row / of its scales.  Replace kv_value_bytes / kv_scale_bytes
 * (src/cuda/ops.cuh:103-104, src/cuda/ops.cu:966-974).  0 for an unknown type. */
size_t qwa_kv_value_bytes(int kvt);
size_t qwa_kv_scale_bytes(int kvt);

/* Replaces attn_prep (src/cuda/ops.cuh:117-118): q/k per-head RMSNorm, NeoX RoPE on dims [0,64), gate split,
 * K/V quantize-on-append at cache position `pos`.  qg [24][512] (q | gate per head), k, v [4][256]. */
int qwa_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, int pos,
                  float theta, float eps, int kvt, const qwa_kv_layer* kv, float* q_out, float* gate, void* stream);

/* Replaces attn_prep_multi (src/cuda/ops.cuh:122-124): n tokens at cache positions pos0.. and rotary positions
 * rope_pos0..; qg / k / v rows of 12288 / 1024 / 1024 floats from split device / mapped-host sources. */
int qwa_attn_prep_multi(const qwa_row_src* qg, const qwa_row_src* k, const qwa_row_src* v, const float* q_norm,
                        const float* k_norm, int pos0, int rope_pos0, int n, float theta, float eps, int kvt,
                        const qwa_kv_layer* kv, float* q_out, float* gate, void* stream);

/* Replaces attn_work_bytes (src/cuda/ops.cuh:129): size of the decode scratch for contexts up to n_pos positions
 * (covers up to 8 queries per call and the FP32 test kernel). */
size_t qwa_attn_work_bytes(int n_pos);
/* Replaces attn_max_positions (src/cuda/ops.cuh:131): 262144. */
int qwa_attn_max_positions(void);

/* Replaces attn_decode (src/cuda/ops.cuh:132-133): one query over positions [0, n_pos). */
int qwa_attn_decode(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int n_pos, void* work,
                    float* out, const qwa_act_q8* oq, void* stream);

/* Replaces attn_decode_multi (src/cuda/ops.cuh:136-137): nq (1..8) queries at positions pos0..pos0+nq-1, query t
 * seeing keys [0, pos0+t].  q / gate / out rows of 6144 floats; optional ActQ8 rows and a copy of out in mapped host
 * memory.  Each query's result is bit-identical to qwa_attn_decode on it alone. */
int qwa_attn_decode_multi(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int pos0, int nq,
                          void* work, float* out, const qwa_act_q8* oq, void* stream, float* out_host);

/* No counterpart in the reference.  attn_decode_multi without the `work` argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the partial records
 * live in a static device array of the library (qwa_attn_work_bytes() bytes, 25.6 MB per GPU, held until the process
 * ends), which covers every valid call.  The call allocates nothing.  All calls on one GPU share that array, so calls
 * that overlap on one GPU (different streams, unordered threads) race; results equal attn_decode_multi's bits. */
int qwa_attn_decode_multi_noalloc(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int pos0, int nq,
                                  float* out, const qwa_act_q8* oq, void* stream, float* out_host);

/* Replaces attn_decode_simple (src/cuda/ops.cuh:139-140): FP32 vector-ALU kernel kept for tests. */
int qwa_attn_decode_simple(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int n_pos, void* work,
                           float* out, const qwa_act_q8* oq, void* stream);

/* Replace rope_table / rope_table_pos (src/cuda/prefill.cuh:46-52): rope [B][64] = cos[32] | sin[32] of
 * pos * theta^(-2i/64); pos = p0 + t, or (M-RoPE) pos3[t*3 + i%3] from a device array [B][3]. */
int qwa_rope_table(int p0, int B, float theta, float* rope, void* stream);
int qwa_rope_table_pos(const int* pos3, int B, float theta, float* rope, void* stream);

/* Replaces attn_prep_rows (src/cuda/prefill.cuh:55-56): prep of B prefill tokens at cache positions p0.. using a
 * rope table; qg [B][12288], k / v [B][1024]; writes q / gate [B][6144] and appends K/V. */
int qwa_attn_prep_rows(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm,
                       int B, int p0, const float* rope, float eps, int kvt, const qwa_kv_layer* kv, float* q,
                       float* gate, void* stream);

/* Replaces attn_prefill (src/cuda/prefill.cuh:59-60, src/cuda/prefill.cu:899-908): causal attention of B queries at
 * positions p0..p0+B-1 over the cache [0, p0+B), output * sigmoid(gate) as fp16 bits [B][6144].  fp16 MFMA, fp32
 * accumulation.  The reference's signature has no work buffer; this kernel needs one (fp16 tile images of the KV
 * range and split partial states), held by the library per (device, stream), so calls on different streams never
 * share one.  A call the stream's workspace does not cover (the first call on a stream without a reservation, or a
 * longer context) widens it first: hipMalloc of a workspace for max(p0 + B, twice the previous max_pos) positions
 * (so a prompt prefilled chunk by chunk allocates O(log n) times); the buffer it replaces stays allocated until
 * qwa_attn_prefill_release.  Under graph capture such a call returns QWA_ERR_RANGE instead (reserve before
 * capturing).  Calls within the reservation allocate nothing. */
int qwa_attn_prefill(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                     uint16_t* out16, void* stream);

/* Set-up for qwa_attn_prefill (no reference counterpart; the engine calls it where it reserves attn_work_bytes,
 * src/runtime/engine.cpp:724): allocates (hipMalloc) the workspace of `stream` on the current device for calls with
 * B <= max_B and p0 + B <= max_pos.  A second call for the same stream keeps a large-enough workspace or allocates a
 * larger one; the smaller one is not freed (a captured graph may still use it) until qwa_attn_prefill_release, which
 * synchronises the stream and frees every workspace of the stream.  A graph that captured a prefill on the stream
 * must not be replayed after its release.  Full context (262144 positions, B = 1024) costs ~1.2 GB per stream. */
int qwa_attn_prefill_reserve(int max_B, int max_pos, void* stream);
int qwa_attn_prefill_release(void* stream);

/* attn_prefill with a caller-owned workspace (no reference counterpart): `work` of at least
 * qwa_attn_prefill_work_bytes(B, p0 + B) bytes of device memory, used only by this call's stream-ordered kernels.
 * Calls that run concurrently need distinct workspaces.  The size grows with B (up to 1024) and with p0 + B. */
size_t qwa_attn_prefill_work_bytes(int B, int n_pos);
int qwa_attn_prefill_ws(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                        uint16_t* out16, void* work, size_t work_bytes, void* stream);

/* Replaces attn_prefill_simple (src/cuda/prefill.cuh:61-62): FP32 vector-ALU version kept for tests. */
int qwa_attn_prefill_simple(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                            uint16_t* out16, void* stream);

/* Quantize-on-append of raw rows, without the norm / RoPE of prep: rows x [n][4][256] stored at positions pos0..
 * of every KV head, for K (xk) and V (xv); either may be NULL.  The store is the reference's kv_store_row
 * (src/cuda/common.cuh:54-80), exposed on its own so callers holding already-roped K can append them. */
int qwa_kv_append(const float* xk, const float* xv, int pos0, int n, int kvt, const qwa_kv_layer* kv, void* stream);

/* KV-cache lifecycle (no operator counterpart: the engine's resize, src/runtime/engine.cpp:248-275, parks "only the
 * P positions in use, per KV head" in host memory with per-head cudaMemcpy calls and restores them into a layer of
 * the new capacity; these calls do that move with the same packed layout).
 * The packed layout is the engine's park layout: K values [4][n_pos][vb], V values [4][n_pos][vb], then for Q8_0 /
 * Q4_0 K scales [4][n_pos][16 B] and V scales [4][n_pos][16 B]; qwa_kv_packed_bytes gives its size.  dst / src may
 * be device memory or pinned host memory (hipHostMalloc); the copies are stream-ordered pitched DMA transfers.
 * n_pos must fit the layer's capacity. */
long long qwa_kv_packed_bytes(int kvt, int n_pos);
int qwa_kv_pack(const qwa_kv_layer* kv, int kvt, int n_pos, void* dst, void* stream);
int qwa_kv_unpack(const void* src, const qwa_kv_layer* kv, int kvt, int n_pos, void* stream);

/* ---- Gated DeltaNet (the recurrent token mixer of the other layers) ---------------------------------------------- */

/* New tokens per qwa_deltanet_multi call (the reference's DN_MAXN = Engine::MAX_BATCH, src/cuda/ops.cu:148). */
#define QWA_DN_MAXN 7

/* Parameters of one Gated DeltaNet layer (device pointers).  Replaces q38rt::cuda::DeltaNetParams
 * (src/cuda/ops.cuh:54-62): conv_w [10240][4], dt_bias [48], ssm_a [48] (= -exp(A_log)), ssm_norm [128],
 * conv_state [2][3][10240] ping-pong (buffer = parity; rows oldest input first), ssm_state [48][128 col j][128 row i]
 * fp32 (j = value dim, i = key dim). */
typedef struct {
    const float* conv_w;
    const float* dt_bias;
    const float* ssm_a;
    const float* ssm_norm;
    float* conv_state;
    float* ssm_state;
} qwa_dn_params;

/* Token inputs of qwa_deltanet_multi.  Replaces q38rt::cuda::DNTokens (src/cuda/ops.cuh:74-91).  Pending tokens
 * (output by an earlier pass, applied to the state now): sqkv [n][10240], sbeta / salpha [n][64].  New tokens:
 * qkv [n][10240], z [n][6144], beta / alpha [n][64] (raw projections; the first 48 of each row are used).
 * oqkv / obeta / oalpha (optional, NULL when unused) receive the new tokens' inputs for a later commit; they must not
 * alias the pending inputs.  New tokens' qkv channels >= qkv_split are read from qkv_host [n][qkv_ld] (mapped host
 * memory), z channels >= z_split from z_host [n][z_ld]; a split of 10240 / 6144 or more means no host part (the
 * reference's default is 1 << 30).  o_host (optional) receives a copy of the outputs, rows of 6144. */
typedef struct {
    const float* sqkv;
    const float* sbeta;
    const float* salpha;
    const float* qkv;
    const float* z;
    const float* beta;
    const float* alpha;
    float* oqkv;
    float* obeta;
    float* oalpha;
    const float* qkv_host;
    int qkv_split, qkv_ld;
    const float* z_host;
    int z_split, z_ld;
    float* o_host;
} qwa_dn_tokens;

/* Replaces deltanet_step (src/cuda/ops.cuh:67-68): one token; the conv window is read from buffer `parity` and
 * written to buffer parity ^ 1, the state is updated in place.  o [6144] fp32, optional ActQ8 rows. */
int qwa_deltanet_step(const qwa_dn_params* p, const float* qkv, const float* z, const float* beta_raw,
                      const float* alpha_raw, int parity, float eps, float* o, const qwa_act_q8* oq, void* stream);

/* Replaces deltanet_multi (src/cuda/ops.cuh:96-97): applies n_commit pending tokens then n_new (<= QWA_DN_MAXN) new
 * tokens (outputs o [n_new][6144], optional ActQ8 rows); the conv window (to buffer cin ^ 1) and the state (in place)
 * are written back after `write_after` tokens (0 = leave both unchanged).  Bit-identical to the same tokens applied
 * one per call.  n_commit + n_new = 0 does nothing. */
int qwa_deltanet_multi(const qwa_dn_params* p, int cin, const qwa_dn_tokens* in, int n_commit, int n_new,
                       int write_after, float eps, float* o, const qwa_act_q8* oq, void* stream);

/* Replaces dn_work_bytes (src/cuda/prefill.cuh:41): scratch bytes of qwa_deltanet_rows for B tokens. */
size_t qwa_dn_work_bytes(int B);

/* Replaces deltanet_rows (src/cuda/prefill.cuh:42-44): B prefill tokens.  qkv [B][10240], z [B][6144], beta / alpha
 * raw [B][48].  Updates the conv window (read from buffer cin, the window after the B tokens written to buffer
 * cin ^ 1) and the state.  work: >= qwa_dn_work_bytes(B).  core_out [B][6144] fp32 scratch, written after qkv was
 * last read (may alias qkv).  o16 [B][6144] fp16 gated-normed output (must not overlap core_out). */
int qwa_deltanet_rows(const qwa_dn_params* p, const float* qkv, const float* z, const float* beta_raw,
                      const float* alpha_raw, int B, int cin, float eps, void* work, float* core_out, uint16_t* o16,
                      void* stream);

/* ---- Consumers of the attention output: decode GEMV over ActQ8 activations, prefill weight dequantizer --------- */

/* Weight formats, the reference's QuantFormat values (include/q38rt/q38rt_types.h:36-66), ggml block layouts
 * (src/quant/quant_formats.h:92-104).  Of the grid formats, IQ2_XXS / IQ2_XS / IQ2_S / IQ3_XXS / IQ3_S are supported
 * (the formats of the model's attention output projection); IQ1_S / IQ1_M are not. */
#define QWA_W_Q2_K 10
#define QWA_W_Q4_K 12
#define QWA_W_Q6_K 14
#define QWA_W_IQ2_XXS 16
#define QWA_W_IQ2_XS 17
#define QWA_W_IQ3_XXS 18
#define QWA_W_IQ3_S 21
#define QWA_W_IQ2_S 22
#define QWA_W_IQ4_XS 23
#define QWA_W_BF16 30

/* Bytes of one row of K weights in format fmt (0: unsupported format, or K not a multiple of the 256-weight block). */
size_t qwa_w_row_bytes(int fmt, long long K);

/* Replaces gemv_q8_supported (src/cuda/gemv.cuh:38-39): 1 if qwa_gemv_q8 has a kernel for fmt. */
int qwa_gemv_q8_supported(int fmt);

/* Replaces quantize_act_q8 (src/cuda/gemv.cuh:20-21): n_rows rows of K fp32 values (stride K) into ActQ8 (same
 * layout; d = amax / 127, q = round-half-even(x / d), s = d * sum(q) per 32 values).  K a multiple of 32. */
int qwa_quantize_act_q8(const float* x, int K, int n_rows, const qwa_act_q8* out, void* stream);

/* Replaces gemv_q8 (src/cuda/gemv.cuh:23-27): y[r] (+)= W[r, :] . act for r < N; W row-major, row_bytes apart, in
 * format fmt with K weights per row (K a multiple of 256).  QWA_ERR_INVALID for a format without a kernel. */
int qwa_gemv_q8(int fmt, const void* W, size_t row_bytes, int K, int N, const qwa_act_q8* act, float* y, void* stream,
                int accumulate);

/* Replaces gemv_q8n (src/cuda/gemv.cuh:33-36): nb (1..4) activation columns at act->q + c * act_ld (d / s at
 * + c * act_ld / 32); y[c * y_ld + r] (+)= W[r, :] . x_c.  Each column's result is bit-identical to qwa_gemv_q8 on it. */
int qwa_gemv_q8n(int fmt, const void* W, size_t row_bytes, int K, int N, const qwa_act_q8* act, int nb, int act_ld,
                 float* y, int y_ld, void* stream, int accumulate);

/* Replaces gemv_bf16 (src/cuda/gemv.cuh:29-30): y[r] = W[r, :] . x for BF16 weights [N][K] (K a multiple of 8). */
int qwa_gemv_bf16(const uint16_t* W, int K, int N, const float* x, float* y, void* stream);

/* Replaces dequant_rows_f16 (src/cuda/prefill.cuh:16-18): rows of K weights to fp16 [rows][K]; each value is the
 * reference dequantizer's fp32 value rounded to fp16 (nearest-even).  BF16 rows are accepted (row_bytes = 2 K). */
int qwa_dequant_rows_f16(int fmt, const void* W, size_t row_bytes, int K, int rows, uint16_t* out, void* stream);

/* FP16 GEMM of the prefill projections on hipBLASLt (replaces cublas_create / cublas_bind / cublas_destroy /
 * gemm_f16, src/cuda/prefill.cuh:20-29): Y[b][n] (+)= sum_k X[b][k] W[n][k] for W [N][K] fp16, X [B][ldx] fp16,
 * Y [B][ldy] fp32 (accumulate: beta = 1).  qwa_gemm_bind sets the default stream and a caller-owned workspace; after
 * it no call allocates.  A NULL stream argument to qwa_gemm_f16 means the bound stream.  NULL from qwa_gemm_create
 * means hipBLASLt could not be initialised. */
void* qwa_gemm_create(void);
int qwa_gemm_bind(void* handle, void* stream, void* workspace, size_t bytes);
void qwa_gemm_destroy(void* handle);
int qwa_gemm_f16(void* handle, const uint16_t* W, int N, int K, const uint16_t* X, int ldx, int B, float* Y, int ldy,
                 int accumulate, void* stream);
/* Set-up companion of qwa_gemm_f16 (no reference counterpart: cuBLAS picks its own kernel): times up to
 * max_candidates (<= 64; < 1 means 16) of hipBLASLt's algorithms for this shape on the caller's buffers (Y is
 * overwritten) and keeps the fastest for later qwa_gemm_f16 calls of the shape.  Synchronises the stream; refused
 * (QWA_ERR_INVALID) while the stream is capturing.  best_us (may be NULL) receives the winner's time per call. */
int qwa_gemm_tune(void* handle, const uint16_t* W, int N, int K, const uint16_t* X, int ldx, int B, float* Y, int ldy,
                  int max_candidates, void* stream, float* best_us);

/* Opt-in kernel timing (no reference counterpart; the reference times phases with env-gated GPU timers,
 * src/runtime/engine.cpp:2477-2480): between qwa_profile_begin() and qwa_profile_end(), every launch of an
 * attention call's main kernel (decode: the split-K kernel; prefill: the MFMA kernel) is launched with two HIP events
 * that take the kernel's own start and end timestamps on its stream (hipExtLaunchKernelGGL; not while the stream is
 * capturing), and each of its workgroups records the device's realtime clock when it starts and ends.
 * qwa_profile_end() synchronizes the device and returns the summed event-to-event kernel time in ms and the number
 * of timed launches; qwa_profile_device_ms() then returns the same window's summed device-clock time (per launch:
 * last workgroup end - first workgroup start), which excludes the dispatch and completion latency the events include,
 * and qwa_profile_clock_mhz() the shader clock the window's workgroups ran at (shader-clock ticks over realtime
 * ticks, summed over every workgroup's lifetime), the clock against which MFMA busy cycles convert to time.
 * At most 1024 launches of at most 4096 workgroups per window; the first qwa_profile_begin() allocates the stamp
 * buffer (128 MiB) on the current device, and events are created on first use; the library keeps both (a window
 * opened on another device moves them there).  Launches on a device other than the window's go untimed.  The calls
 * are serialised by a lock and may come from any host thread. */
int qwa_profile_begin(void);
int qwa_profile_end(double* total_ms, int* launches);
int qwa_profile_device_ms(double* total_ms);
int qwa_profile_clock_mhz(double* mhz);

/* Human-readable text of a status code, and of the last error recorded by this library in the calling thread. */
const char* qwa_status_string(int status);
const char* qwa_last_error(void);

#ifdef __cplusplus
}
#endif
#endif

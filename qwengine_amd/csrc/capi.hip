// C ABI (include/qwattn.h): argument validation, then the kernel launchers.  No operator call allocates memory.  Two
// set-up calls do: qwa_attn_prefill_reserve (the per-stream prefill workspace, freed by qwa_attn_prefill_release)
// and the opt-in timing window (qwa_profile_begin), which keeps one stamp buffer for the life of the process.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "launch.hpp"
#include "pf_workspace.hpp"
#include "qwattn_common.hpp"

namespace {

thread_local char g_err[256] = "";

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return status;
}

int from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return QWA_OK;
    return fail(QWA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool kvt_ok(int kvt) { return kvt == QWA_KV_F16 || kvt == QWA_KV_Q8_0 || kvt == QWA_KV_Q4_0; }

int check_kv(const qwa_kv_layer* kv, int kvt, const char* fn) {
    if (!kvt_ok(kvt)) return fail(QWA_ERR_INVALID, "%s: unknown KV type %d", fn, kvt);
    if (kv == nullptr || kv->k == nullptr || kv->v == nullptr)
        return fail(QWA_ERR_INVALID, "%s: KV layer without value buffers", fn);
    if (kvt != QWA_KV_F16 && (kv->ks == nullptr || kv->vs == nullptr))
        return fail(QWA_ERR_INVALID, "%s: quantized KV layer without scale buffers", fn);
    if (kv->capacity <= 0) return fail(QWA_ERR_INVALID, "%s: KV capacity %d", fn, kv->capacity);
    return QWA_OK;
}

int check_src(const qwa_row_src* s, int n, const char* what, const char* fn) {
    if (s == nullptr || (s->split > 0 && s->dev == nullptr))
        return fail(QWA_ERR_INVALID, "%s: %s row source without device pointer", fn, what);
    if (s->split < 0 || s->split > n) return fail(QWA_ERR_INVALID, "%s: %s split %d", fn, what, s->split);
    if (s->split < n && s->host == nullptr)
        return fail(QWA_ERR_INVALID, "%s: %s row source without host tail", fn, what);
    return QWA_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Prefill workspaces, one per (device, stream): the drop-in attn_prefill keeps the reference's signature (no work
// argument) and finds its stream's workspace here, so calls on different streams never share scratch.  A stream gets
// its workspace from qwa_attn_prefill_reserve at set-up, or on its first prefill that the reservation does not cover
// (outside graph capture).  Buffers are freed only by qwa_attn_prefill_release (pf_workspace.hpp).
int pf_alloc(void** p, size_t bytes) { return (int)hipMalloc(p, bytes); }
int pf_free(void* p) { return (int)hipFree(p); }
size_t pf_size(int B, int n_pos) { return qwa::prefill_work_bytes(B, n_pos); }
using PfTable = qwa::PfWorkspaces<int (*)(void**, size_t), int (*)(void*), size_t (*)(int, int)>;
std::mutex g_pf_mu;  // held from a workspace lookup until the call's kernels are enqueued
PfTable g_pf(pf_alloc, pf_free, pf_size);

// kernel timing window: each timed launch gets a slot of per-workgroup (start, end) stamps in a device buffer
constexpr int PROF_MAX = 1024;     // launches per window
struct Profile {
    bool on = false;
    int n = 0;
    unsigned long long* stamps = nullptr;  // [PROF_MAX][PROF_MAX_WG][PROF_STAMPS], allocated on the first window
    std::vector<int> nwg;                  // workgroups of each timed launch
    std::vector<hipEvent_t> ev;            // 2 per launch (around it on its stream), created on first use
    double device_ms = 0.0;                // device-clock total of the last closed window
    double clock_mhz = 0.0;                // shader clock over the workgroups' lifetimes in the last window
    int device = -1;                       // the device the stamp buffer lives on
} g_prof;
std::mutex g_prof_mu;  // the window's state is shared by every host thread that launches attention calls

}  // namespace

namespace qwa {

ProfSlot profile_slot(int nwg, hipStream_t st) {
    ProfSlot ps;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (!g_prof.on || g_prof.stamps == nullptr || g_prof.n >= PROF_MAX || nwg > PROF_MAX_WG) return ps;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != g_prof.device) return ps;  // launches on other devices go untimed
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return ps;
    const size_t idx = 2 * (size_t)g_prof.n;
    while (g_prof.ev.size() <= idx + 1) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return ps;
        g_prof.ev.push_back(e);
    }
    g_prof.nwg.push_back(nwg);
    ps.start = g_prof.ev[idx];
    ps.stop = g_prof.ev[idx + 1];
    ps.stamps = g_prof.stamps + (size_t)g_prof.n++ * PROF_MAX_WG * PROF_STAMPS;
    return ps;
}

}  // namespace qwa

extern "C" {

size_t qwa_kv_value_bytes(int kvt) { return kvt_ok(kvt) ? (size_t)qwa::value_bytes(kvt) : 0; }
size_t qwa_kv_scale_bytes(int kvt) { return kvt == QWA_KV_Q8_0 || kvt == QWA_KV_Q4_0 ? 16 : 0; }

int qwa_attn_prep_multi(const qwa_row_src* qg, const qwa_row_src* k, const qwa_row_src* v, const float* q_norm,
                        const float* k_norm, int pos0, int rope_pos0, int n, float theta, float eps, int kvt,
                        const qwa_kv_layer* kv, float* q_out, float* gate, void* stream) {
    const char* fn = "attn_prep_multi";
    int st;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (n <= 0) return fail(QWA_ERR_INVALID, "%s: n = %d", fn, n);
    if ((st = check_src(qg, 2 * qwa::NH * qwa::HD, "qg", fn)) || (st = check_src(k, qwa::NKV * qwa::HD, "k", fn)) ||
        (st = check_src(v, qwa::NKV * qwa::HD, "v", fn)))
        return st;
    if (!q_norm || !k_norm || !q_out || !gate) return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    if (pos0 < 0 || (long)pos0 + n > kv->capacity)
        return fail(QWA_ERR_RANGE, "%s: positions [%d, %d) outside the cache capacity %d", fn, pos0, pos0 + n,
                    kv->capacity);
    return from_hip(qwa::launch_prep(*qg, *k, *v, q_norm, k_norm, pos0, rope_pos0, n, theta, eps, kvt, *kv, q_out,
                                     gate, as_stream(stream)),
                    fn);
}

int qwa_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm, int pos,
                  float theta, float eps, int kvt, const qwa_kv_layer* kv, float* q_out, float* gate, void* stream) {
    const qwa_row_src sq{qg, nullptr, 2 * qwa::NH * qwa::HD, 0};
    const qwa_row_src sk{k, nullptr, qwa::NKV * qwa::HD, 0};
    const qwa_row_src sv{v, nullptr, qwa::NKV * qwa::HD, 0};
    return qwa_attn_prep_multi(&sq, &sk, &sv, q_norm, k_norm, pos, pos, 1, theta, eps, kvt, kv, q_out, gate, stream);
}

size_t qwa_attn_work_bytes(int n_pos) {
    if (n_pos < 1) n_pos = 1;
    return qwa::dec_work_bytes(n_pos);
}

int qwa_attn_max_positions(void) { return qwa::MAX_POS; }

static int check_decode(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int pos0, int nq,
                        float* out, const qwa_act_q8* oq, const char* fn) {
    int st;
    if (nq < 1 || nq > qwa::MAXQ) return fail(QWA_ERR_INVALID, "%s: %d queries (1..%d)", fn, nq, qwa::MAXQ);
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (!q || !gate || !out) return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    if (oq && (!oq->q || !oq->d || !oq->s)) return fail(QWA_ERR_INVALID, "%s: incomplete ActQ8 output", fn);
    if (pos0 < 0 || (long)pos0 + nq > qwa::MAX_POS)
        return fail(QWA_ERR_RANGE, "%s: context beyond %d positions", fn, qwa::MAX_POS);
    if ((long)pos0 + nq > kv->capacity)
        return fail(QWA_ERR_RANGE, "%s: positions up to %d beyond the cache capacity %d", fn, pos0 + nq, kv->capacity);
    return QWA_OK;
}

int qwa_attn_decode_multi(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int pos0, int nq,
                          void* work, float* out, const qwa_act_q8* oq, void* stream, float* out_host) {
    const char* fn = "attn_decode_multi";
    int st;
    if ((st = check_decode(q, gate, kv, kvt, pos0, nq, out, oq, fn))) return st;
    if (!work) return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    return from_hip(qwa::launch_decode(q, gate, *kv, kvt, pos0, nq, work, out, oq, out_host, as_stream(stream)), fn);
}

int qwa_attn_decode_multi_noalloc(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int pos0, int nq,
                                  float* out, const qwa_act_q8* oq, void* stream, float* out_host) {
    const char* fn = "attn_decode_multi_noalloc";
    int st;
    if ((st = check_decode(q, gate, kv, kvt, pos0, nq, out, oq, fn))) return st;
    // the scratch array covers every call check_decode accepts (a static_assert next to it says so)
    return from_hip(qwa::launch_decode_noalloc(q, gate, *kv, kvt, pos0, nq, out, oq, out_host, as_stream(stream)), fn);
}

int qwa_attn_decode(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int n_pos, void* work,
                    float* out, const qwa_act_q8* oq, void* stream) {
    if (n_pos < 1) return fail(QWA_ERR_INVALID, "attn_decode: n_pos = %d", n_pos);
    return qwa_attn_decode_multi(q, gate, kv, kvt, n_pos - 1, 1, work, out, oq, stream, nullptr);
}

int qwa_attn_decode_simple(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int n_pos, void* work,
                           float* out, const qwa_act_q8* oq, void* stream) {
    const char* fn = "attn_decode_simple";
    int st;
    (void)work;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (!q || !gate || !out) return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    if (oq && (!oq->q || !oq->d || !oq->s)) return fail(QWA_ERR_INVALID, "%s: incomplete ActQ8 output", fn);
    if (n_pos < 1 || n_pos > kv->capacity || n_pos > qwa::MAX_POS)
        return fail(QWA_ERR_RANGE, "%s: n_pos = %d (capacity %d)", fn, n_pos, kv->capacity);
    return from_hip(qwa::launch_decode_simple(q, gate, *kv, kvt, n_pos, out, oq, as_stream(stream)), fn);
}

int qwa_rope_table(int p0, int B, float theta, float* rope, void* stream) {
    if (B <= 0 || !rope || p0 < 0) return fail(QWA_ERR_INVALID, "rope_table: B = %d, p0 = %d", B, p0);
    return from_hip(qwa::launch_rope_table(p0, B, theta, rope, as_stream(stream)), "rope_table");
}

int qwa_rope_table_pos(const int* pos3, int B, float theta, float* rope, void* stream) {
    if (B <= 0 || !rope || !pos3) return fail(QWA_ERR_INVALID, "rope_table_pos: B = %d", B);
    return from_hip(qwa::launch_rope_table_pos(pos3, B, theta, rope, as_stream(stream)), "rope_table_pos");
}

int qwa_attn_prep_rows(const float* qg, const float* k, const float* v, const float* q_norm, const float* k_norm,
                       int B, int p0, const float* rope, float eps, int kvt, const qwa_kv_layer* kv, float* q,
                       float* gate, void* stream) {
    const char* fn = "attn_prep_rows";
    int st;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (B <= 0) return fail(QWA_ERR_INVALID, "%s: B = %d", fn, B);
    if (!qg || !k || !v || !q_norm || !k_norm || !rope || !q || !gate)
        return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    if (p0 < 0 || (long)p0 + B > kv->capacity)
        return fail(QWA_ERR_RANGE, "%s: positions [%d, %d) outside the cache capacity %d", fn, p0, p0 + B,
                    kv->capacity);
    return from_hip(qwa::launch_prep_rows(qg, k, v, q_norm, k_norm, B, p0, rope, eps, kvt, *kv, q, gate,
                                          as_stream(stream)),
                    fn);
}

static int check_prefill(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                         uint16_t* out16, const char* fn) {
    int st;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (B <= 0) return fail(QWA_ERR_INVALID, "%s: B = %d", fn, B);
    if (!q || !gate || !out16) return fail(QWA_ERR_INVALID, "%s: null pointer", fn);
    if (p0 < 0 || (long)p0 + B > kv->capacity || (long)p0 + B > qwa::MAX_POS)
        return fail(QWA_ERR_RANGE, "%s: positions [%d, %d) outside the cache capacity %d", fn, p0, p0 + B,
                    kv->capacity);
    return QWA_OK;
}

size_t qwa_attn_prefill_work_bytes(int B, int n_pos) {
    if (B <= 0 || n_pos < B || n_pos > qwa::MAX_POS) return 0;
    return qwa::prefill_work_bytes(B, n_pos);
}

int qwa_attn_prefill_ws(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                        uint16_t* out16, void* work, size_t work_bytes, void* stream) {
    const char* fn = "attn_prefill_ws";
    int st;
    if ((st = check_prefill(q, gate, kv, kvt, B, p0, out16, fn))) return st;
    if (work == nullptr) return fail(QWA_ERR_INVALID, "%s: null workspace", fn);
    const size_t need = qwa::prefill_work_bytes(B, p0 + B);
    if (work_bytes < need)
        return fail(QWA_ERR_RANGE, "%s: workspace of %zu bytes, the call needs %zu", fn, work_bytes, need);
    return from_hip(qwa::launch_prefill(q, gate, *kv, kvt, B, p0, out16, work, as_stream(stream)), fn);
}

int qwa_attn_prefill_reserve(int max_B, int max_pos, void* stream) {
    const char* fn = "attn_prefill_reserve";
    if (max_B <= 0 || max_pos < max_B || max_pos > qwa::MAX_POS)
        return fail(QWA_ERR_RANGE, "%s: max_B %d, max_pos %d", fn, max_B, max_pos);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return from_hip(e, fn);
    std::lock_guard<std::mutex> lock(g_pf_mu);
    // a second reservation on the stream widens the first; a workspace it replaces stays allocated until release
    return from_hip((hipError_t)g_pf.reserve(dev, stream, max_B, max_pos), fn);
}

int qwa_attn_prefill_release(void* stream) {
    const char* fn = "attn_prefill_release";
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return from_hip(e, fn);
    std::lock_guard<std::mutex> lock(g_pf_mu);
    if (g_pf.find(dev, stream) == nullptr) return QWA_OK;
    if ((e = hipStreamSynchronize(as_stream(stream))) != hipSuccess) return from_hip(e, fn);
    return from_hip((hipError_t)g_pf.release(dev, stream), fn);
}

int qwa_attn_prefill(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                     uint16_t* out16, void* stream) {
    const char* fn = "attn_prefill";
    int st;
    if ((st = check_prefill(q, gate, kv, kvt, B, p0, out16, fn))) return st;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return from_hip(e, fn);
    std::lock_guard<std::mutex> lock(g_pf_mu);  // until the kernels are enqueued (a release then waits for them)
    qwa::PfSlot* r = g_pf.find(dev, stream);
    if (!g_pf.covers(r, B, p0 + B)) {
        // first use on this stream, or a call past its reservation: widen it, unless the stream is being captured
        // (the graph would hold an allocation made inside the capture)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(as_stream(stream), &cs)) != hipSuccess) return from_hip(e, fn);
        if (cs != hipStreamCaptureStatusNone)
            return fail(QWA_ERR_RANGE, "%s: B = %d, p0 + B = %d during graph capture, beyond the stream's prefill "
                                       "workspace (call qwa_attn_prefill_reserve before capturing)", fn, B, p0 + B);
        // positions grow geometrically, so a prefill that walks a long prompt chunk by chunk allocates O(log n)
        // times; the buffers it outgrows stay allocated until release
        const int grow = r != nullptr ? std::min(qwa::MAX_POS, 2 * r->max_pos) : 0;
        if ((e = (hipError_t)g_pf.reserve(dev, stream, B, std::max(p0 + B, grow))) != hipSuccess) return from_hip(e, fn);
        r = g_pf.find(dev, stream);
    }
    return from_hip(qwa::launch_prefill(q, gate, *kv, kvt, B, p0, out16, r->ptr, as_stream(stream)), fn);
}

int qwa_attn_prefill_simple(const float* q, const float* gate, const qwa_kv_layer* kv, int kvt, int B, int p0,
                            uint16_t* out16, void* stream) {
    int st;
    if ((st = check_prefill(q, gate, kv, kvt, B, p0, out16, "attn_prefill_simple"))) return st;
    return from_hip(qwa::launch_prefill_simple(q, gate, *kv, kvt, B, p0, out16, as_stream(stream)),
                    "attn_prefill_simple");
}

int qwa_kv_append(const float* xk, const float* xv, int pos0, int n, int kvt, const qwa_kv_layer* kv, void* stream) {
    const char* fn = "kv_append";
    int st;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (n <= 0) return fail(QWA_ERR_INVALID, "%s: n = %d", fn, n);
    if (!xk && !xv) return fail(QWA_ERR_INVALID, "%s: neither K nor V rows given", fn);
    if (pos0 < 0 || (long)pos0 + n > kv->capacity)
        return fail(QWA_ERR_RANGE, "%s: positions [%d, %d) outside the cache capacity %d", fn, pos0, pos0 + n,
                    kv->capacity);
    return from_hip(qwa::launch_kv_append(xk, xv, pos0, n, kvt, *kv, as_stream(stream)), fn);
}

long long qwa_kv_packed_bytes(int kvt, int n_pos) {
    if (!kvt_ok(kvt) || n_pos < 0) return -1;
    return (long long)qwa::NKV * n_pos * 2 * (long long)(qwa_kv_value_bytes(kvt) + qwa_kv_scale_bytes(kvt));
}

namespace {
// one pitched copy per buffer: 4 rows (KV heads) of n_pos * row bytes, at pitch capacity * row bytes in the layer
// and n_pos * row bytes in the packed buffer
int kv_move(const qwa_kv_layer* kv, int kvt, int n_pos, uint8_t* packed, bool to_packed, void* stream,
            const char* fn) {
    int st;
    if ((st = check_kv(kv, kvt, fn))) return st;
    if (!packed) return fail(QWA_ERR_INVALID, "%s: null packed buffer", fn);
    if (n_pos < 0 || n_pos > kv->capacity)
        return fail(QWA_ERR_RANGE, "%s: %d positions do not fit the capacity %d", fn, n_pos, kv->capacity);
    if (n_pos == 0) return QWA_OK;
    const size_t vb = qwa_kv_value_bytes(kvt), sb = qwa_kv_scale_bytes(kvt), P = (size_t)n_pos;
    const size_t cap = (size_t)kv->capacity;
    uint8_t* bufs[4] = {kv->k, kv->v, reinterpret_cast<uint8_t*>(kv->ks), reinterpret_cast<uint8_t*>(kv->vs)};
    const size_t row[4] = {vb, vb, sb, sb};
    size_t off = 0;
    for (int i = 0; i < (sb ? 4 : 2); i++) {
        const size_t w = P * row[i];
        hipError_t e;
        if (to_packed)
            e = hipMemcpy2DAsync(packed + off, w, bufs[i], cap * row[i], w, qwa::NKV, hipMemcpyDefault,
                                 as_stream(stream));
        else
            e = hipMemcpy2DAsync(bufs[i], cap * row[i], packed + off, w, w, qwa::NKV, hipMemcpyDefault,
                                 as_stream(stream));
        if (e != hipSuccess) return from_hip(e, fn);
        off += (size_t)qwa::NKV * w;
    }
    return QWA_OK;
}
}  // namespace

int qwa_kv_pack(const qwa_kv_layer* kv, int kvt, int n_pos, void* dst, void* stream) {
    return kv_move(kv, kvt, n_pos, static_cast<uint8_t*>(dst), true, stream, "kv_pack");
}

int qwa_kv_unpack(const void* src, const qwa_kv_layer* kv, int kvt, int n_pos, void* stream) {
    return kv_move(kv, kvt, n_pos, static_cast<uint8_t*>(const_cast<void*>(src)), false, stream, "kv_unpack");
}

// ---- Gated DeltaNet
namespace {
int check_dn_params(const qwa_dn_params* p, const char* fn) {
    if (p == nullptr || !p->conv_w || !p->dt_bias || !p->ssm_a || !p->ssm_norm || !p->conv_state || !p->ssm_state)
        return fail(QWA_ERR_INVALID, "%s: incomplete DeltaNet parameters", fn);
    return QWA_OK;
}
}  // namespace

int qwa_deltanet_multi(const qwa_dn_params* p, int cin, const qwa_dn_tokens* in, int n_commit, int n_new,
                       int write_after, float eps, float* o, const qwa_act_q8* oq, void* stream) {
    const char* fn = "deltanet_multi";
    int st;
    if ((st = check_dn_params(p, fn))) return st;
    if (in == nullptr) return fail(QWA_ERR_INVALID, "%s: no token inputs", fn);
    if (n_commit < 0 || n_new < 0) return fail(QWA_ERR_INVALID, "%s: n_commit %d, n_new %d", fn, n_commit, n_new);
    if (n_new > QWA_DN_MAXN) return fail(QWA_ERR_RANGE, "%s: %d new tokens > %d", fn, n_new, QWA_DN_MAXN);
    if (n_commit + n_new == 0) return QWA_OK;  // nothing to apply (the reference returns too)
    if (cin != 0 && cin != 1) return fail(QWA_ERR_INVALID, "%s: conv buffer %d (0 or 1)", fn, cin);
    if (write_after < 0 || write_after > n_commit + n_new)
        return fail(QWA_ERR_RANGE, "%s: write_after %d outside [0, %d]", fn, write_after, n_commit + n_new);
    if (n_commit > 0 && (!in->sqkv || !in->sbeta || !in->salpha))
        return fail(QWA_ERR_INVALID, "%s: pending tokens without saved inputs", fn);
    if (n_new > 0 && (!in->qkv || !in->z || !in->beta || !in->alpha || !o))
        return fail(QWA_ERR_INVALID, "%s: new tokens without inputs or output", fn);
    if (n_new > 0 && in->qkv_split < 10240 && (in->qkv_split < 0 || !in->qkv_host || in->qkv_ld < 10240 - in->qkv_split))
        return fail(QWA_ERR_INVALID, "%s: qkv host part (split %d, ld %d)", fn, in->qkv_split, in->qkv_ld);
    if (n_new > 0 && in->z_split < 6144 && (in->z_split < 0 || !in->z_host || in->z_ld < 6144 - in->z_split))
        return fail(QWA_ERR_INVALID, "%s: z host part (split %d, ld %d)", fn, in->z_split, in->z_ld);
    if ((in->obeta == nullptr) != (in->oalpha == nullptr))
        return fail(QWA_ERR_INVALID, "%s: obeta and oalpha must be given together", fn);
    if (oq && (!oq->q || !oq->d || !oq->s)) return fail(QWA_ERR_INVALID, "%s: incomplete ActQ8 output", fn);
    return from_hip(qwa::launch_dn_multi(*p, cin, *in, n_commit, n_new, write_after, eps, o, oq, as_stream(stream)),
                    fn);
}

int qwa_deltanet_step(const qwa_dn_params* p, const float* qkv, const float* z, const float* beta_raw,
                      const float* alpha_raw, int parity, float eps, float* o, const qwa_act_q8* oq, void* stream) {
    qwa_dn_tokens in = {};
    in.qkv = qkv;
    in.z = z;
    in.beta = beta_raw;
    in.alpha = alpha_raw;
    in.qkv_split = 1 << 30;
    in.z_split = 1 << 30;
    return qwa_deltanet_multi(p, parity, &in, 0, 1, 1, eps, o, oq, stream);
}

size_t qwa_dn_work_bytes(int B) { return B > 0 ? qwa::dn_work_bytes(B) : 0; }

int qwa_deltanet_rows(const qwa_dn_params* p, const float* qkv, const float* z, const float* beta_raw,
                      const float* alpha_raw, int B, int cin, float eps, void* work, float* core_out, uint16_t* o16,
                      void* stream) {
    const char* fn = "deltanet_rows";
    int st;
    if ((st = check_dn_params(p, fn))) return st;
    if (B <= 0 || B > 65535) return fail(QWA_ERR_RANGE, "%s: B = %d", fn, B);
    if (cin != 0 && cin != 1) return fail(QWA_ERR_INVALID, "%s: conv buffer %d (0 or 1)", fn, cin);
    if (!qkv || !z || !beta_raw || !alpha_raw || !work || !core_out || !o16)
        return fail(QWA_ERR_INVALID, "%s: missing buffer", fn);
    return from_hip(qwa::launch_dn_rows(*p, qkv, z, beta_raw, alpha_raw, B, cin, eps, work, core_out, o16,
                                        as_stream(stream)),
                    fn);
}

// status and message for the host-only sources of the library (gemm.cpp)
extern "C" __attribute__((visibility("hidden"))) int qwa_fail_status(int status, const char* what) {
    return fail(status, "%s", what);
}

// ---- consumers of the attention output (gemv.hip)
size_t qwa_w_row_bytes(int fmt, long long K) { return qwa::w_row_bytes(fmt, K); }

int qwa_gemv_q8_supported(int fmt) { return qwa::gemv_q8_supported(fmt) ? 1 : 0; }

int qwa_quantize_act_q8(const float* x, int K, int n_rows, const qwa_act_q8* out, void* stream) {
    const char* fn = "quantize_act_q8";
    if (K <= 0 || K % 32 || n_rows <= 0) return fail(QWA_ERR_RANGE, "%s: K = %d, n_rows = %d", fn, K, n_rows);
    if (!x || !out || !out->q || !out->d || !out->s) return fail(QWA_ERR_INVALID, "%s: missing buffer", fn);
    if ((long long)K * n_rows / 32 > 8LL * 65535 * 1024) return fail(QWA_ERR_RANGE, "%s: too many values", fn);
    return from_hip(qwa::launch_act_q8(x, (long long)K * n_rows, *out, as_stream(stream)), fn);
}

int qwa_gemv_q8n(int fmt, const void* W, size_t row_bytes, int K, int N, const qwa_act_q8* act, int nb, int act_ld,
                 float* y, int y_ld, void* stream, int accumulate) {
    const char* fn = "gemv_q8";
    if (!qwa::gemv_q8_supported(fmt)) return fail(QWA_ERR_INVALID, "%s: no kernel for weight format %d", fn, fmt);
    if (K <= 0 || K % 256 || N <= 0) return fail(QWA_ERR_RANGE, "%s: K = %d, N = %d", fn, K, N);
    if (row_bytes < qwa::w_row_bytes(fmt, K))
        return fail(QWA_ERR_RANGE, "%s: row_bytes %zu < %zu", fn, row_bytes, qwa::w_row_bytes(fmt, K));
    if (nb < 1 || nb > 4) return fail(QWA_ERR_RANGE, "%s: %d columns (1..4)", fn, nb);
    if (nb > 1 && (act_ld < K || act_ld % 32)) return fail(QWA_ERR_RANGE, "%s: act_ld %d", fn, act_ld);
    if (nb > 1 && y_ld < N) return fail(QWA_ERR_RANGE, "%s: y_ld %d < N %d", fn, y_ld, N);
    if (!W || !act || !act->q || !act->d || !act->s || !y) return fail(QWA_ERR_INVALID, "%s: missing buffer", fn);
    return from_hip(qwa::launch_gemv_q8(fmt, W, row_bytes, K, N, *act, nb, nb > 1 ? act_ld : K, y, nb > 1 ? y_ld : N,
                                        accumulate ? 1 : 0, as_stream(stream)),
                    fn);
}

int qwa_gemv_q8(int fmt, const void* W, size_t row_bytes, int K, int N, const qwa_act_q8* act, float* y, void* stream,
                int accumulate) {
    return qwa_gemv_q8n(fmt, W, row_bytes, K, N, act, 1, K, y, N, stream, accumulate);
}

int qwa_gemv_bf16(const uint16_t* W, int K, int N, const float* x, float* y, void* stream) {
    const char* fn = "gemv_bf16";
    if (K <= 0 || K % 8 || N <= 0) return fail(QWA_ERR_RANGE, "%s: K = %d, N = %d", fn, K, N);
    if (!W || !x || !y) return fail(QWA_ERR_INVALID, "%s: missing buffer", fn);
    return from_hip(qwa::launch_gemv_bf16(W, K, N, x, y, as_stream(stream)), fn);
}

int qwa_dequant_rows_f16(int fmt, const void* W, size_t row_bytes, int K, int rows, uint16_t* out, void* stream) {
    const char* fn = "dequant_rows_f16";
    if (qwa::w_row_bytes(fmt, K) == 0) return fail(QWA_ERR_INVALID, "%s: weight format %d, K = %d", fn, fmt, K);
    if (rows <= 0) return fail(QWA_ERR_RANGE, "%s: rows = %d", fn, rows);
    if (row_bytes < qwa::w_row_bytes(fmt, K))
        return fail(QWA_ERR_RANGE, "%s: row_bytes %zu < %zu", fn, row_bytes, qwa::w_row_bytes(fmt, K));
    if (fmt == QWA_W_BF16 && row_bytes != (size_t)K * 2)
        return fail(QWA_ERR_RANGE, "%s: BF16 rows must be contiguous (row_bytes = 2 K)", fn);
    if (!W || !out) return fail(QWA_ERR_INVALID, "%s: missing buffer", fn);
    return from_hip(qwa::launch_dequant_f16(fmt, W, row_bytes, K, rows, out, as_stream(stream)), fn);
}

int qwa_profile_begin(void) {
    const size_t bytes = (size_t)PROF_MAX * qwa::PROF_MAX_WG * qwa::PROF_STAMPS * sizeof(unsigned long long);
    std::lock_guard<std::mutex> lk(g_prof_mu);
    int dev = -1;
    hipError_t de = hipGetDevice(&dev);
    if (de != hipSuccess) return from_hip(de, "profile_begin");
    if (g_prof.stamps != nullptr && dev != g_prof.device) {
        // a window on another device: the stamp buffer and events follow it
        int cur = dev;
        de = hipSetDevice(g_prof.device);
        if (de == hipSuccess) {
            (void)hipFree(g_prof.stamps);
            for (hipEvent_t ev : g_prof.ev) (void)hipEventDestroy(ev);
            de = hipSetDevice(cur);
        }
        g_prof.stamps = nullptr;
        g_prof.ev.clear();
        if (de != hipSuccess) return from_hip(de, "profile_begin");
    }
    if (g_prof.stamps == nullptr) {
        const hipError_t e = hipMalloc(&g_prof.stamps, bytes);
        if (e != hipSuccess) {
            g_prof.stamps = nullptr;
            return from_hip(e, "profile_begin");
        }
        g_prof.device = dev;
    }
    const hipError_t e = hipMemset(g_prof.stamps, 0, bytes);
    if (e != hipSuccess) return from_hip(e, "profile_begin");
    g_prof.on = true;
    g_prof.n = 0;
    g_prof.nwg.clear();
    return QWA_OK;
}

int qwa_profile_end(double* total_ms, int* launches) {
    constexpr int NS = qwa::PROF_STAMPS;
    std::lock_guard<std::mutex> lk(g_prof_mu);
    g_prof.on = false;
    double tot = 0.0, dev_tot = 0.0, clk_ticks = 0.0, rt_ticks = 0.0;
    const int n = g_prof.n;
    g_prof.device_ms = 0.0;
    g_prof.clock_mhz = 0.0;
    int khz = 0;
    if (n > 0) {
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return from_hip(e, "profile_end");
        int dev = 0;
        e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
        if (e != hipSuccess) return from_hip(e, "profile_end");
        if (khz <= 0) return fail(QWA_ERR_HIP, "profile_end: no wall-clock rate");
        std::vector<unsigned long long> h((size_t)n * qwa::PROF_MAX_WG * NS);
        e = hipMemcpy(h.data(), g_prof.stamps, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost);
        if (e != hipSuccess) return from_hip(e, "profile_end");
        for (int i = 0; i < n; i++) {
            const unsigned long long* st = h.data() + (size_t)i * qwa::PROF_MAX_WG * NS;
            unsigned long long t0 = ~0ull, t1 = 0;
            for (int w = 0; w < g_prof.nwg[i]; w++) {
                const unsigned long long* s = st + (size_t)NS * w;
                if (s[0] == 0 || s[1] == 0) return fail(QWA_ERR_HIP, "profile_end: missing stamp");
                t0 = s[0] < t0 ? s[0] : t0;
                t1 = s[1] > t1 ? s[1] : t1;
                rt_ticks += (double)(s[1] - s[0]);
                clk_ticks += (double)(s[3] - s[2]);
            }
            dev_tot += (double)(t1 - t0) / (double)khz;  // ticks / kHz = ms
            float ms = 0.0f;
            e = hipEventElapsedTime(&ms, g_prof.ev[2 * (size_t)i], g_prof.ev[2 * (size_t)i + 1]);
            if (e != hipSuccess) return from_hip(e, "profile_end");
            tot += ms;
        }
    }
    g_prof.device_ms = dev_tot;
    // shader-clock ticks per realtime tick over every workgroup's lifetime, times the realtime rate
    g_prof.clock_mhz = rt_ticks > 0.0 ? clk_ticks / rt_ticks * (double)khz / 1000.0 : 0.0;
    if (total_ms) *total_ms = tot;
    if (launches) *launches = n;
    g_prof.n = 0;
    g_prof.nwg.clear();
    return QWA_OK;
}

int qwa_profile_device_ms(double* total_ms) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (total_ms) *total_ms = g_prof.device_ms;
    return QWA_OK;
}

int qwa_profile_clock_mhz(double* mhz) {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (mhz) *mhz = g_prof.clock_mhz;
    return QWA_OK;
}

const char* qwa_status_string(int status) {
    switch (status) {
        case QWA_OK: return "ok";
        case QWA_ERR_INVALID: return "invalid argument";
        case QWA_ERR_RANGE: return "out of range";
        case QWA_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* qwa_last_error(void) { return g_err; }

}  // extern "C"

// End-to-end drive of the attention path through the C++ shim (include/q38rt_attn.hpp), written the way the
// reference engine calls its operators (src/runtime/engine.cpp:1587-1592 for decode, :2457-2479 for prefill):
//   prefill of B tokens:  rope_table -> attn_prep_rows -> attn_prefill (drop-in call, workspace reserved on first use)
//   decode of nq tokens:  attn_prep_multi (device RowSrc) -> attn_decode_multi (with the ActQ8 epilogue)
// Test infrastructure: tests/test_gpu_shim_e2e.py writes the inputs, runs this program on the GPU and checks its
// outputs against the ctypes path and the oracle.
//
// usage: shim_e2e <in.bin> <out.bin>
//   in.bin:  int32 kvt, B, nq, capacity; float32 qg_pf[B][12288], k_pf[B][1024], v_pf[B][1024], q_norm[256],
//            k_norm[256], qg_dec[nq][12288], k_dec[nq][1024], v_dec[nq][1024]
//   out.bin: uint16 out16[B][6144]; float32 q_pf[B][6144], gate_pf[B][6144], q_dec[nq][6144], gate_dec[nq][6144],
//            out[nq][6144]; int8 act_q[nq*6144]; float32 act_d[nq*192], act_s[nq*192];
//            uint8 k[4][cap][vb], v[4][cap][vb]; uint16 ks[4][cap][8], vs[4][cap][8] (quantized formats only)
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "q38rt_attn.hpp"

using namespace q38rt;

#define HIP_OK(x)                                                                               \
    do {                                                                                        \
        hipError_t e_ = (x);                                                                    \
        if (e_ != hipSuccess) {                                                                 \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                       \
        }                                                                                       \
    } while (0)

template <class T>
static T* dev_alloc(size_t n) {
    void* p = nullptr;
    HIP_OK(hipMalloc(&p, n * sizeof(T) + 16));
    HIP_OK(hipMemset(p, 0, n * sizeof(T) + 16));
    return static_cast<T*>(p);
}

template <class T>
static T* upload(FILE* f, size_t n) {
    std::vector<T> h(n);
    if (std::fread(h.data(), sizeof(T), n, f) != n) {
        std::fprintf(stderr, "short input\n");
        std::exit(3);
    }
    T* d = dev_alloc<T>(n);
    HIP_OK(hipMemcpy(d, h.data(), n * sizeof(T), hipMemcpyHostToDevice));
    return d;
}

template <class T>
static void download(FILE* f, const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    std::fwrite(h.data(), sizeof(T), n, f);
}

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s in.bin out.bin\n", argv[0]);
        return 1;
    }
    FILE* in = std::fopen(argv[1], "rb");
    if (!in) return 1;
    int32_t hdr[4];
    if (std::fread(hdr, sizeof(int32_t), 4, in) != 4) return 3;
    const auto kvt = static_cast<cuda::KVType>(hdr[0]);
    const int B = hdr[1], nq = hdr[2], cap = hdr[3];
    const float theta = 1e7f, eps = 1e-6f;

    const float* qg_pf = upload<float>(in, (size_t)B * 12288);
    const float* k_pf = upload<float>(in, (size_t)B * 1024);
    const float* v_pf = upload<float>(in, (size_t)B * 1024);
    const float* qn = upload<float>(in, 256);
    const float* kn = upload<float>(in, 256);
    const float* qg_dec = upload<float>(in, (size_t)nq * 12288);
    const float* k_dec = upload<float>(in, (size_t)nq * 1024);
    const float* v_dec = upload<float>(in, (size_t)nq * 1024);
    std::fclose(in);

    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    cuda::KVLayer kv;
    const size_t vb = cuda::kv_value_bytes(kvt), sb = cuda::kv_scale_bytes(kvt);
    kv.capacity = cap;
    kv.k = dev_alloc<uint8_t>((size_t)4 * cap * vb);
    kv.v = dev_alloc<uint8_t>((size_t)4 * cap * vb);
    if (sb) {
        kv.ks = dev_alloc<uint16_t>((size_t)4 * cap * 8);
        kv.vs = dev_alloc<uint16_t>((size_t)4 * cap * 8);
    }

    // ---- prefill of B tokens at positions 0..B-1
    float* rope = dev_alloc<float>((size_t)B * 64);
    float* q_pf = dev_alloc<float>((size_t)B * 6144);
    float* gate_pf = dev_alloc<float>((size_t)B * 6144);
    uint16_t* out16 = dev_alloc<uint16_t>((size_t)B * 6144);
    cuda::rope_table(0, B, theta, rope, st);
    cuda::attn_prep_rows(qg_pf, k_pf, v_pf, qn, kn, B, 0, rope, eps, kvt, kv, q_pf, gate_pf, st);
    // no set-up call, as in the unchanged engine: the first prefill on the stream reserves its workspace
    cuda::attn_prefill(q_pf, gate_pf, kv, kvt, B, 0, reinterpret_cast<__half*>(out16), st);

    // ---- decode / verify of nq tokens at positions B..B+nq-1
    float* q_dec = dev_alloc<float>((size_t)nq * 6144);
    float* gate_dec = dev_alloc<float>((size_t)nq * 6144);
    float* out = dev_alloc<float>((size_t)nq * 6144);
    cuda::ActQ8 act;
    act.q = dev_alloc<int8_t>((size_t)nq * 6144);
    act.d = dev_alloc<float>((size_t)nq * 192);
    act.s = dev_alloc<float>((size_t)nq * 192);
    void* work = dev_alloc<uint8_t>(cuda::attn_work_bytes(B + nq));
    cuda::attn_prep_multi(cuda::RowSrc::device(qg_dec, 12288), cuda::RowSrc::device(k_dec, 1024),
                          cuda::RowSrc::device(v_dec, 1024), qn, kn, B, B, nq, theta, eps, kvt, kv, q_dec, gate_dec,
                          st);
    cuda::attn_decode_multi(q_dec, gate_dec, kv, kvt, B, nq, work, out, &act, st);
    HIP_OK(hipStreamSynchronize(st));

    FILE* o = std::fopen(argv[2], "wb");
    if (!o) return 1;
    download(o, out16, (size_t)B * 6144);
    download(o, q_pf, (size_t)B * 6144);
    download(o, gate_pf, (size_t)B * 6144);
    download(o, q_dec, (size_t)nq * 6144);
    download(o, gate_dec, (size_t)nq * 6144);
    download(o, out, (size_t)nq * 6144);
    download(o, act.q, (size_t)nq * 6144);
    download(o, act.d, (size_t)nq * 192);
    download(o, act.s, (size_t)nq * 192);
    download(o, kv.k, (size_t)4 * cap * vb);
    download(o, kv.v, (size_t)4 * cap * vb);
    if (sb) {
        download(o, kv.ks, (size_t)4 * cap * 8);
        download(o, kv.vs, (size_t)4 * cap * 8);
    }
    std::fclose(o);
    cuda::attn_prefill_release(st);
    HIP_OK(hipStreamDestroy(st));
    std::printf("shim_e2e ok: kvt %d, B %d, nq %d\n", hdr[0], B, nq);
    return 0;
}

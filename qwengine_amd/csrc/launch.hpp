// Internal launchers (host side).  Argument validation lives in capi.hip; these assume valid arguments.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "qwattn.h"

namespace qwa {

// opt-in kernel timing (qwa_profile_begin / qwa_profile_end): before a main kernel launch of nwg workgroups the
// launcher asks for a slot of PROF_STAMPS * nwg stamps and a pair of HIP events (stamps == nullptr when timing is off
// or the stream is capturing), and launches through QWA_LAUNCH_MAIN: under a window the launch goes through
// hipExtLaunchKernelGGL, which gives the two events the kernel's own start and end timestamps on its stream.  Wave 0
// of workgroup w writes, at its start, the realtime clock to slot[4 w] and the shader clock to slot[4 w + 2], and
// after the workgroup's last store the same two clocks to slot[4 w + 1] and slot[4 w + 3]: their ratio is the shader
// clock the launch ran at.
constexpr int PROF_MAX_WG = 4096;
constexpr int PROF_STAMPS = 4;
struct ProfSlot {
    unsigned long long* stamps = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
};
ProfSlot profile_slot(int nwg, hipStream_t st);

// launch of a main kernel whose last argument is the stamp slot
#define QWA_LAUNCH_MAIN(PS, K, GRID, BLOCK, ST, ...)                                                           \
    do {                                                                                                       \
        if ((PS).stamps != nullptr)                                                                            \
            hipExtLaunchKernelGGL(K, GRID, BLOCK, 0, ST, (PS).start, (PS).stop, 0u, __VA_ARGS__, (PS).stamps); \
        else                                                                                                   \
            hipLaunchKernelGGL(K, GRID, BLOCK, 0, ST, __VA_ARGS__, (unsigned long long*)nullptr);              \
    } while (0)

__device__ __forceinline__ int prof_wg() { return blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z); }
// (wave 0 stores with all its lanes: a wave-uniform branch keeps the kernels' scalar operands uniform)
__device__ __forceinline__ bool prof_wave0() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) == 0; }
__device__ __forceinline__ void prof_start(unsigned long long* prof) {
    if (prof != nullptr && prof_wave0()) {
        prof[PROF_STAMPS * prof_wg()] = __builtin_amdgcn_s_memrealtime();
        prof[PROF_STAMPS * prof_wg() + 2] = __builtin_amdgcn_s_memtime();
    }
}
__device__ __forceinline__ void prof_end(unsigned long long* prof) {
    if (prof != nullptr) {
        __syncthreads();
        if (prof_wave0()) {
            prof[PROF_STAMPS * prof_wg() + 1] = __builtin_amdgcn_s_memrealtime();
            prof[PROF_STAMPS * prof_wg() + 3] = __builtin_amdgcn_s_memtime();
        }
    }
}

hipError_t launch_prep(const qwa_row_src& qg, const qwa_row_src& k, const qwa_row_src& v, const float* qn,
                       const float* kn, int pos0, int rpos0, int n, float theta, float eps, int kvt,
                       const qwa_kv_layer& kv, float* q_out, float* gate, hipStream_t st);
hipError_t launch_prep_rows(const float* qg, const float* k, const float* v, const float* qn, const float* kn, int B,
                            int p0, const float* rope, float eps, int kvt, const qwa_kv_layer& kv, float* q,
                            float* gate, hipStream_t st);
hipError_t launch_rope_table(int p0, int B, float theta, float* rope, hipStream_t st);
hipError_t launch_rope_table_pos(const int* pos3, int B, float theta, float* rope, hipStream_t st);
hipError_t launch_kv_append(const float* xk, const float* xv, int pos0, int n, int kvt, const qwa_kv_layer& kv,
                            hipStream_t st);

// split-K decode: 16-key chunks in DEC_CLASSES fixed residue classes per KV head (chunk index mod DEC_CLASSES)
constexpr int DEC_CLASSES = 512;
size_t dec_work_bytes(int n_pos);
hipError_t launch_decode(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int pos0, int nq,
                         void* work, float* out, const qwa_act_q8* oq, float* out_host, hipStream_t st);
// the same decode on the library's static scratch (no allocation, no work argument)
hipError_t launch_decode_noalloc(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int pos0, int nq,
                                 float* out, const qwa_act_q8* oq, float* out_host, hipStream_t st);
hipError_t launch_decode_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int n_pos,
                                float* out, const qwa_act_q8* oq, hipStream_t st);

// Gated DeltaNet (deltanet.hip)
size_t dn_work_bytes(int B);
hipError_t launch_dn_multi(const qwa_dn_params& p, int cin, const qwa_dn_tokens& in, int n_commit, int n_new,
                           int write_after, float eps, float* o, const qwa_act_q8* oq, hipStream_t st);
hipError_t launch_dn_rows(const qwa_dn_params& p, const float* qkv, const float* z, const float* beta_raw,
                          const float* alpha_raw, int B, int cin, float eps, void* work, float* core_out,
                          uint16_t* o16, hipStream_t st);

size_t prefill_work_bytes(int B, int n_pos);
hipError_t launch_prefill(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                          uint16_t* out16, void* work, hipStream_t st);
hipError_t launch_prefill_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                                 uint16_t* out16, hipStream_t st);

// gemv.hip
size_t w_row_bytes(int fmt, long long K);
bool gemv_q8_supported(int fmt);
hipError_t launch_gemv_q8(int fmt, const void* W, size_t rb, int K, int N, const qwa_act_q8& a, int nb, int act_ld,
                          float* y, int y_ld, int accumulate, hipStream_t st);
hipError_t launch_act_q8(const float* x, long long n, const qwa_act_q8& out, hipStream_t st);
hipError_t launch_gemv_bf16(const uint16_t* W, int K, int N, const float* x, float* y, hipStream_t st);
hipError_t launch_dequant_f16(int fmt, const void* W, size_t rb, int K, int rows, uint16_t* out, hipStream_t st);

}  // namespace qwa

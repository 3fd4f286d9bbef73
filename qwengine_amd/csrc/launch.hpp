// Internal launchers (host side).  Argument validation lives in capi.hip; these assume valid arguments.
#pragma once

#include <hip/hip_runtime.h>

#include "qwattn.h"

namespace qwa {

// opt-in kernel timing (qwa_profile_begin / qwa_profile_end): marks around a main kernel launch
void profile_mark_begin(hipStream_t st);
void profile_mark_end(hipStream_t st);

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
hipError_t launch_decode_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int n_pos,
                                float* out, const qwa_act_q8* oq, hipStream_t st);

hipError_t launch_prefill(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                          uint16_t* out16, hipStream_t st);
hipError_t launch_prefill_simple(const float* q, const float* gate, const qwa_kv_layer& kv, int kvt, int B, int p0,
                                 uint16_t* out16, hipStream_t st);

}  // namespace qwa

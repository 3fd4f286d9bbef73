// The F16 one-pass three-tile verify kernels (k_dec3h<F16>, 6..8 queries from 12288 positions on, and the half-record
// k_dec<F16, 3, 4, 1> it replaced, kept for builds with QWA_DEC3H=0), compiled
// from the same definitions as attn_decode.hip with LLVM's iterative-ILP machine scheduler selected for this file
// alone (a schedule that favours latency hiding over register economy; 1.5-1.8 us faster per layer).
// attn_decode.hip declares the instantiation extern and launches it.  Only the instruction order differs; the results
// are bit-identical.
#define QWA_DEC_KERNELS_ONLY 1
#include "attn_decode.hip"

namespace qwa {
#ifndef QWA_TRACE
template __global__ void k_dec<QWA_KV_F16, 3, 4, 1>(const float* __restrict__, qwa_kv_layer, int, int, int,
                                                    float* __restrict__, unsigned long long*);
template __global__ void k_dec3h<QWA_KV_F16>(const float* __restrict__, qwa_kv_layer, int, int, int,
                                             float* __restrict__, unsigned long long*);
#endif
}  // namespace qwa

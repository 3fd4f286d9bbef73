// The one-column decode GEMV kernels of IQ4_XS and IQ2_S (k_gemv_q8<FMT, 1, U>), compiled from the same definitions
// as gemv.hip with LLVM's max-memory-clause machine scheduler selected for this file alone (it groups a lane's
// weight and activation loads into longer clauses).  gemv.hip declares these instantiations extern and launches
// them.  Only the instruction order differs; the results are bit-identical.
#define QWA_GV_KERNELS_ONLY 1
#include "gemv.hip"

namespace qwa {
QWA_GV_ONE_COLUMN(template, QWA_W_IQ4_XS)
QWA_GV_ONE_COLUMN(template, QWA_W_IQ2_S)
}  // namespace qwa

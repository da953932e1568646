// matvec_q41.hip -- the Q4_1 instantiations of matvec_kernel.h.
#include "matvec_kernel.h"

namespace mi {

int launch_matvec_q41(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                     const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  return launch_kind<MI_Q4_1>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
}

}  // namespace mi

// matvec_rows_more.hip -- the batch-1 kernel of matvec_rows.h for Q4_1, Q5_0,
// Q5_1 and Q5_K (their units are in matvec_units.h); a translation unit of its
// own so the kinds compile in parallel.
#include "matvec_rows.h"

namespace mi {

int launch_rows_more(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                     const void* xq, float* y, int32_t epi, const float* aux) {
  const RowSegs sg = rows::one_matrix(w, row_bytes, rows);
  switch (kind) {
    case MI_Q4_1: return rows::launch_any<MI_Q4_1, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q5_0: return rows::launch_any<MI_Q5_0, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q5_1: return rows::launch_any<MI_Q5_1, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q5_K: return rows::launch_any<MI_Q5_K, false>(s, sg, rows, cols, xq, y, epi, aux);
  }
  return fail(MI_ERR_KIND, "matvec: ggml type %d has no batch-1 row kernel", kind);
}

}  // namespace mi

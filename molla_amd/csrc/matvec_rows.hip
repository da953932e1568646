// matvec_rows.hip -- launchers of the batch-1 kernel in matvec_rows.h: one
// matrix of Q4_K, Q4_0 or Q8_0 (the other kinds in matvec_rows_more.hip), up
// to three Q4_K matrices concatenated by rows (a layer's q, k, v), and the
// gate/up pair with the GLU applied (a layer's MLP input side).
#include "matvec_rows.h"

namespace mi {
using rows::launch_any;
using rows::launch_rk;
using rows::rows_kernel;

bool rows_fits(int kind, int32_t cols) {
  const bool k = kind == MI_Q4_K || kind == MI_Q5_K;
  const bool b32 = kind == MI_Q4_0 || kind == MI_Q4_1 || kind == MI_Q5_0 || kind == MI_Q5_1 || kind == MI_Q8_0;
  return (k || b32) && cols > 0 && cols % (k ? 256 : 64) == 0 && cols / 64 <= 4 * 64;
}
bool q4k_rows_fits(int32_t cols) { return rows_fits(MI_Q4_K, cols); }

int launch_rows(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                const void* xq, float* y, int32_t epi, const float* aux) {
  const RowSegs sg = rows::one_matrix(w, row_bytes, rows);
  switch (kind) {
    case MI_Q4_K: return launch_any<MI_Q4_K, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q4_0: return launch_any<MI_Q4_0, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q8_0: return launch_any<MI_Q8_0, false>(s, sg, rows, cols, xq, y, epi, aux);
  }
  return launch_rows_more(s, kind, w, row_bytes, rows, cols, xq, y, epi, aux);
}

int launch_q4k_rows_segs(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, float* y) {
  return launch_any<MI_Q4_K, false>(s, sg, sg.end[sg.nseg - 1], cols, xq, y, MI_EPI_NONE, nullptr);
}

bool q4k_qkv_rope_fits(int32_t cols, int32_t head_dim, int32_t rope_dim) {
  return q4k_rows_fits(cols) && cols <= 4096 && head_dim % 4 == 0 && rope_dim % 2 == 0;
}

int launch_q4k_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, float* q,
                        const QkvRope& rp) {
  const int rows = sg.end[sg.nseg - 1];
  if (!q4k_qkv_rope_fits(cols, rp.head_dim, rp.rope_dim))
    return fail(MI_ERR_SHAPE, "matvec: no fused rope for %d columns, head_dim %d", cols, rp.head_dim);
  // four rows per wave: pairs never straddle a wave (head_dim is even)
  return launch_rk<MI_Q4_K, 4, 1, false, true>(s, sg, rows, cols, xq, q, MI_EPI_NONE, nullptr, rp);
}

int launch_q4k_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                   int32_t cols, const void* xq, float* y, int32_t epi, void* xq_out) {
  RowSegs sg{};
  sg.w[0] = (const uint8_t*)gate;
  sg.w[1] = sg.w[2] = (const uint8_t*)up;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 2;
  if (xq_out) {
    if (rows % 32 || !rows_fits(MI_Q4_K, cols) || cols > 4096)
      return fail(MI_ERR_SHAPE, "matvec: no quantized GLU output for %d x %d", rows, cols);
    constexpr int kRpw = 4;  // 8 waves per 32-row group
    hipLaunchKernelGGL((rows_kernel<MI_Q4_K, kRpw, 1, true, false, true>), dim3(rows / 32), dim3(32 / kRpw * 64),
                       0, s, sg, cols, (const uint8_t*)xq, y, epi, nullptr, QkvRope{}, (uint8_t*)xq_out);
    return hip_check(hipGetLastError(), "matvec launch");
  }
  return launch_any<MI_Q4_K, true>(s, sg, rows, cols, xq, y, epi, nullptr);
}

}  // namespace mi

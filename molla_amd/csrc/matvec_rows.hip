// matvec_rows.hip -- launchers of the batch-1 kernel in matvec_rows.h: one
// matrix of Q4_K, Q4_0 or Q8_0, up to three matrices concatenated by rows (a layer's q, k, v),
// and the gate/up pair with the GLU applied (a layer's MLP input side).
#include "matvec_rows.h"

namespace mi {
namespace {
using rows::rows_kernel;

template <int KIND, int RPW, int KS, bool GLU, bool ROPE = false>
int launch_rk(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux, const QkvRope& rp = QkvRope{}) {
  const int blocks = (rows + RPW - 1) / RPW;
  hipLaunchKernelGGL((rows_kernel<KIND, RPW, KS, GLU, ROPE>), dim3(blocks), dim3(KS * 64), 0, s, sg, cols,
                     (const uint8_t*)xq, y, epi, aux, rp, nullptr);
  return hip_check(hipGetLastError(), "matvec launch");
}

// Rows per wave: 4 keeps a 14336-row matrix resident in one round (3584
// waves at 4 per SIMD); smaller matrices take fewer rows per wave so that
// there are still enough waves to spread over 256 CUs.
template <int KIND, int KS, bool GLU>
int launch_ks(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux) {
  if constexpr (GLU) {
    return launch_rk<KIND, 2, KS, true>(s, sg, rows, cols, xq, y, epi, aux);
  } else {
    if (rows >= 4096) return launch_rk<KIND, 4, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
    if (rows >= 2048) return launch_rk<KIND, 2, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
    return launch_rk<KIND, 1, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
  }
}

template <int KIND, bool GLU>
int launch_any(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
               const float* aux) {
  if (!rows_fits(KIND, cols)) return fail(MI_ERR_SHAPE, "matvec: %d columns is beyond the batch-1 kernel", cols);
  switch ((cols / 64 + 63) / 64) {
    case 1: return launch_ks<KIND, 1, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    case 2: return launch_ks<KIND, 2, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    case 3: return launch_ks<KIND, 3, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    default: return launch_ks<KIND, 4, GLU>(s, sg, rows, cols, xq, y, epi, aux);
  }
}

}  // namespace

bool rows_fits(int kind, int32_t cols) {
  const int align = kind == MI_Q4_K ? 256 : 64;
  return (kind == MI_Q4_K || kind == MI_Q4_0 || kind == MI_Q8_0) && cols > 0 && cols % align == 0 &&
         cols / 64 <= 4 * 64;
}
bool q4k_rows_fits(int32_t cols) { return rows_fits(MI_Q4_K, cols); }

int launch_rows(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                const void* xq, float* y, int32_t epi, const float* aux) {
  RowSegs sg{};
  sg.w[0] = sg.w[1] = sg.w[2] = (const uint8_t*)w;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 1;
  switch (kind) {
    case MI_Q4_K: return launch_any<MI_Q4_K, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q4_0: return launch_any<MI_Q4_0, false>(s, sg, rows, cols, xq, y, epi, aux);
    case MI_Q8_0: return launch_any<MI_Q8_0, false>(s, sg, rows, cols, xq, y, epi, aux);
  }
  return fail(MI_ERR_KIND, "matvec: ggml type %d has no batch-1 row kernel", kind);
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

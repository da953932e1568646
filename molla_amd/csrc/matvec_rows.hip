// matvec_rows.hip -- launchers of the batch-1 Q4_K kernel in matvec_rows.h:
// one matrix, up to three matrices concatenated by rows (a layer's q, k, v),
// and the gate/up pair with the GLU applied (a layer's MLP input side).
#include "matvec_rows.h"

namespace mi {
namespace {
using rows::q4k_rows_kernel;

template <int RPW, int KS, bool GLU>
int launch_rk(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux) {
  const int blocks = (rows + RPW - 1) / RPW;
  hipLaunchKernelGGL((q4k_rows_kernel<RPW, KS, GLU>), dim3(blocks), dim3(KS * 64), 0, s, sg, cols,
                     (const uint8_t*)xq, y, epi, aux);
  return hip_check(hipGetLastError(), "matvec launch");
}

// Rows per wave: 4 keeps a 14336-row matrix resident in one round (3584
// waves at 4 per SIMD); smaller matrices take fewer rows per wave so that
// there are still enough waves to spread over 256 CUs.
template <int KS, bool GLU>
int launch_ks(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux) {
  if (GLU) return launch_rk<2, KS, true>(s, sg, rows, cols, xq, y, epi, aux);
  if (rows >= 4096) return launch_rk<4, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
  if (rows >= 2048) return launch_rk<2, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
  return launch_rk<1, KS, false>(s, sg, rows, cols, xq, y, epi, aux);
}

template <bool GLU>
int launch_any(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, float* y, int epi,
               const float* aux) {
  if (!q4k_rows_fits(cols)) return fail(MI_ERR_SHAPE, "matvec: %d columns is beyond the batch-1 Q4_K kernel", cols);
  switch ((cols / 64 + 63) / 64) {
    case 1: return launch_ks<1, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    case 2: return launch_ks<2, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    case 3: return launch_ks<3, GLU>(s, sg, rows, cols, xq, y, epi, aux);
    default: return launch_ks<4, GLU>(s, sg, rows, cols, xq, y, epi, aux);
  }
}

}  // namespace

bool q4k_rows_fits(int32_t cols) { return cols > 0 && cols % 256 == 0 && cols / 64 <= 4 * 64; }

int launch_q4k_rows(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    float* y, int32_t epi, const float* aux) {
  RowSegs sg{};
  sg.w[0] = sg.w[1] = sg.w[2] = (const uint8_t*)w;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 1;
  return launch_any<false>(s, sg, rows, cols, xq, y, epi, aux);
}

int launch_q4k_rows_segs(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, float* y) {
  return launch_any<false>(s, sg, sg.end[sg.nseg - 1], cols, xq, y, MI_EPI_NONE, nullptr);
}

int launch_q4k_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                   int32_t cols, const void* xq, float* y, int32_t epi) {
  RowSegs sg{};
  sg.w[0] = (const uint8_t*)gate;
  sg.w[1] = sg.w[2] = (const uint8_t*)up;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 2;
  return launch_any<true>(s, sg, rows, cols, xq, y, epi, nullptr);
}

}  // namespace mi

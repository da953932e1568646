// matvec_rows.hip -- the batch-1 Q4_K matvec (the decode hot loop), gfx950.
//
// Same arithmetic as matvec_kernel<MI_Q4_K, R, 1> (matvec_units.h Q4KUnit),
// organised for a single token, where the whole cost is streaming the
// weights once:
//
//  * A wave owns RPW consecutive rows and one K-slice of at most 64 units
//    (4096 values): lane l keeps the activation of unit u0 + l in registers
//    for the whole wave (loaded once, before any weight), so the activation
//    is never re-read per row.
//  * All RPW rows' weight loads are issued up front, straight-line; rows are
//    then computed in order, each waiting only for its own loads (the
//    compiler's vmcnt counts down row by row), so compute of row r overlaps
//    the arrival of rows r+1..RPW-1 and of every other wave's data.
//  * No LDS staging and at most ~125 VGPRs: 4 waves per SIMD stay resident,
//    so a 14336-row matrix (3584 waves at RPW = 4) is in flight in one round
//    and each CU gets the same number of waves (single-wave blocks are
//    handed out evenly; bigger blocks left whole CUs with an extra block).
//  * cols > 4096 splits K over KS waves of one block (the down projection,
//    14336 = 4 x 3584); their partial sums meet in LDS and wave 0 adds them
//    in a fixed order, so results do not depend on timing.
//
// Replaces the reference's planar_matvec_kernel (src/molla/nn/gpu.mojo:1533)
// for Q4_K at batch 1; the epilogue is gpu.mojo:1005 write_epilogue.
#include "matvec_units.h"

namespace mi {
namespace {
using namespace mv;

// Activation of one lane's 64-value unit (groups 2u and 2u + 1).
struct XUnitRegs {
  uint4 l[2][3][2];
  XMeta m[2];
  __device__ __forceinline__ uint4 limb(int, int j, int hh, int g) const { return l[g & 1][j][hh]; }
  __device__ __forceinline__ XMeta meta(int, int g) const { return m[g & 1]; }
};

template <int RPW, int KS>
__global__ __launch_bounds__(KS * 64) void q4k_rows_kernel(const uint8_t* __restrict__ w, int64_t rb, int rows,
                                                           int cols, const uint8_t* __restrict__ xq,
                                                           float* __restrict__ y, int epi,
                                                           const float* __restrict__ aux) {
  __shared__ float part[KS > 1 ? KS * RPW : 1];
  const int lane = threadIdx.x & 63;
  const int ks = KS > 1 ? (threadIdx.x >> 6) : 0;
  const int row0 = blockIdx.x * RPW;
  const int units = cols >> 6;
  const int u0 = ks * units / KS, u1 = (ks + 1) * units / KS;
  const bool act = u0 + lane < u1;
  const int u = act ? u0 + lane : u1 - 1;
  const int last = rows - 1;

  XUnitRegs xr;
  const XAcc xa{xq, 4 * (int64_t)cols, (int64_t)(cols >> 5) * 16};
#pragma unroll
  for (int e = 0; e < 2; e++) {
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int hh = 0; hh < 2; hh++) xr.l[e][j][hh] = xa.limb(0, j, hh, 2 * u + e);
    xr.m[e] = xa.meta(0, 2 * u + e);
  }
  Q4KUnit<1> un[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) un[r].load(w, rb, min(row0 + r, last), last, u);

  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    float a[1][1] = {{0.0f}};
    un[r].template compute<1>(xr, u, a);
    acc[r] = act ? a[0][0] : 0.0f;
    // keep row r's work ahead of row r+1's (and its wait for row r+1's loads)
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < RPW; r++) acc[r] = wave_sum(acc[r]);

  // lane r holds row row0 + r
  float v = acc[0];
#pragma unroll
  for (int r = 1; r < RPW; r++)
    if (lane == r) v = acc[r];
  if constexpr (KS > 1) {
    if (ks > 0 && lane < RPW) part[ks * RPW + lane] = v;
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k = 1; k < KS; k++)
      if (lane < RPW) v += part[k * RPW + lane];
  }
  if (lane < RPW && row0 + lane < rows) epilogue(y, aux, epi, row0 + lane, row0 + lane, v);
}

template <int RPW, int KS>
int launch_rk(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux) {
  const int blocks = (rows + RPW - 1) / RPW;
  hipLaunchKernelGGL((q4k_rows_kernel<RPW, KS>), dim3(blocks), dim3(KS * 64), 0, s, (const uint8_t*)w, rb, rows,
                     cols, (const uint8_t*)xq, y, epi, aux);
  return hip_check(hipGetLastError(), "matvec launch");
}

template <int KS>
int launch_ks(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y, int epi,
              const float* aux) {
  if (rows >= 4096) return launch_rk<4, KS>(s, w, rb, rows, cols, xq, y, epi, aux);
  if (rows >= 2048) return launch_rk<2, KS>(s, w, rb, rows, cols, xq, y, epi, aux);
  return launch_rk<1, KS>(s, w, rb, rows, cols, xq, y, epi, aux);
}

}  // namespace

bool q4k_rows_fits(int32_t cols) { return cols % 256 == 0 && cols / 64 <= 4 * 64; }

int launch_q4k_rows(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    float* y, int32_t epi, const float* aux) {
  const int ks = (cols / 64 + 63) / 64;
  switch (ks) {
    case 1: return launch_ks<1>(s, w, row_bytes, rows, cols, xq, y, epi, aux);
    case 2: return launch_ks<2>(s, w, row_bytes, rows, cols, xq, y, epi, aux);
    case 3: return launch_ks<3>(s, w, row_bytes, rows, cols, xq, y, epi, aux);
    case 4: return launch_ks<4>(s, w, row_bytes, rows, cols, xq, y, epi, aux);
  }
  return fail(MI_ERR_SHAPE, "matvec: %d columns is beyond the batch-1 Q4_K kernel", cols);
}

}  // namespace mi

// matvec_kernel.h -- fused dequantize-and-dot over raw GGUF blocks, gfx950.
// Included once per quant kind (matvec_<kind>.hip) so the kinds compile in
// parallel; matvec.hip routes a call to its kind.
//
// Replaces the reference's planar_matvec_kernel / planar_matmul_kernel
// (src/molla/nn/gpu.mojo:1533, :1809) for every block-quantized kind.
//
// Work decomposition.  A wavefront owns R consecutive output rows and walks
// them together in "units" of 64 values (128 for Q6_K, whose bit planes
// interleave over a half superblock): lane l takes units l, l+64, ... of all R
// rows, so each lane loads whole 16-byte pieces of packed blocks and reuses
// every activation load R times.  Weights are never expanded to floats:
// nibbles / 6-bit codes are masked into bytes and multiplied against the
// activation's int8 limbs with v_dot4c_i32_i8 (four products per
// instruction, exact), and the block scales are applied once per 16 or 32
// values.  A final wave reduction gives each row its dot, and the epilogue
// of gpu.mojo:1005 write_epilogue (bias / residual add / gated activation)
// is applied by lane 0.
//
// Alignment: Q4_K rows must be 16-byte aligned (144-byte superblocks are a
// whole number of 16-byte pieces).  The other kinds only need 4-byte aligned
// rows; their 18/34/210-byte blocks are realigned in registers with
// v_alignbyte_b32.
#pragma once

#include "matvec_units.h"

namespace mi {
namespace {
using namespace mv;

// LDS budget for the staged activation copy; larger activations are read
// from global memory (L2-resident) instead.
constexpr int kMaxLdsX = 64 * 1024;

template <int KIND, int R, int T, int WPB, bool XLDS>
__global__ __launch_bounds__(WPB * 64) void matvec_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                          int rows, int cols,
                                                          const uint8_t* __restrict__ xq,
                                                          float* __restrict__ y, int64_t ldy, int epi,
                                                          const float* __restrict__ aux) {
  using Unit = typename UnitOf<KIND, R>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t xs_lds[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * WPB + wave) * R;
  const int last_row = rows - 1;
  const int units = cols / Unit::kElems;
  const int64_t tok = xq_token_bytes(cols);
  const int64_t plane = (int64_t)(cols >> 5) * 16;
  // First unit's weights go in flight before anything else.
  Unit cur;
  const bool live = row0 < rows;
  if (live && lane < units) cur.load(w, rb, row0, last_row, lane);
  float acc[R][T];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int t = 0; t < T; t++) acc[r][t] = 0.0f;
  if constexpr (XLDS) {
    const int n16 = (int)(T * tok / 16);
    const uint4* src = (const uint4*)xq;
    uint4* dst = (uint4*)xs_lds;
    for (int i = threadIdx.x; i < n16; i += WPB * 64) dst[i] = src[i];
    __syncthreads();
  }
  if (!live) return;
  auto body = [&](const auto& xa) {
    int u = lane;
    while (u < units) {
      const int un = u + kWave;
      if (un < units) {
        Unit nxt;
        nxt.load(w, rb, row0, last_row, un);
        cur.template compute<T>(xa, u, acc);
        cur = nxt;
      } else {
        cur.template compute<T>(xa, u, acc);
      }
      u = un;
    }
  };
  if constexpr (XLDS) body(XLds{xs_lds, (int)tok, (int)plane});
  else body(XAcc{xq, tok, plane});
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float v = wave_sum(acc[r][t]);
      if (lane == 0 && row0 + r < rows) epilogue(y, aux, epi, (int64_t)t * ldy + row0 + r, row0 + r, v);
    }
}

template <int KIND, int R, int T, int WPB>
int launch_rt(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y,
              int64_t ldy, int epi, const float* aux) {
  const int per_block = WPB * R;
  const int blocks = (rows + per_block - 1) / per_block;
  const size_t xbytes = (size_t)T * xq_token_bytes(cols);
  if (xbytes <= (size_t)kMaxLdsX) {
    hipLaunchKernelGGL((matvec_kernel<KIND, R, T, WPB, true>), dim3(blocks), dim3(WPB * kWave), xbytes, s,
                       (const uint8_t*)w, rb, rows, cols, (const uint8_t*)xq, y, ldy, epi, aux);
  } else {
    hipLaunchKernelGGL((matvec_kernel<KIND, R, T, WPB, false>), dim3(blocks), dim3(WPB * kWave), 0, s,
                       (const uint8_t*)w, rb, rows, cols, (const uint8_t*)xq, y, ldy, epi, aux);
  }
  return hip_check(hipGetLastError(), "matvec launch");
}

template <int KIND, int T>
int launch_t(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y,
             int64_t ldy, int epi, const float* aux) {
  // Rows per wave: enough waves to fill 256 CUs several times over, and
  // as many rows as that allows so each activation load serves them all.
  if (rows >= 8192) return launch_rt<KIND, 4, T, 4>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  if (rows >= 4096) return launch_rt<KIND, 2, T, 4>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  return launch_rt<KIND, 1, T, 4>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
}

template <int KIND>
int launch_kind(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq,
                int tokens, float* y, int64_t ldy, int epi, const float* aux) {
  switch (tokens) {
    case 1: return launch_t<KIND, 1>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 2: return launch_t<KIND, 2>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 3: return launch_t<KIND, 3>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 4: return launch_t<KIND, 4>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 5: return launch_t<KIND, 5>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 6: return launch_t<KIND, 6>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 7: return launch_t<KIND, 7>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
    case 8: return launch_t<KIND, 8>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  }
  return fail(MI_ERR_ARG, "matvec: tokens %d outside 1..8", tokens);
}

}  // namespace
}  // namespace mi

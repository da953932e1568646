// matvec_q6k_rows.hip -- batch-1 Q6_K matvec for wide, tall matrices (the
// output head: 128256 x 4096), gfx950.
//
// Q6_K superblock (210 bytes / 256 values, quant.mojo:371 dequant_q6_k):
// ql[128] @0, qh[64] @128, sc[16] int8 @192, d f16 @208.  For half n of the
// superblock and l < 32 (h = qh[32n + l]):
//   value 128n + l      = (ql[64n + l]      & 15 | (h      & 3) << 4) - 32,  scale sc[8n + l/16]
//   value 128n + l + 32 = (ql[64n + l + 32] & 15 | (h >> 2 & 3) << 4) - 32,  scale sc[8n + l/16 + 2]
//   value 128n + l + 64 = (ql[64n + l]      >> 4 | (h >> 4 & 3) << 4) - 32,  scale sc[8n + l/16 + 4]
//   value 128n + l + 96 = (ql[64n + l + 32] >> 4 | (h >> 6 & 3) << 4) - 32,  scale sc[8n + l/16 + 6]
// times d.  A "unit" here is 64 values: half n, part a in {0, 1}: the 32
// bytes ql[64n + 32a ..] give activation groups 4n + a (low nibbles) and
// 4n + a + 2 (high nibbles), with bits 2a and 4 + 2a of qh[32n + l] on top.
//
// Work decomposition: a lane owns one unit position (64 units = 4096
// columns per row) and keeps that unit's activation in registers; each wave
// then walks rows w, w + NW, w + 2 NW, ... (NW = all waves of the grid),
// with the next row's loads in flight while the current row is computed.
// The activation is read once per wave instead of once per row, which for
// 128256 rows is what keeps its traffic well below the weights'.
//
// Replaces planar_matvec_kernel (src/molla/nn/gpu.mojo:1533) for Q6_K at
// batch 1; arithmetic as matvec_units.h Q6KUnit (integer dots on the
// activation's limbs, the -32 offset through the limb sums).
#include <algorithm>

#include "matvec_units.h"

namespace mi {
namespace {
using namespace mv;

// The activation of one lane's unit: groups g0 = 4n + a and g1 = g0 + 2 of
// its superblock.
struct XQ6Regs {
  uint4 l[2][3][2];  // [group][limb][16-value half]
  float scale[2];
  int lsum1[2][2], lsum23[2][2];
};

// The 22 dwords of one row's unit, 4-byte aligned; `sh` realigns them.
struct Q6Piece {
  uint32_t ql[9], qh[9], sc[3], d;
};

__device__ __forceinline__ void load_piece(Q6Piece& p, const uint8_t* blk4, uint32_t sh, int n, int a) {
  const uint8_t* q = blk4 + 64 * n + 32 * a;
  const uint4 q0 = ld16a4(q), q1 = ld16a4(q + 16);
  p.ql[0] = q0.x; p.ql[1] = q0.y; p.ql[2] = q0.z; p.ql[3] = q0.w;
  p.ql[4] = q1.x; p.ql[5] = q1.y; p.ql[6] = q1.z; p.ql[7] = q1.w;
  p.ql[8] = ld4(q + 32);
  const uint8_t* h = blk4 + 128 + 32 * n;
  const uint4 h0 = ld16a4(h), h1 = ld16a4(h + 16);
  p.qh[0] = h0.x; p.qh[1] = h0.y; p.qh[2] = h0.z; p.qh[3] = h0.w;
  p.qh[4] = h1.x; p.qh[5] = h1.y; p.qh[6] = h1.z; p.qh[7] = h1.w;
  p.qh[8] = ld4(h + 32);
  // sc[8n .. 8n+7] spans three dwords only when the block is 2 bytes off
  // alignment; aligned, the third would read past the superblock (past the
  // tensor, for its last one), so it re-reads the second instead.
  const uint8_t* s = blk4 + 192 + 8 * n;
  p.sc[0] = ld4(s);
  p.sc[1] = ld4(s + 4);
  p.sc[2] = ld4(s + (sh ? 8 : 4));
  // d as a 16-bit load at its own (even) address, for the same reason
  p.d = *(const uint16_t*)(blk4 + sh + 208);
}

__device__ __forceinline__ float piece_dot(const Q6Piece& p, uint32_t sh, int a, const XQ6Regs& x) {
  const uint32_t s_lo = 2u * a, s_hi = 4u + 2u * a;
  uint32_t scw[2];
  scw[0] = align(p.sc[1], p.sc[0], sh);  // sc[8n .. 8n+3]
  scw[1] = align(p.sc[2], p.sc[1], sh);  // sc[8n+4 .. 8n+7]
  const float d = half_bits_to_float(p.d);
  float part = 0.0f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    int s0[3] = {0, 0, 0}, s1[3] = {0, 0, 0};
#pragma unroll
    for (int ii = 0; ii < 4; ii++) {
      const int i = 4 * hh + ii;
      const uint32_t A = align(p.ql[i + 1], p.ql[i], sh);
      const uint32_t H = align(p.qh[i + 1], p.qh[i], sh);
      const uint32_t q0 = (A & 0x0F0F0F0Fu) | (((H >> s_lo) & 0x03030303u) << 4);
      const uint32_t q1 = ((A >> 4) & 0x0F0F0F0Fu) | (((H >> s_hi) & 0x03030303u) << 4);
#pragma unroll
      for (int j = 0; j < 3; j++) {
        s0[j] = dot4(q0, comp(x.l[0][j][hh], ii), s0[j]);
        s1[j] = dot4(q1, comp(x.l[1][j][hh], ii), s1[j]);
      }
    }
    // sc[8n + hh + 2a] for group g0, sc[8n + hh + 4 + 2a] for g1
    const uint32_t b0 = hh + 2u * a, b1 = hh + 4u + 2u * a;
    const float sc0 = (float)(int8_t)((scw[b0 >> 2] >> (8 * (b0 & 3))) & 0xFF);
    const float sc1 = (float)(int8_t)((scw[b1 >> 2] >> (8 * (b1 & 3))) & 0xFF);
    const float f0 = limbs_to_float(s0[0] - 32 * x.lsum1[0][hh], s0[1] * 256 + s0[2] - 32 * x.lsum23[0][hh]);
    const float f1 = limbs_to_float(s1[0] - 32 * x.lsum1[1][hh], s1[1] * 256 + s1[2] - 32 * x.lsum23[1][hh]);
    part = fmaf(sc0 * x.scale[0], f0, part);
    part = fmaf(sc1 * x.scale[1], f1, part);
  }
  return d * part;
}

// KS > 1 (rows longer than 4096 columns, the down projection's 14336): the
// four waves of a block take one row together, wave k the units
// [k U, (k + 1) U) with U = ceil(units / KS); their sums meet in LDS and wave
// 0 adds them in wave order, so the result does not depend on timing.  The
// block walks rows blockIdx.x, blockIdx.x + gridDim.x, ... with the next
// row's loads in flight, as the single-wave form does.
template <int KS>
__global__ __launch_bounds__(256) void q6k_rows_kernel(const uint8_t* __restrict__ w, int64_t rb, int rows,
                                                       int cols, const uint8_t* __restrict__ xq,
                                                       float* __restrict__ y, int epi,
                                                       const float* __restrict__ aux) {
  static_assert(KS == 1 || KS <= 4, "up to four waves split a row");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = KS == 1 ? gridDim.x * 4 : gridDim.x;
  const int wv = KS == 1 ? blockIdx.x * 4 + wave : blockIdx.x;
  const int units = cols >> 6;
  const int per = (units + KS - 1) / KS;  // units of a wave's K-slice
  const int ks = KS == 1 ? 0 : wave;
  const bool act = lane < per && ks * per + lane < units;
  const int u = act ? ks * per + lane : units - 1;
  const int sb = u >> 2, n = (u >> 1) & 1, a = u & 1;
  const int g0 = 8 * sb + 4 * n + a, g1 = g0 + 2;
  __shared__ float part[2][KS > 1 ? KS : 1];

  XQ6Regs x;
  {
    const XAcc xa{xq, 4 * (int64_t)cols, (int64_t)(cols >> 5) * 16};
    const int gs[2] = {g0, g1};
#pragma unroll
    for (int e = 0; e < 2; e++) {
#pragma unroll
      for (int j = 0; j < 3; j++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) x.l[e][j][hh] = xa.limb(0, j, hh, gs[e]);
      const XMeta m = xa.meta(0, gs[e]);
      const int2 l23 = xa.lsum23(0, gs[e]);
      x.scale[e] = m.scale;
      x.lsum1[e][0] = m.lsum1[0];
      x.lsum1[e][1] = m.lsum1[1];
      x.lsum23[e][0] = l23.x;
      x.lsum23[e][1] = l23.y;
    }
  }
  // a unit's block address within any row: rb is a multiple of 2, rows are
  // 4-byte aligned at the base, so each (row, unit) realigns by 0 or 2 bytes
  const int64_t uoff = (int64_t)sb * 210;
  // (pointer arithmetic, not integer casts: a pointer rebuilt from an
  // integer loses its global address space and its loads become flat ones)
  auto blk = [&](int row, uint32_t& sh) {
    const uint8_t* p = w + (int64_t)row * rb + uoff;
    sh = (uint32_t)((uintptr_t)p & 3u);
    return p - sh;
  };

  int row = wv;
  if (row >= rows) return;  // uniform over a block when KS > 1
  Q6Piece cur, nxt;
  uint32_t sh_cur, sh_nxt;
  {
    const uint8_t* b = blk(row, sh_cur);
    load_piece(cur, b, sh_cur, n, a);
  }
  for (int it = 0;; it++) {
    const int nrow = row + nw;
    const bool more = nrow < rows;
    if (more) {
      const uint8_t* b = blk(nrow, sh_nxt);
      load_piece(nxt, b, sh_nxt, n, a);
    }
    float v = act ? piece_dot(cur, sh_cur, a, x) : 0.0f;
    v = wave_sum(v);
    if constexpr (KS > 1) {
      // part alternates between two buffers: a row's buffer is written
      // again two rows later, after every wave has passed the next row's
      // barrier, which wave 0 reaches only once it has read this one
      // a block always holds four waves; with KS < 4 the spare ones own no
      // units and must not write (their slot would be the other buffer's)
      if (lane == 0 && ks < KS) part[it & 1][ks] = v;
      __syncthreads();
      if (ks == 0 && lane == 0) {
        float t = part[it & 1][0];
#pragma unroll
        for (int k = 1; k < KS; k++) t += part[it & 1][k];
        epilogue(y, aux, epi, row, row, t);
      }
    } else {
      if (lane == 0) epilogue(y, aux, epi, row, row, v);
    }
    if (!more) break;
    cur = nxt;
    sh_cur = sh_nxt;
    row = nrow;
  }
}

constexpr int kQ6RowsPerWave = 128;  // rows a wave of q6k_rows2_kernel takes at most

// One wave a row (4096 columns or fewer) with NP - 1 rows' loads in flight
// behind the one being computed: NP pieces a lane in a fixed rotation (the
// loop body takes NP rows, so no piece is copied and each compute waits
// only for its own loads).  A row past the end is clamped to the last one
// and its sum dropped, so no load sits under a branch; the sums wait in LDS
// and go out at the end.  Plain rows only (no epilogue operand to load).
// The 128256x4096 head, cold: 84.7 us for q6k_rows_kernel<1> (four waves a
// SIMD, one row ahead), 75.2 us with NP = 3 at two waves a SIMD (NP = 4 or
// 5 at two waves, or 4 or 6 at one wave, 76-79 us).
template <int NP>
__global__ __launch_bounds__(256) void q6k_rows2_kernel(const uint8_t* __restrict__ w, int64_t rb, int rows,
                                                        int cols, const uint8_t* __restrict__ xq,
                                                        float* __restrict__ y) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nw = gridDim.x * 4;
  const int units = cols >> 6;
  const bool act = lane < units;
  const int u = act ? lane : units - 1;
  const int sb = u >> 2, n = (u >> 1) & 1, a = u & 1;
  const int g0 = 8 * sb + 4 * n + a, g1 = g0 + 2;

  XQ6Regs x;
  {
    const XAcc xa{xq, 4 * (int64_t)cols, (int64_t)(cols >> 5) * 16};
    const int gs[2] = {g0, g1};
#pragma unroll
    for (int e = 0; e < 2; e++) {
#pragma unroll
      for (int j = 0; j < 3; j++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) x.l[e][j][hh] = xa.limb(0, j, hh, gs[e]);
      const XMeta m = xa.meta(0, gs[e]);
      const int2 l23 = xa.lsum23(0, gs[e]);
      x.scale[e] = m.scale;
      x.lsum1[e][0] = m.lsum1[0];
      x.lsum1[e][1] = m.lsum1[1];
      x.lsum23[e][0] = l23.x;
      x.lsum23[e][1] = l23.y;
    }
  }
  const int64_t uoff = (int64_t)sb * 210;
  auto load_row = [&](Q6Piece& p, uint32_t& sh, int row) __attribute__((always_inline)) {
    const uint8_t* q = w + (int64_t)min(row, rows - 1) * rb + uoff;
    sh = (uint32_t)((uintptr_t)q & 3u);
    load_piece(p, q - sh, sh, n, a);
  };
  int row = blockIdx.x * 4 + wave;
  if (row >= rows) return;
  const int row0 = row;
  __shared__ float res[4][kQ6RowsPerWave];
  int k = 0;
  Q6Piece pc[NP];
  uint32_t sh[NP];
#pragma unroll
  for (int j = 0; j < NP - 1; j++) load_row(pc[j], sh[j], row + j * nw);
  // compute `use` (row r), after sending for row r + (NP - 1) nw into `refill`
  auto step = [&](Q6Piece& use, uint32_t& su, Q6Piece& refill, uint32_t& sr) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    load_row(refill, sr, row + (NP - 1) * nw);
    __builtin_amdgcn_sched_barrier(0);
    float v = piece_dot(use, su, a, x);
    v = wave_sum(act ? v : 0.0f);
    if (lane == 0) res[wave][k] = v;
    __builtin_amdgcn_sched_barrier(0);
    k++;
    row += nw;
    return row < rows;
  };
  // one pass over the ring: piece j computed, piece j - 1 refilled
  auto ring = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NP; j++)
      if (!step(pc[j], sh[j], pc[(j + NP - 1) % NP], sh[(j + NP - 1) % NP])) return false;
    return true;
  };
  // the first pass peeled, so the loop is entered from the state its back
  // edge leaves (the compiler's waits at a loop head cover every path)
  if (ring())
    while (ring()) {}
  // the sums go out at the end: a global store inside the loop let the
  // compiler wait for the loads in flight before reusing its registers
  for (int i = lane; i < k; i += 64) y[row0 + i * nw] = res[wave][i];
}

}  // namespace

bool q6k_rows_fits(int32_t cols, int64_t row_bytes) {
  return cols > 0 && cols % 256 == 0 && cols / 64 <= 4 * 64 && row_bytes % 4 == 0;
}

#ifndef MI_Q6_DEEP
#define MI_Q6_DEEP 1
#endif
#ifndef MI_Q6_DEEP_WAVES
#define MI_Q6_DEEP_WAVES 2
#endif
constexpr bool kQ6Deep = MI_Q6_DEEP;
constexpr int kQ6DeepWaves = MI_Q6_DEEP_WAVES;
#ifndef MI_Q6_PIECES
#define MI_Q6_PIECES 3
#endif
constexpr int kQ6Pieces = MI_Q6_PIECES;

int launch_q6k_rows(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    float* y, int32_t epi, const float* aux) {
  if (((uintptr_t)w & 3) || row_bytes % 4) return fail(MI_ERR_ALIGN, "matvec: Q6_K rows must be 4-byte aligned");
  const int ks = (cols / 64 + 63) / 64;  // waves a row takes
  const int deep_waves = std::min(rows, 256 * 4 * kQ6DeepWaves);
  if (ks == 1 && kQ6Deep && epi == MI_EPI_NONE && rows <= (int64_t)deep_waves * kQ6RowsPerWave) {
    // three waves per SIMD (the three-piece ring takes ~150 registers)
    const int waves = deep_waves;
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL(q6k_rows2_kernel<kQ6Pieces>, dim3(blocks), dim3(256), 0, s, (const uint8_t*)w, row_bytes, rows, cols,
                       (const uint8_t*)xq, y);
  } else if (ks == 1) {
    // four waves per SIMD over the whole chip; each wave then streams rows
    const int waves = std::min(rows, 256 * 4 * 4);
    const int blocks = (waves + 3) / 4;
    hipLaunchKernelGGL(q6k_rows_kernel<1>, dim3(blocks), dim3(256), 0, s, (const uint8_t*)w, row_bytes, rows, cols,
                       (const uint8_t*)xq, y, epi, aux);
  } else {
    // a block of four waves a row, as many blocks as four waves a SIMD hold
    const int blocks = std::min(rows, 256 * 4);
#define MI_Q6R(K)                                                                                              \
  hipLaunchKernelGGL(q6k_rows_kernel<K>, dim3(blocks), dim3(256), 0, s, (const uint8_t*)w, row_bytes, rows, cols, \
                     (const uint8_t*)xq, y, epi, aux)
    if (ks == 2) MI_Q6R(2);
    else if (ks == 3) MI_Q6R(3);
    else MI_Q6R(4);
#undef MI_Q6R
  }
  return hip_check(hipGetLastError(), "matvec launch");
}

}  // namespace mi

// matvec_rows.hip -- launchers of the batch-1 kernel in matvec_rows.h: one
// matrix of Q4_K, Q4_0 or Q8_0 (the other kinds in matvec_rows_more.hip), up
// to three Q4_K matrices concatenated by rows (a layer's q, k, v), and the
// gate/up pair with the GLU applied (a layer's MLP input side).
#include <algorithm>

#include "matvec_rows.h"

namespace mi {
using rows::launch_any;
using rows::launch_rk;
using rows::rows_kernel;

namespace {
using namespace mv;

// The gate|up GLU of one decoding token with the layer's ffn RMSNorm folded
// in (Q4_K, cols <= 4096).  A block is 8 waves, each owning four rows of
// gate and of up in a 32-row group, as rows_kernel<Q4_K, 4, 1, GLU, -, GQ>;
// the grid is at most one block per CU and a block loops over groups
// blockIdx.x, blockIdx.x + gridDim.x, ...  The block issues the first PRE
// rows of each wave's weights, normalises the row into LDS in matvec form
// (norm_row_to_lds), issues the rest of its first group's weights, and keeps
// the activation in registers for every group it takes: the norm costs no
// launch
// and is computed once per CU, not once per group.  After each group, wave 0
// writes its act(gate) * up in matvec form for the down projection.
// The folded norms put x * gain into the matvec form and scale each row's
// sum by the norm's scale (norm_row_to_lds DEFER): the sum of squares runs
// beside the quantize, one barrier fewer (decode step 1.673 -> 1.652 ms at
// batch 1).
constexpr bool kNormDefer = true;
constexpr int kGluIts = 8;  // groups a block of glu_norm_kernel takes at most (one per wave)
template <int PRE>
__global__ __launch_bounds__(8 * 64) void glu_norm_kernel(const RowSegs sg, int cols, float* __restrict__ y,
                                                          int epi, const NormIn nm, uint8_t* __restrict__ xq_out) {
  constexpr int RPW = 4, NR = 2 * RPW, kNT = 8 * 64;
  __shared__ __align__(16) uint8_t xs[4 * 4096];
  __shared__ double red[kNT / 64];
  __shared__ float grp[kGluIts][32];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rows = sg.end[0];
  const int groups = rows >> 5;
  const int units = cols >> 6;
  const bool act = lane < units;
  const int u = act ? lane : units - 1;

  rows::XUnitRegs<false> xr;
  UnitOf<MI_Q4_K, 1>::type un[NR];
  // PRE of a wave's rows (its gate rows), then the norm, then the rest: with
  // every weight load issued first, the norm finished about 2 us later (its
  // row loads and code wait behind the whole chip's weight requests) and the
  // block computes nothing before it; with none, the first weights only set
  // out after the norm.  14336 x 4096 cold: 19.3 us with none, 17.4 with 4,
  // 20.4 with all 8.
  const NormRow nr = norm_row_load(nm.x, nm.gain, cols);
  int g = blockIdx.x;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < PRE; r++) {
    const int row = (g * 8 + wave) * RPW + r % RPW;
    un[r].load(sg.w[r / RPW] + (int64_t)row * sg.rb[r / RPW], 0, 0, 0, u);
  }
  __builtin_amdgcn_sched_barrier(0);
  const float nsc = norm_row_to_lds<kNT, kNormDefer>(nr, cols, nm.eps, xs, red);
  rows::load_x(xr, XLds{xs, 0, (cols >> 5) * 16}, u);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = PRE; r < NR; r++) {
    const int row = (g * 8 + wave) * RPW + r % RPW;
    un[r].load(sg.w[r / RPW] + (int64_t)row * sg.rb[r / RPW], 0, 0, 0, u);
  }
  // No barrier inside the loop: each wave sends for its next group's weights
  // as soon as it has used this group's, and leaves its act(gate) * up in
  // LDS; the quantize of every group (wave k takes the block's k-th group)
  // waits for one barrier after the last group.  A barrier per group held
  // every wave of the block, and the next group's loads, until the slowest
  // wave's weights had arrived.  The launcher keeps a block to at most
  // kGluIts groups.
  // this group's sums, store and act(gate) * up into LDS
  // the eight sums by a transposed reduction (wave_sum_rows8): gate row r
  // in lanes 8 h + 16 k with r = k + 2 h, its up row 32 lanes higher
  auto finish = [&](float (&acc)[NR], int it) __attribute__((always_inline)) {
    float v = rows::wave_sum_rows8(acc);
    if constexpr (kNormDefer) v *= nsc;
    const float upv = __shfl_down(v, 32);
    const float o = ((epi & MI_ACT_GELU) ? gelu(v) : silu(v)) * upv;
    const int row0 = (g * 8 + wave) * RPW;
    const int r = ((lane >> 4) & 1) + 2 * ((lane >> 3) & 1);
    if (lane < 32 && (lane & 7) == 0) {
      if (epi & MI_EPI_ADD) y[row0 + r] += o;
      else y[row0 + r] = o;
      grp[it][wave * RPW + r] = o;
    }
  };
  int it = 0;
  for (;; it++) {
    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
      float a[1][1] = {{0.0f}};
      un[r].template compute<1>(xr, u, a);
      acc[r] = act ? a[0][0] : 0.0f;
      __builtin_amdgcn_sched_barrier(0);
    }
    const int gn = g + gridDim.x;
    // the exit and the next loads on one branch: with the loads under a
    // branch of their own, the old weights stayed live across it (spills)
    if (gn >= groups) {
      finish(acc, it);
      break;
    }
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const int row = (gn * 8 + wave) * RPW + r % RPW;
      un[r].load(sg.w[r / RPW] + (int64_t)row * sg.rb[r / RPW], 0, 0, 0, u);
    }
    finish(acc, it);
    g = gn;
  }
  __syncthreads();
  if (wave <= it) {
    const int gq = blockIdx.x + wave * gridDim.x;
    quantize_group32(grp[wave][lane & 31], lane & 31, gq, groups, xq_out, lane < 32);
  }
}

// The q|k|v matvec of one decoding token with the layer's attention RMSNorm
// folded in (Q4_K, cols <= 4096), and the rope and cache store of
// rows_kernel<…, ROPE> in its epilogue.  A block is 12 waves of two rows
// (one rope pair) each; the grid is at most one block per CU, each block
// looping over 24-row groups.  As in glu_norm_kernel, a wave issues its
// first PRE rows' weights, the block normalises the row into LDS in matvec
// form (norm_row_to_lds), then the rest go out (PRE = 1 of the wave's two
// rows measured best).  A wave's (cos, sin) comes
// from scalar loads of pos, steps and factors and float64 trig, as
// rms_norm_kernel computes its table, so it never waits for weights.
// Q8 (a q8_0 cache): 16 waves and 32-row groups, so that a group of k or v
// rows is one q8_0 block of the cache row (qw and kvw multiples of 32); the
// block gathers the group's 32 outputs in LDS and one half-wave stores it as
// rope_store_kernel's q8 branch does (store_kv_q8: repack.mojo:174-218).
template <int PRE, bool Q8 = false>
__global__ __launch_bounds__((Q8 ? 16 : 12) * 64) void qkv_norm_kernel(const RowSegs sg, int cols,
                                                                       float* __restrict__ y, const NormIn nm,
                                                                       const QkvRope rp) {
#pragma clang fp contract(off)
  constexpr int W = Q8 ? 16 : 12, RPW = 2, kNT = W * 64;
  __shared__ __align__(16) uint8_t xs[4 * 4096];
  __shared__ double red[kNT / 64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rows = sg.end[sg.nseg - 1];
  const int groups = (rows + W * RPW - 1) / (W * RPW);
  const int units = cols >> 6;
  const bool act = lane < units;
  const int u = act ? lane : units - 1;
  const int pos = rp.pos[0];

  // Group g's wave rows, and whether (and which pair) the rope rotates them.
  struct Pair {
    int row0;
    bool is_q, is_k, rot;
    int pair;
  };
  auto pair_of = [&](int gg) __attribute__((always_inline)) {
    Pair p;
    p.row0 = (gg * W + wave) * RPW;  // even: a wave's two rows are one rope pair
    p.is_q = p.row0 < rp.qw;
    p.is_k = !p.is_q && p.row0 < rp.qw + rp.kvw;
    const int e0 = (p.is_q ? p.row0 : p.row0 - rp.qw) % rp.head_dim;
    p.rot = (p.is_q || p.is_k) && e0 < rp.rope_dim;
    p.pair = p.rot ? e0 >> 1 : 0;
    return p;
  };

  rows::XUnitRegs<false> xr;
  UnitOf<MI_Q4_K, 1>::type un[RPW];
  int g = blockIdx.x;
  Pair pr = pair_of(g);
  // the row, this group's rope step and factor, then the weights: loads
  // complete in issue order, so nothing waited for before the compute
  // waits for a weight
  const NormRow nr = norm_row_load(nm.x, nm.gain, cols);
  float step = rp.steps[pr.pair], factor = rp.factors ? rp.factors[pr.pair] : 1.0f;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < PRE; r++) un[r].load(rows::seg_row(sg, min(pr.row0 + r, rows - 1)), 0, 0, 0, u);
  __builtin_amdgcn_sched_barrier(0);
  // rope_theta's arithmetic on the step and factor (scalar loads): done
  // while the row's loads are in flight, not after the norm
  float c = 1.0f, sn = 0.0f;
  auto angle = [&]() __attribute__((always_inline)) {
    c = 1.0f;
    sn = 0.0f;
    if (pr.rot) {
      float theta = (float)pos * step;
      if (rp.factors) theta = theta / factor;
      c = (float)cos((double)theta);
      sn = (float)sin((double)theta);
    }
  };
  angle();
  __builtin_amdgcn_sched_barrier(0);
  const float nsc = norm_row_to_lds<kNT, kNormDefer>(nr, cols, nm.eps, xs, red);
  rows::load_x(xr, XLds{xs, 0, (cols >> 5) * 16}, u);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = PRE; r < RPW; r++) un[r].load(rows::seg_row(sg, min(pr.row0 + r, rows - 1)), 0, 0, 0, u);
  const int64_t slot = (int64_t)(rp.kv_index ? rp.kv_index[pos] : pos) * (Q8 ? cache_row(MI_CACHE_Q8, rp.kvw) : rp.kvw);
  __shared__ float q8buf[Q8 ? 2 : 1][32];
  // q8buf alternates: a block's groups go q rows first, then k and v rows
  // (each with a barrier), so a buffer is written again only after every
  // wave has passed the next group's barrier, which wave 0 reaches once it
  // has read the buffer
  for (int it = 0;; it++) {
    if (it > 0) angle();
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; r++) {
      float a[1][1] = {{0.0f}};
      un[r].template compute<1>(xr, u, a);
      acc[r] = act ? a[0][0] : 0.0f;
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int r = 0; r < RPW; r++) acc[r] = wave_sum(acc[r]);
    // rope.mojo:294 rotate_scaled, adjacent pairs: (a, b) <- (a c - b s, a s + b c)
    const float a = kNormDefer ? acc[0] * nsc : acc[0], b = kNormDefer ? acc[1] * nsc : acc[1];
    const float o = !pr.rot ? (lane == 0 ? a : b) : (lane == 0 ? a * c - b * sn : a * sn + b * c);
    const int row = pr.row0 + lane;
    if constexpr (Q8) {
      // the group is all q, all k or all v rows (block-uniform)
      const int grow0 = g * W * RPW;
      if (grow0 < rp.qw) {
        if (lane < RPW && row < rows) y[row] = o;
      } else {
        float* qb = q8buf[it & 1];
        if (lane < RPW) qb[wave * RPW + lane] = o;
        __syncthreads();
        if (wave == 0) {
          // q8_0 of the 32 values (both half-waves compute the same block)
          const int l32 = lane & 31;
          const float x = qb[l32];
          const float amax = lanes::reduce<32>(fabsf(x), lanes::Max{});
          const float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
          const float yv = x * inv;
          const float r = yv >= 0.0f ? yv + 0.5f : yv - 0.5f;
          const int qi = max(-127, min(127, (int)r));
          const bool is_k = grow0 < rp.qw + rp.kvw;
          __half* rowp = (is_k ? rp.k_cache : rp.v_cache) + slot;
          const int b = (grow0 - rp.qw - (is_k ? 0 : rp.kvw)) >> 5;
          if (lane < 32) ((int8_t*)rowp)[b * 32 + l32] = (int8_t)qi;
          if (lane == 0) rowp[(rp.kvw >> 1) + b] = __float2half_rn(amax / 127.0f);
        }
      }
    } else if (lane < RPW && row < rows) {
      if (pr.is_q) y[row] = o;
      else if (pr.is_k) rp.k_cache[slot + (row - rp.qw)] = __float2half_rn(o);
      else rp.v_cache[slot + (row - rp.qw - rp.kvw)] = __float2half_rn(o);
    }
    g += gridDim.x;
    if (g >= groups) break;
    pr = pair_of(g);
    step = rp.steps[pr.pair];
    factor = rp.factors ? rp.factors[pr.pair] : 1.0f;
#pragma unroll
    for (int r = 0; r < RPW; r++) un[r].load(rows::seg_row(sg, min(pr.row0 + r, rows - 1)), 0, 0, 0, u);
  }
}


}  // namespace

// Compute units of the current device (cached per device).
int cu_count() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

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

int launch_q4k_glu_norm(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                        int32_t cols, const float* x, const float* gain, float eps, float* y, void* xq_out) {
  if (!q4k_glu_norm_fits(rows, cols, x, gain))
    return fail(MI_ERR_SHAPE, "matvec: no normed GLU for %d x %d", rows, cols);
  RowSegs sg{};
  sg.w[0] = (const uint8_t*)gate;
  sg.w[1] = sg.w[2] = (const uint8_t*)up;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 2;
  const int groups = rows / 32;
  const int grid = std::max(std::min(groups, cu_count()), (groups + kGluIts - 1) / kGluIts);
  hipLaunchKernelGGL(glu_norm_kernel<4>, dim3(grid), dim3(8 * 64), 0, s, sg, cols, y,
                     MI_EPI_NONE, NormIn{x, gain, eps}, (uint8_t*)xq_out);
  return hip_check(hipGetLastError(), "matvec launch");
}

bool q4k_qkv_norm_fits(int32_t cols, int32_t head_dim, int32_t rope_dim, const void* x, const void* gain) {
  return q4k_qkv_rope_fits(cols, head_dim, rope_dim) && !(((uintptr_t)x | (uintptr_t)gain) & 15);
}

int launch_q4k_qkv_norm(hipStream_t s, const RowSegs& sg, int32_t cols, const float* x, const float* gain,
                        float eps, float* q, const QkvRope& rp, bool q8) {
  if (!q4k_qkv_norm_fits(cols, rp.head_dim, rp.rope_dim, x, gain) || !rp.steps)
    return fail(MI_ERR_SHAPE, "matvec: no normed q|k|v for %d columns, head_dim %d", cols, rp.head_dim);
  const int rows = sg.end[sg.nseg - 1];
  if (q8) {
    if (rp.qw % 32 || rp.kvw % 32)
      return fail(MI_ERR_SHAPE, "matvec: q8_0 q|k|v needs q and kv widths of whole 32-value blocks");
    hipLaunchKernelGGL((qkv_norm_kernel<1, true>), dim3(std::min((rows + 31) / 32, cu_count())), dim3(16 * 64), 0,
                       s, sg, cols, q, NormIn{x, gain, eps}, rp);
    return hip_check(hipGetLastError(), "matvec launch");
  }
  const int groups = (rows + 23) / 24;
  hipLaunchKernelGGL(qkv_norm_kernel<1>, dim3(std::min(groups, cu_count())), dim3(12 * 64), 0, s, sg, cols, q,
                     NormIn{x, gain, eps}, rp);
  return hip_check(hipGetLastError(), "matvec launch");
}

bool q4k_glu_norm_fits(int32_t rows, int32_t cols, const void* x, const void* gain) {
  // 512 threads of 8 values cover 4096 columns; the row loads are float4
  return rows % 32 == 0 && rows > 0 && rows_fits(MI_Q4_K, cols) && cols <= 4096 && !(((uintptr_t)x | (uintptr_t)gain) & 15);
}

}  // namespace mi

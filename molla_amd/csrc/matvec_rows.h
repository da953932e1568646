// matvec_rows.h -- the batch-1 matvec kernel (the decode hot loop) for the
// kinds with 64-value units: Q4_K, Q4_0, Q8_0; gfx950; launched from
// matvec_rows.hip.
//
// Same arithmetic as matvec_kernel<KIND, R, 1> (matvec_units.h units),
// organised for a single token, where the whole cost is streaming the
// weights once:
//
//  * A wave owns RPW consecutive rows and one K-slice of at most 64 units
//    (4096 values): lane l keeps the activation of unit u0 + l in registers
//    for the whole wave (loaded once, before any weight), so the activation
//    is never re-read per row.
//  * All of the wave's weight loads are issued up front, straight-line; rows
//    are then computed in order, each waiting only for its own loads (the
//    compiler's vmcnt counts down row by row), so compute of one row overlaps
//    the arrival of the next rows and of every other wave's data.
//  * No LDS staging and few enough VGPRs that every wave of a 14336-row
//    matrix is resident at once; single-wave blocks are handed out evenly
//    over the CUs (multi-wave blocks left whole CUs with an extra block).
//  * cols > 4096 splits K over KS waves of one block (the down projection,
//    14336 = 4 x 3584); their partial sums meet in LDS and wave 0 adds them
//    in a fixed order, so results do not depend on timing.
//  * Rows may come from up to three matrices laid end to end in the output
//    (q, k and v of a layer in one launch), and in GLU mode each wave takes
//    the same rows of two matrices (gate, up) and writes act(gate) * up.
//
// Replaces the reference's planar_matvec_kernel (src/molla/nn/gpu.mojo:1533)
// at batch 1; the epilogue is gpu.mojo:1005 write_epilogue.
#pragma once

#include "matvec_units.h"

namespace mi {

// Up to three row-major GGUF matrices of the same width whose rows are
// numbered consecutively: rows [end[s-1], end[s]) come from w[s].
struct RowSegs {
  const uint8_t* w[3];
  int64_t rb[3];
  int32_t end[3];
  int32_t nseg;
};

// The q|k|v launch's epilogue for one decoding token (Llama pairing,
// adjacent elements): rows [0, qw) are q, rotated and written to y; rows
// [qw, qw + kvw) are k, rotated and stored as halves into k_cache at slot
// pos[0]; rows [qw + kvw, qw + 2 kvw) are v, stored as halves into v_cache.
// trig holds (cos, sin) of pos * step for each pair (rms_norm wrote it).
struct QkvRope {
  int qw, kvw, head_dim, rope_dim;
  const float2* trig;
  const int32_t* pos;
  __half* k_cache;
  __half* v_cache;
  const int32_t* kv_index;  // paged: the cell of position pos[0] is kv_index[pos[0]]; null: slot pos[0]
  const float* steps;       // qkv_norm_kernel and the batched tile compute (cos, sin) from these
  const float* factors;     // rope_freqs.weight, or null
  // batched tile: token t's cache row is kv_index[t * index_stride + pos[t]]
  // (paged) or t * cache_stride + pos[t] * kvw halves (stride 0: one
  // sequence's chunk)
  int64_t cache_stride, index_stride;
};

// The RMSNorm that glu_norm_kernel applies to its input row itself (the
// residual x, the norm's gain and epsilon) instead of reading xq.
struct NormIn {
  const float* x;
  const float* gain;
  float eps;
};

namespace rows {
using namespace mv;

// The wave sums of four values a lane, transposed: lane l ends with the sum
// of value l / 16 over the wave.  Two half swaps pair rows 0|2 and 1|3 (the
// lower 32 lanes keep rows 0 and 1), one row swap pairs those (16-lane row
// g keeps value g), and a 16-lane sum finishes each.
__device__ __forceinline__ float wave_sum_rows4(float a0, float a1, float a2, float a3) {
  const auto p02 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a0), __float_as_uint(a2), false, false);
  const auto p13 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a1), __float_as_uint(a3), false, false);
  const float x = __uint_as_float(p02[0]) + __uint_as_float(p02[1]);  // lanes < 32: row 0, else row 2
  const float y = __uint_as_float(p13[0]) + __uint_as_float(p13[1]);  // lanes < 32: row 1, else row 3
  const auto pb = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  const float z = __uint_as_float(pb[0]) + __uint_as_float(pb[1]);
  return lanes::reduce<16>(z, lanes::Add{});
}

// The same for eight values: lane l ends with the sum of value
// (g & 1) + 2 h + 4 (g >> 1), g = l / 16, h = l / 8 % 2, so value r sits 32
// lanes below value r + 4.  After the half and row swaps, each 8-lane half
// of a row keeps one of its two values and adds its partner half's (row
// rotate by 8), and an 8-lane sum finishes.
__device__ __forceinline__ float wave_sum_rows8(const float (&a)[8]) {
  float x[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a[i]), __float_as_uint(a[i + 4]), false, false);
    x[i] = __uint_as_float(p[0]) + __uint_as_float(p[1]);  // lanes < 32: value i, else i + 4
  }
  const auto p01 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[0]), __float_as_uint(x[1]), false, false);
  const auto p23 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[2]), __float_as_uint(x[3]), false, false);
  const float z0 = __uint_as_float(p01[0]) + __uint_as_float(p01[1]);  // rows 0, 1, 4, 5 of 16 lanes
  const float z1 = __uint_as_float(p23[0]) + __uint_as_float(p23[1]);  // rows 2, 3, 6, 7
  const bool hi = (__lane_id() & 8) != 0;
  const float keep = hi ? z1 : z0, send = hi ? z0 : z1;
  const float w = keep + __uint_as_float(lanes::dpp<0x128>(__float_as_uint(send)));  // row_ror:8
  return lanes::reduce<8>(w, lanes::Add{});
}

// Activation of one lane's 64-value unit (groups 2u and 2u + 1); the
// per-half limb sums of plane 7 only for the kinds with an offset (Q4_0).
template <bool L23>
struct XUnitRegs {
  uint4 l[2][3][2];
  XMeta m[2];
  int2 s23[L23 ? 2 : 1];
  __device__ __forceinline__ uint4 limb(int, int j, int hh, int g) const { return l[g & 1][j][hh]; }
  __device__ __forceinline__ XMeta meta(int, int g) const { return m[g & 1]; }
  __device__ __forceinline__ int2 lsum23(int, int g) const { return s23[L23 ? (g & 1) : 0]; }
};

// Row `row` of the segmented matrix: base address of its blocks.  The
// segment fields are picked by constant index: indexing the kernel-argument
// arrays with a per-lane value would fetch them with vector loads, whose
// wait (vmcnt) then also waits for every weight load already in flight.
__device__ __forceinline__ const uint8_t* seg_row(const RowSegs& sg, int row) {
  const bool s0 = row < sg.end[0], s1 = !s0 && row < sg.end[1];
  const uint8_t* w = s0 ? sg.w[0] : (s1 ? sg.w[1] : sg.w[2]);
  const int64_t rb = s0 ? sg.rb[0] : (s1 ? sg.rb[1] : sg.rb[2]);
  const int start = s0 ? 0 : (s1 ? sg.end[0] : sg.end[1]);
  return w + (int64_t)(row - start) * rb;
}

// The activation of unit u (groups 2u, 2u + 1) into a lane's registers.
template <bool L23, class XA>
__device__ __forceinline__ void load_x(XUnitRegs<L23>& xr, const XA& xa, int u) {
#pragma unroll
  for (int e = 0; e < 2; e++) {
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int hh = 0; hh < 2; hh++) xr.l[e][j][hh] = xa.limb(0, j, hh, 2 * u + e);
    xr.m[e] = xa.meta(0, 2 * u + e);
    if constexpr (L23) xr.s23[e] = xa.lsum23(0, 2 * u + e);
  }
}

// GLU: sg.w[0] = gate, sg.w[1] = up, both with sg.end[0] rows.  KIND is
// any kind with 64-value units (Q4_K, Q4_0, Q8_0; matvec_units.h).
// ROPE: the QkvRope epilogue instead of write_epilogue (RPW even).
// GQ (GLU, KS == 1): a block is 32 / RPW waves owning one 32-row group, and
// it also writes that group of y in matvec form into xq_out (the down
// projection's input), so no quantize launch follows.
template <int KIND, int RPW, int KS, bool GLU, bool ROPE = false, bool GQ = false>
__global__ __launch_bounds__(GQ ? 32 / RPW * 64 : KS * 64) void rows_kernel(
    const RowSegs sg, int cols, const uint8_t* __restrict__ xq, float* __restrict__ y, int epi,
    const float* __restrict__ aux, const QkvRope rp, uint8_t* __restrict__ xq_out) {
  static_assert(!GQ || (GLU && KS == 1 && 32 % RPW == 0), "GQ: GLU, one K-slice, whole groups");
  constexpr int NR = GLU ? 2 * RPW : RPW;
  __shared__ float part[KS > 1 ? KS * NR : 1];
  const int lane = threadIdx.x & 63;
  const int ks = KS > 1 ? (threadIdx.x >> 6) : 0;
  const int rows = GLU ? sg.end[0] : sg.end[sg.nseg - 1];
  const int wib = GQ ? (threadIdx.x >> 6) : 0;  // wave in the group block
  const int row0 = (GQ ? blockIdx.x * (32 / RPW) + wib : blockIdx.x) * RPW;
  const int units = cols >> 6;
  const int u0 = ks * units / KS, u1 = (ks + 1) * units / KS;
  const bool act = u0 + lane < u1;
  const int u = act ? u0 + lane : u1 - 1;

  constexpr bool kL23 = KIND == MI_Q4_0 || KIND == MI_Q5_0;  // kinds with a fixed offset
  XUnitRegs<kL23> xr;
  typename UnitOf<KIND, 1>::type un[NR];
  // the epilogue's operand (plain rows): loaded first, so the store at the
  // end waits for nothing queued behind the weights
  // (branch-free: a load under a branch makes the compiler wait for every
  // load in flight at the join)
  float pre = 0.0f;
  if constexpr (!GLU && !ROPE) {
    const float* src = (epi & (MI_EPI_BIAS | MI_EPI_GLU)) ? aux : y;
    pre = src[min(row0 + (NR == 4 ? lane >> 4 : lane & (RPW - 1)), rows - 1)];  // the row it stores (kT4)
  }
  load_x(xr, XAcc{xq, 4 * (int64_t)cols, (int64_t)(cols >> 5) * 16}, u);
#pragma unroll
  for (int r = 0; r < NR; r++) {
    const int row = min(row0 + (GLU ? r % RPW : r), rows - 1);
    const uint8_t* base = GLU ? sg.w[r / RPW] + (int64_t)row * sg.rb[r / RPW] : seg_row(sg, row);
    un[r].load(base, 0, 0, 0, u);
  }

  float acc[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    float a[1][1] = {{0.0f}};
    un[r].template compute<1>(xr, u, a);
    acc[r] = act ? a[0][0] : 0.0f;
    // keep row r's work ahead of row r+1's (and its wait for row r+1's loads)
    __builtin_amdgcn_sched_barrier(0);
  }
  // four plain rows: a transposed reduction leaves row lane / 16 in every
  // lane of each 16-lane row (10 instructions against 4 full wave sums; the
  // 14336x4096 launch 9.0 -> 8.8 us); otherwise lane r holds matrix-row r
  // of this wave (GLU: r < RPW gate, r >= RPW up)
  constexpr bool kT4 = NR == 4 && !GLU && !ROPE;
  // the lanes that hold a row: r (or 16 r), and which row
  const bool holds = kT4 ? (lane & 15) == 0 : lane < NR;
  const int hrow = kT4 ? lane >> 4 : lane;
  float v;
  if constexpr (kT4) {
    v = wave_sum_rows4(acc[0], acc[1], acc[2], acc[3]);
  } else {
#pragma unroll
    for (int r = 0; r < NR; r++) acc[r] = wave_sum(acc[r]);
    v = acc[0];
#pragma unroll
    for (int r = 1; r < NR; r++)
      if (lane == r) v = acc[r];
  }
  if constexpr (KS > 1) {
    if (ks > 0 && holds) part[ks * NR + hrow] = v;
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int k = 1; k < KS; k++)
      if (holds) v += part[k * NR + hrow];
  }
  if constexpr (ROPE) {
    // rope.mojo:294 rotate_scaled, adjacent pairs: (a, b) <- (a c - b s, a s + b c)
#pragma clang fp contract(off)
    const int row = row0 + lane;
    const float partner = __shfl_xor(v, 1);
    if (lane < RPW && row < rows) {
      const bool is_q = row < rp.qw, is_k = !is_q && row < rp.qw + rp.kvw;
      float o = v;
      if (is_q || is_k) {
        const int e = (is_q ? row : row - rp.qw) % rp.head_dim;
        if (e < rp.rope_dim) {
          const float2 cs = rp.trig[e >> 1];
          const float a = (e & 1) ? partner : v, b = (e & 1) ? v : partner;
          o = (e & 1) ? a * cs.y + b * cs.x : a * cs.x - b * cs.y;
        }
      }
      const int64_t slot = (int64_t)(rp.kv_index ? rp.kv_index[rp.pos[0]] : rp.pos[0]) * rp.kvw;
      if (is_q) y[row] = o;
      else if (is_k) rp.k_cache[slot + (row - rp.qw)] = __float2half_rn(o);
      else rp.v_cache[slot + (row - rp.qw - rp.kvw)] = __float2half_rn(o);
    }
  } else if constexpr (GLU) {
    const float upv = __shfl_down(v, RPW);
    const float o = ((epi & MI_ACT_GELU) ? gelu(v) : silu(v)) * upv;
    if (lane < RPW && row0 + lane < rows) {
      if (epi & MI_EPI_ADD) y[row0 + lane] += o;
      else y[row0 + lane] = o;
    }
    if constexpr (GQ) {
      __shared__ float grp[32];
      if (lane < RPW) grp[wib * RPW + lane] = o;
      __syncthreads();
      if (wib == 0) quantize_group32(grp[lane & 31], lane & 31, blockIdx.x, rows >> 5, xq_out, lane < 32);
    }
  } else if constexpr (kT4) {
    if (holds && row0 + hrow < rows) epilogue_with(y, epi, row0 + hrow, pre, v);
  } else {
    if (lane < RPW && row0 + lane < rows) epilogue_with(y, epi, row0 + lane, pre, v);
  }
}

// ---- launchers (shared by matvec_rows.hip and matvec_rows_more.hip) ----------

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

// K split over KS = ceil(units / 64) waves of one block.
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

inline RowSegs one_matrix(const void* w, int64_t row_bytes, int32_t rows) {
  RowSegs sg{};
  sg.w[0] = sg.w[1] = sg.w[2] = (const uint8_t*)w;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 1;
  return sg;
}

}  // namespace rows

// Batch-1 rows for Q4_1, Q5_0, Q5_1 and Q5_K (matvec_rows_more.hip).
int launch_rows_more(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                     const void* xq, float* y, int32_t epi, const float* aux);
}  // namespace mi

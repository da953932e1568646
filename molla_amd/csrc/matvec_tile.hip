// matvec_tile.hip -- the batched (2..8 tokens) Q4_K matvec on the matrix
// cores (v_mfma_i32_32x32x32_i8), gfx950.
//
// At batch b the matvec becomes a small dense contraction: per 32-value
// group, 32 rows of 4-bit codes against b tokens' three int8 limbs.  One
// MFMA multiplies a 32(M) x 32(K) int8 A by a 32(K) x 32(N) int8 B:
//   N = 32 rows of the tile (lane l supplies row l % 32's codes for values
//       16 (l / 32) .. +16 of the group: the low or high nibbles of 16 bytes),
//   M = 8 slots x 4: slot s holds (token s % T, group s / T of an 8/T-group
//       window), rows 4s + j of A are that token's limb j (j = 3 is zero),
//   K = the 32 values of one group.
// A window's MFMAs each add one group, whose A is non-zero only in that
// group's slots, so after 8/T MFMAs the int32 accumulator holds every
// (token, group) pair of the window in its own slot; lane (row n, half h)
// then owns slots 2a + h (a = 0..3) in C[4a .. 4a+2] and applies the
// group's scales once per slot.  Integer products are exact, as in the
// VALU kernels; the result agrees with them to float rounding.
//
// Work decomposition: a block is one tile of 32 rows; its (up to 8) waves
// split the superblocks of the row, SBW per wave.  A wave keeps the next
// superblock's weights and activation limbs in flight while it computes the
// current one.  Every token's per-group (scale, sum) is staged in LDS once
// per block; the limbs come from global memory (L2): eight tokens of 4096
// values are 128 KB, too much to stage per block.  Partial sums meet in LDS
// and wave 0 adds them in a fixed order.
//
// Replaces the batched planar_matmul_kernel (src/molla/nn/gpu.mojo:1809) for
// Q4_K; output y[t * ldy + r] and epilogues as gpu.mojo:1005.
#include "matvec_rows.h"

namespace mi {
namespace {
using namespace mv;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i as_v4i(uint4 u) {
  v4i r;
  r[0] = (int)u.x;
  r[1] = (int)u.y;
  r[2] = (int)u.z;
  r[3] = (int)u.w;
  return r;
}

// (sc, m) of group j (0..7) from scales[0..11] held in y, z, w4
// (quant.mojo:161 _k_scale), without a lane-divergent branch.
__device__ __forceinline__ void kscale(uint32_t y, uint32_t z, uint32_t w4, int j, uint32_t& sc, uint32_t& m) {
  const uint32_t s = 8u * (uint32_t)(j & 3);
  const uint32_t hi = (uint32_t)(j >> 2);  // 1 for groups 4..7
  sc = __builtin_amdgcn_ubfe(hi ? w4 : y, s, 4) | (__builtin_amdgcn_ubfe(y, s + 4 + 2 * hi, 2) << 4);
  m = __builtin_amdgcn_ubfe(hi ? w4 : z, s + 4 * hi, 4) | (__builtin_amdgcn_ubfe(z, s + 4 + 2 * hi, 2) << 4);
}

// The segment fields as scalar values for a per-lane row: selects between
// the kernel argument's array elements by a per-lane row were folded back
// into a per-lane index, which copied the whole struct to scratch memory
// (72 bytes a lane) and read it back with vector loads at every launch.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const uint8_t* uni(const uint8_t* p) {
  const uint64_t v = (uint64_t)p;
  return (const uint8_t*)((uint64_t)(uint32_t)uni((int)v) | ((uint64_t)(uint32_t)uni((int)(v >> 32)) << 32));
}
__device__ __forceinline__ int64_t uni(int64_t v) { return (int64_t)(uint64_t)uni((const uint8_t*)v); }

__device__ __forceinline__ const uint8_t* lane_seg_row(const RowSegs& sg, int row) {
  const int e0 = uni(sg.end[0]), e1 = uni(sg.end[1]);
  const bool s0 = row < e0, s1 = !s0 && row < e1;
  const uint8_t* w = s0 ? uni(sg.w[0]) : (s1 ? uni(sg.w[1]) : uni(sg.w[2]));
  const int64_t rb = s0 ? uni(sg.rb[0]) : (s1 ? uni(sg.rb[1]) : uni(sg.rb[2]));
  return w + (int64_t)(row - (s0 ? 0 : (s1 ? e0 : e1))) * rb;
}
__device__ __forceinline__ int lane_seg_rows(const RowSegs& sg) {
  const int n = uni(sg.nseg);
  return n >= 3 ? uni(sg.end[2]) : (n == 2 ? uni(sg.end[1]) : uni(sg.end[0]));
}

constexpr int kTileWaves = 8;  // waves per block for matrices of many tiles
constexpr int kWideWaves = 16;  // ... and for few (<= 8192 rows): more waves split K

// Rows come from RowSegs (one matrix, or q|k|v end to end).  GLU: sg.w[0] =
// gate, sg.w[1] = up, both with sg.end[0] rows; every wave walks its
// superblocks of the gate row, then of the up row, and the block writes
// act(gate) * up.
// ROPE (q|k|v, Llama pairing, f16 cache): the epilogue rotates q and k rows
// with each token's own position and writes q to y, k and v to the cache, as
// rope_store_kernel does after an unrotated q|k|v; no separate launch.
template <int T, int SBW, bool GLU, int KW, bool ROPE = false>
__global__ __launch_bounds__(KW * 64) void q4k_tile_kernel(const RowSegs sg, int cols, int tn,
                                                                   const uint8_t* __restrict__ xq,
                                                                   float* __restrict__ y, int64_t ldy, int epi,
                                                                   const float* __restrict__ aux,
                                                                   uint8_t* __restrict__ xq_out, const QkvRope rp) {
  constexpr int GW = 8 / T;    // groups per window
  constexpr int NW = 8 / GW;   // windows per superblock
  constexpr int NSL = GW * T;  // slots in use
  constexpr int NP = GLU ? 2 : 1;  // passes: gate, then up
  extern __shared__ float2 meta_lds[];  // [T][G] (scale, xsum)
  __shared__ float red[NP][KW][T][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ks = blockDim.x >> 6;
  const int n = lane & 31, kh = lane >> 5;
  const int rows = GLU ? sg.end[0] : lane_seg_rows(sg);
  const int row = min(blockIdx.x * 32 + n, rows - 1);
  const uint8_t* wrow[NP];
  wrow[0] = GLU ? sg.w[0] + (int64_t)row * sg.rb[0] : lane_seg_row(sg, row);
  if (GLU) wrow[NP - 1] = sg.w[1] + (int64_t)row * sg.rb[1];
  const int nsb = cols >> 8, G = cols >> 5;
  // gridDim.y > 1 splits K over blocks: block y takes waves y * ks .. of the
  // row and writes its raw sums to y + blockIdx.y * tn * ldy (epi NONE)
  const int sb0 = (blockIdx.y * ks + wave) * SBW;
  if (gridDim.y > 1) y += (int64_t)blockIdx.y * tn * ldy;
  // activation offsets in 32 bits (8 tokens of 16384 values are 512 KB), so
  // each load is one base register plus a 32-bit offset
  const int tok = 4 * cols, plane = (cols >> 5) * 16;

  // two superblocks of weights in flight: the next one's loads are issued
  // before the current one is computed; step i < SBW * NP is superblock
  // i % SBW of pass i / SBW
  uint4 hdr[2], qp[2][4];
  auto load_w = [&](int i, int slot) {
    const uint8_t* blk = wrow[i / SBW] + (int64_t)min(sb0 + i % SBW, nsb - 1) * 144;
    hdr[slot] = ld16(blk);
#pragma unroll
    for (int h = 0; h < 4; h++) qp[slot][h] = ld16(blk + 16 + 32 * h + 16 * kh);
  };
  // this lane's A role: slot s = m / 4, limb m % 4; it feeds one MFMA per
  // window (group a_gi of the window), so a superblock needs NW loads
  const int m = lane & 31, s = m >> 2, jj = m & 3;
  const int a_tok = s % T, a_gi = s / T;
  const bool a_live = jj < 3 && s < NSL && a_tok < tn;
  const int a_off = a_tok * tok + (jj * 2 + kh) * plane + a_gi * 16;
  uint4 av[2][NW];
  auto load_a = [&](int i, int slot) {
    const int sb = min(sb0 + i % SBW, nsb - 1);
#pragma unroll
    for (int win = 0; win < NW; win++)
      av[slot][win] = a_live ? ld16(xq + (uint32_t)(a_off + (sb * 8 + win * GW) * 16)) : make_uint4(0, 0, 0, 0);
  };
  // every token's (scale, xsum) per group, once per block: loaded first,
  // since a wave's loads complete in order and the barrier below would
  // otherwise also wait for the weights issued ahead of them
  float2 mreg[2];
  int mi[2];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    mi[k] = (int)threadIdx.x + k * (int)blockDim.x;
    const int i = min(mi[k], tn * G - 1), t = i / G, g = i - t * G;
    mreg[k] = *(const float2*)(xq + (uint32_t)(t * tok + 6 * plane + g * 16));
  }
  load_w(0, 0);
  load_a(0, 0);
  if (SBW * NP > 1) {  // the second step (next superblock, or the up row)
    load_w(1, 1);
    load_a(1, 1);
  }
#pragma unroll
  for (int k = 0; k < 2; k++)
    if (mi[k] < tn * G) meta_lds[mi[k]] = mreg[k];
  for (int i = (int)threadIdx.x + 2 * (int)blockDim.x; i < tn * G; i += blockDim.x) {
    const int t = i / G, g = i - t * G;
    meta_lds[i] = *(const float2*)(xq + (uint32_t)(t * tok + 6 * plane + g * 16));
  }
  __syncthreads();

  float acc[NP][4];
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int a = 0; a < 4; a++) acc[p][a] = 0.0f;
#pragma unroll
  for (int i = 0; i < SBW * NP; i++) {
    const int pass = i / SBW;
    const int sb = sb0 + i % SBW;
    const int sl = i & 1;
    if (sb < nsb) {
      const float d = half_bits_to_float(hdr[sl].x), dmin = half_bits_to_float(hdr[sl].x >> 16);
#pragma unroll
      for (int win = 0; win < NW; win++) {
        v16i C = {};
#pragma unroll
        for (int gi = 0; gi < GW; gi++) {
          const int g = win * GW + gi;
          const uint4 q = qp[sl][g >> 1];
          const uint4 bq = (g & 1) ? make_uint4((q.x >> 4) & 0x0F0F0F0Fu, (q.y >> 4) & 0x0F0F0F0Fu,
                                                (q.z >> 4) & 0x0F0F0F0Fu, (q.w >> 4) & 0x0F0F0F0Fu)
                                   : make_uint4(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, q.z & 0x0F0F0F0Fu,
                                                q.w & 0x0F0F0F0Fu);
          const uint4 a = a_gi == gi ? av[sl][win] : make_uint4(0, 0, 0, 0);
          C = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(a), as_v4i(bq), C, 0, 0, 0);
        }
#pragma unroll
        for (int a = 0; a < 4; a++) {
          const int slot = 2 * a + kh;
          const int t = slot % T;
          if (slot < NSL && t < tn) {
            const int g = win * GW + slot / T;
            uint32_t sc, mn;
            kscale(hdr[sl].y, hdr[sl].z, hdr[sl].w, g, sc, mn);
            const float2 mt = meta_lds[t * G + sb * 8 + g];
            const float v = limbs_to_float(C[4 * a], C[4 * a + 1] * 256 + C[4 * a + 2]);
            acc[pass][a] = fmaf(d * (float)sc * mt.x, v, fmaf(-dmin * (float)mn, mt.y, acc[pass][a]));
          }
        }
      }
    }
    if (i + 2 < SBW * NP) {
      load_w(i + 2, sl);
      load_a(i + 2, sl);
    }
  }
  // per token: the slots of this lane holding token t, then both halves
#pragma unroll
  for (int p = 0; p < NP; p++)
#pragma unroll
    for (int t = 0; t < T; t++) {
      float v = 0.0f;
#pragma unroll
      for (int a = 0; a < 4; a++)
        if ((2 * a + kh) < NSL && (2 * a + kh) % T == t) v += acc[p][a];
      v += __shfl_xor(v, 32);
      if (kh == 0) red[p][wave][t][n] = v;
    }
  __syncthreads();
  // 32 T outputs; a block of fewer waves than T / 2 loops
  for (int o = threadIdx.x; o < 32 * tn; o += blockDim.x) {
    const int t = o >> 5, nn = o & 31;
    float v = 0.0f;
    for (int k = 0; k < ks; k++) v += red[0][k][t][nn];
    const int r = blockIdx.x * 32 + nn;
    if constexpr (ROPE) {
#pragma clang fp contract(off)
      // rope.mojo:294 rotate_scaled, adjacent pairs: (a, b) <- (a c - b s, a s + b c);
      // the partner row is the neighbouring lane (o ^ 1, the same token)
      const float partner = __shfl_xor(v, 1);
      if (r >= rows) continue;
      const int p = rp.pos[t];
      const bool is_q = r < rp.qw, is_k = !is_q && r < rp.qw + rp.kvw;
      float out = v;
      if (is_q || is_k) {
        const int e = (is_q ? r : r - rp.qw) % rp.head_dim;
        if (e < rp.rope_dim) {
          const float theta = rope_theta(p, rp.steps, rp.factors, e >> 1);
          const float c = (float)cos((double)theta), sn = (float)sin((double)theta);
          const float a = (e & 1) ? partner : v, b = (e & 1) ? v : partner;
          out = (e & 1) ? a * sn + b * c : a * c - b * sn;
        }
      }
      if (is_q) {
        y[(int64_t)t * ldy + r] = out;
      } else {
        const int64_t at = rp.kv_index ? (int64_t)rp.kv_index[t * rp.index_stride + p] * rp.kvw
                                       : (int64_t)t * rp.cache_stride + (int64_t)p * rp.kvw;
        if (is_k) rp.k_cache[at + (r - rp.qw)] = __float2half_rn(out);
        else rp.v_cache[at + (r - rp.qw - rp.kvw)] = __float2half_rn(out);
      }
      continue;
    }
    if (r >= rows) continue;
    if constexpr (GLU) {
      float u = 0.0f;
      for (int k = 0; k < ks; k++) u += red[NP - 1][k][t][nn];
      const float o2 = ((epi & MI_ACT_GELU) ? gelu(v) : silu(v)) * u;
      const int64_t at = (int64_t)t * ldy + r;
      if (epi & MI_EPI_ADD) y[at] += o2;
      else y[at] = o2;
      // a half-wave holds one token's 32 rows of this tile: one xq group
      // (rows % 32 == 0, so every lane of it is live)
      if (xq_out)
        quantize_group32(o2, nn, r >> 5, rows >> 5, xq_out + (int64_t)t * xq_token_bytes(rows), true,
                         (epi & kEpiHx) ? xq_out + (int64_t)(tn + t) * xq_token_bytes(rows) : nullptr);
    } else {
      epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
    }
  }
}

// Split-K partials in y order: out = epilogue(part[0] + part[1]) (the two K
// halves added in that order, so the result does not depend on timing).
__global__ void tile_split_reduce_kernel(const float* __restrict__ part, int tn, int rows, float* __restrict__ y,
                                         int64_t ldy, int epi, const float* __restrict__ aux) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tn * rows) return;
  const int t = i / rows, r = i - t * rows;
  const float v = part[i] + part[(int64_t)tn * rows + i];
  epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
}

template <int T, int SBW>
int launch_split(hipStream_t s, const RowSegs& sg, int rows, int cols, int tn, const void* xq, float* y,
                 int64_t ldy, int epi, const float* aux, float* part) {
  const int waves = (cols / 256 + SBW - 1) / SBW;
  const int ks = (waves + 1) / 2;
  const size_t shm = (size_t)T * (cols / 32) * sizeof(float2);
  hipLaunchKernelGGL((q4k_tile_kernel<T, SBW, false, kWideWaves>), dim3((rows + 31) / 32, 2), dim3(ks * 64), shm, s,
                     sg, cols, tn, (const uint8_t*)xq, part, (int64_t)rows, MI_EPI_NONE, nullptr, nullptr, QkvRope{});
  int rc = hip_check(hipGetLastError(), "matvec launch");
  if (rc) return rc;
  hipLaunchKernelGGL(tile_split_reduce_kernel, dim3((tn * rows + 255) / 256), dim3(256), 0, s, part, tn, rows, y,
                     ldy, epi, aux);
  return hip_check(hipGetLastError(), "matvec split reduce");
}

template <int T, int SBW, bool GLU, int KW>
int launch_ts(hipStream_t s, const RowSegs& sg, int rows, int cols, int tn, const void* xq, float* y, int64_t ldy,
              int epi, const float* aux, void* xq_out, const QkvRope* rp = nullptr) {
  const int ks = (cols / 256 + SBW - 1) / SBW;
  const size_t shm = (size_t)T * (cols / 32) * sizeof(float2);
  if constexpr (!GLU) {
    if (rp) {
      hipLaunchKernelGGL((q4k_tile_kernel<T, SBW, false, KW, true>), dim3((rows + 31) / 32), dim3(ks * 64), shm, s,
                         sg, cols, tn, (const uint8_t*)xq, y, ldy, MI_EPI_NONE, nullptr, nullptr, *rp);
      return hip_check(hipGetLastError(), "matvec launch");
    }
  }
  hipLaunchKernelGGL((q4k_tile_kernel<T, SBW, GLU, KW>), dim3((rows + 31) / 32), dim3(ks * 64), shm, s, sg, cols, tn,
                     (const uint8_t*)xq, y, ldy, epi, aux, (uint8_t*)xq_out, QkvRope{});
  return hip_check(hipGetLastError(), "matvec launch");
}

// T is the token capacity of the slot layout (2, 3, 4 or 8); tn <= T tokens
// are live and the rest of the slots stay empty.
template <int T, bool GLU>
int launch_t(hipStream_t s, const RowSegs& sg, int rows, int cols, int tn, const void* xq, float* y,
             int64_t ldy, int epi, const float* aux, void* xq_out, const QkvRope* rp = nullptr) {
  const int nsb = cols / 256;
  // Few tiles (a 4096-row matrix is 128 blocks for 256 CUs): up to 16 waves
  // per block split K, so the whole chip streams.
  // (16-wave blocks have 128 registers per lane: the 8-token GLU form fits
  // only one superblock per wave, the 8-token plain form two.)
  constexpr int kWideSbw = T == 8 ? (GLU ? 1 : 2) : 4;
  if (rows <= 8192 && nsb <= kWideSbw * kWideWaves) {
    if (nsb <= kWideWaves) return launch_ts<T, 1, GLU, kWideWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
    if constexpr (kWideSbw >= 2)
      if (nsb <= 2 * kWideWaves)
        return launch_ts<T, 2, GLU, kWideWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
    if constexpr (kWideSbw >= 4) return launch_ts<T, 4, GLU, kWideWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
  }
  if (nsb <= 2 * kTileWaves) return launch_ts<T, 2, GLU, kTileWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
  if (nsb <= 4 * kTileWaves) return launch_ts<T, 4, GLU, kTileWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
  return launch_ts<T, 8, GLU, kTileWaves>(s, sg, rows, cols, tn, xq, y, ldy, epi, aux, xq_out, rp);
}

template <bool GLU>
int launch_g(hipStream_t s, const RowSegs& sg, int rows, int cols, const void* xq, int tokens, float* y,
             int64_t ldy, int epi, const float* aux, void* xq_out = nullptr, const QkvRope* rp = nullptr) {
  switch (tokens) {
    case 2: return launch_t<2, GLU>(s, sg, rows, cols, 2, xq, y, ldy, epi, aux, xq_out, rp);
    case 3: return launch_t<3, GLU>(s, sg, rows, cols, 3, xq, y, ldy, epi, aux, xq_out, rp);
    case 4: return launch_t<4, GLU>(s, sg, rows, cols, 4, xq, y, ldy, epi, aux, xq_out, rp);
    case 5:
    case 6:
    case 7:
    case 8: return launch_t<8, GLU>(s, sg, rows, cols, tokens, xq, y, ldy, epi, aux, xq_out, rp);
  }
  return fail(MI_ERR_ARG, "matvec: tokens %d outside 2..8 for the batched tile", tokens);
}

}  // namespace

// K split over two blocks per 32-row tile: for matrices of few tiles and a
// long K (the down projection: 128 tiles, 14336 values), so that all 256
// CUs share the VALU work of the tiles instead of 128.
bool q4k_tile_split_fits(int32_t rows, int32_t cols, int32_t tokens) {
  const int nsb = cols / 256;
  const int sbw = tokens > 4 ? 2 : 4;
  return q4k_tile_fits(cols, tokens) && rows <= 4096 && nsb >= 32 && (nsb + sbw - 1) / sbw <= 2 * kWideWaves;
}

size_t q4k_tile_split_bytes(int32_t rows, int32_t tokens) { return sizeof(float) * 2 * (size_t)rows * tokens; }

int launch_q4k_tile_split(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                          const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux,
                          float* part) {
  if (!q4k_tile_split_fits(rows, cols, tokens))
    return fail(MI_ERR_SHAPE, "matvec: no split-K tile for %d x %d at %d tokens", rows, cols, tokens);
  RowSegs sg{};
  sg.w[0] = sg.w[1] = sg.w[2] = (const uint8_t*)w;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 1;
  switch (tokens) {
    case 2: return launch_split<2, 4>(s, sg, rows, cols, 2, xq, y, ldy, epi, aux, part);
    case 3: return launch_split<3, 4>(s, sg, rows, cols, 3, xq, y, ldy, epi, aux, part);
    case 4: return launch_split<4, 4>(s, sg, rows, cols, 4, xq, y, ldy, epi, aux, part);
    default: return launch_split<8, 2>(s, sg, rows, cols, tokens, xq, y, ldy, epi, aux, part);
  }
}

bool q4k_tile_fits(int32_t cols, int32_t tokens) {
  return tokens >= 2 && tokens <= 8 && cols % 256 == 0 && cols / 256 <= 8 * kTileWaves;
}

int launch_q4k_tile(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  RowSegs sg{};
  sg.w[0] = sg.w[1] = sg.w[2] = (const uint8_t*)w;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 1;
  return launch_g<false>(s, sg, rows, cols, xq, tokens, y, ldy, epi, aux);
}

int launch_q4k_tile_segs(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, int32_t tokens, float* y,
                         int64_t ldy) {
  return launch_g<false>(s, sg, sg.end[sg.nseg - 1], cols, xq, tokens, y, ldy, MI_EPI_NONE, nullptr);
}

int launch_q4k_tile_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, int32_t tokens,
                             float* q, int64_t ldq, const QkvRope& rp) {
  if (rp.head_dim % 2 || rp.rope_dim % 2 || !rp.steps || !rp.pos)
    return fail(MI_ERR_SHAPE, "matvec: no fused rope for head_dim %d, rope_dim %d", rp.head_dim, rp.rope_dim);
  return launch_g<false>(s, sg, sg.end[sg.nseg - 1], cols, xq, tokens, q, ldq, MI_EPI_NONE, nullptr, nullptr, &rp);
}

int launch_q4k_tile_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows,
                        int32_t cols, const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                        void* xq_out) {
  if (xq_out && rows % 32) return fail(MI_ERR_SHAPE, "matvec: quantized GLU output needs rows %% 32 == 0");
  RowSegs sg{};
  sg.w[0] = (const uint8_t*)gate;
  sg.w[1] = sg.w[2] = (const uint8_t*)up;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = sg.end[1] = sg.end[2] = rows;
  sg.nseg = 2;
  return launch_g<true>(s, sg, rows, cols, xq, tokens, y, ldy, epi, nullptr, xq_out);
}

}  // namespace mi

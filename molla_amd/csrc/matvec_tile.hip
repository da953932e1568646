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
#include "matvec_units.h"

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

constexpr int kTileWaves = 8;

template <int T, int SBW>
__global__ __launch_bounds__(kTileWaves * 64) void q4k_tile_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                                   int rows, int cols, int tn,
                                                                   const uint8_t* __restrict__ xq,
                                                                   float* __restrict__ y, int64_t ldy, int epi,
                                                                   const float* __restrict__ aux) {
  constexpr int GW = 8 / T;    // groups per window
  constexpr int NW = 8 / GW;   // windows per superblock
  constexpr int NSL = GW * T;  // slots in use
  extern __shared__ float2 meta_lds[];  // [T][G] (scale, xsum)
  __shared__ float red[kTileWaves][T][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ks = blockDim.x >> 6;
  const int n = lane & 31, kh = lane >> 5;
  const int row = blockIdx.x * 32 + n;
  const uint8_t* wrow = w + (int64_t)min(row, rows - 1) * rb;
  const int nsb = cols >> 8, G = cols >> 5;
  const int sb0 = wave * SBW;
  // activation offsets in 32 bits (8 tokens of 16384 values are 512 KB), so
  // each load is one base register plus a 32-bit offset
  const int tok = 4 * cols, plane = (cols >> 5) * 16;

  // two superblocks of weights in flight: the next one's loads are issued
  // before the current one is computed
  uint4 hdr[2], qp[2][4];
  auto load_w = [&](int i, int slot) {
    const uint8_t* blk = wrow + (int64_t)min(sb0 + i, nsb - 1) * 144;
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
    const int sb = min(sb0 + i, nsb - 1);
#pragma unroll
    for (int win = 0; win < NW; win++)
      av[slot][win] = a_live ? ld16(xq + (uint32_t)(a_off + (sb * 8 + win * GW) * 16)) : make_uint4(0, 0, 0, 0);
  };
  load_w(0, 0);
  load_a(0, 0);
  if (SBW > 1) {
    load_w(1, 1);
    load_a(1, 1);
  }
  // every token's (scale, xsum) per group, once per block
  for (int i = threadIdx.x; i < tn * G; i += blockDim.x) {
    const int t = i / G, g = i - t * G;
    meta_lds[i] = *(const float2*)(xq + (uint32_t)(t * tok + 6 * plane + g * 16));
  }
  __syncthreads();

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < SBW; i++) {
    const int sb = sb0 + i;
    if (sb >= nsb) break;
    const int sl = i & 1;
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
          acc[a] = fmaf(d * (float)sc * mt.x, v, fmaf(-dmin * (float)mn, mt.y, acc[a]));
        }
      }
    }
    if (i + 2 < SBW) {
      load_w(i + 2, sl);
      load_a(i + 2, sl);
    }
  }
  // per token: the slots of this lane holding token t, then both halves
#pragma unroll
  for (int t = 0; t < T; t++) {
    float v = 0.0f;
#pragma unroll
    for (int a = 0; a < 4; a++)
      if ((2 * a + kh) < NSL && (2 * a + kh) % T == t) v += acc[a];
    v += __shfl_xor(v, 32);
    if (kh == 0) red[wave][t][n] = v;
  }
  __syncthreads();
  // 32 T outputs; a block of fewer waves than T / 2 loops
  for (int o = threadIdx.x; o < 32 * tn; o += blockDim.x) {
    const int t = o >> 5, nn = o & 31;
    float v = 0.0f;
    for (int k = 0; k < ks; k++) v += red[k][t][nn];
    const int r = blockIdx.x * 32 + nn;
    if (r < rows) epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
  }
}

template <int T, int SBW>
int launch_ts(hipStream_t s, const void* w, int64_t rb, int rows, int cols, int tn, const void* xq, float* y,
              int64_t ldy, int epi, const float* aux) {
  const int ks = (cols / 256 + SBW - 1) / SBW;
  const size_t shm = (size_t)T * (cols / 32) * sizeof(float2);
  hipLaunchKernelGGL((q4k_tile_kernel<T, SBW>), dim3((rows + 31) / 32), dim3(ks * 64), shm, s, (const uint8_t*)w,
                     rb, rows, cols, tn, (const uint8_t*)xq, y, ldy, epi, aux);
  return hip_check(hipGetLastError(), "matvec launch");
}

// T is the token capacity of the slot layout (2, 3, 4 or 8); tn <= T tokens
// are live and the rest of the slots stay empty.
template <int T>
int launch_t(hipStream_t s, const void* w, int64_t rb, int rows, int cols, int tn, const void* xq, float* y,
             int64_t ldy, int epi, const float* aux) {
  const int nsb = cols / 256;
  if (nsb <= 2 * kTileWaves) return launch_ts<T, 2>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
  if (nsb <= 4 * kTileWaves) return launch_ts<T, 4>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
  return launch_ts<T, 8>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
}

}  // namespace

bool q4k_tile_fits(int32_t cols, int32_t tokens) {
  return tokens >= 2 && tokens <= 8 && cols % 256 == 0 && cols / 256 <= 8 * kTileWaves;
}

int launch_q4k_tile(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  switch (tokens) {
    case 2: return launch_t<2>(s, w, row_bytes, rows, cols, 2, xq, y, ldy, epi, aux);
    case 3: return launch_t<3>(s, w, row_bytes, rows, cols, 3, xq, y, ldy, epi, aux);
    case 4: return launch_t<4>(s, w, row_bytes, rows, cols, 4, xq, y, ldy, epi, aux);
    case 5:
    case 6:
    case 7:
    case 8: return launch_t<8>(s, w, row_bytes, rows, cols, tokens, xq, y, ldy, epi, aux);
  }
  return fail(MI_ERR_ARG, "matvec: tokens %d outside 2..8 for the batched tile", tokens);
}

}  // namespace mi

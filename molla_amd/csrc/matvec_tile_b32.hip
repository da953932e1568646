// matvec_tile_b32.hip -- the batched (2..8 tokens) matvec on the matrix cores
// for the 32-value block kinds, gfx950:
//   Q4_0: 18 bytes / 32 values, d f16 @0, qs[16] @2: value l (l < 16) =
//         ((qs[l] & 15) - 8) d, value l + 16 = ((qs[l] >> 4) - 8) d
//         (quant.mojo:232 dequant_q4_0);
//   Q8_0: 34 bytes / 32 values, d f16 @0, qs[32] int8 @2: value l = qs[l] d
//         (quant.mojo:304 dequant_q8_0).
//
// The slot layout is the Q4_K tile's (matvec_tile.hip): one MFMA
// (v_mfma_i32_32x32x32_i8) per block, N = 32 rows, K = the block's 32
// values, M = 8 slots of (token, block of an 8/T-block window) x 4 limb rows.
// Q4_0 codes enter unsigned (0..15) and the -8 comes off through the
// activation's limb sums; Q8_0 codes are already int8.  A wave walks chunks
// of 8 blocks (256 values), keeping the next chunk's loads in flight; both
// 18- and 34-byte blocks land 2 bytes off alignment every other block and
// are realigned from 4-byte aligned dwords.
//
// Replaces the batched planar_matmul_kernel (src/molla/nn/gpu.mojo:1809) for
// Q4_0 and Q8_0; output y[t * ldy + r] and epilogues as gpu.mojo:1005.
#include "matvec_units.h"

namespace mi {
namespace {
using namespace mv;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v4i as_v4i(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  v4i r;
  r[0] = (int)a;
  r[1] = (int)b;
  r[2] = (int)c;
  r[3] = (int)d;
  return r;
}

constexpr int kB32Waves = 8;

template <int KIND>
struct B32;

// Q4_0: a lane holds the whole 144-byte chunk (36 dwords, 16-byte aligned:
// rows are whole numbers of 36-byte block pairs and chunks of 144 bytes).
template <>
struct B32<MI_Q4_0> {
  static constexpr int kBytes = 18;
  uint32_t v[36];
  __device__ __forceinline__ void load(const uint8_t* chunk, int) {
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const uint4 q = ld16(chunk + 16 * i);
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
  }
  // codes of block g for K half kb: low nibbles (kb 0) or high (kb 1) of qs
  __device__ __forceinline__ void codes(int g, int kb, uint32_t (&b)[4]) const {
    const int o = 18 * g + 2;  // qs byte offset: 2 mod 4 for even g, 0 for odd g
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t q = (o & 3) ? align(v[(o >> 2) + k + 1], v[(o >> 2) + k], 2) : v[(o >> 2) + k];
      b[k] = kb ? (q >> 4) & 0x0F0F0F0Fu : q & 0x0F0F0F0Fu;
    }
  }
  __device__ __forceinline__ float scale(int g) const {
    const int o = 18 * g;
    return half_bits_to_float(v[o >> 2] >> (8 * (o & 3)));
  }
  static constexpr int kOffset = 8;  // value = code - 8
};

// Q8_0: the 34-byte blocks at 2 + 34 g; a lane needs its K half (16 int8)
// of each block, five dwords, plus the scale's dword.
template <>
struct B32<MI_Q8_0> {
  static constexpr int kBytes = 34;
  uint32_t q[8][5];
  uint32_t dw[8];
  __device__ __forceinline__ void load(const uint8_t* chunk, int kb) {
#pragma unroll
    for (int g = 0; g < 8; g++) {
      const int o = 34 * g + 2 + 16 * kb;  // 2 mod 4 for even g, 0 for odd g
      const uint8_t* p = chunk + (o & ~3);
      const uint4 a = ld16a4(p);
      q[g][0] = a.x;
      q[g][1] = a.y;
      q[g][2] = a.z;
      q[g][3] = a.w;
      // the fifth dword only matters 2 bytes off alignment (even g); for odd
      // g it would lie past the block (past the tensor, for its last one)
      q[g][4] = (g & 1) ? a.w : ld4(p + 16);
      dw[g] = ld4(chunk + ((34 * g) & ~3));
    }
  }
  __device__ __forceinline__ void codes(int g, int, uint32_t (&b)[4]) const {
#pragma unroll
    for (int k = 0; k < 4; k++) b[k] = (g & 1) ? q[g][k] : align(q[g][k + 1], q[g][k], 2);
  }
  __device__ __forceinline__ float scale(int g) const { return half_bits_to_float(dw[g] >> (8 * ((34 * g) & 3))); }
  static constexpr int kOffset = 0;
};

template <int KIND, int T, int CPW>
__global__ __launch_bounds__(kB32Waves * 64) void b32_tile_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                                  int rows, int cols, int tn,
                                                                  const uint8_t* __restrict__ xq,
                                                                  float* __restrict__ y, int64_t ldy, int epi,
                                                                  const float* __restrict__ aux) {
  using Blk = B32<KIND>;
  constexpr int GW = 8 / T;    // blocks per window
  constexpr int NW = 8 / GW;   // windows per chunk
  constexpr int NSL = GW * T;  // slots in use
  extern __shared__ float2 meta_b32[];  // [T][G]: (scale, offset * limb sums recombined)
  __shared__ float red[kB32Waves][T][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ks = blockDim.x >> 6;
  const int n = lane & 31, kh = lane >> 5;
  const int row = blockIdx.x * 32 + n;
  const uint8_t* wrow = w + (int64_t)min(row, rows - 1) * rb;
  const int G = cols >> 5, nch = G >> 3;
  const int c0 = wave * CPW;
  const int tok = 4 * cols, plane = (cols >> 5) * 16;

  Blk wl[2];
  wl[0].load(wrow + (int64_t)min(c0, nch - 1) * 8 * Blk::kBytes, kh);
  if (CPW > 1) wl[1].load(wrow + (int64_t)min(c0 + 1, nch - 1) * 8 * Blk::kBytes, kh);

  const int m = lane & 31, s = m >> 2, jj = m & 3;
  const int a_tok = s % T, a_gi = s / T;
  const bool a_live = jj < 3 && s < NSL && a_tok < tn;
  const int a_off = a_tok * tok + (jj * 2 + kh) * plane + a_gi * 16;
  uint4 av[2][NW];
  auto load_a = [&](int i, int sl) {
    const int c = min(c0 + i, nch - 1);
#pragma unroll
    for (int win = 0; win < NW; win++)
      av[sl][win] = a_live ? ld16(xq + (uint32_t)(a_off + (c * 8 + win * GW) * 16)) : make_uint4(0, 0, 0, 0);
  };
  load_a(0, 0);
  if (CPW > 1) load_a(1, 1);
  // per (token, block): the activation scale, and the offset's share of the
  // limb sums (both halves: the offset applies to all 32 values)
  for (int i = threadIdx.x; i < tn * G; i += blockDim.x) {
    const int t = i / G, g = i - t * G;
    const XMeta mt = *(const XMeta*)(xq + (uint32_t)(t * tok + 6 * plane + g * 16));
    const int2 l23 = *(const int2*)(xq + (uint32_t)(t * tok + 7 * plane + g * 16));
    meta_b32[2 * i] = make_float2(mt.scale, __int_as_float(Blk::kOffset * (mt.lsum1[0] + mt.lsum1[1])));
    meta_b32[2 * i + 1] = make_float2(__int_as_float(Blk::kOffset * (l23.x + l23.y)), 0.0f);
  }
  __syncthreads();

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int i = 0; i < CPW; i++) {
    const int c = c0 + i;
    if (c >= nch) break;
    const int sl = i & 1;
#pragma unroll
    for (int win = 0; win < NW; win++) {
      v16i C = {};
#pragma unroll
      for (int gi = 0; gi < GW; gi++) {
        const int g = win * GW + gi;
        uint32_t b[4];
        wl[sl].codes(g, kh, b);
        const uint4 a = a_gi == gi ? av[sl][win] : make_uint4(0, 0, 0, 0);
        C = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(a.x, a.y, a.z, a.w), as_v4i(b[0], b[1], b[2], b[3]), C, 0,
                                                  0, 0);
      }
#pragma unroll
      for (int a = 0; a < 4; a++) {
        const int slot = 2 * a + kh;
        const int t = slot % T;
        if (slot < NSL && t < tn) {
          const int g = win * GW + slot / T;
          const int mi = 2 * (t * G + c * 8 + g);
          const float2 m0 = meta_b32[mi], m1 = meta_b32[mi + 1];
          const float v = limbs_to_float(C[4 * a] - __float_as_int(m0.y),
                                         C[4 * a + 1] * 256 + C[4 * a + 2] - __float_as_int(m1.x));
          acc[a] = fmaf(wl[sl].scale(g) * m0.x, v, acc[a]);
        }
      }
    }
    if (i + 2 < CPW) {
      wl[sl].load(wrow + (int64_t)min(c0 + i + 2, nch - 1) * 8 * Blk::kBytes, kh);
      load_a(i + 2, sl);
    }
  }
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
  for (int o = threadIdx.x; o < 32 * tn; o += blockDim.x) {
    const int t = o >> 5, nn = o & 31;
    float v = 0.0f;
    for (int k = 0; k < ks; k++) v += red[k][t][nn];
    const int r = blockIdx.x * 32 + nn;
    if (r < rows) epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
  }
}

template <int KIND, int T, int CPW>
int launch_tc(hipStream_t s, const void* w, int64_t rb, int rows, int cols, int tn, const void* xq, float* y,
              int64_t ldy, int epi, const float* aux) {
  const int ks = (cols / 256 + CPW - 1) / CPW;
  const size_t shm = (size_t)T * (cols / 32) * 2 * sizeof(float2);
  hipLaunchKernelGGL((b32_tile_kernel<KIND, T, CPW>), dim3((rows + 31) / 32), dim3(ks * 64), shm, s,
                     (const uint8_t*)w, rb, rows, cols, tn, (const uint8_t*)xq, y, ldy, epi, aux);
  return hip_check(hipGetLastError(), "matvec launch");
}

template <int KIND, int T>
int launch_t(hipStream_t s, const void* w, int64_t rb, int rows, int cols, int tn, const void* xq, float* y,
             int64_t ldy, int epi, const float* aux) {
  const int nch = cols / 256;
  if (nch <= 2 * kB32Waves) return launch_tc<KIND, T, 2>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
  if (nch <= 4 * kB32Waves) return launch_tc<KIND, T, 4>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
  return launch_tc<KIND, T, 8>(s, w, rb, rows, cols, tn, xq, y, ldy, epi, aux);
}

template <int KIND>
int launch_k(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, int tokens, float* y,
             int64_t ldy, int epi, const float* aux) {
  switch (tokens) {
    case 2: return launch_t<KIND, 2>(s, w, rb, rows, cols, 2, xq, y, ldy, epi, aux);
    // 3 tokens take the 4-token slots: with windows of 8 / 3 blocks the
    // block index of a slot is a run-time division, and the chunk's codes
    // went to scratch memory (304-400 bytes a lane; 54.8 against 35.5 us at
    // 4096 x 14336)
    case 3:
    case 4: return launch_t<KIND, 4>(s, w, rb, rows, cols, tokens, xq, y, ldy, epi, aux);
    case 5:
    case 6:
    case 7:
    case 8: return launch_t<KIND, 8>(s, w, rb, rows, cols, tokens, xq, y, ldy, epi, aux);
  }
  return fail(MI_ERR_ARG, "matvec: tokens %d outside 2..8 for the batched tile", tokens);
}

}  // namespace

bool b32_tile_fits(int kind, int32_t cols, int64_t row_bytes, int32_t tokens) {
  if (tokens < 2 || tokens > 8 || cols % 256 || cols / 256 > 8 * kB32Waves) return false;
  if (kind == MI_Q4_0) return row_bytes % 16 == 0;
  if (kind == MI_Q8_0) return row_bytes % 4 == 0;
  return false;
}

int launch_b32_tile(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                    const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  if (kind == MI_Q4_0) return launch_k<MI_Q4_0>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
  if (kind == MI_Q8_0) return launch_k<MI_Q8_0>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
  return fail(MI_ERR_KIND, "matvec: ggml type %d has no 32-value block tile", kind);
}

}  // namespace mi

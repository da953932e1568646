// matvec.hip -- fused dequantize-and-dot over raw GGUF blocks, gfx950.
//
// Replaces the reference's planar_matvec_kernel / planar_matmul_kernel
// (src/molla/nn/gpu.mojo:1533, :1809) for Q8_0, Q4_0, Q4_K and Q6_K.
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
#include "mi_internal.h"
#include "xq_device.h"

namespace mi {
namespace {

struct __attribute__((aligned(4))) U4a {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ uint4 ld16(const uint8_t* p) { return *(const uint4*)p; }
__device__ __forceinline__ uint4 ld16a4(const uint8_t* p) {
  U4a v = *(const U4a*)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ uint32_t comp(const uint4& v, int k) {
  return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}
__device__ __forceinline__ uint32_t align(uint32_t hi, uint32_t lo, uint32_t s) {
  return __builtin_amdgcn_alignbyte(hi, lo, s);
}

template <int KIND>
struct UnitElems;
template <> struct UnitElems<MI_Q4_K> { static constexpr int v = 64; };
template <> struct UnitElems<MI_Q4_0> { static constexpr int v = 64; };
template <> struct UnitElems<MI_Q8_0> { static constexpr int v = 64; };
template <> struct UnitElems<MI_Q6_K> { static constexpr int v = 128; };

// ---- Q4_K: unit u = quarter h of superblock sb (64 values, groups 2u, 2u+1)
template <int R, int T>
__device__ __forceinline__ void q4k_unit(const uint8_t* __restrict__ w, int64_t rb, int row0,
                                         int last_row, int u, const XPlanes (&xp)[T],
                                         float (&acc)[R][T]) {
  const int sb = u >> 2, h = u & 3;
  uint4 hdr[R];
  uint32_t lo[R][8], hi[R][8];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint8_t* blk = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)sb * 144;
    hdr[r] = ld16(blk);
    uint4 a = ld16(blk + 16 + 32 * h), b = ld16(blk + 32 + 32 * h);
    uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      lo[r][i] = q[i] & 0x0F0F0F0Fu;
      hi[r][i] = (q[i] >> 4) & 0x0F0F0F0Fu;
    }
  }
  // six-bit scale/min pair for group j = 2h + e (quant.mojo:161 _k_scale):
  // the byte shift is 16*(h&1) + 8e for both packings.
  float dsc[R][2], dmn[R][2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const float d = half_bits_to_float(hdr[r].x), dmin = half_bits_to_float(hdr[r].x >> 16);
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const uint32_t sh = 16u * (h & 1) + 8u * e;
      uint32_t sc_lo = __builtin_amdgcn_ubfe(hdr[r].y, sh, 6);
      uint32_t m_lo = __builtin_amdgcn_ubfe(hdr[r].z, sh, 6);
      uint32_t sc_hi = __builtin_amdgcn_ubfe(hdr[r].w, sh, 4) | (__builtin_amdgcn_ubfe(hdr[r].y, sh + 6, 2) << 4);
      uint32_t m_hi = __builtin_amdgcn_ubfe(hdr[r].w, sh + 4, 4) | (__builtin_amdgcn_ubfe(hdr[r].z, sh + 6, 2) << 4);
      const bool high = h >= 2;
      dsc[r][e] = d * (float)(high ? sc_hi : sc_lo);
      dmn[r][e] = dmin * (float)(high ? m_hi : m_lo);
    }
  }
  const int gA = 2 * u;
#pragma unroll
  for (int t = 0; t < T; t++) {
    uint4 xa[3][2], xb[3][2];
#pragma unroll
    for (int j = 0; j < 3; j++)
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        xa[j][hh] = xp[t].limb(j, hh, gA);
        xb[j][hh] = xp[t].limb(j, hh, gA + 1);
      }
    const XMeta ma = xp[t].meta(gA), mb = xp[t].meta(gA + 1);
#pragma unroll
    for (int r = 0; r < R; r++) {
      int sa[3] = {0, 0, 0}, sbb[3] = {0, 0, 0};
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 3; j++) {
          sa[j] = dot4(lo[r][i], comp(xa[j][i >> 2], i & 3), sa[j]);
          sbb[j] = dot4(hi[r][i], comp(xb[j][i >> 2], i & 3), sbb[j]);
        }
      const float va = limbs_to_float(sa[0], sa[1] * 256 + sa[2]);
      const float vb = limbs_to_float(sbb[0], sbb[1] * 256 + sbb[2]);
      float part = dsc[r][0] * (ma.scale * va) - dmn[r][0] * ma.xsum;
      part += dsc[r][1] * (mb.scale * vb) - dmn[r][1] * mb.xsum;
      acc[r][t] += part;
    }
  }
}

// ---- Q4_0: unit u = blocks 2u, 2u+1 (36 bytes, groups 2u, 2u+1)
template <int R, int T>
__device__ __forceinline__ void q40_unit(const uint8_t* __restrict__ w, int64_t rb, int row0,
                                         int last_row, int u, const XPlanes (&xp)[T],
                                         float (&acc)[R][T]) {
  uint32_t lo[R][2][4], hi[R][2][4];
  float d[R][2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * 36;
    uint4 a = ld16a4(p), b = ld16a4(p + 16);
    uint32_t c = ld4(p + 32);
    uint32_t W[9] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c};
    d[r][0] = half_bits_to_float(W[0]);
    d[r][1] = half_bits_to_float(W[4] >> 16);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint32_t qa = align(W[i + 1], W[i], 2), qb = W[5 + i];
      lo[r][0][i] = qa & 0x0F0F0F0Fu;
      hi[r][0][i] = (qa >> 4) & 0x0F0F0F0Fu;
      lo[r][1][i] = qb & 0x0F0F0F0Fu;
      hi[r][1][i] = (qb >> 4) & 0x0F0F0F0Fu;
    }
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
#pragma unroll
    for (int bk = 0; bk < 2; bk++) {
      const int g = 2 * u + bk;
      uint4 x0[3], x1[3];
#pragma unroll
      for (int j = 0; j < 3; j++) {
        x0[j] = xp[t].limb(j, 0, g);
        x1[j] = xp[t].limb(j, 1, g);
      }
      const XMeta m = xp[t].meta(g);
      const int2 l23 = xp[t].lsum23(g);
      const int c1 = 8 * (m.lsum1[0] + m.lsum1[1]), c23 = 8 * (l23.x + l23.y);
#pragma unroll
      for (int r = 0; r < R; r++) {
        int s[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) {
            s[j] = dot4(lo[r][bk][i], comp(x0[j], i), s[j]);
            s[j] = dot4(hi[r][bk][i], comp(x1[j], i), s[j]);
          }
        const float v = limbs_to_float(s[0] - c1, s[1] * 256 + s[2] - c23);
        acc[r][t] += d[r][bk] * (m.scale * v);
      }
    }
  }
}

// ---- Q8_0: unit u = blocks 2u, 2u+1 (68 bytes)
template <int R, int T>
__device__ __forceinline__ void q80_unit(const uint8_t* __restrict__ w, int64_t rb, int row0,
                                         int last_row, int u, const XPlanes (&xp)[T],
                                         float (&acc)[R][T]) {
  uint32_t q[R][2][8];
  float d[R][2];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * 68;
    uint4 a = ld16a4(p), b = ld16a4(p + 16), c = ld16a4(p + 32), e = ld16a4(p + 48);
    uint32_t f = ld4(p + 64);
    uint32_t W[17] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y, c.z, c.w, e.x, e.y, e.z, e.w, f};
    d[r][0] = half_bits_to_float(W[0]);
    d[r][1] = half_bits_to_float(W[8] >> 16);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      q[r][0][i] = align(W[i + 1], W[i], 2);
      q[r][1][i] = W[9 + i];
    }
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
#pragma unroll
    for (int bk = 0; bk < 2; bk++) {
      const int g = 2 * u + bk;
      uint4 x[3][2];
#pragma unroll
      for (int j = 0; j < 3; j++) {
        x[j][0] = xp[t].limb(j, 0, g);
        x[j][1] = xp[t].limb(j, 1, g);
      }
      const float scale = xp[t].meta(g).scale;
#pragma unroll
      for (int r = 0; r < R; r++) {
        int s[3] = {0, 0, 0};
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) s[j] = dot4(q[r][bk][i], comp(x[j][i >> 2], i & 3), s[j]);
        acc[r][t] += d[r][bk] * (scale * limbs_to_float(s[0], s[1] * 256 + s[2]));
      }
    }
  }
}

// ---- Q6_K: unit u = half n of superblock sb (128 values, groups 4u..4u+3)
template <int R, int T>
__device__ __forceinline__ void q6k_unit(const uint8_t* __restrict__ w, int64_t rb, int row0,
                                         int last_row, int u, const XPlanes (&xp)[T],
                                         float (&acc)[R][T]) {
  const int sb = u >> 1, n = u & 1;
  uint32_t ql[R][16], qh[R][8], sc[R][2];
  float d[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    const uint8_t* addr = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)sb * 210;
    const uint32_t s = (uint32_t)((uintptr_t)addr & 3u);
    const uint8_t* base = addr - s;
    const uint8_t* pl = base + 64 * n;
    uint4 a0 = ld16a4(pl), a1 = ld16a4(pl + 16), a2 = ld16a4(pl + 32), a3 = ld16a4(pl + 48);
    uint32_t a4 = ld4(pl + 64);
    uint32_t L[17] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                      a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w, a4};
    const uint8_t* ph = base + 128 + 32 * n;
    uint4 h0 = ld16a4(ph), h1 = ld16a4(ph + 16);
    uint32_t h2 = ld4(ph + 32);
    uint32_t H[9] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w, h2};
    const uint8_t* ps = base + 192 + 8 * n;
    uint32_t S[3] = {ld4(ps), ld4(ps + 4), ld4(ps + 8)};
    uint32_t D = ld4(base + 208);
#pragma unroll
    for (int i = 0; i < 16; i++) ql[r][i] = align(L[i + 1], L[i], s);
#pragma unroll
    for (int i = 0; i < 8; i++) qh[r][i] = align(H[i + 1], H[i], s);
    sc[r][0] = align(S[1], S[0], s);
    sc[r][1] = align(S[2], S[1], s);
    d[r] = half_bits_to_float(align(D, D, s));
  }
#pragma unroll
  for (int t = 0; t < T; t++) {
    float part[R];
#pragma unroll
    for (int r = 0; r < R; r++) part[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int g = 4 * u + k;
      uint4 x[3][2];
#pragma unroll
      for (int j = 0; j < 3; j++) {
        x[j][0] = xp[t].limb(j, 0, g);
        x[j][1] = xp[t].limb(j, 1, g);
      }
      const XMeta m = xp[t].meta(g);
      const int2 l23 = xp[t].lsum23(g);
#pragma unroll
      for (int r = 0; r < R; r++) {
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          int s[3] = {0, 0, 0};
#pragma unroll
          for (int ii = 0; ii < 4; ii++) {
            const int i = 4 * hh + ii;
            const uint32_t A = ql[r][i], B = ql[r][i + 8], Hq = qh[r][i];
            uint32_t qv;
            if (k == 0) qv = (A & 0x0F0F0F0Fu) | ((Hq & 0x03030303u) << 4);
            else if (k == 1) qv = (B & 0x0F0F0F0Fu) | ((Hq & 0x0C0C0C0Cu) << 2);
            else if (k == 2) qv = ((A >> 4) & 0x0F0F0F0Fu) | (Hq & 0x30303030u);
            else qv = ((B >> 4) & 0x0F0F0F0Fu) | ((Hq >> 2) & 0x30303030u);
#pragma unroll
            for (int j = 0; j < 3; j++) s[j] = dot4(qv, comp(x[j][hh], ii), s[j]);
          }
          const int lsum1 = hh ? m.lsum1[1] : m.lsum1[0];
          const int lsum23 = hh ? l23.y : l23.x;
          const float f = limbs_to_float(s[0] - 32 * lsum1, s[1] * 256 + s[2] - 32 * lsum23);
          const int si = hh + 2 * k;  // sc[8n + l/16 + 2k] (quant.mojo:371)
          const float scv = (float)(int8_t)((sc[r][si >> 2] >> (8 * (si & 3))) & 0xFF);
          part[r] += scv * (m.scale * f);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r][t] += d[r] * part[r];
  }
}

template <int KIND, int R, int T>
__device__ __forceinline__ void run_unit(const uint8_t* w, int64_t rb, int row0, int last_row, int u,
                                         const XPlanes (&xp)[T], float (&acc)[R][T]) {
  if constexpr (KIND == MI_Q4_K) q4k_unit<R, T>(w, rb, row0, last_row, u, xp, acc);
  else if constexpr (KIND == MI_Q4_0) q40_unit<R, T>(w, rb, row0, last_row, u, xp, acc);
  else if constexpr (KIND == MI_Q8_0) q80_unit<R, T>(w, rb, row0, last_row, u, xp, acc);
  else q6k_unit<R, T>(w, rb, row0, last_row, u, xp, acc);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }
__device__ __forceinline__ float gelu(float v) {
  const float c = 0.7978845608028654f;
  const float inner = c * (v + 0.044715f * v * v * v);
  const float e = 2.0f / (1.0f + expf(-2.0f * inner));
  return 0.5f * v * (1.0f + (e - 1.0f));
}

// gpu.mojo:1005 write_epilogue
__device__ __forceinline__ void epilogue(float* __restrict__ y, const float* __restrict__ aux, int epi,
                                         int64_t at, int r, float v) {
  if (epi & MI_EPI_BIAS) v += aux[r];
  else if (epi & MI_EPI_GLU) v = ((epi & MI_ACT_GELU) ? gelu(v) : silu(v)) * aux[at];
  if (epi & MI_EPI_ADD) y[at] = y[at] + v;
  else y[at] = v;
}

constexpr int kWavesPerBlock = 4;

template <int KIND, int R, int T>
__global__ __launch_bounds__(256) void matvec_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                     int rows, int cols,
                                                     const uint8_t* __restrict__ xq,
                                                     float* __restrict__ y, int64_t ldy, int epi,
                                                     const float* __restrict__ aux) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWavesPerBlock + wave) * R;
  if (row0 >= rows) return;
  const int G = cols >> 5;
  XPlanes xp[T];
#pragma unroll
  for (int t = 0; t < T; t++) {
    xp[t].xt = xq + (int64_t)t * xq_token_bytes(cols);
    xp[t].plane = (int64_t)G * 16;
  }
  float acc[R][T];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int t = 0; t < T; t++) acc[r][t] = 0.0f;
  const int units = cols / UnitElems<KIND>::v;
  for (int u = lane; u < units; u += kWave) run_unit<KIND, R, T>(w, rb, row0, rows - 1, u, xp, acc);
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int t = 0; t < T; t++) {
      const float v = wave_sum(acc[r][t]);
      if (lane == 0 && row0 + r < rows) epilogue(y, aux, epi, (int64_t)t * ldy + row0 + r, row0 + r, v);
    }
}

template <int KIND, int R, int T>
int launch_rt(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y,
              int64_t ldy, int epi, const float* aux) {
  const int per_block = kWavesPerBlock * R;
  const int blocks = (rows + per_block - 1) / per_block;
  hipLaunchKernelGGL((matvec_kernel<KIND, R, T>), dim3(blocks), dim3(kWavesPerBlock * kWave), 0, s,
                     (const uint8_t*)w, rb, rows, cols, (const uint8_t*)xq, y, ldy, epi, aux);
  return hip_check(hipGetLastError(), "matvec launch");
}

template <int KIND, int T>
int launch_t(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y,
             int64_t ldy, int epi, const float* aux) {
  // Rows per wave: enough waves to fill 256 CUs several times over, and
  // as many rows as that allows so each activation load serves them all.
  if (rows >= 8192) return launch_rt<KIND, 4, T>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  if (rows >= 4096) return launch_rt<KIND, 2, T>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  return launch_rt<KIND, 1, T>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
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

int launch_matvec(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows,
                  int32_t cols, const void* xq, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                  const float* aux) {
  switch (kind) {
    case MI_Q4_K: return launch_kind<MI_Q4_K>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q6_K: return launch_kind<MI_Q6_K>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q4_0: return launch_kind<MI_Q4_0>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
    case MI_Q8_0: return launch_kind<MI_Q8_0>(s, w, row_bytes, rows, cols, xq, tokens, y, ldy, epi, aux);
  }
  return fail(MI_ERR_KIND, "matvec: ggml type %d has no device kernel", kind);
}

}  // namespace mi

// matvec_units.h -- per-kind "unit" code of the GGUF matvec (see matvec.hip):
// the packed bytes one lane reads for one unit of R rows, and the unpack /
// integer dot / block-scale arithmetic on them.
#pragma once

#include "mi_internal.h"
#include "xq_device.h"

namespace mi {
namespace mv {

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

// Each kind is a struct holding one unit's packed bytes for R rows, with
// load() (issue the global loads) separate from compute() (unpack, dot,
// scale), so a kernel can put loads for the next unit in flight before it
// computes the current one.  X is the activation accessor (global memory or
// a copy staged in LDS).

// d * sc and dmin * m of groups 2h and 2h + 1 of a K-quant superblock whose
// first 16 bytes (d, dmin, scales[12]) are hdr (quant.mojo:161 _k_scale):
// the byte shift is 16*(h&1) + 8e for both packings.
__device__ __forceinline__ void kquarter_scales(const uint4& hdr, int h, float (&dsc)[2], float (&dmn)[2]) {
  const uint32_t sh = 16u * (h & 1);
  const bool high = h >= 2;
  const uint32_t hs2 = 2u * (uint32_t)(h >> 1);
  const float d = half_bits_to_float(hdr.x), dmin = half_bits_to_float(hdr.x >> 16);
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const uint32_t s = sh + 8u * e;
    // One formula for both packings: the low four bits come from
    // scales[j] / scales[j+4] (low groups) or scales[j+8] (high groups), the
    // top two from bits 4-5 (low) or 6-7 (high) of scales[j] / scales[j+4].
    // Only a register is selected per lane, never a computation: a
    // lane-divergent branch here makes the compiler hoist this row's scale
    // work (and its wait for this row's loads) above earlier rows' dots.
    const uint32_t sc = __builtin_amdgcn_ubfe(high ? hdr.w : hdr.y, s, 4) |
                        (__builtin_amdgcn_ubfe(hdr.y, s + 4 + hs2, 2) << 4);
    const uint32_t m = __builtin_amdgcn_ubfe(high ? hdr.w : hdr.z, s + 2 * hs2, 4) |
                       (__builtin_amdgcn_ubfe(hdr.z, s + 4 + hs2, 2) << 4);
    dsc[e] = d * (float)sc;
    dmn[e] = dmin * (float)m;
  }
}

// Four fifth bits (bits 0-3 of v) moved to bit 0 of four bytes.
__device__ __forceinline__ uint32_t spread4(uint32_t v) { return (v * 0x00204081u) & 0x01010101u; }

// ---- Q4_K: unit u = quarter h of superblock sb (64 values, groups 2u, 2u+1)
template <int R>
struct Q4KUnit {
  static constexpr int kElems = 64;
  uint4 hdr[R], a[R], b[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
    const int sb = u >> 2, h = u & 3;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* blk = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)sb * 144;
      hdr[r] = ld16(blk);
      a[r] = ld16(blk + 16 + 32 * h);
      b[r] = ld16(blk + 32 + 32 * h);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    const int h = u & 3;
    // six-bit scale/min pair for group j = 2h + e (quant.mojo:161 _k_scale):
    // the byte shift is 16*(h&1) + 8e for both packings.
    float dsc[R][2], dmn[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) kquarter_scales(hdr[r], h, dsc[r], dmn[r]);
    uint32_t lo[R][8], hi[R][8];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t q[8] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        lo[r][i] = q[i] & 0x0F0F0F0Fu;
        hi[r][i] = (q[i] >> 4) & 0x0F0F0F0Fu;
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
          xa[j][hh] = x.limb(t, j, hh, gA);
          xb[j][hh] = x.limb(t, j, hh, gA + 1);
        }
      const XMeta ma = x.meta(t, gA), mb = x.meta(t, gA + 1);
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
        float part = fmaf(dsc[r][0] * ma.scale, va, -dmn[r][0] * ma.xsum);
        part = fmaf(dsc[r][1] * mb.scale, vb, part);
        acc[r][t] += fmaf(-dmn[r][1], mb.xsum, part);
      }
    }
  }
};

// ---- Q4_0: unit u = blocks 2u, 2u+1 (36 bytes, groups 2u, 2u+1)
template <int R>
struct Q40Unit {
  static constexpr int kElems = 64;
  uint4 a[R], b[R];
  uint32_t c[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * 36;
      a[r] = ld16a4(p);
      b[r] = ld16a4(p + 16);
      c[r] = ld4(p + 32);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    uint32_t lo[R][2][4], hi[R][2][4];
    float d[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t W[9] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w, c[r]};
      d[r][0] = half_bits_to_float(W[0]);
      d[r][1] = half_bits_to_float(W[4] >> 16);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t qa = align(W[i + 1], W[i], 2), qb = W[5 + i];
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
          x0[j] = x.limb(t, j, 0, g);
          x1[j] = x.limb(t, j, 1, g);
        }
        const XMeta m = x.meta(t, g);
        const int2 l23 = x.lsum23(t, g);
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
          acc[r][t] = fmaf(d[r][bk] * m.scale, v, acc[r][t]);
        }
      }
    }
  }
};

// ---- Q8_0: unit u = blocks 2u, 2u+1 (68 bytes)
template <int R>
struct Q80Unit {
  static constexpr int kElems = 64;
  uint4 a[R], b[R], c[R], e[R];
  uint32_t f[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * 68;
      a[r] = ld16a4(p);
      b[r] = ld16a4(p + 16);
      c[r] = ld16a4(p + 32);
      e[r] = ld16a4(p + 48);
      f[r] = ld4(p + 64);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    uint32_t q[R][2][8];
    float d[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t W[17] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w,
                              c[r].x, c[r].y, c[r].z, c[r].w, e[r].x, e[r].y, e[r].z, e[r].w, f[r]};
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
        uint4 xv[3][2];
#pragma unroll
        for (int j = 0; j < 3; j++) {
          xv[j][0] = x.limb(t, j, 0, g);
          xv[j][1] = x.limb(t, j, 1, g);
        }
        const float scale = x.meta(t, g).scale;
#pragma unroll
        for (int r = 0; r < R; r++) {
          int s[3] = {0, 0, 0};
#pragma unroll
          for (int i = 0; i < 8; i++)
#pragma unroll
            for (int j = 0; j < 3; j++) s[j] = dot4(q[r][bk][i], comp(xv[j][i >> 2], i & 3), s[j]);
          acc[r][t] = fmaf(d[r][bk] * scale, limbs_to_float(s[0], s[1] * 256 + s[2]), acc[r][t]);
        }
      }
    }
  }
};

// ---- Q6_K: unit u = half n of superblock sb (128 values, groups 4u..4u+3)
template <int R>
struct Q6KUnit {
  static constexpr int kElems = 128;
  uint32_t L[R][17], H[R][9], S[R][3], D[R], sh[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
    const int sb = u >> 1, n = u & 1;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* addr = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)sb * 210;
      sh[r] = (uint32_t)((uintptr_t)addr & 3u);
      const uint8_t* base = addr - sh[r];
      const uint8_t* pl = base + 64 * n;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint4 v = ld16a4(pl + 16 * i);
        L[r][4 * i] = v.x;
        L[r][4 * i + 1] = v.y;
        L[r][4 * i + 2] = v.z;
        L[r][4 * i + 3] = v.w;
      }
      L[r][16] = ld4(pl + 64);
      const uint8_t* ph = base + 128 + 32 * n;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint4 v = ld16a4(ph + 16 * i);
        H[r][4 * i] = v.x;
        H[r][4 * i + 1] = v.y;
        H[r][4 * i + 2] = v.z;
        H[r][4 * i + 3] = v.w;
      }
      H[r][8] = ld4(ph + 32);
      const uint8_t* ps = base + 192 + 8 * n;
      S[r][0] = ld4(ps);
      S[r][1] = ld4(ps + 4);
      S[r][2] = ld4(ps + 8);
      D[r] = ld4(base + 208);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    uint32_t ql[R][16], qh[R][8], sc[R][2];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
      for (int i = 0; i < 16; i++) ql[r][i] = align(L[r][i + 1], L[r][i], sh[r]);
#pragma unroll
      for (int i = 0; i < 8; i++) qh[r][i] = align(H[r][i + 1], H[r][i], sh[r]);
      sc[r][0] = align(S[r][1], S[r][0], sh[r]);
      sc[r][1] = align(S[r][2], S[r][1], sh[r]);
      d[r] = half_bits_to_float(align(D[r], D[r], sh[r]));
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
      float part[R];
#pragma unroll
      for (int r = 0; r < R; r++) part[r] = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int g = 4 * u + k;
        uint4 xv[3][2];
#pragma unroll
        for (int j = 0; j < 3; j++) {
          xv[j][0] = x.limb(t, j, 0, g);
          xv[j][1] = x.limb(t, j, 1, g);
        }
        const XMeta m = x.meta(t, g);
        const int2 l23 = x.lsum23(t, g);
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
              for (int j = 0; j < 3; j++) s[j] = dot4(qv, comp(xv[j][hh], ii), s[j]);
            }
            const int lsum1 = hh ? m.lsum1[1] : m.lsum1[0];
            const int lsum23 = hh ? l23.y : l23.x;
            const float f = limbs_to_float(s[0] - 32 * lsum1, s[1] * 256 + s[2] - 32 * lsum23);
            const int si = hh + 2 * k;  // sc[8n + l/16 + 2k] (quant.mojo:371)
            const float scv = (float)(int8_t)((sc[r][si >> 2] >> (8 * (si & 3))) & 0xFF);
            part[r] = fmaf(scv * m.scale, f, part[r]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < R; r++) acc[r][t] = fmaf(d[r], part[r], acc[r][t]);
    }
  }
};

// ---- Q4_1: unit u = blocks 2u, 2u+1 (40 bytes); value = q * d + m
template <int R>
struct Q41Unit {
  static constexpr int kElems = 64;
  uint4 a[R], b[R];
  uint32_t c[R], e[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * 40;
      a[r] = ld16a4(p);
      b[r] = ld16a4(p + 16);
      c[r] = ld4(p + 32);
      e[r] = ld4(p + 36);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    uint32_t lo[R][2][4], hi[R][2][4];
    float d[R][2], m[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t W[10] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w, c[r], e[r]};
#pragma unroll
      for (int bk = 0; bk < 2; bk++) {
        d[r][bk] = half_bits_to_float(W[5 * bk]);
        m[r][bk] = half_bits_to_float(W[5 * bk] >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t q = W[5 * bk + 1 + i];
          lo[r][bk][i] = q & 0x0F0F0F0Fu;
          hi[r][bk][i] = (q >> 4) & 0x0F0F0F0Fu;
        }
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
          x0[j] = x.limb(t, j, 0, g);
          x1[j] = x.limb(t, j, 1, g);
        }
        const XMeta mt = x.meta(t, g);
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
          const float v = limbs_to_float(s[0], s[1] * 256 + s[2]);
          acc[r][t] = fmaf(d[r][bk] * mt.scale, v, fmaf(m[r][bk], mt.xsum, acc[r][t]));
        }
      }
    }
  }
};

// ---- Q5_0 / Q5_1: unit u = blocks 2u, 2u+1 (44 / 48 bytes); the fifth bit
// of value l is bit l of the block's 32-bit qh.  Q5_0: (q - 16) * d, through
// the per-half limb sums; Q5_1: q * d + m.
template <int R, bool ONE>
struct Q5xUnit {
  static constexpr int kElems = 64;
  static constexpr int kBytes = ONE ? 48 : 44;
  static constexpr int kTail = (kBytes - 32) / 4;  // dwords after the first 32 bytes
  uint4 a[R], b[R];
  uint32_t c[R][kTail];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* p = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)u * kBytes;
      a[r] = ld16a4(p);
      b[r] = ld16a4(p + 16);
#pragma unroll
      for (int k = 0; k < kTail; k++) c[r][k] = ld4(p + 32 + 4 * k);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    uint32_t lo[R][2][4], hi[R][2][4];
    float d[R][2], m[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint32_t W[8 + kTail] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w};
#pragma unroll
      for (int k = 0; k < kTail; k++) W[8 + k] = c[r][k];
#pragma unroll
      for (int bk = 0; bk < 2; bk++) {
        uint32_t qh, qs[4];
        if constexpr (ONE) {  // d, m, qh, qs[16]: 24 bytes, dword aligned
          d[r][bk] = half_bits_to_float(W[6 * bk]);
          m[r][bk] = half_bits_to_float(W[6 * bk] >> 16);
          qh = W[6 * bk + 1];
#pragma unroll
          for (int i = 0; i < 4; i++) qs[i] = W[6 * bk + 2 + i];
        } else if (bk == 0) {  // d, qh, qs[16]: 22 bytes from byte 0
          d[r][0] = half_bits_to_float(W[0]);
          qh = align(W[1], W[0], 2);
#pragma unroll
          for (int i = 0; i < 4; i++) qs[i] = align(W[2 + i], W[1 + i], 2);
        } else {  // from byte 22
          d[r][1] = half_bits_to_float(W[5] >> 16);
          qh = W[6];
#pragma unroll
          for (int i = 0; i < 4; i++) qs[i] = W[7 + i];
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
          lo[r][bk][i] = (qs[i] & 0x0F0F0F0Fu) | (spread4((qh >> (4 * i)) & 0xFu) << 4);
          hi[r][bk][i] = ((qs[i] >> 4) & 0x0F0F0F0Fu) | (spread4((qh >> (16 + 4 * i)) & 0xFu) << 4);
        }
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
          x0[j] = x.limb(t, j, 0, g);
          x1[j] = x.limb(t, j, 1, g);
        }
        const XMeta mt = x.meta(t, g);
        int c1 = 0, c23 = 0;
        if constexpr (!ONE) {
          const int2 l23 = x.lsum23(t, g);
          c1 = 16 * (mt.lsum1[0] + mt.lsum1[1]);
          c23 = 16 * (l23.x + l23.y);
        }
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
          if constexpr (ONE) acc[r][t] = fmaf(d[r][bk] * mt.scale, v, fmaf(m[r][bk], mt.xsum, acc[r][t]));
          else acc[r][t] = fmaf(d[r][bk] * mt.scale, v, acc[r][t]);
        }
      }
    }
  }
};

// ---- Q5_K: unit u = quarter h of superblock sb (64 values, groups 2u,
// 2u+1); Q4_K's nibbles and scales plus a fifth bit per value: bit 2h of qh
// byte l for value 64h + l, bit 2h + 1 for value 64h + 32 + l.
template <int R>
struct Q5KUnit {
  static constexpr int kElems = 64;
  uint4 hdr[R], h0[R], h1[R], a[R], b[R];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int64_t rb, int row0, int last_row,
                                       int u) {
    const int sb = u >> 2, h = u & 3;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint8_t* blk = w + (int64_t)min(row0 + r, last_row) * rb + (int64_t)sb * 176;
      hdr[r] = ld16a4(blk);
      h0[r] = ld16a4(blk + 16);
      h1[r] = ld16a4(blk + 32);
      a[r] = ld16a4(blk + 48 + 32 * h);
      b[r] = ld16a4(blk + 64 + 32 * h);
    }
  }
  template <int T, class X>
  __device__ __forceinline__ void compute(const X& x, int u, float (&acc)[R][T]) const {
    const int h = u & 3;
    float dsc[R][2], dmn[R][2];
#pragma unroll
    for (int r = 0; r < R; r++) kquarter_scales(hdr[r], h, dsc[r], dmn[r]);
    uint32_t lo[R][8], hi[R][8];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const uint32_t q[8] = {a[r].x, a[r].y, a[r].z, a[r].w, b[r].x, b[r].y, b[r].z, b[r].w};
      const uint32_t H[8] = {h0[r].x, h0[r].y, h0[r].z, h0[r].w, h1[r].x, h1[r].y, h1[r].z, h1[r].w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        lo[r][i] = (q[i] & 0x0F0F0F0Fu) | (((H[i] >> (2 * h)) & 0x01010101u) << 4);
        hi[r][i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((H[i] >> (2 * h + 1)) & 0x01010101u) << 4);
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
          xa[j][hh] = x.limb(t, j, hh, gA);
          xb[j][hh] = x.limb(t, j, hh, gA + 1);
        }
      const XMeta ma = x.meta(t, gA), mb = x.meta(t, gA + 1);
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
        float part = fmaf(dsc[r][0] * ma.scale, va, -dmn[r][0] * ma.xsum);
        part = fmaf(dsc[r][1] * mb.scale, vb, part);
        acc[r][t] += fmaf(-dmn[r][1], mb.xsum, part);
      }
    }
  }
};

template <int KIND, int R>
struct UnitOf;
template <int R> struct UnitOf<MI_Q4_K, R> { using type = Q4KUnit<R>; };
template <int R> struct UnitOf<MI_Q4_0, R> { using type = Q40Unit<R>; };
template <int R> struct UnitOf<MI_Q8_0, R> { using type = Q80Unit<R>; };
template <int R> struct UnitOf<MI_Q6_K, R> { using type = Q6KUnit<R>; };
template <int R> struct UnitOf<MI_Q4_1, R> { using type = Q41Unit<R>; };
template <int R> struct UnitOf<MI_Q5_0, R> { using type = Q5xUnit<R, false>; };
template <int R> struct UnitOf<MI_Q5_1, R> { using type = Q5xUnit<R, true>; };
template <int R> struct UnitOf<MI_Q5_K, R> { using type = Q5KUnit<R>; };

// Activation accessor over the xq layout (mi_internal.h), in global memory
// or in an LDS copy: the same byte layout either way.
struct XAcc {
  const uint8_t* base;
  int64_t tok;    // bytes per token = 4 * cols
  int64_t plane;  // bytes per plane = G * 16
  __device__ __forceinline__ uint4 limb(int t, int j, int hh, int g) const {
    return *(const uint4*)(base + t * tok + (int64_t)(j * 2 + hh) * plane + (int64_t)g * 16);
  }
  __device__ __forceinline__ XMeta meta(int t, int g) const {
    return *(const XMeta*)(base + t * tok + 6 * plane + (int64_t)g * 16);
  }
  __device__ __forceinline__ int2 lsum23(int t, int g) const {
    return *(const int2*)(base + t * tok + 7 * plane + (int64_t)g * 16);
  }
};
struct XLds {
  const uint8_t* base;  // points into __shared__ memory
  int tok, plane;
  __device__ __forceinline__ uint4 limb(int t, int j, int hh, int g) const {
    return *(const uint4*)(base + t * tok + (j * 2 + hh) * plane + g * 16);
  }
  __device__ __forceinline__ XMeta meta(int t, int g) const {
    return *(const XMeta*)(base + t * tok + 6 * plane + g * 16);
  }
  __device__ __forceinline__ int2 lsum23(int t, int g) const {
    return *(const int2*)(base + t * tok + 7 * plane + g * 16);
  }
};

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

// The same epilogue with its one memory operand (y for ADD, aux for BIAS or
// GLU) loaded ahead by the caller (pre = aux[at] or y[at]), so the store does
// not wait for a load issued behind the weights.
__device__ __forceinline__ void epilogue_with(float* __restrict__ y, int epi, int64_t at, float pre, float v) {
  if (epi & MI_EPI_BIAS) v += pre;
  else if (epi & MI_EPI_GLU) v = ((epi & MI_ACT_GELU) ? gelu(v) : silu(v)) * pre;
  if (epi & MI_EPI_ADD) y[at] = (epi & (MI_EPI_BIAS | MI_EPI_GLU)) ? y[at] + v : pre + v;
  else y[at] = v;
}

}  // namespace mv
}  // namespace mi

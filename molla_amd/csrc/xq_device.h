// xq_device.h -- device side of the activation format described in
// mi_internal.h: the group quantizer (called by the quantize, rms_norm and
// attention-merge kernels so the producer of an activation writes it in the
// form the next matvec reads) and the plane accessors the matvecs use.
#pragma once

#include "mi_internal.h"

namespace mi {

// All 32 lanes of one half-wave call this together, lane32 = value index in
// the group.  `live` is false for padding lanes, which still take part in the
// shuffles but write nothing.  xtok points at the token's 4*cols bytes.
__device__ __forceinline__ void quantize_group32(float v, int lane32, int g, int G,
                                                 uint8_t* __restrict__ xtok, bool live) {
  float a = fabsf(v);
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) a = fmaxf(a, __shfl_xor(a, m));
  int E;
  (void)frexpf(a, &E);                // a = f * 2^E, f in [0.5, 1)
  const int e = (a > 0.0f) ? E - 22 : 0;  // a * 2^-e in [2^21, 2^22)
  const int X = (int)rintf(ldexpf(v, -e));  // exact scaling, one rounding
  const int L3 = (int)(int8_t)(X & 0xFF);
  const int X1 = (X - L3) >> 8;
  const int L2 = (int)(int8_t)(X1 & 0xFF);
  const int L1 = (X1 - L2) >> 8;
  int s1 = L1, s23 = L2 * 256 + L3, sx = X;
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) {
    s1 += __shfl_xor(s1, m);
    s23 += __shfl_xor(s23, m);
  }
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) sx += __shfl_xor(sx, m);
  const int other1 = __shfl_xor(s1, 16);
  const int other23 = __shfl_xor(s23, 16);
  // Gather each limb's bytes four lanes to a dword: byte stores from every
  // lane cost the memory system far more than a quarter as many dword stores.
  uint32_t w[3] = {(uint32_t)L1 & 0xFFu, (uint32_t)L2 & 0xFFu, (uint32_t)L3 & 0xFFu};
#pragma unroll
  for (int j = 0; j < 3; j++) {
    w[j] |= (uint32_t)__shfl_down((int)w[j], 1, 4) << 8;
    w[j] |= (uint32_t)__shfl_down((int)w[j], 2, 4) << 16;
  }
  if (!live) return;
  const int hh = lane32 >> 4, b = lane32 & 15;
  const int64_t plane = (int64_t)G * 16;
  if ((b & 3) == 0) {
    uint8_t* e0 = xtok + (int64_t)g * 16 + b;
    *(uint32_t*)(e0 + (0 * 2 + hh) * plane) = w[0];
    *(uint32_t*)(e0 + (1 * 2 + hh) * plane) = w[1];
    *(uint32_t*)(e0 + (2 * 2 + hh) * plane) = w[2];
  }
  if (lane32 == 0) {
    const float scale = ldexpf(1.0f, e);
    XMeta mt;
    mt.scale = scale;
    mt.xsum = scale * (float)sx;
    mt.lsum1[0] = s1;
    mt.lsum1[1] = other1;
    *(XMeta*)(xtok + 6 * plane + (int64_t)g * 16) = mt;
    int4 l23 = make_int4(s23, other23, 0, 0);
    *(int4*)(xtok + 7 * plane + (int64_t)g * 16) = l23;
  }
}

// Plane accessors.  `xt` = token base, G = groups per token.
struct XPlanes {
  const uint8_t* __restrict__ xt;
  int64_t plane;  // G * 16
  __device__ __forceinline__ uint4 limb(int j, int hh, int g) const {
    return *(const uint4*)(xt + (int64_t)(j * 2 + hh) * plane + (int64_t)g * 16);
  }
  __device__ __forceinline__ XMeta meta(int g) const {
    return *(const XMeta*)(xt + 6 * plane + (int64_t)g * 16);
  }
  __device__ __forceinline__ int2 lsum23(int g) const {
    return *(const int2*)(xt + 7 * plane + (int64_t)g * 16);
  }
};

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// S1*65536 + (S2*256 + S3), the three limb sums recombined (exact ints in,
// one float rounding out).
__device__ __forceinline__ float limbs_to_float(int s1, int s23) {
  return fmaf((float)s1, 65536.0f, (float)s23);
}

}  // namespace mi

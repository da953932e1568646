// xq_device.h -- device side of the activation format described in
// mi_internal.h: the group quantizer (called by the quantize, rms_norm and
// attention-merge kernels so the producer of an activation writes it in the
// form the next matvec reads) and the plane accessors the matvecs use.
#pragma once

#include "mi_internal.h"

namespace mi {

// The "hx" form of a token (read by the f16 matrix-core tile,
// matvec_htile.hip), 4 cols bytes like the xq form: group g at g * 128 is
// [kq 0..3][hi, lo][8 halves], value 8 kq + u of the group being X * 2^-8 =
// hi + lo exactly (hi = f16(X / 256), lo = f16(X / 256 - hi)), X the group's
// xq integer.  The group's scale stays in the xq form's plane 6.
__device__ __forceinline__ void hx_group32(int X, int lane32, int g, uint8_t* __restrict__ hxtok, bool live) {
  const float xs = (float)X * (1.0f / 256.0f);  // exact: |X| < 2^22
  const _Float16 hi = (_Float16)xs;
  const _Float16 lo = (_Float16)(xs - (float)hi);
  const uint32_t pair = (uint32_t)__builtin_bit_cast(uint16_t, hi) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
  // lanes 2j and 2j + 1: (hi, hi') and (lo, lo') as two dwords
  const uint32_t other = lanes::dpp<lanes::kDown1>(pair);
  if (!live || (lane32 & 1)) return;
  const int kq = lane32 >> 3, u = lane32 & 7;
  uint8_t* e = hxtok + (int64_t)g * 128 + kq * 32 + u * 2;
  *(uint32_t*)e = (pair & 0xFFFFu) | (other << 16);
  *(uint32_t*)(e + 16) = (pair >> 16) | (other & 0xFFFF0000u);
}

// All 32 lanes of one half-wave call this together, lane32 = value index in
// the group.  `live` is false for padding lanes, which still take part in the
// shuffles but write nothing.  xtok points at the token's 4*cols bytes; hxtok,
// when not null, at the token's hx form (hx_group32).
__device__ __forceinline__ void quantize_group32(float v, int lane32, int g, int G,
                                                 uint8_t* __restrict__ xtok, bool live,
                                                 uint8_t* __restrict__ hxtok = nullptr) {
  const float a = lanes::reduce<32>(fabsf(v), lanes::Max{});
  int E;
  (void)frexpf(a, &E);                // a = f * 2^E, f in [0.5, 1)
  const int e = (a > 0.0f) ? E - 22 : 0;  // a * 2^-e in [2^21, 2^22)
  const int X = (int)rintf(ldexpf(v, -e));  // exact scaling, one rounding
  const int L3 = (int)(int8_t)(X & 0xFF);
  const int X1 = (X - L3) >> 8;
  const int L2 = (int)(int8_t)(X1 & 0xFF);
  const int L1 = (X1 - L2) >> 8;
  // this half's limb sums (16 values) and the other half's: the group's
  // sum less this half's (exact integers)
  const int s1 = lanes::reduce<16>(L1, lanes::Add{}), s23 = lanes::reduce<16>(L2 * 256 + L3, lanes::Add{});
  const int other1 = lanes::reduce<32>(L1, lanes::Add{}) - s1;
  const int other23 = lanes::reduce<32>(L2 * 256 + L3, lanes::Add{}) - s23;
  const int sx = lanes::reduce<32>(X, lanes::Add{});
  if (hxtok) hx_group32(X, lane32, g, hxtok, live);
  // Gather each limb's bytes four lanes to a dword: byte stores from every
  // lane cost the memory system far more than a quarter as many dword stores.
  uint32_t w[3] = {(uint32_t)L1 & 0xFFu, (uint32_t)L2 & 0xFFu, (uint32_t)L3 & 0xFFu};
#pragma unroll
  for (int j = 0; j < 3; j++) {
    w[j] |= lanes::dpp<lanes::kDown1>(w[j]) << 8;
    w[j] |= lanes::dpp<lanes::kDown2>(w[j]) << 16;
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

// RMSNorm of one row folded into a matvec block, in two steps: a thread
// first issues the loads of its 8 values of the row x and of the norm's gain
// (norm_row_load; n <= 8 NT values, n a multiple of 32, both pointers
// 16-byte aligned), the caller then issues its own weight loads, and only
// then does norm_row_to_lds wait for the row.  Vector-memory loads of a wave
// complete in issue order, so the row's loads must go out first.
//
// norm_row_to_lds: the NT threads take rms_norm_kernel's scale (float64 sum
// of squares, scale = f32(1/sqrt(sum/n + eps))) and write the row in matvec
// form into the LDS `xs` (4 n bytes, the planes of an xq token): x * scale *
// gain, byte for byte what quantize_group32 writes for it, or (DEFER, below)
// x * gain with the scale left to the caller.  Thread t holds values
// 8t..8t+7, so a 32-value group is 4 lanes and its reductions are two
// shuffles.  Every block sums in the same order, so every block derives the
// same scale.  `red` is NT / 64 doubles of LDS; the step ends with a
// barrier.
struct NormRow {
  float4 x0, x1, g0, g1;
};

__device__ __forceinline__ NormRow norm_row_load(const float* __restrict__ x, const float* __restrict__ gain,
                                                 int n) {
  const int at = min((int)threadIdx.x * 8, n - 8);
  NormRow r;
  r.x0 = *(const float4*)(x + at);
  r.x1 = *(const float4*)(x + at + 4);
  r.g0 = *(const float4*)(gain + at);
  r.g1 = *(const float4*)(gain + at + 4);
  return r;
}

// Thread t's 8 consecutive values v (of a row of n, n a multiple of 32)
// in matvec form into the LDS `xs` (4 n bytes, the planes of an xq token),
// byte for byte what quantize_group32 writes for them: a 32-value group is
// 4 lanes, so its reductions are two shuffles.  Every lane of the wave takes
// part; only `live` ones write.  No barrier.
__device__ __forceinline__ void quantize8_to_lds(const float (&v)[8], bool live, int t, int n, uint8_t* xs) {
#pragma clang fp contract(off)
  const int i0 = t * 8;
  float a = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; k++) a = fmaxf(a, fabsf(v[k]));
  a = lanes::reduce<4>(a, lanes::Max{});
  int E;
  (void)frexpf(a, &E);
  const int e = (a > 0.0f) ? E - 22 : 0;
  uint32_t w[3][2] = {{0, 0}, {0, 0}, {0, 0}};
  int s1 = 0, s23 = 0, sx = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int X = (int)rintf(ldexpf(v[k], -e));
    const int L3 = (int)(int8_t)(X & 0xFF);
    const int X1 = (X - L3) >> 8;
    const int L2 = (int)(int8_t)(X1 & 0xFF);
    const int L1 = (X1 - L2) >> 8;
    s1 += L1;
    s23 += L2 * 256 + L3;
    sx += X;
    const int sh = (k & 3) * 8;
    w[0][k >> 2] |= ((uint32_t)L1 & 0xFFu) << sh;
    w[1][k >> 2] |= ((uint32_t)L2 & 0xFFu) << sh;
    w[2][k >> 2] |= ((uint32_t)L3 & 0xFFu) << sh;
  }
  // lanes 4q, 4q+1 hold half 0 of group q, lanes 4q+2, 4q+3 half 1
  const int h1 = lanes::reduce<2>(s1, lanes::Add{}), h23 = lanes::reduce<2>(s23, lanes::Add{});
  const int other1 = lanes::reduce<4>(s1, lanes::Add{}) - h1;
  const int other23 = lanes::reduce<4>(s23, lanes::Add{}) - h23;
  s1 = h1;
  s23 = h23;
  sx = lanes::reduce<4>(sx, lanes::Add{});
  if (live) {
    const int grp = i0 >> 5, k4 = t & 3, hh = k4 >> 1;
    const int plane = (n >> 5) * 16;
    uint8_t* e0 = xs + grp * 16 + (k4 & 1) * 8;
#pragma unroll
    for (int j = 0; j < 3; j++) *(uint2*)(e0 + (j * 2 + hh) * plane) = make_uint2(w[j][0], w[j][1]);
    if (k4 == 0) {
      const float sc = ldexpf(1.0f, e);
      XMeta mt;
      mt.scale = sc;
      mt.xsum = sc * (float)sx;
      mt.lsum1[0] = s1;
      mt.lsum1[1] = other1;
      *(XMeta*)(xs + 6 * plane + grp * 16) = mt;
      *(int4*)(xs + 7 * plane + grp * 16) = make_int4(s23, other23, 0, 0);
    }
  }
}

//
// DEFER: the row goes into LDS as x * gain, without the norm's scale, and
// the scale is returned for the caller to apply to each matvec result
// (W (s x g) = s (W (x g)); the matvec form's per-group power-of-two scale
// gives x g the same relative precision as s x g).  The sum of squares then
// runs beside the quantize instead of ahead of it, and the step has one
// barrier.  Without DEFER the scale is applied first, as rms_norm_kernel
// does, and 1 is returned.
template <int NT, bool DEFER = false>
__device__ __forceinline__ float norm_row_to_lds(const NormRow& nr, int n, float eps, uint8_t* xs, double* red) {
#pragma clang fp contract(off)
  const int t = threadIdx.x;
  const int i0 = t * 8;
  const bool live = i0 < n;
  const float4 x0 = nr.x0, x1 = nr.x1, g0 = nr.g0, g1 = nr.g1;
  float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  const float g[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < 8; k++) acc += live ? (double)v[k] * (double)v[k] : 0.0;
  acc = lanes::reduce_sum<64>(acc);
  if ((t & 63) == 0) red[t >> 6] = acc;
  if constexpr (DEFER) {
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = v[k] * g[k];
    quantize8_to_lds(v, live, t, n, xs);
  }
  __syncthreads();
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < NT / 64; i++) sum += red[i];
  const float scale = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
  if constexpr (DEFER) return scale;
#pragma unroll
  for (int k = 0; k < 8; k++) v[k] = v[k] * scale * g[k];
  quantize8_to_lds(v, live, t, n, xs);
  __syncthreads();
  return 1.0f;
}

// rope.mojo:253 angle with scale 1 and no YaRN mix: f32(pos) * step / freq,
// freq being the pair's rope_freqs.weight factor (none: 1, no division).
// Shared by the norm, rope and fused q|k|v kernels.
__device__ __forceinline__ float rope_theta(int pos, const float* __restrict__ steps,
                                            const float* __restrict__ factors, int pair) {
#pragma clang fp contract(off)
  const float theta = (float)pos * steps[pair];
  return factors ? theta / factors[pair] : theta;
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

// quant.hip -- bit-exact GGUF dequant and the activation quantizer.
//
// Dequant follows src/molla/nn/quant.mojo:184-409 operation for operation
// (Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K, Q6_K):
// every product is rounded on its own (no fused multiply-add), so the output
// is bit-identical to the host decoder.  That is enforced with
// `#pragma clang fp contract(off)` on the functions that compute values.
#include <math.h>

#include "mi_internal.h"
#include "xq_device.h"

namespace mi {
namespace {

__device__ __forceinline__ float f16_at(const uint8_t* p) {
  return half_bits_to_float((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}

// quant.mojo:161 _k_scale
__device__ __forceinline__ void k_scale(const uint8_t* s, int j, int& sc, int& m) {
  if (j < 4) {
    sc = s[j] & 63;
    m = s[j + 4] & 63;
  } else {
    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

// One thread decodes one 32-value group.  `gi` indexes groups of the run.
__global__ void dequant_kernel(int kind, const uint8_t* __restrict__ w, int64_t groups,
                               float* __restrict__ out) {
#pragma clang fp contract(off)
  int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gi >= groups) return;
  float v[32];
  if (kind == MI_Q8_0) {  // quant.mojo:304 _q8_0
    const uint8_t* b = w + gi * 34;
    float d = f16_at(b);
#pragma unroll
    for (int l = 0; l < 32; l++) v[l] = (float)(int8_t)b[2 + l] * d;
  } else if (kind == MI_Q4_0) {  // quant.mojo:232 _q4_0
    const uint8_t* b = w + gi * 18;
    float d = f16_at(b);
#pragma unroll
    for (int l = 0; l < 16; l++) {
      int q = b[2 + l];
      v[l] = (float)((q & 0xF) - 8) * d;
      v[l + 16] = (float)((q >> 4) - 8) * d;
    }
  } else if (kind == MI_Q4_1) {  // quant.mojo:247 _q4_1
    const uint8_t* b = w + gi * 20;
    float d = f16_at(b), m = f16_at(b + 2);
#pragma unroll
    for (int l = 0; l < 16; l++) {
      int q = b[4 + l];
      v[l] = (float)(q & 0xF) * d + m;
      v[l + 16] = (float)(q >> 4) * d + m;
    }
  } else if (kind == MI_Q5_0 || kind == MI_Q5_1) {  // quant.mojo:272 _q5_0, :290 _q5_1
    const bool one = kind == MI_Q5_1;
    const uint8_t* b = w + gi * (one ? 24 : 22);
    float d = f16_at(b), m = one ? f16_at(b + 2) : 0.0f;
    const uint8_t* h = b + (one ? 4 : 2);
    const uint32_t qh = (uint32_t)h[0] | ((uint32_t)h[1] << 8) | ((uint32_t)h[2] << 16) | ((uint32_t)h[3] << 24);
    const uint8_t* qs = h + 4;
#pragma unroll
    for (int l = 0; l < 16; l++) {
      int q = qs[l];
      int lo = (q & 0xF) | (int)(((qh >> l) << 4) & 0x10);
      int hi = (q >> 4) | (int)((qh >> (l + 12)) & 0x10);
      if (one) {
        v[l] = (float)lo * d + m;
        v[l + 16] = (float)hi * d + m;
      } else {
        v[l] = (float)(lo - 16) * d;
        v[l + 16] = (float)(hi - 16) * d;
      }
    }
  } else if (kind == MI_Q5_K) {  // quant.mojo:331 _q5_k
    const uint8_t* b = w + (gi >> 3) * 176;
    int j = (int)(gi & 7), half = j >> 1;
    float d = f16_at(b), dmin = f16_at(b + 2);
    int sc, m;
    k_scale(b + 4, j, sc, m);
    float d1 = d * (float)sc;
    float m1 = dmin * (float)m;
    const uint8_t* qh = b + 16;
    const uint8_t* q = b + 48 + half * 32;
    int shift = (j & 1) * 4, bit = 2 * half + (j & 1);
#pragma unroll
    for (int l = 0; l < 32; l++) v[l] = d1 * (float)(((q[l] >> shift) & 0xF) + (((qh[l] >> bit) & 1) << 4)) - m1;
  } else if (kind == MI_Q4_K) {  // quant.mojo:310 _q4_k
    const uint8_t* b = w + (gi >> 3) * 144;
    int j = (int)(gi & 7), half = j >> 1;
    float d = f16_at(b), dmin = f16_at(b + 2);
    int sc, m;
    k_scale(b + 4, j, sc, m);
    float d1 = d * (float)sc;
    float m1 = dmin * (float)m;
    const uint8_t* q = b + 16 + half * 32;
    int shift = (j & 1) * 4;
#pragma unroll
    for (int l = 0; l < 32; l++) v[l] = d1 * (float)((q[l] >> shift) & 0xF) - m1;
  } else {  // MI_Q6_K, quant.mojo:371 _q6_k; group j = (half n, quarter k)
    const uint8_t* b = w + (gi >> 3) * 210;
    int j = (int)(gi & 7), n = j >> 2, k = j & 3;
    float d = f16_at(b + 208);
    const uint8_t* lo = b + n * 64;
    const uint8_t* hi = b + 128 + n * 32;
    const int8_t* sc = (const int8_t*)(b + 192 + n * 8);
#pragma unroll
    for (int l = 0; l < 32; l++) {
      int h = hi[l];
      int low4 = (k & 1) ? lo[l + 32] : lo[l];
      low4 = (k & 2) ? (low4 >> 4) : (low4 & 0xF);
      int q = (low4 | (((h >> (2 * k)) & 3) << 4)) - 32;
      v[l] = d * (float)sc[(l >> 4) + 2 * k] * (float)q;
    }
  }
  float4* o = (float4*)(out + gi * 32);
#pragma unroll
  for (int i = 0; i < 8; i++) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

// Quantize x (tokens rows of cols floats) into the xq layout.  Each 32-lane
// half of a wave owns one group.
__global__ void quantize_kernel(const float* __restrict__ x, int32_t cols, int32_t tokens,
                                uint8_t* __restrict__ xq, uint8_t* __restrict__ hx) {
  const int G = cols >> 5;
  const int64_t gg = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // global group
  const int lane32 = threadIdx.x & 31;
  const bool live = gg < (int64_t)G * tokens;
  const int64_t t = live ? gg / G : 0;
  const int g = live ? (int)(gg - t * G) : 0;
  float v = live ? x[t * cols + (int64_t)g * 32 + lane32] : 0.0f;
  quantize_group32(v, lane32, g, G, xq + t * xq_token_bytes(cols), live,
                   hx ? hx + t * xq_token_bytes(cols) : nullptr);
}

}  // namespace

int launch_dequant(hipStream_t s, int kind, const void* w, int64_t count, float* out) {
  int64_t groups = count / 32;
  if (groups == 0) return MI_OK;
  int threads = 128;
  int64_t blocks = (groups + threads - 1) / threads;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, kind,
                     (const uint8_t*)w, groups, out);
  return hip_check(hipGetLastError(), "dequant launch");
}

int launch_quantize(hipStream_t s, const float* x, int32_t cols, int32_t tokens, void* xq, void* hx) {
  int64_t lanes = (int64_t)(cols / 32) * tokens * 32;
  int threads = 256;
  int64_t blocks = (lanes + threads - 1) / threads;
  hipLaunchKernelGGL(quantize_kernel, dim3((unsigned)blocks), dim3(threads), 0, s, x, cols, tokens,
                     (uint8_t*)xq, (uint8_t*)hx);
  return hip_check(hipGetLastError(), "quantize launch");
}

}  // namespace mi

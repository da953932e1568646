/*
 * molla_oracle.c -- CPU restatement of molla's host decode path.
 *
 * TEST INFRASTRUCTURE ONLY (see molla_oracle.h).  It is the checker for the
 * HIP kernels and the CPU baseline that bench.py times; the product path never
 * loads it.
 *
 * Built with -O2 -ffp-contract=off -fno-fast-math: every expression below is
 * evaluated in the order the cited Mojo source writes it, left to right, with
 * each float32 product and sum rounded separately.  Where the Mojo source
 * widens to float64 (rms_norm's sum of squares, rope's trig, the step table)
 * this does the same.
 */
#include "molla_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* quant.mojo:78 block_elements */
int or_block_elements(int kind) {
  switch (kind) {
    case OR_F32: case OR_F16: case OR_BF16: return 1;
    case OR_Q4_0: case OR_Q4_1: case OR_Q8_0: case OR_Q5_0: case OR_Q5_1: return 32;
    case OR_Q4_K: case OR_Q5_K: case OR_Q6_K: return 256;
    default: return 0;
  }
}

/* quant.mojo:97 block_bytes */
int or_block_bytes(int kind) {
  switch (kind) {
    case OR_F32: return 4;
    case OR_F16: case OR_BF16: return 2;
    case OR_Q4_0: return 18;
    case OR_Q4_1: return 20;
    case OR_Q5_0: return 22;
    case OR_Q5_1: return 24;
    case OR_Q8_0: return 34;
    case OR_Q4_K: return 144;
    case OR_Q5_K: return 176;
    case OR_Q6_K: return 210;
    default: return 0;
  }
}

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* quant.mojo:135 f16_at: IEEE binary16 widened to binary32 (exact). */
float or_f16(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0) {
    if (man == 0) return u2f(sign);
    /* subnormal: value = man * 2^-24, exact in float32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return u2f(sign | 0x7F800000u | (man << 13));
  return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* float32 -> float16, round to nearest even: what a device half store does
 * (gpu_ops.mojo:1491 store_kv_kernel narrows with a plain cast). */
uint16_t or_f32_to_f16(float v) {
  uint32_t x = f2u(v);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds past 65504 */
  if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal half */
    if (ax < 0x33000000u) return (uint16_t)sign;             /* below 2^-25 rounds to zero */
    uint32_t e = ax >> 23;
    uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - e;                               /* 14 - (e - 127) + 13 */
    uint32_t half = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t mid = 1u << (shift - 1u);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((ax >> 13) - (112u << 10));
  uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return (uint16_t)(sign | half);
}

static inline float bf16_at(const uint8_t* p) {
  uint32_t bits = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
  return u2f(bits << 16);
}
static inline float f16_at(const uint8_t* p) {
  return or_f16((uint16_t)(p[0] | (p[1] << 8)));
}
static inline float f32_at(const uint8_t* p) {
  uint32_t b = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
  return u2f(b);
}
static inline int i8_at(const uint8_t* p) { return (int)(int8_t)p[0]; }

/* quant.mojo:161 _k_scale (ggml get_scale_min_k4) */
static inline void k_scale(const uint8_t* s, int j, float* sc, float* m) {
  if (j < 4) {
    *sc = (float)(s[j] & 63);
    *m = (float)(s[j + 4] & 63);
    return;
  }
  int d = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
  int mm = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  *sc = (float)d;
  *m = (float)mm;
}

static inline uint32_t qh32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* quant.mojo:232 _q4_0 */
static void dq_q4_0(const uint8_t* p, float* out) {
  float d = f16_at(p);
  for (int l = 0; l < 16; l++) {
    int b = p[2 + l];
    out[l] = (float)((b & 0xF) - 8) * d;
    out[l + 16] = (float)((b >> 4) - 8) * d;
  }
}
/* quant.mojo:247 _q4_1 */
static void dq_q4_1(const uint8_t* p, float* out) {
  float d = f16_at(p), m = f16_at(p + 2);
  for (int l = 0; l < 16; l++) {
    int b = p[4 + l];
    out[l] = (float)(b & 0xF) * d + m;
    out[l + 16] = (float)(b >> 4) * d + m;
  }
}
/* quant.mojo:272 _q5_0 */
static void dq_q5_0(const uint8_t* p, float* out) {
  float d = f16_at(p);
  uint32_t qh = qh32(p + 2);
  for (int l = 0; l < 16; l++) {
    int b = p[6 + l];
    int hl = (int)(((qh >> l) << 4) & 0x10u);
    int hh = (int)((qh >> (l + 12)) & 0x10u);
    out[l] = (float)(((b & 0xF) | hl) - 16) * d;
    out[l + 16] = (float)(((b >> 4) | hh) - 16) * d;
  }
}
/* quant.mojo:290 _q5_1 */
static void dq_q5_1(const uint8_t* p, float* out) {
  float d = f16_at(p), m = f16_at(p + 2);
  uint32_t qh = qh32(p + 4);
  for (int l = 0; l < 16; l++) {
    int b = p[8 + l];
    int hl = (int)(((qh >> l) << 4) & 0x10u);
    int hh = (int)((qh >> (l + 12)) & 0x10u);
    out[l] = (float)((b & 0xF) | hl) * d + m;
    out[l + 16] = (float)((b >> 4) | hh) * d + m;
  }
}
/* quant.mojo:304 _q8_0 */
static void dq_q8_0(const uint8_t* p, float* out) {
  float d = f16_at(p);
  for (int l = 0; l < 32; l++) out[l] = (float)i8_at(p + 2 + l) * d;
}
/* quant.mojo:310 _q4_k */
static void dq_q4_k(const uint8_t* p, float* out) {
  float d = f16_at(p), dmin = f16_at(p + 2);
  const uint8_t* scales = p + 4;
  const uint8_t* qs = p + 16;
  for (int half = 0; half < 4; half++) {
    float s0, m0, s1, m1;
    k_scale(scales, half * 2, &s0, &m0);
    k_scale(scales, half * 2 + 1, &s1, &m1);
    float d1 = d * s0, mm1 = dmin * m0, d2 = d * s1, mm2 = dmin * m1;
    const uint8_t* q = qs + half * 32;
    float* base = out + half * 64;
    for (int l = 0; l < 32; l++) {
      int b = q[l];
      base[l] = d1 * (float)(b & 0xF) - mm1;
      base[l + 32] = d2 * (float)(b >> 4) - mm2;
    }
  }
}
/* quant.mojo:336 _q5_k */
static void dq_q5_k(const uint8_t* p, float* out) {
  float d = f16_at(p), dmin = f16_at(p + 2);
  const uint8_t* scales = p + 4;
  const uint8_t* qh = p + 16;
  const uint8_t* qs = p + 48;
  for (int half = 0; half < 4; half++) {
    float s0, m0, s1, m1;
    k_scale(scales, half * 2, &s0, &m0);
    k_scale(scales, half * 2 + 1, &s1, &m1);
    float d1 = d * s0, mm1 = dmin * m0, d2 = d * s1, mm2 = dmin * m1;
    int u1 = 1 << (half * 2), u2 = u1 << 1;
    const uint8_t* q = qs + half * 32;
    float* base = out + half * 64;
    for (int l = 0; l < 32; l++) {
      int b = q[l], h = qh[l];
      int v1 = (b & 0xF) + ((h & u1) ? 16 : 0);
      int v2 = (b >> 4) + ((h & u2) ? 16 : 0);
      base[l] = d1 * (float)v1 - mm1;
      base[l + 32] = d2 * (float)v2 - mm2;
    }
  }
}
/* quant.mojo:371 _q6_k */
static void dq_q6_k(const uint8_t* p, float* out) {
  float d = f16_at(p + 208);
  for (int n = 0; n < 2; n++) {
    const uint8_t* lo = p + n * 64;
    const uint8_t* hi = p + 128 + n * 32;
    const uint8_t* sc = p + 192 + n * 8;
    float* base = out + n * 128;
    for (int l = 0; l < 32; l++) {
      int g = l / 16;
      int h = hi[l];
      int q1 = ((lo[l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
      int q2 = ((lo[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
      int q3 = ((lo[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
      int q4 = ((lo[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
      base[l] = d * (float)i8_at(sc + g) * (float)q1;
      base[l + 32] = d * (float)i8_at(sc + g + 2) * (float)q2;
      base[l + 64] = d * (float)i8_at(sc + g + 4) * (float)q3;
      base[l + 96] = d * (float)i8_at(sc + g + 6) * (float)q4;
    }
  }
}

/* quant.mojo:184 dequant_block + :412 dequant_run */
int or_dequant_run(int kind, const uint8_t* p, int64_t count, float* out) {
  int per = or_block_elements(kind);
  if (per == 0) return -1;
  if (count % per != 0) return -2;
  int stride = or_block_bytes(kind);
  int64_t blocks = count / per;
  for (int64_t i = 0; i < blocks; i++) {
    const uint8_t* b = p + i * stride;
    float* o = out + i * per;
    switch (kind) {
      case OR_F32: o[0] = f32_at(b); break;
      case OR_F16: o[0] = f16_at(b); break;
      case OR_BF16: o[0] = bf16_at(b); break;
      case OR_Q4_0: dq_q4_0(b, o); break;
      case OR_Q4_1: dq_q4_1(b, o); break;
      case OR_Q5_0: dq_q5_0(b, o); break;
      case OR_Q5_1: dq_q5_1(b, o); break;
      case OR_Q8_0: dq_q8_0(b, o); break;
      case OR_Q4_K: dq_q4_k(b, o); break;
      case OR_Q5_K: dq_q5_k(b, o); break;
      case OR_Q6_K: dq_q6_k(b, o); break;
      default: return -1;
    }
  }
  return 0;
}

/* kernel.mojo:138 _dot_q4_0 */
static float dot_q4_0(const uint8_t* p, const float* x) {
  float d = f16_at(p), qx = 0.0f, sx = 0.0f;
  for (int l = 0; l < 16; l++) {
    int b = p[2 + l];
    float lo = x[l], hi = x[l + 16];
    qx += (float)(b & 0xF) * lo + (float)(b >> 4) * hi;
    sx += lo + hi;
  }
  return d * (qx - 8.0f * sx);
}
/* kernel.mojo:153 _dot_q4_1 */
static float dot_q4_1(const uint8_t* p, const float* x) {
  float d = f16_at(p), m = f16_at(p + 2), qx = 0.0f, sx = 0.0f;
  for (int l = 0; l < 16; l++) {
    int b = p[4 + l];
    float lo = x[l], hi = x[l + 16];
    qx += (float)(b & 0xF) * lo + (float)(b >> 4) * hi;
    sx += lo + hi;
  }
  return d * qx + m * sx;
}
/* kernel.mojo:168 _dot_q5_0 */
static float dot_q5_0(const uint8_t* p, const float* x) {
  float d = f16_at(p), qx = 0.0f, sx = 0.0f;
  uint32_t qh = qh32(p + 2);
  for (int l = 0; l < 16; l++) {
    int b = p[6 + l];
    float lo = x[l], hi = x[l + 16];
    int ql = (b & 0xF) | (int)(((qh >> l) << 4) & 0x10u);
    int qhh = (b >> 4) | (int)((qh >> (l + 12)) & 0x10u);
    qx += (float)ql * lo + (float)qhh * hi;
    sx += lo + hi;
  }
  return d * (qx - 16.0f * sx);
}
/* kernel.mojo:185 _dot_q5_1 */
static float dot_q5_1(const uint8_t* p, const float* x) {
  float d = f16_at(p), m = f16_at(p + 2), qx = 0.0f, sx = 0.0f;
  uint32_t qh = qh32(p + 4);
  for (int l = 0; l < 16; l++) {
    int b = p[8 + l];
    float lo = x[l], hi = x[l + 16];
    int ql = (b & 0xF) | (int)(((qh >> l) << 4) & 0x10u);
    int qhh = (b >> 4) | (int)((qh >> (l + 12)) & 0x10u);
    qx += (float)ql * lo + (float)qhh * hi;
    sx += lo + hi;
  }
  return d * qx + m * sx;
}
/* kernel.mojo:202 _dot_q8_0 */
static float dot_q8_0(const uint8_t* p, const float* x) {
  float d = f16_at(p), acc = 0.0f;
  for (int l = 0; l < 32; l++) acc += (float)i8_at(p + 2 + l) * x[l];
  return d * acc;
}
/* kernel.mojo:210 _dot_q4_k */
static float dot_q4_k(const uint8_t* p, const float* x) {
  float d = f16_at(p), dmin = f16_at(p + 2), total = 0.0f;
  const uint8_t* scales = p + 4;
  const uint8_t* qs = p + 16;
  for (int half = 0; half < 4; half++) {
    float s0, m0, s1, m1;
    k_scale(scales, half * 2, &s0, &m0);
    k_scale(scales, half * 2 + 1, &s1, &m1);
    const uint8_t* q = qs + half * 32;
    const float* a_lo = x + half * 64;
    const float* a_hi = a_lo + 32;
    float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
    for (int l = 0; l < 32; l++) {
      int b = q[l];
      float a = a_lo[l], c = a_hi[l];
      qx1 += (float)(b & 0xF) * a;
      sx1 += a;
      qx2 += (float)(b >> 4) * c;
      sx2 += c;
    }
    total += d * s0 * qx1 - dmin * m0 * sx1;
    total += d * s1 * qx2 - dmin * m1 * sx2;
  }
  return total;
}
/* kernel.mojo:244 _dot_q5_k */
static float dot_q5_k(const uint8_t* p, const float* x) {
  float d = f16_at(p), dmin = f16_at(p + 2), total = 0.0f;
  const uint8_t* scales = p + 4;
  const uint8_t* qh = p + 16;
  const uint8_t* qs = p + 48;
  for (int half = 0; half < 4; half++) {
    float s0, m0, s1, m1;
    k_scale(scales, half * 2, &s0, &m0);
    k_scale(scales, half * 2 + 1, &s1, &m1);
    int u1 = 1 << (half * 2), u2 = u1 << 1;
    const uint8_t* q = qs + half * 32;
    const float* a_lo = x + half * 64;
    const float* a_hi = a_lo + 32;
    float qx1 = 0.0f, sx1 = 0.0f, qx2 = 0.0f, sx2 = 0.0f;
    for (int l = 0; l < 32; l++) {
      int b = q[l], h = qh[l];
      float a = a_lo[l], c = a_hi[l];
      int v1 = (b & 0xF) + ((h & u1) ? 16 : 0);
      int v2 = (b >> 4) + ((h & u2) ? 16 : 0);
      qx1 += (float)v1 * a;
      sx1 += a;
      qx2 += (float)v2 * c;
      sx2 += c;
    }
    total += d * s0 * qx1 - dmin * m0 * sx1;
    total += d * s1 * qx2 - dmin * m1 * sx2;
  }
  return total;
}
/* kernel.mojo:281 _dot_q6_k */
static float dot_q6_k(const uint8_t* p, const float* x) {
  float d = f16_at(p + 208), total = 0.0f;
  for (int n = 0; n < 2; n++) {
    const uint8_t* lo = p + n * 64;
    const uint8_t* hi = p + 128 + n * 32;
    const uint8_t* sc = p + 192 + n * 8;
    const float* o = x + n * 128;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int l = 0; l < 32; l++) {
      int g = l / 16;
      int h = hi[l];
      int q1 = ((lo[l] & 0xF) | (((h >> 0) & 3) << 4)) - 32;
      int q2 = ((lo[l + 32] & 0xF) | (((h >> 2) & 3) << 4)) - 32;
      int q3 = ((lo[l] >> 4) | (((h >> 4) & 3) << 4)) - 32;
      int q4 = ((lo[l + 32] >> 4) | (((h >> 6) & 3) << 4)) - 32;
      acc[g] += (float)q1 * o[l];
      acc[g + 2] += (float)q2 * o[l + 32];
      acc[g + 4] += (float)q3 * o[l + 64];
      acc[g + 6] += (float)q4 * o[l + 96];
    }
    for (int g = 0; g < 8; g++) total += d * (float)i8_at(sc + g) * acc[g];
  }
  return total;
}

/* kernel.mojo:75 row_dot */
int or_row_dot(int kind, const uint8_t* p, const float* x, int64_t n, float* out) {
  int per = or_block_elements(kind);
  if (per == 0) return -1;
  if (n % per != 0) return -2;
  float acc = 0.0f;
  if (kind == OR_F32) {
    for (int64_t i = 0; i < n; i++) acc += f32_at(p + i * 4) * x[i];
    *out = acc;
    return 0;
  }
  if (kind == OR_F16) {
    for (int64_t i = 0; i < n; i++) acc += f16_at(p + i * 2) * x[i];
    *out = acc;
    return 0;
  }
  if (kind == OR_BF16) {
    for (int64_t i = 0; i < n; i++) acc += bf16_at(p + i * 2) * x[i];
    *out = acc;
    return 0;
  }
  int stride = or_block_bytes(kind);
  int64_t blocks = n / per;
  for (int64_t b = 0; b < blocks; b++) {
    const uint8_t* blk = p + b * stride;
    const float* xb = x + b * per;
    switch (kind) {
      case OR_Q4_0: acc += dot_q4_0(blk, xb); break;
      case OR_Q4_1: acc += dot_q4_1(blk, xb); break;
      case OR_Q5_0: acc += dot_q5_0(blk, xb); break;
      case OR_Q5_1: acc += dot_q5_1(blk, xb); break;
      case OR_Q8_0: acc += dot_q8_0(blk, xb); break;
      case OR_Q4_K: acc += dot_q4_k(blk, xb); break;
      case OR_Q5_K: acc += dot_q5_k(blk, xb); break;
      case OR_Q6_K: acc += dot_q6_k(blk, xb); break;
      default: return -1;
    }
  }
  *out = acc;
  return 0;
}

/* kernel.mojo:316 matvec: one row at a time, in row order. */
int or_matvec(int kind, const uint8_t* w, int64_t row_bytes, int32_t rows,
              int32_t cols, const float* x, float* y, int32_t threads) {
  int per = or_block_elements(kind);
  if (per == 0) return -1;
  if (cols % per != 0) return -2;
  if ((int64_t)(cols / per) * or_block_bytes(kind) != row_bytes) return -3;
  int bad = 0;
#ifdef _OPENMP
  if (threads > 1) {
#pragma omp parallel for num_threads(threads) schedule(static) reduction(| : bad)
    for (int32_t r = 0; r < rows; r++)
      bad |= or_row_dot(kind, w + (int64_t)r * row_bytes, x, cols, &y[r]) != 0;
    return bad ? -1 : 0;
  }
#else
  (void)threads;
#endif
  for (int32_t r = 0; r < rows; r++)
    bad |= or_row_dot(kind, w + (int64_t)r * row_bytes, x, cols, &y[r]) != 0;
  return bad ? -1 : 0;
}

/* kernel.mojo:400 rms_norm: float64 sum of squares, float32 scale. */
void or_rms_norm(float* out, const float* x, const float* gain, int32_t n, float eps) {
  double sum = 0.0;
  for (int32_t i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
  float scale = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
  for (int32_t i = 0; i < n; i++) out[i] = x[i] * scale * gain[i];
}

/* kernel.mojo:470 softmax */
void or_softmax(float* x, int32_t n) {
  if (n <= 0) return;
  float top = x[0];
  for (int32_t i = 1; i < n; i++)
    if (x[i] > top) top = x[i];
  float sum = 0.0f;
  for (int32_t i = 0; i < n; i++) {
    float e = expf(x[i] - top);
    x[i] = e;
    sum += e;
  }
  float inv = 1.0f / sum;
  for (int32_t i = 0; i < n; i++) x[i] *= inv;
}

/* kernel.mojo:494 silu */
float or_silu(float v) { return v / (1.0f + expf(-v)); }

/* kernel.mojo:499 gelu (tanh form) */
float or_gelu(float v) {
  float c = 0.7978845608028654f;
  float inner = c * (v + 0.044715f * v * v * v);
  float t = 2.0f / (1.0f + expf(-2.0f * inner)) - 1.0f;
  return 0.5f * v * (1.0f + t);
}

/* kernel.mojo:512 swiglu */
void or_swiglu(float* gate, const float* up, int32_t n) {
  for (int32_t i = 0; i < n; i++) gate[i] = or_silu(gate[i]) * up[i];
}

/* kernel.mojo:571 argmax: ties go to the lower index. */
int32_t or_argmax(const float* x, int32_t n) {
  if (n <= 0) return -1;
  int32_t best = 0;
  for (int32_t i = 1; i < n; i++)
    if (x[i] > x[best]) best = i;
  return best;
}

/* rope.mojo:153 _powf */
static float powf_ref(float x, float y) {
  if (x <= 0.0f) return 0.0f;
  return (float)exp((double)y * log((double)x));
}

/* rope.mojo:230 step_table */
void or_rope_steps(float* steps, int32_t dim, float base) {
  for (int32_t pair = 0; pair < dim / 2; pair++)
    steps[pair] = powf_ref(base, -2.0f * (float)pair / (float)dim);
}

/* rope.mojo:253 angle, with scale 1, ext_factor 0, attn_factor 1; freq is
 * the pair's rope_freqs.weight factor (1 when the model has none). */
void or_rope_angle_scaled(int32_t dim, float base, int32_t pos, int32_t pair, float freq, float* c, float* s) {
  float step = powf_ref(base, -2.0f * (float)pair / (float)dim);
  float extrap = (float)pos * step / freq;
  float interp = 1.0f * extrap;
  float theta = interp;
  *c = (float)cos((double)theta) * 1.0f;
  *s = (float)sin((double)theta) * 1.0f;
}

void or_rope_angle(int32_t dim, float base, int32_t pos, int32_t pair, float* c, float* s) {
  or_rope_angle_scaled(dim, base, pos, pair, 1.0f, c, s);
}

/* rope.mojo:294 rotate_scaled over every head (rope.mojo:374 rotate_run);
 * factors: one per pair (rope_freqs.weight), or NULL for none. */
void or_rotate_run_scaled(float* x, int32_t heads, int32_t head_dim, int32_t dim,
                          float base, int32_t neox, int32_t pos, const float* factors) {
  int32_t pairs = dim / 2;
  for (int32_t h = 0; h < heads; h++) {
    float* at = x + (int64_t)h * head_dim;
    for (int32_t pair = 0; pair < pairs; pair++) {
      float c, s;
      or_rope_angle_scaled(dim, base, pos, pair, factors ? factors[pair] : 1.0f, &c, &s);
      int32_t lo, hi;
      if (neox) {
        lo = pair;
        hi = pair + pairs;
      } else {
        lo = pair * 2;
        hi = lo + 1;
      }
      float a = at[lo], b = at[hi];
      at[lo] = a * c - b * s;
      at[hi] = a * s + b * c;
    }
  }
}

void or_rotate_run(float* x, int32_t heads, int32_t head_dim, int32_t dim,
                   float base, int32_t neox, int32_t pos) {
  or_rotate_run_scaled(x, heads, head_dim, dim, base, neox, pos, NULL);
}

/* attention.mojo:144 attend over a contiguous run of positions 0..count-1. */
void or_attend(int32_t heads, int32_t kv_heads, int32_t head_dim, float scale,
               const float* q, const float* keys, const float* values,
               int32_t count, float* out, float* scores) {
  int32_t kv_width = kv_heads * head_dim;
  int32_t group = heads / kv_heads;
  for (int32_t h = 0; h < heads; h++) {
    int32_t kvh = h / group;
    const float* qa = q + (int64_t)h * head_dim;
    for (int32_t t = 0; t < count; t++) {
      const float* ka = keys + (int64_t)t * kv_width + (int64_t)kvh * head_dim;
      float s = 0.0f;
      for (int32_t d = 0; d < head_dim; d++) s += qa[d] * ka[d];
      s *= scale;
      scores[t] = s;
    }
    or_softmax(scores, count);
    float* oa = out + (int64_t)h * head_dim;
    for (int32_t d = 0; d < head_dim; d++) oa[d] = 0.0f;
    for (int32_t t = 0; t < count; t++) {
      float p = scores[t];
      const float* va = values + (int64_t)t * kv_width + (int64_t)kvh * head_dim;
      for (int32_t d = 0; d < head_dim; d++) oa[d] += p * va[d];
    }
  }
}

static int mv(const or_weight* w, const float* x, float* y, int32_t threads) {
  return or_matvec(w->kind, (const uint8_t*)w->data, w->row_bytes, w->rows, w->cols, x, y, threads);
}

static float f16_round(float v) { return or_f16(or_f32_to_f16(v)); }

/* What a q8_0 cache row holds for n values (gpu_ops.mojo:1531
 * store_kv_q8_kernel; the host restatement is tests/test_gpu_ops.mojo
 * _quantize_q8): per 32-value block a factor amax / 127 kept as float16, the
 * values times 127 / amax rounded half away from zero and clamped to
 * [-127, 127]; read back as float(q) * float(f16 factor).  In place. */
void or_q8_cache_round(float* v, int32_t n) {
  for (int32_t i = 0; i + 32 <= n; i += 32) {
    float amax = 0.0f;
    for (int k = 0; k < 32; k++) {
      float a = v[i + k] < 0 ? -v[i + k] : v[i + k];
      if (a > amax) amax = a;
    }
    float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
    float s = f16_round(amax / 127.0f);
    for (int k = 0; k < 32; k++) {
      float x = v[i + k] * inv;
      float r = x >= 0 ? x + 0.5f : x - 0.5f;
      int q = (int)r;
      if (q > 127) q = 127;
      if (q < -127) q = -127;
      v[i + k] = (float)q * s;
    }
  }
}

/* kernel.mojo:400 rms_norm_at: the same norm over a run of n values, in
 * place (a head of q or k, or a sublayer's whole output). */
static void rms_norm_at(float* x, const float* gain, int32_t n, float eps) {
  or_rms_norm(x, x, gain, n, eps);
}

/* kernel.mojo:526 add_bias_at */
static void add_bias_at(float* x, const float* bias, int32_t n) {
  for (int32_t i = 0; i < n; i++) x[i] += bias[i];
}

static float act_of(int32_t act, float v) { return act ? or_gelu(v) : or_silu(v); }

/* block.mojo:466 layer = attention_layer (:319) then mlp_layer (:429);
 * parts: 1 the attention sublayer only, 2 the mlp sublayer only, 3 both. */
int or_layer_part(const or_layer* L, float* x, float* keys, float* values,
                  int32_t slot, int32_t pos, int32_t f16_store, int32_t threads, int32_t parts) {
  int32_t width = L->width, qw = L->heads * L->head_dim, kvw = L->kv_heads * L->head_dim;
  int32_t hidden = L->hidden;
  float* norm = (float*)malloc(sizeof(float) * width);
  float* q = (float*)malloc(sizeof(float) * qw);
  float* heads_out = (float*)malloc(sizeof(float) * qw);
  float* projected = (float*)malloc(sizeof(float) * width);
  float* gate = (float*)malloc(sizeof(float) * hidden);
  float* up = (float*)malloc(sizeof(float) * hidden);
  float* scores = (float*)malloc(sizeof(float) * (slot + 1));
  int rc = 0;
  if (!norm || !q || !heads_out || !projected || !gate || !up || !scores) { rc = -9; goto done; }

  if (!(parts & 1)) goto mlp;
  /* attention_layer */
  or_rms_norm(norm, x, L->attn_norm, width, L->eps);
  if ((rc = mv(&L->wq, norm, q, threads))) goto done;
  float* kslot = keys + (int64_t)slot * kvw;
  float* vslot = values + (int64_t)slot * kvw;
  if ((rc = mv(&L->wk, norm, kslot, threads))) goto done;
  if ((rc = mv(&L->wv, norm, vslot, threads))) goto done;
  /* block.mojo:363-366: the bias is part of the projection */
  if (L->q_bias) add_bias_at(q, L->q_bias, qw);
  if (L->k_bias) add_bias_at(kslot, L->k_bias, kvw);
  if (L->v_bias) add_bias_at(vslot, L->v_bias, kvw);
  /* block.mojo:367-384: each head of q and k normed before rope */
  if (L->q_norm) {
    for (int32_t h = 0; h < L->heads; h++) rms_norm_at(q + (int64_t)h * L->head_dim, L->q_norm, L->head_dim, L->eps);
    for (int32_t h = 0; h < L->kv_heads; h++)
      rms_norm_at(kslot + (int64_t)h * L->head_dim, L->k_norm, L->head_dim, L->eps);
  }
  or_rotate_run_scaled(q, L->heads, L->head_dim, L->rope_dim, L->rope_base, L->neox, pos, L->rope_factors);
  or_rotate_run_scaled(kslot, L->kv_heads, L->head_dim, L->rope_dim, L->rope_base, L->neox, pos,
                       L->rope_factors);
  if (f16_store == 2) {  /* a q8_0 cache */
    or_q8_cache_round(kslot, kvw);
    or_q8_cache_round(vslot, kvw);
  } else if (f16_store) {
    for (int32_t i = 0; i < kvw; i++) {
      kslot[i] = f16_round(kslot[i]);
      vslot[i] = f16_round(vslot[i]);
    }
  }
  or_attend(L->heads, L->kv_heads, L->head_dim, L->attn_scale, q, keys, values,
            slot + 1, heads_out, scores);
  if ((rc = mv(&L->wo, heads_out, projected, threads))) goto done;
  /* block.mojo:405-406: a sublayer's output normed on its way in */
  if (L->attn_post_norm) rms_norm_at(projected, L->attn_post_norm, width, L->eps);
  for (int32_t i = 0; i < width; i++) x[i] += projected[i];

mlp:
  if (!(parts & 2)) goto done;
  /* mlp_layer (:429-463) */
  or_rms_norm(norm, x, L->ffn_norm, width, L->eps);
  if ((rc = mv(&L->up, norm, up, threads))) goto done;
  if (!L->ungated) {
    if ((rc = mv(&L->gate, norm, gate, threads))) goto done;
    if (L->act)
      for (int32_t i = 0; i < hidden; i++) gate[i] = or_gelu(gate[i]) * up[i];
    else
      or_swiglu(gate, up, hidden);
    if ((rc = mv(&L->down, gate, projected, threads))) goto done;
  } else {
    for (int32_t i = 0; i < hidden; i++) up[i] = act_of(L->act, up[i]);
    if ((rc = mv(&L->down, up, projected, threads))) goto done;
  }
  if (L->ffn_post_norm) rms_norm_at(projected, L->ffn_post_norm, width, L->eps);
  for (int32_t i = 0; i < width; i++) x[i] += projected[i];

done:
  free(norm); free(q); free(heads_out); free(projected); free(gate); free(up); free(scores);
  return rc;
}

int or_layer_step(const or_layer* L, float* x, float* keys, float* values,
                  int32_t slot, int32_t pos, int32_t f16_store, int32_t threads) {
  return or_layer_part(L, x, keys, values, slot, pos, f16_store, threads, 3);
}

/* model.mojo:178 forward: embed (:102, an f32 row copy), the layers, head (:136). */
int or_forward(const or_layer* layers, int32_t n_layers, const float* embedding,
               int32_t vocab, const float* output_norm, const or_weight* output,
               int32_t token, int32_t pos, int32_t slot, float** keys,
               float** values, int32_t f16_store, float* logits, int32_t threads) {
  if (n_layers <= 0 || token < 0 || token >= vocab || pos < 0) return -1;
  int32_t width = layers[0].width;
  float* x = (float*)malloc(sizeof(float) * width);
  float* normed = (float*)malloc(sizeof(float) * width);
  int rc = 0;
  if (!x || !normed) { rc = -9; goto done; }
  memcpy(x, embedding + (int64_t)token * width, sizeof(float) * width);
  for (int32_t i = 0; i < n_layers; i++) {
    rc = or_layer_step(&layers[i], x, keys[i], values[i], slot, pos, f16_store, threads);
    if (rc) goto done;
  }
  or_rms_norm(normed, x, output_norm, width, layers[0].eps);
  rc = mv(output, normed, logits, threads);
done:
  free(x); free(normed);
  return rc;
}

/* tests/test_kernel.mojo:69 Rng.next (xorshift64) */
uint64_t or_xorshift_next(uint64_t* s) {
  *s ^= *s << 13;
  *s ^= *s >> 7;
  *s ^= *s << 17;
  return *s;
}

/* tests/test_kernel.mojo:96 _scale_bits */
static int scale_bits(int pick) {
  if (pick == 0) return 0x3C00;
  if (pick == 1) return 0xB800;
  if (pick == 2) return 0x2E66;
  return 0x3555;
}

static void put16(uint8_t* b, int64_t at, int v) {
  b[at] = (uint8_t)(v & 0xFF);
  b[at + 1] = (uint8_t)((v >> 8) & 0xFF);
}

/* tests/test_kernel.mojo:106 _blocks */
void or_test_blocks(int kind, int32_t count, uint64_t seed, uint8_t* out) {
  int stride = or_block_bytes(kind);
  uint64_t st = seed;
  for (int64_t i = 0; i < (int64_t)count * stride; i++) out[i] = (uint8_t)(or_xorshift_next(&st) & 0xFF);
  for (int32_t b = 0; b < count; b++) {
    int64_t at = (int64_t)b * stride;
    if (kind == OR_Q6_K) {
      put16(out, at + 208, scale_bits((int)(or_xorshift_next(&st) & 3)));
    } else {
      put16(out, at, scale_bits((int)(or_xorshift_next(&st) & 3)));
      if (kind == OR_Q4_K || kind == OR_Q5_K || kind == OR_Q4_1 || kind == OR_Q5_1)
        put16(out, at + 2, scale_bits((int)(or_xorshift_next(&st) & 3)));
    }
  }
}

/* tests/test_kernel.mojo:85 Rng.unit: a float in [-1, 1). */
void or_test_units(uint64_t seed, int32_t n, float* out) {
  uint64_t st = seed;
  for (int32_t i = 0; i < n; i++)
    out[i] = (float)(int64_t)(or_xorshift_next(&st) & 0xFFFF) / 32768.0f - 1.0f;
}

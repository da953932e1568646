// prefill.hip -- the many-token matmul (prefill chunks, tokens > 8) on the
// matrix cores: v_mfma_f32_32x32x16_f16, gfx950.
//
// y[t * ldy + r] = epilogue(sum_k W[r][k] * x[t][k]) for every kind of the
// decode path, at roughly float32 accuracy although the multiplier takes
// half precision operands:
//
//  * Activations.  Token t is scaled by a power of two 2^-e_t so its largest
//    |x| lies in [2^13, 2^14), then each value is split into two halves,
//    x' = hi + lo with hi = f16(x') and lo = f16(x' - hi): 22 significant bits
//    (prefill_x_kernel).  The scale comes back once, on the finished sum.
//  * Weights enter as the integer codes of the format, which half precision
//    holds exactly: sc * q for Q4_K and Q5_K (at most 63 * 31), the signed
//    code for the 32-value kinds (q - 8, q - 16, the int8 of Q8_0, or q), and
//    sc * (q - 32) for Q6_K split into its even part and its low bit (up to
//    4096 in magnitude, one bit more than half precision carries).  Every
//    product code * hi, code * lo is then exact in the float32 accumulator.
//  * The scale of a weight block multiplies the accumulator once per block
//    (per 256 values for the K-quants, per 32 for the others), and the
//    min terms (dmin * m of the K-quants, m of Q4_1 / Q5_1) are one more MFMA
//    per 256 values against the per-32 means of x (hi and lo in the 16
//    K-slots; a sum of 32 scaled values would overflow a half).
//
// Against the float32 host dot this differs by float32 rounding of the sums.
// The reference's own tensor-core tile (src/molla/nn/gpu.mojo:2665
// planar_nvmma_kernel) rounds the activations and weights to half precision
// and is held to 2e-3 of the peak; this form keeps the 1e-5 gate of its float
// tiles (tests/test_gpu.mojo:255-300).
//
// Work decomposition.  One MFMA is 32 tokens (M) x 32 rows (N) x 16 values
// (K): lane l holds token / row l % 32 and values 8 (l / 32) .. +8 of the
// step, and accumulator element j belongs to token 8 (j / 4) + 4 (l / 32) +
// j % 4, row l % 32.  A wave owns 2 row tiles x 2 token tiles (64 rows x 64
// tokens); a block of W waves shares the 64 tokens, whose activation halves
// are staged through LDS 64 values at a time (double-buffered), while each
// wave decodes its own rows' weight codes straight from global memory, one
// stage ahead.  Long reductions over few output tiles split K across
// blockIdx.z, with partial sums in the workspace and a second kernel adding
// them in split order (deterministic) before the epilogue.  Rows may come
// from up to three matrices of one kind laid end to end (RowSegs: a layer's
// q|k|v in one launch), and one activation prep (prefill_prepare) can serve
// several launches over the same input.
//
// Replaces device_matmul_into's batched kernels (src/molla/nn/gpu.mojo:1809
// planar_matmul_kernel, :2665 planar_nvmma_kernel; dispatch :3015) for
// tokens above the decode batch; output layout and epilogues as
// gpu.mojo:1005 and :2955-2961.
#include <algorithm>
#include <type_traits>

#include "matvec_rows.h"

namespace mi {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kTileTok = 32;     // tokens of one MFMA tile
constexpr int kStage = 64;       // values of K per LDS stage (4 MFMA steps)
constexpr int kChunk = 256;      // values per min-term MFMA / K-quant superblock
constexpr int kPadTiles = 4;     // token tiles the activation prep pads to (the widest block's)
constexpr int kRing = 2;         // register slots: the stage computed and the one in flight

__device__ __forceinline__ v16f mfma(v8h a, v8h b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v8h as_v8h4(v4u u) { return __builtin_bit_cast(v8h, u); }
__device__ __forceinline__ v8h as_v8h(uint4 u) {
  union {
    uint4 u;
    v8h h;
  } c;
  c.u = u;
  return c.h;
}

// 8 bytes from a 2-byte aligned address, as two dwords (the 34/18/22-byte
// blocks sit 2 bytes off alignment every other block).
__device__ __forceinline__ uint2 ld8(const uint8_t* p) {
  const uintptr_t a = (uintptr_t)p;
  const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
  const uint32_t sh = (uint32_t)(a & 3);
  // branch-free: aligned, the third load repeats the second (in bounds) and
  // a zero shift passes the low dword through
  const uint32_t d0 = q[0], d1 = q[1], d2 = q[sh ? 2 : 1];
  return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, sh), __builtin_amdgcn_alignbyte(d2, d1, sh));
}
__device__ __forceinline__ uint32_t ld4u(const uint8_t* p) {
  const uintptr_t a = (uintptr_t)p;
  const uint32_t* q = (const uint32_t*)(a & ~(uintptr_t)3);
  const uint32_t sh = (uint32_t)(a & 3);
  return __builtin_amdgcn_alignbyte(q[sh ? 1 : 0], q[0], sh);
}
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { return *(const uint16_t*)p; }
__device__ __forceinline__ float f16f(uint32_t bits) { return half_bits_to_float(bits & 0xFFFF); }

// (sc, m) of group j of a K-quant superblock from scales[0..11] in y, z, w
// (quant.mojo:161 _k_scale).
__device__ __forceinline__ void kscale(uint32_t y, uint32_t z, uint32_t w, int j, uint32_t& sc, uint32_t& m) {
  const uint32_t s = 8u * (uint32_t)(j & 3);
  const uint32_t hi = (uint32_t)(j >> 2);
  sc = __builtin_amdgcn_ubfe(hi ? w : y, s, 4) | (__builtin_amdgcn_ubfe(y, s + 4 + 2 * hi, 2) << 4);
  m = __builtin_amdgcn_ubfe(hi ? w : z, s + 4 * hi, 4) | (__builtin_amdgcn_ubfe(z, s + 4 + 2 * hi, 2) << 4);
}

typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// Eight byte codes u (0..255, bytes of t0 then t1) as the halves 1024 + u:
// 0x64 above each byte is the exponent of 1024, the byte the mantissa.
__device__ __forceinline__ v8h magic8(uint32_t t0, uint32_t t1) {
  return as_v8h(make_uint4(__builtin_amdgcn_perm(0x64646464u, t0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, t0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, t1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, t1, 0x04030402u)));
}
__device__ __forceinline__ v8h splat8(_Float16 v) { return v8h{v, v, v, v, v, v, v, v}; }
// (1024 + u) * a + b, once rounded: exact when the result is a small integer.
__device__ __forceinline__ v8h fma8(v8h v, _Float16 a, _Float16 b) {
  return __builtin_elementwise_fma(v, splat8(a), splat8(b));
}

// ---- per-kind weight access ------------------------------------------------
// Raw: what one lane reads of one row for one stage (64 values of K);
// load(raw, row, stage, kh); codes(raw, stage, s4, kh, b0, b1) for MFMA step
// s4 (0..3) of the stage, b1 only when LIMBS == 2.  Codes are made in half
// precision from "magic" halves 1024 + u (magic8), so each pair of values
// costs a byte permute and one packed multiply-add.
// GROUP: values per block scale.  MIN: 0 none, 1 K-quant dmin * m (scaled per
// superblock), 2 m per 32-value block (Q4_1, Q5_1).

__device__ __forceinline__ v8h kquant_codes(uint32_t t0, uint32_t t1, uint32_t sc) {
  // sc * u = (1024 + u) * sc - 1024 * sc; both terms exact halves (sc < 64)
  return fma8(magic8(t0, t1), (_Float16)(float)sc, (_Float16)(-1024.0f * (float)sc));
}

struct KQ4K {
  static constexpr int GROUP = 256, LIMBS = 1, MIN = 1, BLOCK = 144;
  struct Raw {
    uint4 hdr;
    uint2 q[2];
  };
  static __device__ __forceinline__ void load(Raw& r, const uint8_t* row, int st, int kh) {
    const uint8_t* b = row + (int64_t)(st >> 2) * BLOCK;
    r.hdr = *(const uint4*)b;
    const uint8_t* q = b + 16 + 32 * (st & 3) + 8 * kh;
    r.q[0] = *(const uint2*)q;
    r.q[1] = *(const uint2*)(q + 16);
  }
  static __device__ __forceinline__ void codes(const Raw& r, int st, int s4, int, v8h& b0, v8h&) {
    const int j = 2 * (st & 3) + (s4 >> 1);
    uint32_t sc, m;
    kscale(r.hdr.y, r.hdr.z, r.hdr.w, j, sc, m);
    const uint2 q = r.q[s4 & 1];
    const int sh = 4 * (s4 >> 1);
    b0 = kquant_codes((q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu, sc);
  }
  static __device__ __forceinline__ float d(const Raw& r) { return f16f(r.hdr.x); }
  static __device__ __forceinline__ float dmin(const Raw& r) { return f16f(r.hdr.x >> 16); }
  static __device__ __forceinline__ v8h mins(const Raw& r) {
    v8h c;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      uint32_t sc, m;
      kscale(r.hdr.y, r.hdr.z, r.hdr.w, j, sc, m);
      c[j] = (_Float16)(float)m;
    }
    return c;
  }
};

struct KQ5K {
  static constexpr int GROUP = 256, LIMBS = 1, MIN = 1, BLOCK = 176;
  struct Raw {
    uint4 hdr;
    uint2 qh[2], q[2];
  };
  static __device__ __forceinline__ void load(Raw& r, const uint8_t* row, int st, int kh) {
    const uint8_t* b = row + (int64_t)(st >> 2) * BLOCK;
    r.hdr = *(const uint4*)b;
    r.qh[0] = *(const uint2*)(b + 16 + 8 * kh);
    r.qh[1] = *(const uint2*)(b + 32 + 8 * kh);
    const uint8_t* q = b + 48 + 32 * (st & 3) + 8 * kh;
    r.q[0] = *(const uint2*)q;
    r.q[1] = *(const uint2*)(q + 16);
  }
  static __device__ __forceinline__ void codes(const Raw& r, int st, int s4, int, v8h& b0, v8h&) {
    const int j = 2 * (st & 3) + (s4 >> 1);
    uint32_t sc, m;
    kscale(r.hdr.y, r.hdr.z, r.hdr.w, j, sc, m);
    const uint2 q = r.q[s4 & 1], h = r.qh[s4 & 1];
    const int sh = 4 * (s4 >> 1);
    // the fifth bit of value i is bit j of qh byte i
    const uint32_t t0 = ((q.x >> sh) & 0x0F0F0F0Fu) | (((h.x >> j) & 0x01010101u) << 4);
    const uint32_t t1 = ((q.y >> sh) & 0x0F0F0F0Fu) | (((h.y >> j) & 0x01010101u) << 4);
    b0 = kquant_codes(t0, t1, sc);
  }
  static __device__ __forceinline__ float d(const Raw& r) { return f16f(r.hdr.x); }
  static __device__ __forceinline__ float dmin(const Raw& r) { return f16f(r.hdr.x >> 16); }
  static __device__ __forceinline__ v8h mins(const Raw& r) { return KQ4K::mins(*(const KQ4K::Raw*)&r); }
};

// Q6_K (quant.mojo:371): stage st' = st % 4 of a superblock covers half
// n = st' / 2 and quarters 2 (st' % 2) + {0, 1}; step s4 is quarter
// 2 (st' % 2) + s4 / 2, values 16 (s4 % 2) + 8 kh .. +8 of it, whose scale is
// sc[8n + 4 (st' % 2) + s4].  sc * (q - 32) reaches 4096 in magnitude: b0 is
// its nearest half, b1 the remainder (-1, 0 or 1), both exact.
struct KQ6K {
  static constexpr int GROUP = 256, LIMBS = 2, MIN = 0, BLOCK = 210;
  struct Raw {
    uint2 ql[2][2], qh[2];
    uint32_t sc, dbits;
  };
  static __device__ __forceinline__ void load(Raw& r, const uint8_t* row, int st, int kh) {
    const uint8_t* b = row + (int64_t)(st >> 2) * BLOCK;
    const int sp = st & 3, n = sp >> 1;
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int c = 0; c < 2; c++) r.ql[a][c] = ld8(b + 64 * n + 32 * a + 16 * c + 8 * kh);
#pragma unroll
    for (int c = 0; c < 2; c++) r.qh[c] = ld8(b + 128 + 32 * n + 16 * c + 8 * kh);
    r.sc = ld4u(b + 192 + 8 * n + 4 * (sp & 1));
    r.dbits = ld2(b + 208);
  }
  static __device__ __forceinline__ void codes(const Raw& r, int st, int s4, int, v8h& b0, v8h& b1) {
    const int sp = st & 3, a = s4 >> 1, c = s4 & 1;
    const int kq = 2 * (sp & 1) + a;
    const int nib = 4 * (sp & 1);
    const _Float16 sc = (_Float16)(float)(int8_t)(r.sc >> (8 * s4));
    const uint2 ql = r.ql[a][c], qh = r.qh[c];
    const uint32_t t0 = ((ql.x >> nib) & 0x0F0F0F0Fu) | (((qh.x >> (2 * kq)) & 0x03030303u) << 4);
    const uint32_t t1 = ((ql.y >> nib) & 0x0F0F0F0Fu) | (((qh.y >> (2 * kq)) & 0x03030303u) << 4);
    const v8h q = magic8(t0, t1) - splat8((_Float16)1056.0f);  // q - 32, exact
    b0 = q * splat8(sc);
    b1 = __builtin_elementwise_fma(q, splat8(sc), -b0);
  }
  static __device__ __forceinline__ float d(const Raw& r) { return f16f(r.dbits); }
  static __device__ __forceinline__ float dmin(const Raw&) { return 0.0f; }
  static __device__ __forceinline__ v8h mins(const Raw&) { return v8h{}; }
};

// The 32-value kinds: a stage is two blocks; step s4 is block s4 / 2, values
// 16 (s4 % 2) + 8 kh .. +8 of it.
template <int KIND>
struct KB32 {
  static constexpr int GROUP = 32, LIMBS = 1;
  static constexpr int MIN = (KIND == MI_Q4_1 || KIND == MI_Q5_1) ? 2 : 0;
  static constexpr int BLOCK = KIND == MI_Q8_0 ? 34 : KIND == MI_Q4_0 ? 18 : KIND == MI_Q4_1 ? 20
                               : KIND == MI_Q5_0 ? 22 : 24;
  // u of the magic halves is the unsigned code; the signed one is u - BIAS
  static constexpr float BIAS = KIND == MI_Q8_0 ? 128.0f : KIND == MI_Q4_0 ? 8.0f : KIND == MI_Q5_0 ? 16.0f : 0.0f;
  struct Raw {
    uint32_t dm[2];    // d | m << 16
    uint32_t qh[2];    // Q5_0 / Q5_1 fifth bits
    uint2 q[2][2];     // [block][Q8_0: half of the block; else [0] = the 8 nibble bytes]
  };
  static __device__ __forceinline__ void load(Raw& r, const uint8_t* row, int st, int kh) {
#pragma unroll
    for (int bb = 0; bb < 2; bb++) {
      const uint8_t* b = row + (int64_t)(2 * st + bb) * BLOCK;
      if (KIND == MI_Q8_0) {
        r.dm[bb] = ld2(b);
        r.q[bb][0] = ld8(b + 2 + 8 * kh);
        r.q[bb][1] = ld8(b + 18 + 8 * kh);
      } else if (KIND == MI_Q4_0) {
        r.dm[bb] = ld2(b);
        r.q[bb][0] = ld8(b + 2 + 8 * kh);
      } else if (KIND == MI_Q4_1) {
        r.dm[bb] = *(const uint32_t*)b;
        r.q[bb][0] = *(const uint2*)(b + 4 + 8 * kh);
      } else if (KIND == MI_Q5_0) {
        r.dm[bb] = ld2(b);
        r.qh[bb] = ld4u(b + 2);
        r.q[bb][0] = ld8(b + 6 + 8 * kh);
      } else {
        r.dm[bb] = *(const uint32_t*)b;
        r.qh[bb] = *(const uint32_t*)(b + 4);
        r.q[bb][0] = *(const uint2*)(b + 8 + 8 * kh);
      }
    }
  }
  static __device__ __forceinline__ void codes(const Raw& r, int, int s4, int kh, v8h& b0, v8h&) {
    const int bb = s4 >> 1, hf = s4 & 1;
    uint32_t t0, t1;
    if (KIND == MI_Q8_0) {
      t0 = r.q[bb][hf].x ^ 0x80808080u;  // int8 + 128
      t1 = r.q[bb][hf].y ^ 0x80808080u;
    } else {
      t0 = (r.q[bb][0].x >> (4 * hf)) & 0x0F0F0F0Fu;
      t1 = (r.q[bb][0].y >> (4 * hf)) & 0x0F0F0F0Fu;
      if (KIND == MI_Q5_0 || KIND == MI_Q5_1) {  // bit l of qh is value l's fifth
        const uint32_t bits = (r.qh[bb] >> (16 * hf + 8 * kh)) & 0xFFu;
        t0 |= mv::spread4(bits & 0xFu) << 4;
        t1 |= mv::spread4(bits >> 4) << 4;
      }
    }
    b0 = magic8(t0, t1) - splat8((_Float16)(1024.0f + BIAS));
  }
  static __device__ __forceinline__ float d(const Raw& r, int bb) { return f16f(r.dm[bb]); }
  static __device__ __forceinline__ uint32_t mbits(const Raw& r, int bb) { return r.dm[bb] >> 16; }
};

template <int KIND> struct KindOf;
template <> struct KindOf<MI_Q4_K> { using T = KQ4K; };
template <> struct KindOf<MI_Q5_K> { using T = KQ5K; };
template <> struct KindOf<MI_Q6_K> { using T = KQ6K; };
template <> struct KindOf<MI_Q8_0> { using T = KB32<MI_Q8_0>; };
template <> struct KindOf<MI_Q4_0> { using T = KB32<MI_Q4_0>; };
template <> struct KindOf<MI_Q4_1> { using T = KB32<MI_Q4_1>; };
template <> struct KindOf<MI_Q5_0> { using T = KB32<MI_Q5_0>; };
template <> struct KindOf<MI_Q5_1> { using T = KB32<MI_Q5_1>; };

// ---- activations -----------------------------------------------------------
// Layout (ttp token tiles of 32, ks = cols / 16 steps, nch = ceil(cols/256)):
//   xp: [tile][step][limb][lane][8 halves]: lane (kh, m) holds token
//       32 tile + m, values 16 step + 8 kh .. +8; limb 0 = hi, 1 = lo.
//   xm: [tile][chunk][lane][8 halves]: lane (0, m) holds hi of the means of
//       the chunk's eight 32-value blocks for token 32 tile + m, lane (1, m)
//       their lo (zero past cols).
//   xs: [32 ttp] the power of two each token's sums are multiplied by.
struct Prep {
  int ttp, ks, nch;
  size_t xp, xm, xs, total;
};

__host__ __device__ inline Prep prep_layout(int cols, int tokens) {
  Prep p;
  const int tt = (tokens + kTileTok - 1) / kTileTok;
  p.ttp = (tt + kPadTiles - 1) / kPadTiles * kPadTiles;
  p.ks = cols / 16;
  p.nch = (cols + kChunk - 1) / kChunk;
  p.xp = 0;
  p.xm = p.xp + (size_t)p.ttp * p.ks * 2048;
  p.xs = p.xm + (size_t)p.ttp * p.nch * 1024;
  p.total = (p.xs + (size_t)p.ttp * kTileTok * 4 + 255) & ~(size_t)255;
  return p;
}

__device__ __forceinline__ void split_half(float v, _Float16& hi, _Float16& lo) {
  hi = (_Float16)v;
  lo = (_Float16)(v - (float)hi);
}

// Each token's scale: the power of two 2^e with its largest |x| * 2^-e in
// [2^13, 2^14) (e clamped so the scale stays a normal float; 1 for a zero or
// padding token).  One block per token, xs[t] = 2^e.
__global__ __launch_bounds__(256) void prefill_scale_kernel(const float* __restrict__ x, int cols, int tokens,
                                                            uint8_t* __restrict__ work) {
  const Prep P = prep_layout(cols, tokens);
  const int t = blockIdx.x;
  __shared__ float red[4];
  float mx = 0.0f;
  if (t < tokens) {
    const float4* row = (const float4*)(x + (int64_t)t * cols);
    for (int c = threadIdx.x; c < (cols >> 2); c += blockDim.x) {
      const float4 a = row[c];
      mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int e = mx > 0.0f ? min(max(ilogbf(mx) - 13, -100), 100) : 0;
    ((float*)(work + P.xs))[t] = ldexpf(1.0f, e);
  }
}

// The halves and block means of one 256-value chunk of one 32-token tile
// (grid: chunks x tiles).  Thread f of 1024 fragments per chunk holds step
// f / 64, lane f % 64; consecutive threads write consecutive 16 bytes.
__global__ __launch_bounds__(256) void prefill_x_kernel(const float* __restrict__ x, int cols, int tokens,
                                                        uint8_t* __restrict__ work) {
  const Prep P = prep_layout(cols, tokens);
  const int ch = blockIdx.x, tile = blockIdx.y;
  const int steps = min(16, (cols >> 4) - ch * 16);  // the last chunk may be short
  const float* xs = (const float*)(work + P.xs);
  __shared__ float part[16][2][32];  // [step][kh][token] sums of 8 values
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int f = threadIdx.x + 256 * q;
    const int s = f >> 6, L = f & 63, m = L & 31, kh = L >> 5;
    if (s >= steps) continue;
    const int t = tile * 32 + m;
    float v[8];
    if (t < tokens) {
      const float* src = x + (int64_t)t * cols + ch * 256 + 16 * s + 8 * kh;
      const float4 a = *(const float4*)src, b = *(const float4*)(src + 4);
      const int e = ilogbf(xs[t]);
      v[0] = ldexpf(a.x, -e), v[1] = ldexpf(a.y, -e), v[2] = ldexpf(a.z, -e), v[3] = ldexpf(a.w, -e);
      v[4] = ldexpf(b.x, -e), v[5] = ldexpf(b.y, -e), v[6] = ldexpf(b.z, -e), v[7] = ldexpf(b.w, -e);
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = 0.0f;
    }
    v8h hi, lo;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      _Float16 h, l;
      split_half(v[i], h, l);
      hi[i] = h;
      lo[i] = l;
      sum += v[i];
    }
    uint8_t* dst = work + P.xp + ((size_t)(tile * P.ks + ch * 16 + s) * 2) * 1024 + L * 16;
    *(v8h*)dst = hi;
    *(v8h*)(dst + 1024) = lo;
    part[s][kh][m] = sum;
  }
  __syncthreads();
  // thread (g, m): the mean of 32-value block g of the chunk for token m (a
  // mean, since 32 values of up to 2^14 overflow a half); zero past cols
  const int g = threadIdx.x >> 5, m = threadIdx.x & 31;
  float mean = 0.0f;
  if (2 * g + 1 < steps)
    mean = ((part[2 * g][0][m] + part[2 * g][1][m]) + (part[2 * g + 1][0][m] + part[2 * g + 1][1][m])) *
           (1.0f / 32.0f);
  _Float16 h, l;
  split_half(mean, h, l);
  _Float16* mdst = (_Float16*)(work + P.xm + (size_t)(tile * P.nch + ch) * 1024);
  mdst[m * 8 + g] = h;
  mdst[(32 + m) * 8 + g] = l;
}

// ---- the matmul ------------------------------------------------------------
template <int KIND, int W, int RT, int TT>
__global__ __launch_bounds__(W * 64, KIND == MI_Q6_K ? 2 : 1) void prefill_kernel(const RowSegs sg,
                                                         int cols, int tokens, const uint8_t* __restrict__ work,
                                                         int stages_per_split, float* __restrict__ y, int64_t ldy,
                                                         int epi, const float* __restrict__ aux,
                                                         float* __restrict__ part) {
  using K = typename KindOf<KIND>::T;
  constexpr int kWaveRows = RT, kWaveTok = TT;  // row and token tiles per wave
  constexpr int kStageBytes = TT * 4 * 2 * 1024;  // one LDS buffer: TT tiles x 4 steps x 2 halves
  __shared__ __attribute__((aligned(16))) uint8_t xl[2][kStageBytes];
  const Prep P = prep_layout(cols, tokens);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 31, kh = lane >> 5;
  const int tile0 = blockIdx.y * kWaveTok;
  const int nst = cols / kStage;
  const int st0 = blockIdx.z * stages_per_split;
  const int st1 = min(st0 + stages_per_split, nst);
  const int rows = sg.end[sg.nseg - 1];
  const int row_base = (blockIdx.x * W + wave) * (kWaveRows * 32);
  const uint8_t* wrow[kWaveRows];
#pragma unroll
  for (int rt = 0; rt < kWaveRows; rt++) wrow[rt] = rows::seg_row(sg, min(row_base + rt * 32 + n, rows - 1));

  // activation stage copy: 16 KB, four 16-byte pieces a thread
  const uint8_t* xp = work + P.xp;
  constexpr int kPieces = kStageBytes / 16 / (W * 64);
  static_assert(kPieces * 16 * W * 64 == kStageBytes, "stage copy");
  // the register ring (a native vector type: HIP's uint4 struct is copied through memory)
  v4u xr0[kPieces], xr1[kPieces];
  // piece q of a stage's activation copy: 16 bytes of tile tt, offset within
  const size_t x_tile = (size_t)P.ks * 2048;
  const uint8_t* xsrc[kPieces];
  int xdst[kPieces];
#pragma unroll
  for (int q = 0; q < kPieces; q++) {
    const int idx = threadIdx.x + q * W * 64;
    const int tt = idx >> 9, within = idx & 511;
    xsrc[q] = xp + (tile0 + tt) * x_tile + within * 16;
    xdst[q] = idx * 16;
  }
#define PF_LOAD_X(ST, DST)                                                       \
  {                                                                              \
    const size_t o_ = (size_t)(ST) * 8192;                                       \
    _Pragma("unroll") for (int q = 0; q < kPieces; q++) DST[q] = *(const v4u*)(xsrc[q] + o_); \
  }
#define PF_STORE_X(SRC, BUF) \
  { _Pragma("unroll") for (int q = 0; q < kPieces; q++) *(v4u*)(&xl[BUF][xdst[q]]) = SRC[q]; }

  typename K::Raw raw[kRing][kWaveRows];
  v16f tot[kWaveRows][kWaveTok], acc[kWaveRows][kWaveTok];
  const v16f zero = {};
#pragma unroll
  for (int rt = 0; rt < kWaveRows; rt++)
#pragma unroll
    for (int tt = 0; tt < kWaveTok; tt++) tot[rt][tt] = acc[rt][tt] = zero;
  // min-term A fragments: the current chunk's, and the next one's in flight
  // (loaded a chunk ahead so the min MFMA never waits on a fresh load)
  v4u am[kWaveTok], am_next[kWaveTok];
  auto load_am = [&](int chunk, v4u (&dst)[kWaveTok]) __attribute__((always_inline)) {
    chunk = min(chunk, P.nch - 1);
#pragma unroll
    for (int tt = 0; tt < kWaveTok; tt++)
      dst[tt] = *(const v4u*)(work + P.xm + (size_t)((tile0 + tt) * P.nch + chunk) * 1024 + lane * 16);
  };
  if (K::MIN) load_am(st0 >> 2, am);
  uint32_t mrec[kWaveRows][4];
#pragma unroll
  for (int rt = 0; rt < kWaveRows; rt++)
#pragma unroll
    for (int q = 0; q < 4; q++) mrec[rt][q] = 0;

  // One stage of the reduction, stage C (static) of its 256-value chunk: x
  // from LDS buffer C % 2, weights from rw.  Stages past st1 (the tail of a
  // short last chunk) run on clamped loads and count with factor zero.
  auto stage = [&](auto cc, int st, const typename K::Raw (&rw)[kWaveRows]) __attribute__((always_inline)) {
    constexpr int C = decltype(cc)::value;
    const bool live = st < st1;
    if constexpr (K::MIN != 0 && C == 0) load_am((st >> 2) + 1, am_next);
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      v8h b0[kWaveRows], b1[kWaveRows];
#pragma unroll
      for (int rt = 0; rt < kWaveRows; rt++) K::codes(rw[rt], C, s4, kh, b0[rt], b1[rt]);
#pragma unroll
      for (int tt = 0; tt < kWaveTok; tt++) {
        const uint8_t* base = &xl[C & 1][((tt * 4 + s4) * 2) * 1024 + lane * 16];
        const v8h ahi = as_v8h4(*(const v4u*)base), alo = as_v8h4(*(const v4u*)(base + 1024));
#pragma unroll
        for (int rt = 0; rt < kWaveRows; rt++) {
          acc[rt][tt] = mfma(ahi, b0[rt], acc[rt][tt]);
          acc[rt][tt] = mfma(alo, b0[rt], acc[rt][tt]);
          if constexpr (K::LIMBS == 2) acc[rt][tt] = mfma(ahi, b1[rt], acc[rt][tt]);
        }
      }
      if constexpr (K::GROUP == 32) {
       if (s4 & 1) {  // a 32-value block ends
        const int bb = s4 >> 1;
#pragma unroll
        for (int rt = 0; rt < kWaveRows; rt++) {
          const float dv = live ? K::d(rw[rt], bb) : 0.0f;
#pragma unroll
          for (int tt = 0; tt < kWaveTok; tt++) {
            tot[rt][tt] += dv * acc[rt][tt];
            acc[rt][tt] = zero;
          }
          if constexpr (K::MIN == 2) {
            const int slot = 2 * C + bb;  // block of the chunk
            const uint32_t mb = live ? K::mbits(rw[rt], bb) : 0u;
            mrec[rt][slot >> 1] = (slot & 1) ? (mrec[rt][slot >> 1] | (mb << 16)) : mb;
          }
        }
       }
      }
    }
    if constexpr (K::GROUP == 256) {
     if constexpr (C == 3) {  // a superblock ends
#pragma unroll
      for (int rt = 0; rt < kWaveRows; rt++) {
        const float dv = K::d(rw[rt]);
        const float dm = K::dmin(rw[rt]);
        const v8h bm = K::mins(rw[rt]);
#pragma unroll
        for (int tt = 0; tt < kWaveTok; tt++) {
          tot[rt][tt] += dv * acc[rt][tt];
          acc[rt][tt] = zero;
          if constexpr (K::MIN == 1) {
            const v16f mn = mfma(as_v8h4(am[tt]), bm, zero);
            tot[rt][tt] -= (32.0f * dm) * mn;
          }
        }
      }
     }
    }
    if constexpr (K::MIN == 2) {
     if constexpr (C == 3) {  // a chunk of eight blocks ends
#pragma unroll
      for (int rt = 0; rt < kWaveRows; rt++) {
        const v8h bm = as_v8h(make_uint4(mrec[rt][0], mrec[rt][1], mrec[rt][2], mrec[rt][3]));
#pragma unroll
        for (int tt = 0; tt < kWaveTok; tt++) tot[rt][tt] += 32.0f * mfma(as_v8h4(am[tt]), bm, zero);
      }
     }
    }
  };

  // Pipeline, branch-free within a chunk of four stages: stage st + 1's
  // weights and activations are loaded into the other register slot while
  // stage st computes (loads past st1 are clamped to its last stage), the
  // activations then move to the other LDS buffer, and one barrier closes
  // each stage.  st0 is a whole chunk.  Two slots rather than a deeper ring
  // keep a wave under 256 registers, so two blocks share a CU and hide each
  // other's load latency (measured: faster than four slots at one block).
#define PF_ISSUE(ST, RW, XD)                                                           \
  {                                                                                    \
    const int ist = min((ST), st1 - 1);                                                \
    PF_LOAD_X(ist, XD)                                                                 \
    _Pragma("unroll") for (int rt = 0; rt < kWaveRows; rt++) K::load(RW[rt], wrow[rt], ist, kh); \
  }
  PF_ISSUE(st0, raw[0], xr0)
  PF_STORE_X(xr0, 0)
  __syncthreads();
  for (int base = st0; base < st1; base += 4) {
    PF_ISSUE(base + 1, raw[1], xr1)
    stage(std::integral_constant<int, 0>{}, base, raw[0]);
    PF_STORE_X(xr1, 1)
    __syncthreads();
    PF_ISSUE(base + 2, raw[0], xr0)
    stage(std::integral_constant<int, 1>{}, base + 1, raw[1]);
    PF_STORE_X(xr0, 0)
    __syncthreads();
    PF_ISSUE(base + 3, raw[1], xr1)
    stage(std::integral_constant<int, 2>{}, base + 2, raw[0]);
    PF_STORE_X(xr1, 1)
    __syncthreads();
    PF_ISSUE(base + 4, raw[0], xr0)
    stage(std::integral_constant<int, 3>{}, base + 3, raw[1]);
    if (K::MIN) {
#pragma unroll
      for (int tt = 0; tt < kWaveTok; tt++) am[tt] = am_next[tt];
    }
    PF_STORE_X(xr0, 0)
    __syncthreads();
  }
#undef PF_ISSUE
#undef PF_LOAD_X
#undef PF_STORE_X

  // results: element j of tile (rt, tt) is token 32 (tile0 + tt) + 8 (j / 4) +
  // 4 kh + j % 4, row row_base + 32 rt + n
  const float* xs = (const float*)(work + P.xs);
#pragma unroll
  for (int tt = 0; tt < kWaveTok; tt++) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const int t = (tile0 + tt) * 32 + 8 * (j >> 2) + 4 * kh + (j & 3);
      if (t >= tokens) continue;
      const float sc = xs[t];
#pragma unroll
      for (int rt = 0; rt < kWaveRows; rt++) {
        const int r = row_base + rt * 32 + n;
        if (r >= rows) continue;
        const float v = tot[rt][tt][j] * sc;
        if (part) part[((size_t)blockIdx.z * tokens + t) * rows + r] = v;
        else mv::epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
      }
    }
  }
}

// Adds the splits' partial sums in split order and applies the epilogue.
__global__ __launch_bounds__(256) void prefill_reduce_kernel(const float* __restrict__ part, int splits, int rows,
                                                             int tokens, float* __restrict__ y, int64_t ldy, int epi,
                                                             const float* __restrict__ aux) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n = (int64_t)rows * tokens;
  if (i >= n) return;
  float v = part[i];
  for (int z = 1; z < splits; z++) v += part[z * n + i];
  const int t = (int)(i / rows), r = (int)(i - (int64_t)t * rows);
  mv::epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
}

constexpr int kWaves = 4;
// Wave tile shapes: (row tiles, token tiles) of 32.  2 x 2 (64 rows x 64
// tokens) or 1 x 4 (32 rows x 128 tokens: each decoded weight serves twice
// the tokens, the block's activation stage is twice as large).
struct Shape {
  int rt, tt;
  int block_rows() const { return kWaves * rt * 32; }
};
// Measured at 256 tokens: Q6_K (three products per step, the heavier
// decode) gains from 1 x 4 (4096x14336: 152 against 208 us); Q4_K loses
// (14336x4096: 140 against 108 us: 195 registers a wave, one wave per SIMD).
Shape shape_for(int kind, int tokens) {
  if (kind == MI_Q6_K && tokens > 64) return Shape{1, 4};
  return Shape{2, 2};
}

template <int KIND>
int launch_kind(hipStream_t s, const RowSegs& sg, int cols, int tokens, const void* work, int splits, int sps,
                float* y, int64_t ldy, int epi, const float* aux, float* part) {
  const Prep P = prep_layout(cols, tokens);
  const int rows = sg.end[sg.nseg - 1];
  const Shape sh = shape_for(KIND, tokens);
  const int tiles = (tokens + kTileTok - 1) / kTileTok;
  dim3 grid((rows + sh.block_rows() - 1) / sh.block_rows(), (tiles + sh.tt - 1) / sh.tt, splits);
  (void)P;
  if constexpr (KIND == MI_Q6_K) {
    if (sh.tt == 4) {
      hipLaunchKernelGGL((prefill_kernel<KIND, kWaves, 1, 4>), grid, dim3(kWaves * 64), 0, s, sg, cols, tokens,
                         (const uint8_t*)work, sps, y, ldy, epi, aux, splits > 1 ? part : nullptr);
      return hip_check(hipGetLastError(), "prefill launch");
    }
  }
  hipLaunchKernelGGL((prefill_kernel<KIND, kWaves, 2, 2>), grid, dim3(kWaves * 64), 0, s, sg, cols, tokens,
                     (const uint8_t*)work, sps, y, ldy, epi, aux, splits > 1 ? part : nullptr);
  return hip_check(hipGetLastError(), "prefill launch");
}

// Splits of K (in whole 256-value chunks): the largest power of two whose
// blocks still fit one round of the chip's block slots (two blocks per CU on
// 256 CUs), each split at least one chunk.  A partial second round costs more
// than fewer, longer blocks: measured at 256 tokens, 14336x4096 runs in
// 110 us at 2 splits (448 blocks) against 125 us at 4, while 4096x14336 wants
// 8 (512 blocks: 212 us) over 4 (232 us).
constexpr int kBlockSlots = 2 * 256;
int choose_splits(int kind, int rows, int cols, int tokens) {
  const Prep P = prep_layout(cols, tokens);
  const Shape sh = shape_for(kind, tokens);
  const int tiles = (tokens + kTileTok - 1) / kTileTok;
  const int64_t blocks = (int64_t)((rows + sh.block_rows() - 1) / sh.block_rows()) * ((tiles + sh.tt - 1) / sh.tt);
  (void)P;
  const int chunks = (cols + kChunk - 1) / kChunk;
  int s = 1;
  while (blocks * 2 * s <= kBlockSlots && chunks >= 2 * s) s *= 2;
  return s;
}

}  // namespace

bool prefill_fits(int kind, int32_t cols, int64_t row_bytes, const void* w) {
  if (cols % kStage) return false;
  switch (kind) {
    case MI_Q4_K:
    case MI_Q5_K:
      return cols % 256 == 0 && ((uintptr_t)w & 15) == 0 && row_bytes % 16 == 0;
    case MI_Q6_K:
      return cols % 256 == 0 && ((uintptr_t)w & 1) == 0 && row_bytes % 2 == 0;
    case MI_Q4_1:
      return ((uintptr_t)w & 3) == 0 && row_bytes % 4 == 0;
    case MI_Q5_1:
      return ((uintptr_t)w & 7) == 0 && row_bytes % 8 == 0;
    case MI_Q8_0:
    case MI_Q4_0:
    case MI_Q5_0:
      return ((uintptr_t)w & 1) == 0 && row_bytes % 2 == 0;
  }
  return false;
}

size_t prefill_workspace(int32_t rows, int32_t cols, int32_t tokens) {
  const Prep P = prep_layout(cols, tokens);
  int splits = 1;
  for (int k : {MI_Q4_K, MI_Q6_K}) splits = std::max(splits, rows > 0 ? choose_splits(k, rows, cols, tokens) : 1);
  size_t part = splits > 1 ? (size_t)splits * tokens * rows * 4 : 0;
  return P.total + ((part + 255) & ~(size_t)255);
}

size_t prefill_prep_bytes(int32_t cols, int32_t tokens) { return prep_layout(cols, tokens).total; }

int prefill_prepare(hipStream_t s, const float* x, int32_t cols, int32_t tokens, void* work) {
  const Prep P = prep_layout(cols, tokens);
  hipLaunchKernelGGL(prefill_scale_kernel, dim3(P.ttp * kTileTok), dim3(256), 0, s, x, cols, tokens,
                     (uint8_t*)work);
  hipLaunchKernelGGL(prefill_x_kernel, dim3(P.nch, P.ttp), dim3(256), 0, s, x, cols, tokens, (uint8_t*)work);
  return hip_check(hipGetLastError(), "prefill activation launch");
}

int launch_prefill_segs(hipStream_t s, int kind, const RowSegs& sg, int32_t cols, int32_t tokens, float* y,
                        int64_t ldy, int32_t epi, const float* aux, void* work, size_t work_bytes) {
  const Prep P = prep_layout(cols, tokens);
  const int rows = sg.end[sg.nseg - 1];
  int splits = choose_splits(kind, rows, cols, tokens);
  const size_t need = (size_t)splits * tokens * rows * 4;
  if (splits > 1 && work_bytes < P.total + need) splits = 1;  // no room for partial sums
  const int nst = cols / kStage;
  int sps = (nst + splits - 1) / splits;
  sps = (sps + 3) & ~3;  // whole 256-value chunks
  splits = (nst + sps - 1) / sps;
  float* part = (float*)((uint8_t*)work + P.total);
  int rc;
  switch (kind) {
    case MI_Q4_K: rc = launch_kind<MI_Q4_K>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q5_K: rc = launch_kind<MI_Q5_K>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q6_K: rc = launch_kind<MI_Q6_K>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q8_0: rc = launch_kind<MI_Q8_0>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q4_0: rc = launch_kind<MI_Q4_0>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q4_1: rc = launch_kind<MI_Q4_1>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q5_0: rc = launch_kind<MI_Q5_0>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    case MI_Q5_1: rc = launch_kind<MI_Q5_1>(s, sg, cols, tokens, work, splits, sps, y, ldy, epi, aux, part); break;
    default: return fail(MI_ERR_KIND, "prefill: ggml type %d has no tile", kind);
  }
  if (rc || splits == 1) return rc;
  const int64_t n = (int64_t)rows * tokens;
  hipLaunchKernelGGL(prefill_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, splits, rows,
                     tokens, y, ldy, epi, aux);
  return hip_check(hipGetLastError(), "prefill reduce launch");
}

int launch_prefill(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                   const float* x, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux, void* work,
                   size_t work_bytes) {
  int rc = prefill_prepare(s, x, cols, tokens, work);
  if (rc) return rc;
  return launch_prefill_segs(s, kind, rows::one_matrix(w, row_bytes, rows), cols, tokens, y, ldy, epi, aux, work,
                             work_bytes);
}

}  // namespace mi

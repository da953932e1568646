// matvec_htile.hip -- the batched (2..8 tokens) Q4_K and Q6_K matvec on the
// f16 matrix cores (v_mfma_f32_16x16x32_f16), gfx950.
//
// The int8 tile (matvec_tile.hip) multiplies exactly but has to recombine
// three activation limbs per (row, token, group) on the VALU afterwards.
// This tile feeds the matrix core half-precision numbers that are exact, so
// everything after the MFMA is one scale per superblock:
//
//  * Activations ("hx" form, written next to the xq form by its producers,
//    xq_device.h quantize_group32): the xq integers X of a group split into
//    two halves hi + lo = X * 2^-8 exactly (X has at most 22 significant
//    bits; hi carries the top 11, lo the rest).  The tile rescales each
//    group to its superblock's largest group scale (a power of two, so exact
//    while the group is within 2^16 of the largest).
//  * Weights enter as the integer codes sc * q (at most 63 * 15), exact in
//    half precision, so every product is exact and d scales the superblock's
//    sum once.
//  * The min term dmin * sum_g m_g * sum(x in group g) is one more MFMA per
//    superblock: the 8 mins of a row against the 8 group sums of each column
//    (each sum divided by 256 and split into two halves, hi and lo, so 16 of
//    the 32 k slots).
//
// MFMA fragments (16x16x32): lane l holds row / column l % 16 and values
// 8 (l / 16) .. +8 of the 32; result element i of lane l is row 4 (l / 16) +
// i, column l % 16.  Here M = 16 rows of the tile, N = 16 columns: token t
// hi (2t) and lo (2t + 1), K = the 32 values of one Q4_K group (group 2h + e
// of a superblock is the low (e = 0) or high nibbles of bytes 32h..32h+31;
// lane l supplies bytes 32h + 8 (l / 16) .. +8).
//
// Work decomposition: a block is cols / 512 waves, wave w owning superblocks
// 2w, 2w + 1 (512 values) of every row: it builds its activation fragments
// once and keeps them in registers for every tile the block takes.  Blocks
// loop over 16-row tiles (tile, tile + gridDim.x, ...).  A tile's 16 rows are
// one run of memory: the block reads it with contiguous loads into LDS (a
// fragment read straight from memory touches 16 rows per instruction, a
// part of a cache line each, at about half the speed), keeping the next
// tile's weights in flight while it computes the current one.  The waves'
// partial sums meet in LDS, where 16 * tokens (row, token) sums add them in
// a fixed order and apply the epilogue.
//
// Q6_K (sb_product_q6k) has no min term; its codes need two MFMAs a group.
//
// Replaces the batched planar_matmul_kernel (src/molla/nn/gpu.mojo:1809) for
// Q4_K and Q6_K; output y[t * ldy + r] and epilogues as gpu.mojo:1005.
#include <type_traits>

#include "matvec_rows.h"

namespace mi {
namespace {
using namespace mv;

typedef _Float16 hh8 __attribute__((ext_vector_type(8)));
typedef _Float16 hh2 __attribute__((ext_vector_type(2)));
typedef float ff4 __attribute__((ext_vector_type(4)));
typedef uint32_t uu4 __attribute__((ext_vector_type(4)));
struct __attribute__((aligned(4))) U2a {
  uint32_t x, y;
};

constexpr int kSBW = 2;                                  // superblocks per wave
constexpr int kMaxHWaves = 8;                            // cols <= 8 * 512
constexpr int kMaxRopePairs = 128;                       // rope_dim <= 256 for the rope epilogue

// Per kind: superblock bytes, and the LDS row stride of a tile (the row at
// 4096 columns, so that a fragment read's 16 rows start 8 banks apart: Q4_K
// rows of 2304 bytes take 32 bytes of padding, Q6_K rows of 3360 bytes are
// 8 banks apart already).
template <int KIND>
struct HGeo;
template <>
struct HGeo<MI_Q4_K> {
  static constexpr int SB = 144, ROW = kMaxHWaves * kSBW * 144 + 32;
};
template <>
struct HGeo<MI_Q6_K> {
  static constexpr int SB = 210, ROW = kMaxHWaves * kSBW * 210;
};
constexpr int kTileBuf = 16 * HGeo<MI_Q6_K>::ROW;  // one tile buffer, the larger kind
// 8-byte loads per lane per tile: a tile is 16 rows of cols / 256
// superblocks, a block cols / 8 lanes, so SB / 16 words a lane
template <int KIND>
constexpr int kLoadsOf = (HGeo<KIND>::SB + 15) / 16;

__device__ __forceinline__ ff4 mfma16(hh8 a, hh8 b, ff4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ hh8 as_hh8(uint4 u) { return __builtin_bit_cast(hh8, u); }
__device__ __forceinline__ hh2 as_hh2(uint32_t u) { return __builtin_bit_cast(hh2, u); }
__device__ __forceinline__ uint32_t as_u32(hh2 h) { return __builtin_bit_cast(uint32_t, h); }

// Two bytes of x (picked by the perm selector) as the halves 1024 + byte:
// 0x64 above a byte is the exponent of 1024, the byte the mantissa.
__device__ __forceinline__ uint32_t magic2(uint32_t x, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, x, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;
__device__ __forceinline__ uint32_t sel_splat(int k) { return 0x04000400u | ((uint32_t)k << 16) | (uint32_t)k; }

// sc * u for the eight nibble codes u in the bytes of t0, t1: (1024 + u) *
// sc - 1024 * sc, one rounding of an exact small integer.
__device__ __forceinline__ hh8 codes8(uint32_t t0, uint32_t t1, hh2 sc, hh2 nsc) {
  uint4 o;
  o.x = as_u32(__builtin_elementwise_fma(as_hh2(magic2(t0, kSel01)), sc, nsc));
  o.y = as_u32(__builtin_elementwise_fma(as_hh2(magic2(t0, kSel23)), sc, nsc));
  o.z = as_u32(__builtin_elementwise_fma(as_hh2(magic2(t1, kSel01)), sc, nsc));
  o.w = as_u32(__builtin_elementwise_fma(as_hh2(magic2(t1, kSel23)), sc, nsc));
  return as_hh8(o);
}

// The 6-bit scales and mins of groups 0..7 from scales[0..11] held in y, z,
// w (quant.mojo:161 _k_scale), four to a dword: sc0..3, sc4..7, m0..3, m4..7.
__device__ __forceinline__ void kscales(uint32_t y, uint32_t z, uint32_t w, uint32_t& sc_lo, uint32_t& sc_hi,
                                        uint32_t& m_lo, uint32_t& m_hi) {
  sc_lo = y & 0x3F3F3F3Fu;
  m_lo = z & 0x3F3F3F3Fu;
  sc_hi = (w & 0x0F0F0F0Fu) | ((y >> 2) & 0x30303030u);
  m_hi = ((w >> 4) & 0x0F0F0F0Fu) | ((z >> 2) & 0x30303030u);
}

// The partial product of superblock `sb` of the 16 rows in LDS (lrows: row
// 0 of the tile) for this lane's result rows 4 kq + i, column lm:
// esc * (d * C - dmin * Cmin).  bm is this lane's fragment of the group sums
// (the min MFMA's B), which are held divided by 256.
__device__ __forceinline__ void sb_product(const uint8_t* lrows, int sb, const hh8 (&b)[8], hh8 bm, float esc,
                                           int lm, int kq, ff4& acc) {
  constexpr int kLdsRow = HGeo<MI_Q4_K>::ROW;
  const uint8_t* lrow = lrows + lm * kLdsRow + sb * 144;
  const uint4 h = *(const uint4*)lrow;
  uint2 q[4];
#pragma unroll
  for (int k = 0; k < 4; k++) q[k] = *(const uint2*)(lrow + 16 + 32 * k + 8 * kq);
  uint32_t dd[4];
#pragma unroll
  for (int i = 0; i < 4; i++) dd[i] = *(const uint32_t*)(lrows + (4 * kq + i) * kLdsRow + sb * 144);

  uint32_t sc_lo, sc_hi, m_lo, m_hi;
  kscales(h.y, h.z, h.w, sc_lo, sc_hi, m_lo, m_hi);
  const hh2 k1024 = {(_Float16)-1024.0f, (_Float16)-1024.0f};
  // the 8 scales as pairs (sc 2i, sc 2i + 1 / 16) and their negated 1024
  // multiples; a group takes one half of its pair to both halves.  An odd
  // group's codes are the high nibbles left in place (16 u, one AND instead
  // of a shift and an AND), so its scale is a sixteenth: 0x54 above the
  // byte is the exponent of 64, whose half step is 1/16, and (1024 + 16 u)
  // sc / 16 - 64 sc = u sc is one exact rounding, as for the even groups.
  const hh2 kOff = {(_Float16)-1024.0f, (_Float16)-64.0f};
  constexpr uint32_t kScSel01 = 0x07010400u, kScSel23 = 0x07030402u;
  hh2 scp[4], nscp[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    scp[i] = as_hh2(__builtin_amdgcn_perm(0x54646464u, i < 2 ? sc_lo : sc_hi, (i & 1) ? kScSel23 : kScSel01)) + kOff;
    nscp[i] = scp[i] * k1024;
  }
  ff4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const hh2 sc = (j & 1) ? __builtin_shufflevector(scp[j >> 1], scp[j >> 1], 1, 1)
                           : __builtin_shufflevector(scp[j >> 1], scp[j >> 1], 0, 0);
    const hh2 nsc = (j & 1) ? __builtin_shufflevector(nscp[j >> 1], nscp[j >> 1], 1, 1)
                            : __builtin_shufflevector(nscp[j >> 1], nscp[j >> 1], 0, 0);
    const uint32_t t0 = q[j >> 1].x, t1 = q[j >> 1].y;
    const uint32_t u0 = t0 & ((j & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
    const uint32_t u1 = t1 & ((j & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
    c = mfma16(codes8(u0, u1, sc, nsc), b[j], c);
  }
  // the mins of groups 0..7 as this lane's A fragment: k 0..7 and 8..15
  // (the hi and lo group sums) both take m0..m7
  const uint4 am = make_uint4(magic2(m_lo, kSel01), magic2(m_lo, kSel23), magic2(m_hi, kSel01),
                              magic2(m_hi, kSel23));
  const _Float16 n = (_Float16)-1024.0f;
  // (lanes kq >= 2 hold k 16..31, where bm is zero: their finite mins add
  // nothing, so they are not cleared)
  const hh8 a_m = as_hh8(am) + hh8{n, n, n, n, n, n, n, n};
  const ff4 cm = mfma16(a_m, bm, ff4{0.0f, 0.0f, 0.0f, 0.0f});
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float di = half_bits_to_float(dd[i]), mi_ = half_bits_to_float(dd[i] >> 16);
    acc[i] = fmaf(esc, fmaf(mi_, cm[i] * -256.0f, di * c[i]), acc[i]);
  }
}

// The same for a Q6_K superblock (ql[128], qh[64], int8 scales[16], f16 d:
// quant.mojo Q6_K; value 32 g + l of a group g of half h = g / 4 takes the low
// (g & 2 = 0) or high nibble of ql[64 h + 32 (g & 1) + l] and bits 2 (g & 3)
// of qh[32 h + l], minus 32, times scale 2 g + l / 16).  sc * (q - 32)
// reaches 4096, past exact halves, so the scale splits into 16 s_hi + s_lo
// and each group is two MFMAs of exact codes (b - 32) s_hi and (b - 32) s_lo.
// Superblocks of 210 bytes sit packed in LDS: one of odd index S starts 2
// bytes past a dword, so its fields are read as dwords and realigned.
template <int S>
__device__ __forceinline__ void sb_product_q6k(const uint8_t* lrows, int sb, const hh8 (&b)[8], float esc,
                                               int lm, int kq, ff4& acc) {
  constexpr int kLdsRow = HGeo<MI_Q6_K>::ROW;
  const uint8_t* p = lrows + lm * kLdsRow + sb * 210;  // 4-aligned + 2 S
  auto ld8 = [&](int off) __attribute__((always_inline)) {
    const uint32_t* a = (const uint32_t*)(p + off - 2 * S);
    if constexpr (S == 0) return make_uint2(a[0], a[1]);
    else return make_uint2(__builtin_amdgcn_alignbyte(a[1], a[0], 2), __builtin_amdgcn_alignbyte(a[2], a[1], 2));
  };
  uint2 ql[2][2], qh[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    ql[h][0] = ld8(64 * h + 8 * kq);
    ql[h][1] = ld8(64 * h + 32 + 8 * kq);
    qh[h] = ld8(128 + 32 * h + 8 * kq);
  }
  uint32_t scw[4];
  {
    const uint32_t* a = (const uint32_t*)(p + 192 - 2 * S);
#pragma unroll
    for (int j = 0; j < 4; j++) scw[j] = S == 0 ? a[j] : __builtin_amdgcn_alignbyte(a[j + 1], a[j], 2);
  }
  float dd[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t w = *(const uint32_t*)(lrows + (4 * kq + i) * kLdsRow + sb * 210 + 208 - 2 * S);
    dd[i] = half_bits_to_float(S == 0 ? w : w >> 16);
  }
  const int kh = kq >> 1;  // which 16-value sub-block of a group this lane's values are in
  ff4 ch = {0.0f, 0.0f, 0.0f, 0.0f}, cl = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int g = 0; g < 8; g++) {
    const int h = g >> 2, qq = g & 3;
    const uint32_t t0 = ql[h][qq & 1].x, t1 = ql[h][qq & 1].y;
    const uint32_t n0 = (qq >> 1) ? (t0 >> 4) & 0x0F0F0F0Fu : t0 & 0x0F0F0F0Fu;
    const uint32_t n1 = (qq >> 1) ? (t1 >> 4) & 0x0F0F0F0Fu : t1 & 0x0F0F0F0Fu;
    const uint32_t b0 = n0 | (((qh[h].x >> (2 * qq)) & 0x03030303u) << 4);
    const uint32_t b1 = n1 | (((qh[h].y >> (2 * qq)) & 0x03030303u) << 4);
    const int sc = __builtin_amdgcn_sbfe((int)scw[g >> 1], 8 * (2 * (g & 1) + kh), 8);
    const _Float16 fh = (_Float16)(float)(sc >> 4), fl = (_Float16)(float)(sc & 15);
    const hh2 shi = {fh, fh}, slo = {fl, fl};
    const hh2 k1056 = {(_Float16)-1056.0f, (_Float16)-1056.0f};
    ch = mfma16(codes8(b0, b1, shi, shi * k1056), b[g], ch);
    cl = mfma16(codes8(b0, b1, slo, slo * k1056), b[g], cl);
  }
#pragma unroll
  for (int i = 0; i < 4; i++) acc[i] = fmaf(esc * dd[i], fmaf(16.0f, ch[i], cl[i]), acc[i]);
}

// GLU (Q4_K): sg holds gate (rows 0 .. end[0]) and up (end[0] .. end[1]);
// a block takes 32-row groups, each as four tiles (gate rows 0-15, up rows
// 0-15, gate rows 16-31, up rows 16-31), and writes act(gate) * up of each
// group only in matvec form, into xq_out (the down projection's input;
// gpu_block.mojo device_swiglu then the quantize), one half-wave a token.
// ROPE (Q4_K, q|k|v rows): the epilogue of the batched int8 tile's rope form
// (matvec_tile.hip): rows of q and k rotated in adjacent pairs at each
// token's position, q to y, k and v to the f16 caches (rp).
// SPLIT: the split-K form (block row blockIdx.y reads a column part of
// longer rows); the tile's rows are then not one run of memory.
// COPY (SPLIT): the blocks also copy aux[0 .. ysplit) (the residual row the
// parts are added to) into the slot after the last part, one value a
// thread, so that the launch which adds the parts can write the residual
// in place while every block of it still reads the old values.
template <int TN, int KIND, bool GLU, bool ROPE = false, bool SPLIT = false, bool COPY = false>
__global__ __launch_bounds__(kMaxHWaves * 64) void htile_kernel(const RowSegs sg, int cols,
                                                                     const uint8_t* __restrict__ xq,
                                                                     const uint8_t* __restrict__ hx,
                                                                     float* __restrict__ y, int64_t ldy, int epi,
                                                                     const float* __restrict__ aux,
                                                                     uint8_t* __restrict__ xq_out, int gtot,
                                                                     int64_t ysplit, const QkvRope rp) {
  constexpr int SB = HGeo<KIND>::SB, kLdsRow = HGeo<KIND>::ROW, kLoads = kLoadsOf<KIND>;
  __shared__ __align__(16) uint8_t wl[2][kTileBuf];
  __shared__ float part[2][kMaxHWaves][16][17];
  __shared__ __align__(16) uint8_t sink[16];  // target of the copies' idle lanes
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int lm = lane & 15, kq = lane >> 4;
  const int rows = sg.end[sg.nseg - 1];
  const int tiles = (rows + 15) >> 4;
  // Split K: block row blockIdx.y takes columns [y cols, (y + 1) cols) of
  // rows gtot * 32 long and writes its partial sums ysplit floats further on.
  const int G = cols >> 5, g0 = (int)blockIdx.y * G;
  const int rb = (cols >> 8) * SB;  // bytes of a row this block reads
  const int64_t rstride = sg.rb[0];  // bytes between rows (every segment's)
  const int64_t tok_bytes = xq_token_bytes(gtot * 32);
  y += (int64_t)blockIdx.y * ysplit;
  const int step = gridDim.x;
  // the k-th tile of this block: tile blockIdx.x + k step, or under GLU tile
  // k % 4 of 32-row group blockIdx.x + (k / 4) step
  const int gl_rows = GLU ? sg.end[0] : 0, jobs = gl_rows >> 5;
  auto tile_of = [&](int kk) __attribute__((always_inline)) {
    if constexpr (GLU) {
      const int j = blockIdx.x + (kk >> 2) * step, q = kk & 3;
      return (q & 1) * (gl_rows >> 4) + 2 * j + (q >> 1);
    } else {
      return (int)blockIdx.x + kk * step;
    }
  };
  auto valid = [&](int kk) __attribute__((always_inline)) {
    if constexpr (GLU) return (int)blockIdx.x + (kk >> 2) * step < jobs;
    else return (int)blockIdx.x + kk * step < tiles;
  };

  // This lane's share of a tile: 8-byte words threadIdx.x + blockDim.x * j,
  // and where each lands in the padded LDS rows.
  int ldso[kLoads];
  // Q4_K (and the split form): each word's byte offset from row 0 of the
  // tile, clamped per tile with one min; Q6_K keeps the word index (the
  // offsets cost its 8-token form 34 spilled VGPRs, 133 -> 210 us on the head)
  constexpr bool kOff = SPLIT || KIND == MI_Q4_K;
  uint32_t wfull[kOff ? kLoads : 1];
#pragma unroll
  for (int j = 0; j < kLoads; j++) {
    // o / rb through a float reciprocal (o < 2^16: exact after one
    // correction), not the long integer division sequence.  A lane past the
    // tile's last word (Q6_K's ragged last round) stores that word again
    // where it belongs.
    const int o = 8 * min((int)threadIdx.x + (int)blockDim.x * j, 2 * rb - 1);
    int row = (int)((float)o * (1.0f / (float)rb));
    row -= row * rb > o;
    row += (row + 1) * rb <= o;
    ldso[j] = row * kLdsRow + (o - row * rb);
    if constexpr (kOff) wfull[j] = (uint32_t)row * (uint32_t)rstride + (uint32_t)(o - row * rb);
  }
  (void)rstride;
  // A last tile of fewer than 16 rows reads its last word again in place of
  // the missing rows (whose sums are never stored): loads stay unconditional.
  auto load_tile = [&](uint2 (&r)[kLoads], int tl) __attribute__((always_inline)) {
    if constexpr (kOff) {
      const uint8_t* src = rows::seg_row(sg, tl * 16) + (int64_t)blockIdx.y * rb;
      // a word of a missing row reads the last word of the last row
      const uint32_t lastw = (uint32_t)(min(16, rows - tl * 16) - 1) * (uint32_t)rstride + (uint32_t)(rb - 8);
#pragma unroll
      for (int j = 0; j < kLoads; j++) {
        const U2a v = *(const U2a*)(src + min(wfull[j], lastw));  // 4-byte aligned (Q6_K parts)
        r[j] = make_uint2(v.x, v.y);
      }
    } else {
      const uint2* src = (const uint2*)rows::seg_row(sg, tl * 16);
      const int words = min(16, rows - tl * 16) * (rb >> 3);
#pragma unroll
      for (int j = 0; j < kLoads; j++) r[j] = src[min((int)threadIdx.x + (int)blockDim.x * j, words - 1)];
    }
  };
  auto store_tile = [&](const uint2 (&r)[kLoads], int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kLoads; j++) *(uint2*)(wl[buf] + ldso[j]) = r[j];
  };

  // Activation fragments: token t = lm / 2, hi (lm even) or lo, groups of
  // the wave's superblocks; columns of absent tokens are zero.  The block
  // copies the group scales and the whole hx form into registers with
  // contiguous loads, all issued before tile 0's weights (loads queue in
  // order, and these are the ones the first tile waits for), then passes
  // them through LDS in chunks of `cw` waves' superblocks that fit the
  // weight buffers' space; each lane reads its fragments there.  (Per-lane
  // gathers of the fragments straight from memory, or a copy loop that
  // waits on each load, cost several times longer.)
  static_assert(!COPY || SPLIT, "COPY is a split-K form");
  float cpv = 0.0f;
  int64_t cpi = 0;
  if constexpr (COPY) {
    // sent for first: the store below, after the first weight loads, then
    // waits for this load only
    cpi = min((int64_t)(blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x, ysplit - 1);
    cpv = aux[cpi];
  }
  const int t = lm >> 1, part_hl = lm & 1;
  const bool live_col = t < TN;
  const int wave_bytes = kSBW * 8 * 128;  // one token's hx for one wave
  // 16-byte word tid + j * blockDim.x of the block's hx is word tid +
  // (j & 1) * blockDim.x of token j / 2 (a token is 2 * blockDim.x words)
  uu4 v[2 * TN];
#pragma unroll
  for (int j = 0; j < 2 * TN; j++) {
    const int u = j >> 1, w = (int)threadIdx.x + (j & 1) * (int)blockDim.x;
    v[j] = *(const uu4*)(hx + u * tok_bytes + g0 * 128 + w * 16);
  }
  const float* scale_src = &((const XMeta*)(xq + 6 * (int64_t)gtot * 16 + g0 * 16))->scale;
  float scl[TN];  // thread g < G: group g's scale of every token
  const int sg_g = min((int)threadIdx.x, G - 1);
#pragma unroll
  for (int u = 0; u < TN; u++) scl[u] = scale_src[u * (tok_bytes / 4) + sg_g * 4];
  uint2 ra[kLoads], rb_[kLoads];
  load_tile(ra, tile_of(0));  // the grid is at most `tiles` (GLU: groups) blocks
  if constexpr (COPY) y[(int64_t)(gridDim.y - blockIdx.y) * ysplit + cpi] = cpv;
  // A block with more tiles than this one sends for tile 1 only after its
  // prologue: the prologue's own loads then compete with fewer weight loads
  // of the whole chip (14336 rows at 4 tokens: 16.4 against 17.5 us).  Split
  // K and GLU blocks always have more.
  const bool late1 = GLU || tiles > (int)gridDim.x;
  if (!late1 && valid(1)) load_tile(rb_, tile_of(1));

  hh8 b[kSBW][8];
  float sc8[kSBW][8];
  {
    float* lsc = (float*)part;  // TN * G scales; part is free until the first tile
#pragma unroll
    for (int u = 0; u < TN; u++) *((int)threadIdx.x < G ? &lsc[u * G + threadIdx.x] : (float*)sink) = scl[u];
    const int cw = min(nw, (int)sizeof(wl) / (TN * (wave_bytes + 128)));
    for (int w0 = 0; w0 < nw; w0 += cw) {
      const int nwc = min(cw, nw - w0);
      const int tstride = nwc * wave_bytes + 128;  // 128 extra: tokens 32 banks apart
      uint8_t* lhx = &wl[0][0];
      if (w0) __syncthreads();  // the previous chunk has been read
#pragma unroll
      for (int j = 0; j < 2 * TN; j++) {
        const int u = j >> 1;
        const int o = ((int)threadIdx.x + (j & 1) * (int)blockDim.x) * 16 - w0 * wave_bytes;  // inside the chunk
        *(uu4*)(o >= 0 && o < nwc * wave_bytes ? lhx + u * tstride + o : sink) = v[j];
      }
      __syncthreads();
      if (wave >= w0 && wave < w0 + nwc) {
#pragma unroll
        for (int s = 0; s < kSBW; s++)
#pragma unroll
          for (int g = 0; g < 8; g++) {
            sc8[s][g] = live_col ? lsc[t * G + (wave * kSBW + s) * 8 + g] : 0.0f;
            b[s][g] = live_col ? as_hh8(*(const uint4*)(lhx + t * tstride + (wave - w0) * wave_bytes +
                                                        (s * 8 + g) * 128 + (kq * 2 + part_hl) * 16))
                               : hh8{0, 0, 0, 0, 0, 0, 0, 0};
          }
      }
    }
    __syncthreads();  // every fragment read before the buffers take weights
  }
  if (late1 && valid(1)) load_tile(rb_, tile_of(1));
  // Rescale each group to its superblock's largest scale (2^(e_g - e_sb),
  // exact) and form the min MFMA's B: column lm's group sums (divided by
  // 256: a sum reaches 2^19, past the largest half), hi in k 0..7 (lanes
  // kq = 0), lo in k 8..15 (kq = 1), zero above.  A group's column sums come
  // from the matrix core too: a block of ones times the group's fragment.
  float esc[kSBW];
  hh8 bm[kSBW];
  const hh8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
  for (int s = 0; s < kSBW; s++) {
    float emax = 0.0f;
#pragma unroll
    for (int g = 0; g < 8; g++) emax = fmaxf(emax, sc8[s][g]);
    esc[s] = 256.0f * emax;
    const float inv = emax > 0.0f ? __builtin_amdgcn_rcpf(emax) : 0.0f;  // exact: a power of two
    hh8 hv = {}, lv = {};
#pragma unroll
    for (int g = 0; g < 8; g++) {
      const _Float16 f = (_Float16)(sc8[s][g] * inv);
      b[s][g] = b[s][g] * hh8{f, f, f, f, f, f, f, f};
      if constexpr (KIND == MI_Q4_K) {
        const float gs = mfma16(ones, b[s][g], ff4{0.0f, 0.0f, 0.0f, 0.0f})[0] * (1.0f / 256.0f);
        hv[g] = (_Float16)gs;
        lv[g] = (_Float16)(gs - (float)hv[g]);
      }
    }
    if constexpr (KIND == MI_Q4_K) bm[s] = kq == 0 ? hv : (kq == 1 ? lv : hh8{0, 0, 0, 0, 0, 0, 0, 0});
    else bm[s] = hh8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  // (row r, token u) sums of tile kk over the waves, in wave order, hi + lo,
  // and the epilogue.  GLU: a gate tile's sums wait in gsum for the up tile
  // of the same rows, whose act(gate) * up go to hbuf (another wave may
  // finish that tile: a barrier lies between the two finishes).
  __shared__ float gsum[GLU ? 2 : 1][16][TN], hbuf[GLU ? 32 : 1][TN];
  // ROPE: (cos, sin) of every (token, pair), once per block, read by the
  // finish of every tile (computed as rope_theta then float64 trig)
  __shared__ float2 trig[ROPE ? TN * kMaxRopePairs : 1];
  if constexpr (ROPE) {
#pragma clang fp contract(off)
    const int np = rp.rope_dim >> 1;
    for (int i = threadIdx.x; i < TN * np; i += blockDim.x) {
      const int u = i / np, pr = i - u * np;
      const float theta = rope_theta(rp.pos[u], rp.steps, rp.factors, pr);
      trig[u * kMaxRopePairs + pr] = make_float2((float)cos((double)theta), (float)sin((double)theta));
    }
  }
  auto finish = [&](int kk, int buf) __attribute__((always_inline)) {
    // The (row, token) sums of a tile are dealt to as few waves as hold them
    // (F of 64 sums each), a different wave for each tile: the finish's
    // instructions cost a wave that runs them however few of its lanes are
    // live, so spreading a few sums over every wave costs all of them.
    constexpr int F = (16 * TN + 63) / 64;
    int f0 = 0;  // this wave's first share
    if constexpr (F == 1) {
      if (wave != kk % nw) return;
    } else {
      f0 = wave - (kk * F) % nw;
      if (f0 < 0) f0 += nw;
      if (f0 >= F) return;
    }
    const int tl = tile_of(kk);
    for (int ix = f0 * 64 + lane; ix < 16 * TN; ix += (F == 1 ? 64 : 64 * nw)) {
      const int rr = ix & 15, u = ix >> 4;
      // every wave's pair is read unconditionally (a wave past nw reads
      // the last one again and adds nothing), so the reads go out together
      // instead of one LDS round trip per wave behind a branch
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < kMaxHWaves; w++) {
        const int ww = min(w, nw - 1);
        const float h = part[buf][ww][rr][2 * u] + part[buf][ww][rr][2 * u + 1];
        v += w < nw ? h : 0.0f;
      }
      if constexpr (ROPE) {
#pragma clang fp contract(off)
        // the partner row's sum, added in the same order as its own thread's
        float pv = 0.0f;
#pragma unroll
        for (int w = 0; w < kMaxHWaves; w++) {
          const int ww = min(w, nw - 1);
          const float h = part[buf][ww][rr ^ 1][2 * u] + part[buf][ww][rr ^ 1][2 * u + 1];
          pv += w < nw ? h : 0.0f;
        }
        const int r = tl * 16 + rr;
        if (r >= rows) continue;
        // rope.mojo:294 rotate_scaled, adjacent pairs: (a, b) <- (a c - b s, a s + b c)
        const int p = rp.pos[u];
        const bool is_q = r < rp.qw, is_k = !is_q && r < rp.qw + rp.kvw;
        float out = v;
        if (is_q || is_k) {
          const int e = (is_q ? r : r - rp.qw) % rp.head_dim;
          if (e < rp.rope_dim) {
            const float2 cs = trig[u * kMaxRopePairs + (e >> 1)];
            const float c = cs.x, sn = cs.y;
            const float a = (e & 1) ? pv : v, b = (e & 1) ? v : pv;
            out = (e & 1) ? a * sn + b * c : a * c - b * sn;
          }
        }
        if (is_q) {
          y[(int64_t)u * ldy + r] = out;
        } else {
          const int64_t at = rp.kv_index ? (int64_t)rp.kv_index[u * rp.index_stride + p] * rp.kvw
                                         : (int64_t)u * rp.cache_stride + (int64_t)p * rp.kvw;
          if (is_k) rp.k_cache[at + (r - rp.qw)] = __float2half_rn(out);
          else rp.v_cache[at + (r - rp.qw - rp.kvw)] = __float2half_rn(out);
        }
      } else if constexpr (GLU) {
        const int q = kk & 3;
        if (!(q & 1)) {
          gsum[q >> 1][rr][u] = v;
        } else {
          const float g = gsum[q >> 1][rr][u];
          hbuf[16 * (q >> 1) + rr][u] = ((epi & MI_ACT_GELU) ? gelu(g) : silu(g)) * v;
        }
      } else {
        const int row = tl * 16 + rr;
        if (row < rows) epilogue(y, aux, epi, (int64_t)u * ldy + row, row, v);
      }
    }
  };
  // GLU: group kk / 4's 32 act(gate) * up per token into xq_out, a half-wave
  // a token (lane = row); hbuf is complete once a barrier follows its tile's
  // finish, and the next group's first write to it is two tiles later.
  auto quantize_group = [&](int kk) __attribute__((always_inline)) {
    if constexpr (GLU) {
      const int j = blockIdx.x + (kk >> 2) * step;
      for (int u0 = 2 * wave; u0 < TN; u0 += 2 * nw) {  // a block of one wave takes every token
        const int u = u0 + (lane >> 5);
        const int uu = u < TN ? u : 0;
        quantize_group32(hbuf[lane & 31][uu], lane & 31, j, jobs, xq_out + (int64_t)uu * xq_token_bytes(gl_rows),
                         u < TN, (epi & kEpiHx) ? xq_out + (int64_t)(TN + uu) * xq_token_bytes(gl_rows) : nullptr);
      }
    }
  };

  // Tile k of this block is computed from LDS buffer k & 1 while tiles
  // k + 1 and k + 2 are in flight in the two register sets; then tile k + 1
  // goes into the other buffer and its registers send for tile k + 3.  With
  // buffers alternating, one barrier per tile keeps every buffer from being
  // overwritten before it has been read.
  int k = 0;
  store_tile(ra, 0);
  if (valid(2)) load_tile(ra, tile_of(2));
  // P = k & 1, the buffer tile k is computed from: step_tile(rb_) always
  // runs at even k and step_tile(ra) at odd k, so it is a constant of each
  // call and the buffers' LDS addresses fold into the instructions' offsets.
  auto step_tile = [&](uint2 (&rn)[kLoads], auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    __syncthreads();
    if (GLU && k >= 2 && ((k - 2) & 3) == 3) quantize_group(k - 2);
    if (k > 0) finish(k - 1, 1 - P);
    ff4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < kSBW; s++) {
      if constexpr (KIND == MI_Q4_K) {
        sb_product(wl[P], wave * kSBW + s, b[s], bm[s], esc[s], lm, kq, acc);
      } else if (s == 0) {
        sb_product_q6k<0>(wl[P], wave * kSBW, b[0], esc[0], lm, kq, acc);
      } else {
        sb_product_q6k<1>(wl[P], wave * kSBW + 1, b[1], esc[1], lm, kq, acc);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) part[P][wave][4 * kq + i][lm] = acc[i];
    if (!valid(k + 1)) return false;
    store_tile(rn, 1 - P);  // tile k + 1
    if (valid(k + 3)) load_tile(rn, tile_of(k + 3));
    k++;
    return true;
  };
  while (step_tile(rb_, std::integral_constant<int, 0>{}) && step_tile(ra, std::integral_constant<int, 1>{})) {
  }
  __syncthreads();
  finish(k, k & 1);
  if constexpr (GLU) {
    __syncthreads();
    quantize_group(k);
  }
}

// The parts of a split-K htile (part[k][t][r], k < nsplit) added in part
// order, then the epilogue.
__global__ void htile_split_reduce_kernel(const float* __restrict__ part, int nsplit, int tn, int rows,
                                          float* __restrict__ y, int64_t ldy, int epi, const float* __restrict__ aux) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= tn * rows) return;
  const int t = i / rows, r = i - t * rows;
  const int64_t n = (int64_t)tn * rows;
  float v = part[i];
  for (int k = 1; k < nsplit; k++) v += part[k * n + i];
  epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
}


}  // namespace

// A tile is copied in 8-byte words, row by row, so a row must be whole
// words: any number of 144-byte Q4_K superblocks, a multiple of four 210-byte
// Q6_K ones (a Q6_K row of 2, 6, 10 or 14 superblocks would straddle words).
bool htile_fits(int kind, int32_t rows, int32_t cols, int32_t tokens) {
  return (kind == MI_Q4_K || (kind == MI_Q6_K && (cols / 256) % 4 == 0)) && tokens >= 2 &&
         tokens <= kMaxTokens && cols % (256 * kSBW) == 0 && cols / (256 * kSBW) <= kMaxHWaves && rows > 0;
}

int launch_htile(hipStream_t s, int kind, const RowSegs& sg, int32_t rows, int32_t cols, const void* xq,
                 const void* hx, int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  const int sbb = kind == MI_Q6_K ? HGeo<MI_Q6_K>::SB : HGeo<MI_Q4_K>::SB;
  for (int i = 0; i < sg.nseg; i++)
    if ((i < sg.nseg - 1 && sg.end[i] % 16) || sg.rb[i] != (int64_t)(cols / 256) * sbb || ((uintptr_t)sg.w[i] & 7))
      return fail(MI_ERR_SHAPE, "htile: segments must be whole 16-row tiles of %d-column rows, 8-byte aligned", cols);
  const int waves = cols / (256 * kSBW);
  const int grid = std::min((rows + 15) / 16, cu_count());
#define MI_HT(T)                                                                                              \
  case T:                                                                                                     \
    if (kind == MI_Q6_K)                                                                                      \
      hipLaunchKernelGGL((htile_kernel<T, MI_Q6_K, false>), dim3(grid), dim3(waves * 64), 0, s, sg, cols,     \
                         (const uint8_t*)xq, (const uint8_t*)hx, y, ldy, epi, aux, nullptr, cols / 32, 0, QkvRope{}); \
    else                                                                                                      \
      hipLaunchKernelGGL((htile_kernel<T, MI_Q4_K, false>), dim3(grid), dim3(waves * 64), 0, s, sg, cols,     \
                         (const uint8_t*)xq, (const uint8_t*)hx, y, ldy, epi, aux, nullptr, cols / 32, 0, QkvRope{}); \
    break;
  switch (tokens) {
    MI_HT(2) MI_HT(3) MI_HT(4) MI_HT(5) MI_HT(6) MI_HT(7) MI_HT(8)
    default: return fail(MI_ERR_ARG, "htile: %d tokens", tokens);
  }
#undef MI_HT
  return hip_check(hipGetLastError(), "htile launch");
}

// Split K for rows longer than one block's 4096 columns (the down
// projection's 14336 = 4 x 3584): parts of a multiple of 512 columns.
// A part's row bytes must be whole 8-byte words (a tile is copied in 8-byte
// words, row by row): any number of 144-byte Q4_K superblocks, a multiple of
// four 210-byte Q6_K ones (14336 columns: seven parts of 2048).
int htile_nsplit(int kind, int32_t cols, int nmin) {
  for (int n = std::max(nmin, (cols + 4095) / 4096); n <= 8; n++)
    if (cols % (n * 256 * kSBW) == 0 && (kind != MI_Q6_K || (cols / n / 256) % 4 == 0)) return n;
  return 0;
}

bool htile_split_fits(int kind, int32_t rows, int32_t cols, int32_t tokens, int nmin) {
  const int n = htile_nsplit(kind, cols, nmin);
  return n > 1 && htile_fits(kind, rows, cols / n, tokens);
}

// Q4_K or Q6_K rows of whole superblocks, at the alignment the split's word
// loads need (a Q6_K part starts 4 bytes past an 8-byte boundary when it
// holds an odd number of 210-byte superblocks)
static bool split_rows_ok(int kind, const void* w, int64_t row_bytes, int32_t cols) {
  const int sbb = kind == MI_Q6_K ? HGeo<MI_Q6_K>::SB : HGeo<MI_Q4_K>::SB;
  return (kind == MI_Q4_K || kind == MI_Q6_K) && row_bytes == (int64_t)(cols / 256) * sbb &&
         !((uintptr_t)w & (kind == MI_Q6_K ? 3 : 7));
}

// the parts, and one more slot for launch_htile_split_norm's residual copy
size_t htile_split_bytes(int32_t rows, int32_t cols, int32_t tokens, int nmin) {
  // room for either kind's parts
  const int n = std::max(htile_nsplit(MI_Q4_K, cols, nmin), htile_nsplit(MI_Q6_K, cols, nmin));
  return sizeof(float) * (size_t)(n + 1) * rows * tokens;
}

static int launch_split_main(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                             const void* xq, const void* hx, int32_t tokens, const float* resid, float* part,
                             int nmin = 1) {
  const int n = htile_nsplit(kind, cols, nmin), pc = cols / n;
  const RowSegs sg = rows::one_matrix(w, row_bytes, rows);
  const int waves = pc / (256 * kSBW);
  const int grid = std::min((rows + 15) / 16, std::max(1, cu_count() / n));
  const int64_t ysplit = (int64_t)tokens * rows;
  if (resid && (int64_t)grid * n * waves * 64 < ysplit)
    return fail(MI_ERR_SHAPE, "htile: %d x %d blocks cannot copy %lld residual values", grid, n, (long long)ysplit);
#define MI_HSK(T, K)                                                                                          \
  if (resid)                                                                                                  \
    hipLaunchKernelGGL((htile_kernel<T, K, false, false, true, true>), dim3(grid, n), dim3(waves * 64), 0, s, \
                       sg, pc, (const uint8_t*)xq, (const uint8_t*)hx, part, (int64_t)rows, MI_EPI_NONE, resid, \
                       nullptr, cols / 32, ysplit, QkvRope{});                                                \
  else                                                                                                        \
    hipLaunchKernelGGL((htile_kernel<T, K, false, false, true>), dim3(grid, n), dim3(waves * 64), 0, s, sg,   \
                       pc, (const uint8_t*)xq, (const uint8_t*)hx, part, (int64_t)rows, MI_EPI_NONE, nullptr,  \
                       nullptr, cols / 32, ysplit, QkvRope{});
#define MI_HS(T)                                                                                              \
  case T:                                                                                                     \
    if (kind == MI_Q6_K) {                                                                                    \
      MI_HSK(T, MI_Q6_K)                                                                                      \
    } else {                                                                                                  \
      MI_HSK(T, MI_Q4_K)                                                                                      \
    }                                                                                                         \
    break;
  switch (tokens) {
    MI_HS(2) MI_HS(3) MI_HS(4) MI_HS(5) MI_HS(6) MI_HS(7) MI_HS(8)
    default: return fail(MI_ERR_ARG, "htile: %d tokens", tokens);
  }
#undef MI_HS
#undef MI_HSK
  return hip_check(hipGetLastError(), "htile launch");
}

int launch_htile_split(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                       const void* xq, const void* hx, int32_t tokens, float* y, int64_t ldy, int32_t epi,
                       const float* aux, float* part) {
  if (!htile_split_fits(kind, rows, cols, tokens) || !split_rows_ok(kind, w, row_bytes, cols))
    return fail(MI_ERR_SHAPE, "htile: no split-K tile for %d x %d at %d tokens", rows, cols, tokens);
  int rc = launch_split_main(s, kind, w, row_bytes, rows, cols, xq, hx, tokens, nullptr, part);
  if (rc) return rc;
  hipLaunchKernelGGL(htile_split_reduce_kernel, dim3((tokens * rows + 255) / 256), dim3(256), 0, s, part,
                     htile_nsplit(kind, cols), tokens, rows, y, ldy, epi, aux);
  return hip_check(hipGetLastError(), "htile split reduce");
}

bool htile_split_norm_fits(int kind, int32_t rows, int32_t cols, int32_t tokens, int nmin) {
  const int n = htile_nsplit(kind, cols, nmin);
  // launch_split_add_norm takes rows of up to 16 * 256 values
  return htile_split_fits(kind, rows, cols, tokens, nmin) && n <= kMaxNormSplit && rows % 32 == 0 && rows <= 4096 &&
         (int64_t)std::min((rows + 15) / 16, std::max(1, cu_count() / n)) * n * (cols / n / 256 / kSBW) * 64 >=
             (int64_t)tokens * rows;
}

int launch_htile_split_norm(hipStream_t s, int kind, const void* w, int64_t row_bytes, int32_t rows, int32_t cols,
                            const void* xq, const void* hx, int32_t tokens, float* resid, const float* gain,
                            float eps, float* part, void* xq_out, void* hx_out, int nmin) {
  if (!htile_split_norm_fits(kind, rows, cols, tokens, nmin) || !split_rows_ok(kind, w, row_bytes, cols))
    return fail(MI_ERR_SHAPE, "htile: no split-K tile with a norm for %d x %d at %d tokens", rows, cols, tokens);
  int rc = launch_split_main(s, kind, w, row_bytes, rows, cols, xq, hx, tokens, resid, part, nmin);
  if (rc) return rc;
  return launch_split_add_norm(s, part, htile_nsplit(kind, cols, nmin), resid, gain, rows, tokens, eps, xq_out,
                               hx_out);
}

bool htile_qkv_rope_fits(const RowSegs& sg, int32_t cols, int32_t tokens, int32_t head_dim, int32_t rope_dim,
                         int kind) {
  const int rows = sg.end[sg.nseg - 1];
  const int sbb = kind == MI_Q6_K ? HGeo<MI_Q6_K>::SB : HGeo<MI_Q4_K>::SB;
  if ((kind != MI_Q4_K && kind != MI_Q6_K) || !htile_fits(kind, rows, cols, tokens) || head_dim % 2 ||
      rope_dim % 2 || rope_dim > 2 * kMaxRopePairs)
    return false;
  for (int i = 0; i < sg.nseg; i++)
    if (sg.end[i] % 16 || sg.rb[i] != (int64_t)(cols / 256) * sbb || ((uintptr_t)sg.w[i] & 7)) return false;
  return true;
}

int launch_htile_qkv_rope(hipStream_t s, const RowSegs& sg, int32_t cols, const void* xq, const void* hx,
                          int32_t tokens, float* q, int64_t ldq, const QkvRope& rp, int kind) {
  if (!htile_qkv_rope_fits(sg, cols, tokens, rp.head_dim, rp.rope_dim, kind))
    return fail(MI_ERR_SHAPE, "htile: no rope tile for %d columns at %d tokens", cols, tokens);
  const int rows = sg.end[sg.nseg - 1];
  const int waves = cols / (256 * kSBW);
  const int grid = std::min((rows + 15) / 16, cu_count());
#define MI_HR(T)                                                                                              \
  case T:                                                                                                     \
    if (kind == MI_Q6_K)                                                                                      \
      hipLaunchKernelGGL((htile_kernel<T, MI_Q6_K, false, true>), dim3(grid), dim3(waves * 64), 0, s, sg, cols, \
                         (const uint8_t*)xq, (const uint8_t*)hx, q, ldq, MI_EPI_NONE, nullptr, nullptr,       \
                         cols / 32, 0, rp);                                                                   \
    else                                                                                                      \
      hipLaunchKernelGGL((htile_kernel<T, MI_Q4_K, false, true>), dim3(grid), dim3(waves * 64), 0, s, sg, cols, \
                         (const uint8_t*)xq, (const uint8_t*)hx, q, ldq, MI_EPI_NONE, nullptr, nullptr,       \
                         cols / 32, 0, rp);                                                                   \
    break;
  switch (tokens) {
    MI_HR(2) MI_HR(3) MI_HR(4) MI_HR(5) MI_HR(6) MI_HR(7) MI_HR(8)
    default: return fail(MI_ERR_ARG, "htile: %d tokens", tokens);
  }
#undef MI_HR
  return hip_check(hipGetLastError(), "htile launch");
}

bool htile_glu_fits(int32_t rows, int32_t cols, int32_t tokens) {
  return htile_fits(MI_Q4_K, 2 * rows, cols, tokens) && rows % 32 == 0;
}

int launch_htile_glu(hipStream_t s, const void* gate, const void* up, int64_t row_bytes, int32_t rows, int32_t cols,
                     const void* xq, const void* hx, int32_t tokens, int32_t act, void* xq_out, bool hx_out) {
  if (!htile_glu_fits(rows, cols, tokens) || row_bytes != (int64_t)(cols / 256) * HGeo<MI_Q4_K>::SB ||
      (((uintptr_t)gate | (uintptr_t)up) & 7))
    return fail(MI_ERR_SHAPE, "htile: no GLU tile for %d x %d at %d tokens", rows, cols, tokens);
  RowSegs sg{};
  sg.w[0] = (const uint8_t*)gate;
  sg.w[1] = sg.w[2] = (const uint8_t*)up;
  sg.rb[0] = sg.rb[1] = sg.rb[2] = row_bytes;
  sg.end[0] = rows;
  sg.end[1] = sg.end[2] = 2 * rows;
  sg.nseg = 2;
  const int waves = cols / (256 * kSBW);
  const int grid = std::min(rows / 32, cu_count());
#define MI_HTG(T)                                                                                             \
  case T:                                                                                                     \
    hipLaunchKernelGGL((htile_kernel<T, MI_Q4_K, true>), dim3(grid), dim3(waves * 64), 0, s, sg, cols,        \
                       (const uint8_t*)xq, (const uint8_t*)hx, nullptr, 0,                                  \
                       (act & MI_ACT_GELU) | (hx_out ? kEpiHx : 0), nullptr,                                  \
                       (uint8_t*)xq_out, cols / 32, 0, QkvRope{});                                            \
    break;
  switch (tokens) {
    MI_HTG(2) MI_HTG(3) MI_HTG(4) MI_HTG(5) MI_HTG(6) MI_HTG(7) MI_HTG(8)
    default: return fail(MI_ERR_ARG, "htile: %d tokens", tokens);
  }
#undef MI_HTG
  return hip_check(hipGetLastError(), "htile launch");
}

}  // namespace mi

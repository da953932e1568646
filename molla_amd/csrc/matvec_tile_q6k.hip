// matvec_tile_q6k.hip -- the batched (2..8 tokens) Q6_K matvec on the matrix
// cores (v_mfma_i32_32x32x32_i8), gfx950: the output head at batch 8.
//
// Q6_K superblock (210 bytes / 256 values, quant.mojo:371): ql[128] @0,
// qh[64] @128, sc[16] int8 @192, d f16 @208.  Its 32-value group g
// (half n = g / 4, part a = g % 4) holds, for l < 32,
//   q = (ql[64n + 32(a & 1) + l] >> 4(a >> 1) & 15) | (qh[32n + l] >> 2a & 3) << 4
// and value (q - 32) * d * sc[2g + l / 16]: two 16-value sub-blocks with
// their own int8 scale.
//
// One MFMA covers one group: N = 32 rows (lane l gives row l % 32's codes q,
// unsigned 0..63, for values 16 (l / 32) .. +16, i.e. one sub-block), K = the
// group's 32 values, M = 8 slots x 4 where slot s is (token s % TC, sub-block
// s / TC) of a chunk of TC <= 4 tokens, its rows the token's three limbs.  A
// slot's A is non-zero only in its own sub-block's 16 values, so each slot's
// C is one (token, sub-block) dot; batch 8 takes two MFMAs per group.  The
// -32 offset comes off through the activation's per-16 limb sums, as in
// matvec_units.h Q6KUnit.
//
// Work decomposition as matvec_tile.hip: a block is 32 rows, its waves split
// the superblocks, each keeping the next superblock's loads in flight;
// per-group activation metadata is staged in LDS once per block.  210-byte
// superblocks are 2-byte aligned at worst: loads are of 4-byte aligned
// dwords, realigned with v_alignbyte.
//
// Replaces the batched planar_matmul_kernel (src/molla/nn/gpu.mojo:1809) for
// Q6_K; output y[t * ldy + r] and epilogues as gpu.mojo:1005.
#include "matvec_units.h"

namespace mi {
namespace {
using namespace mv;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kQ6Waves = 8;

// One lane's bytes of one superblock: its half (16 values) of each of the six
// 32-byte ql/qh runs, five dwords each for realignment, plus sc[0..15] and d.
struct Q6Lane {
  uint32_t ql[4][5];  // ql[32 p + 16 kb ..], p = 0..3
  uint32_t qh[2][5];  // qh[32 n + 16 kb ..], n = 0..1
  uint32_t sc[5];
  uint32_t d;
};

__device__ __forceinline__ void q6_load(Q6Lane& L, const uint8_t* blk, int kb) {
  const uint32_t sh = (uint32_t)((uintptr_t)blk & 3u);
  const uint8_t* b4 = blk - sh;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const uint8_t* q = b4 + 32 * p + 16 * kb;
    const uint4 v = ld16a4(q);
    L.ql[p][0] = v.x;
    L.ql[p][1] = v.y;
    L.ql[p][2] = v.z;
    L.ql[p][3] = v.w;
    L.ql[p][4] = ld4(q + 16);
  }
#pragma unroll
  for (int n = 0; n < 2; n++) {
    const uint8_t* q = b4 + 128 + 32 * n + 16 * kb;
    const uint4 v = ld16a4(q);
    L.qh[n][0] = v.x;
    L.qh[n][1] = v.y;
    L.qh[n][2] = v.z;
    L.qh[n][3] = v.w;
    L.qh[n][4] = ld4(q + 16);
  }
  const uint4 s = ld16a4(b4 + 192);
  L.sc[0] = s.x;
  L.sc[1] = s.y;
  L.sc[2] = s.z;
  L.sc[3] = s.w;
  // the fifth dword is only needed 2 bytes off alignment; aligned, it would
  // lie past the superblock (past the tensor for its last one)
  L.sc[4] = ld4(b4 + (sh ? 208 : 204));
  L.d = *(const uint16_t*)(blk + 208);
}

__device__ __forceinline__ v4i as_v4i(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  v4i r;
  r[0] = (int)a;
  r[1] = (int)b;
  r[2] = (int)c;
  r[3] = (int)d;
  return r;
}

// metadata per (token, group): scale, lsum1[2], lsum23[2]
struct Q6Meta {
  float scale;
  int l1[2], l23[2];
};

// STAGE: the block first copies every token's activation limbs (3 cols bytes
// a token) into LDS, and the group loop reads them from there.  A wave's
// vector loads complete in issue order, so a limb load issued in the group
// loop, after the weight loads of the superblocks ahead, would wait for those
// weights too; from LDS it waits for nothing.
template <int T, int SBW, bool STAGE>
__global__ __launch_bounds__(kQ6Waves * 64) void q6k_tile_kernel(const uint8_t* __restrict__ w, int64_t rb,
                                                                 int rows, int cols, const uint8_t* __restrict__ xq,
                                                                 float* __restrict__ y, int64_t ldy, int epi,
                                                                 const float* __restrict__ aux) {
  constexpr int TC = T < 4 ? T : 4;        // tokens per MFMA
  constexpr int NC = (T + TC - 1) / TC;    // MFMAs per group
  constexpr int NSL = 2 * TC;              // slots in use
  extern __shared__ Q6Meta meta6[];        // [T][G]
  __shared__ float red[kQ6Waves][T][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, ks = blockDim.x >> 6;
  const int n = lane & 31, kh = lane >> 5;
  const int row = blockIdx.x * 32 + n;
  const uint8_t* wrow = w + (int64_t)min(row, rows - 1) * rb;
  const int nsb = cols >> 8, G = cols >> 5;
  const int sb0 = wave * SBW;
  const int tok = 4 * cols, plane = (cols >> 5) * 16;
  uint8_t* xs = (uint8_t*)(meta6 + T * G);  // STAGE: [T][3 cols] limb bytes
  if constexpr (STAGE) {
    // all of a thread's loads first, clamped (a duplicate store of the last
    // vector is harmless), then the stores
    const int per_tok = 3 * cols / 16, total = T * per_tok;
    for (int base = 0; base < total; base += 8 * (int)blockDim.x) {
      uint4 v[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int i = min(base + j * (int)blockDim.x + (int)threadIdx.x, total - 1);
        const int t = i / per_tok;
        v[j] = *(const uint4*)(xq + (uint32_t)(t * tok + (i - t * per_tok) * 16));
      }
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int i = min(base + j * (int)blockDim.x + (int)threadIdx.x, total - 1);
        ((uint4*)xs)[i] = v[j];
      }
    }
  }

  Q6Lane wl[2];
  q6_load(wl[0], wrow + (int64_t)min(sb0, nsb - 1) * 210, kh);
  if (SBW > 1) q6_load(wl[1], wrow + (int64_t)min(sb0 + 1, nsb - 1) * 210, kh);

  // A role: slot s = m / 4 = (token chunk-local s % TC, sub-block s / TC),
  // limb m % 4; lanes of the other sub-block's K half give zeros
  const int m = lane & 31, s = m >> 2, jj = m & 3;
  const int a_t = s % TC, a_sub = s / TC;
  const bool a_live = jj < 3 && s < NSL && a_sub == kh;
  const int a_off = (jj * 2 + kh) * plane;

  for (int i = threadIdx.x; i < T * G; i += blockDim.x) {
    const int t = i / G, g = i - t * G;
    const XMeta mt = *(const XMeta*)(xq + (uint32_t)(t * tok + 6 * plane + g * 16));
    const int2 l23 = *(const int2*)(xq + (uint32_t)(t * tok + 7 * plane + g * 16));
    meta6[i] = Q6Meta{mt.scale, {mt.lsum1[0], mt.lsum1[1]}, {l23.x, l23.y}};
  }
  __syncthreads();

  float acc[NC][4];
#pragma unroll
  for (int c = 0; c < NC; c++)
#pragma unroll
    for (int a = 0; a < 4; a++) acc[c][a] = 0.0f;

#pragma unroll
  for (int i = 0; i < SBW; i++) {
    const int sb = sb0 + i;
    if (sb >= nsb) break;
    const int sl = i & 1;
    const Q6Lane& L = wl[sl];
    const uint32_t sh = (uint32_t)((uintptr_t)(wrow + (int64_t)sb * 210) & 3u);
    const float d = half_bits_to_float(L.d);
    // sc[0..15] realigned
    uint32_t scw[4];
#pragma unroll
    for (int k = 0; k < 4; k++) scw[k] = align(L.sc[k + 1], L.sc[k], sh);
    float part[NC][4];
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int a = 0; a < 4; a++) part[c][a] = 0.0f;
#pragma unroll 1
    for (int g = 0; g < 8; g++) {
      const int hn = g >> 2, pa = g & 3, p = 2 * hn + (pa & 1);
      const uint32_t nib = 4u * (uint32_t)(pa >> 1), hb = 2u * (uint32_t)pa;
      uint32_t bq[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        // runtime p / hn: select among the loaded runs without indexing
        const uint32_t q0 = p == 0 ? align(L.ql[0][k + 1], L.ql[0][k], sh)
                          : p == 1 ? align(L.ql[1][k + 1], L.ql[1][k], sh)
                          : p == 2 ? align(L.ql[2][k + 1], L.ql[2][k], sh)
                                   : align(L.ql[3][k + 1], L.ql[3][k], sh);
        const uint32_t h0 = hn == 0 ? align(L.qh[0][k + 1], L.qh[0][k], sh) : align(L.qh[1][k + 1], L.qh[1][k], sh);
        bq[k] = ((q0 >> nib) & 0x0F0F0F0Fu) | (((h0 >> hb) & 0x03030303u) << 4);
      }
      const int gabs = sb * 8 + g;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int tt = c * TC + a_t;
        uint4 av = make_uint4(0, 0, 0, 0);
        if (a_live && tt < T)
          av = STAGE ? *(const uint4*)(xs + tt * 3 * cols + a_off + gabs * 16)
                     : ld16(xq + (uint32_t)(tt * tok + a_off + gabs * 16));
        v16i C = {};
        C = __builtin_amdgcn_mfma_i32_32x32x32_i8(as_v4i(av.x, av.y, av.z, av.w), as_v4i(bq[0], bq[1], bq[2], bq[3]),
                                                  C, 0, 0, 0);
        // lane (n, kh) owns slots 2a + kh: token (2a + kh) % TC, sub-block (2a + kh) / TC
#pragma unroll
        for (int a = 0; a < 4; a++) {
          const int slot = 2 * a + kh;
          const int t = c * TC + slot % TC, j = slot / TC;
          if (slot < NSL && t < T) {
            const Q6Meta& mt = meta6[t * G + gabs];
            const int l1 = j ? mt.l1[1] : mt.l1[0], l23 = j ? mt.l23[1] : mt.l23[0];
            const float v = limbs_to_float(C[4 * a] - 32 * l1, C[4 * a + 1] * 256 + C[4 * a + 2] - 32 * l23);
            const uint32_t si = 2u * (uint32_t)g + (uint32_t)j;
            const uint32_t sw = si < 4 ? scw[0] : si < 8 ? scw[1] : si < 12 ? scw[2] : scw[3];
            const float scv = (float)(int8_t)((sw >> (8 * (si & 3))) & 0xFF);
            part[c][a] = fmaf(scv * mt.scale, v, part[c][a]);
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int a = 0; a < 4; a++) acc[c][a] = fmaf(d, part[c][a], acc[c][a]);
    if (i + 2 < SBW) q6_load(wl[sl], wrow + (int64_t)min(sb0 + i + 2, nsb - 1) * 210, kh);
  }
  // per token: this lane's slots holding it (both sub-blocks), then both halves
#pragma unroll
  for (int t = 0; t < T; t++) {
    float v = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; c++)
#pragma unroll
      for (int a = 0; a < 4; a++) {
        const int slot = 2 * a + kh;
        if (slot < NSL && c * TC + slot % TC == t) v += acc[c][a];
      }
    v += __shfl_xor(v, 32);
    if (kh == 0) red[wave][t][n] = v;
  }
  __syncthreads();
  for (int o = threadIdx.x; o < 32 * T; o += blockDim.x) {
    const int t = o >> 5, nn = o & 31;
    float v = 0.0f;
    for (int k = 0; k < ks; k++) v += red[k][t][nn];
    const int r = blockIdx.x * 32 + nn;
    if (r < rows) epilogue(y, aux, epi, (int64_t)t * ldy + r, r, v);
  }
}

// Dynamic LDS the staged form may take (the static part, red, is 8 KB at most).
constexpr size_t kQ6StageLds = 144 * 1024;

template <int T, int SBW>
int launch_ts(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y, int64_t ldy,
              int epi, const float* aux) {
  const int ks = (cols / 256 + SBW - 1) / SBW;
  const size_t meta = (size_t)T * (cols / 32) * sizeof(Q6Meta);
  const size_t staged = meta + (size_t)T * 3 * cols;
  if (staged <= kQ6StageLds) {
    static bool done[kMaxDevices];  // more than 64 KB has to be asked for
    if (int rc = allow_lds((const void*)q6k_tile_kernel<T, SBW, true>, (int)kQ6StageLds, done,
                           "q6k tile LDS attribute"))
      return rc;
    hipLaunchKernelGGL((q6k_tile_kernel<T, SBW, true>), dim3((rows + 31) / 32), dim3(ks * 64), staged, s,
                       (const uint8_t*)w, rb, rows, cols, (const uint8_t*)xq, y, ldy, epi, aux);
  } else {
    hipLaunchKernelGGL((q6k_tile_kernel<T, SBW, false>), dim3((rows + 31) / 32), dim3(ks * 64), meta, s,
                       (const uint8_t*)w, rb, rows, cols, (const uint8_t*)xq, y, ldy, epi, aux);
  }
  return hip_check(hipGetLastError(), "matvec launch");
}

template <int T>
int launch_t(hipStream_t s, const void* w, int64_t rb, int rows, int cols, const void* xq, float* y, int64_t ldy,
             int epi, const float* aux) {
  const int nsb = cols / 256;
  if (nsb <= 2 * kQ6Waves) return launch_ts<T, 2>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  if (nsb <= 4 * kQ6Waves) return launch_ts<T, 4>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
  return launch_ts<T, 8>(s, w, rb, rows, cols, xq, y, ldy, epi, aux);
}

}  // namespace

bool q6k_tile_fits(int32_t cols, int64_t row_bytes, int32_t tokens) {
  return tokens >= 2 && tokens <= 8 && cols % 256 == 0 && cols / 256 <= 8 * kQ6Waves && row_bytes % 2 == 0;
}

int launch_q6k_tile(hipStream_t s, const void* w, int64_t row_bytes, int32_t rows, int32_t cols, const void* xq,
                    int32_t tokens, float* y, int64_t ldy, int32_t epi, const float* aux) {
  if (tokens > 4) {
    // Two passes over the weights (4 + 4, 4 + 3, 4 + 2 or 3 + 2 tokens): the
    // forms of more than four tokens are bound by their per-group VALU work,
    // and at 8 tokens two 4-token passes (2 x 159 us for the 128256 x 4096
    // head) beat one 8-token pass (390 us) despite reading the weights twice.
    const int first = tokens >= 6 ? 4 : 3;
    int rc = first == 4 ? launch_t<4>(s, w, row_bytes, rows, cols, xq, y, ldy, epi, aux)
                        : launch_t<3>(s, w, row_bytes, rows, cols, xq, y, ldy, epi, aux);
    if (rc) return rc;
    const uint8_t* xq2 = (const uint8_t*)xq + (size_t)first * 4 * cols;  // the next token's activation
    const float* aux2 = (epi & MI_EPI_GLU) ? aux + first * ldy : aux;   // GLU's aux is per token, a bias per row
    float* y2 = y + first * ldy;
    switch (tokens - first) {
      case 2: return launch_t<2>(s, w, row_bytes, rows, cols, xq2, y2, ldy, epi, aux2);
      case 3: return launch_t<3>(s, w, row_bytes, rows, cols, xq2, y2, ldy, epi, aux2);
      default: return launch_t<4>(s, w, row_bytes, rows, cols, xq2, y2, ldy, epi, aux2);
    }
  }
  switch (tokens) {
    case 2: return launch_t<2>(s, w, row_bytes, rows, cols, xq, y, ldy, epi, aux);
    case 3: return launch_t<3>(s, w, row_bytes, rows, cols, xq, y, ldy, epi, aux);
    case 4: return launch_t<4>(s, w, row_bytes, rows, cols, xq, y, ldy, epi, aux);
  }
  return fail(MI_ERR_ARG, "matvec: tokens %d outside 2..8 for the batched tile", tokens);
}

}  // namespace mi

// ops.hip -- the decoder layer's small kernels, gfx950.
//
// Replaces src/molla/nn/gpu_ops.mojo: rms_norm_kernel (:152), rope_kernel
// (:470), store_kv_kernel (:1491), attend_split_kernel / attend_merge_kernel
// (:929 / :1104), argmax_kernel (:408) and the embedding row copy (:320).
// Producers of a matvec input (norm, attention merge) also write the
// activation in the matvec's block fixed-point form (xq_device.h), so the
// next projection needs no separate quantize launch.
#include <math.h>

#include <algorithm>

#include "mi_internal.h"
#include "xq_device.h"
#include "matvec_units.h"

namespace mi {
namespace {

// ---- RMSNorm ---------------------------------------------------------------
// kernel.mojo:432-467: float64 sum of squares, scale = f32(1/sqrt(sum/n+eps)),
// out = x * scale * gain.  A token's row is spread over `parts` blocks of
// 256 threads.  Every block sums the whole row (16 KB for n = 4096, an L2
// read) in the same order, so all blocks derive the identical scale with no
// cross-block communication; each then normalises and quantizes only its
// own 256-value slice.  Spreading the slices over CUs matters: the
// fixed-point conversion is shuffle-heavy and one CU doing a whole row was
// the slowest part.  All loads are issued before any arithmetic.
constexpr int kNormThreads = 256;
#ifndef MI_NORM_VEC
#define MI_NORM_VEC 1
#endif
constexpr bool kNormVec = MI_NORM_VEC;

// With `trig`, the last block also writes (cos, sin) of the angle of pair p at
// pos[0] for p < pairs, in float64 as rope.mojo:253-285, for the layer's fused
// q|k|v rope; it has no other use for its spare threads' time.
//
// NS > 0: the row is the residual after a split-K matvec's parts are added
// (x = part[k * pstride + ...] for k < NS, the old residual in slot NS; the
// sums in htile_split_reduce_kernel's order), and each block also writes its
// slice of that row to `out` (the residual, in place: no block reads it).
template <int PER, int NS = 0, int NT = kNormThreads>
__global__ __launch_bounds__(NT) void rms_norm_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ gain, int n,
                                                                float eps, float* __restrict__ out,
                                                                uint8_t* __restrict__ xq,
                                                                uint8_t* __restrict__ hx,
                                                                const int32_t* __restrict__ pos,
                                                                const float* __restrict__ steps,
                                                                const float* __restrict__ factors, int pairs,
                                                                float2* __restrict__ trig, int64_t pstride) {
#pragma clang fp contract(off)
  const int t = blockIdx.y;
  if (trig && blockIdx.x == gridDim.x - 1) {
    for (int p = threadIdx.x; p < pairs; p += NT) {
      const float theta = rope_theta(pos[0], steps, factors, p);
      trig[p] = make_float2((float)cos((double)theta), (float)sin((double)theta));
    }
  }
  const float* xr = x + (int64_t)t * n;
  const int mine = blockIdx.x * NT + threadIdx.x;
  const bool live = mine < n;
  float xv[PER];
  __shared__ float own[(NS > 0 && kNormVec) ? NT : 1];
  if constexpr (NS > 0 && kNormVec) {
    // 16-byte loads: thread t sums values 4 (t + NT q) .. +4, q < PER / 4
    // (4 times fewer load instructions than one value a load, which bound
    // the launch), and leaves the ones of its block's slice in LDS for the
    // thread that owns them
    typedef float nf4 __attribute__((ext_vector_type(4)));
    nf4 pv[NS + 1][PER / 4];
#pragma unroll
    for (int j = 0; j <= NS; j++)
#pragma unroll
      for (int q = 0; q < PER / 4; q++) {
        const int i = min(4 * ((int)threadIdx.x + q * NT), n - 4);
        pv[j][q] = *(const nf4*)(xr + j * pstride + i);
      }
#pragma unroll
    for (int q = 0; q < PER / 4; q++) {
      nf4 v = pv[0][q];
#pragma unroll
      for (int j = 1; j < NS; j++) v += pv[j][q];
      const int i0 = 4 * ((int)threadIdx.x + q * NT);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float xe = i0 + e < n ? pv[NS][q][e] + v[e] : 0.0f;
        xv[4 * q + e] = xe;
        const int r = i0 + e - (int)blockIdx.x * NT;
        if (r >= 0 && r < NT) own[r] = xe;
      }
    }
  } else if constexpr (NS > 0) {
    float pv[NS + 1][PER];
#pragma unroll
    for (int j = 0; j <= NS; j++)
#pragma unroll
      for (int k = 0; k < PER; k++) {
        const int i = min((int)threadIdx.x + k * NT, n - 1);
        pv[j][k] = xr[j * pstride + i];
      }
#pragma unroll
    for (int k = 0; k < PER; k++) {
      float v = pv[0][k];
#pragma unroll
      for (int j = 1; j < NS; j++) v += pv[j][k];
      xv[k] = threadIdx.x + k * NT < n ? pv[NS][k] + v : 0.0f;
    }
  } else {
#pragma unroll
    for (int k = 0; k < PER; k++) {
      const int i = threadIdx.x + k * NT;
      xv[k] = i < n ? xr[i] : 0.0f;
    }
  }
  const float gm = live ? gain[mine] : 0.0f;
  // this thread's own value is one it already loaded for the sum (a second
  // load of it measured a microsecond slower); in the 16-byte form it comes
  // from LDS after the barrier below
  float xm = xv[0];
#pragma unroll
  for (int k = 1; k < PER; k++)
    if ((int)blockIdx.x == k) xm = xv[k];
  double acc = 0.0;
#pragma unroll
  for (int k = 0; k < PER; k++) acc += (double)xv[k] * (double)xv[k];
  acc = lanes::reduce_sum<64>(acc);
  __shared__ double part[NT / kWave];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  double sum = 0.0;
#pragma unroll
  for (int i = 0; i < NT / kWave; i++) sum += part[i];
  const float scale = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
  if constexpr (NS > 0 && kNormVec) xm = live ? own[threadIdx.x] : 0.0f;
  const float v = xm * scale * gm;
  if constexpr (NS > 0) {
    if (live) out[(int64_t)t * n + mine] = xm;
  } else {
    if (out && live) out[(int64_t)t * n + mine] = v;
  }
  // A half-wave is one 32-value group; n is a multiple of 32 whenever xq
  // is asked for, so a group is either entirely live or entirely past the end.
  if (xq)
    quantize_group32(v, threadIdx.x & 31, mine >> 5, n >> 5, xq + (int64_t)t * xq_token_bytes(n), live,
                     hx ? hx + (int64_t)t * xq_token_bytes(n) : nullptr);
}

// One q8_0 block of a cache row: the 32 lanes of a half-wave each bring one
// value x of block b; rowp is the position's row (quants, then factors).
__device__ __forceinline__ void q8_store_block(float x, __half* __restrict__ rowp, int b, int kv_width,
                                               int lane32) {
#pragma clang fp contract(off)
  float amax = fabsf(x);
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
  const float inv = amax == 0.0f ? 0.0f : 127.0f / amax;
  const float y = x * inv;
  const float r = y >= 0.0f ? y + 0.5f : y - 0.5f;
  const int qi = max(-127, min(127, (int)r));
  ((int8_t*)rowp)[b * 32 + lane32] = (int8_t)qi;
  if (lane32 == 0) rowp[(kv_width >> 1) + b] = __float2half_rn(amax / 127.0f);
}

// ---- RoPE ------------------------------------------------------------------
// rope.mojo:253-338: theta = f32(pos) * step / freq (scale 1),
// c = f32(cos(f64(theta))), s likewise, (a, b) <- (a*c - b*s, a*s + b*c).
// The trig is done in float64 on the device too, so the rotated values
// match the host's to float32 rounding at any position.
__device__ __forceinline__ void rotate_pair(float* __restrict__ row, int head_dim, int dim, int neox,
                                            const float* __restrict__ steps, const float* __restrict__ factors,
                                            int pos, int head, int pair) {
#pragma clang fp contract(off)
  const float theta = rope_theta(pos, steps, factors, pair);
  const float c = (float)cos((double)theta);
  const float s = (float)sin((double)theta);
  const int pairs = dim >> 1;
  float* at = row + (int64_t)head * head_dim;
  const int lo = neox ? pair : 2 * pair;
  const int hi = neox ? pair + pairs : 2 * pair + 1;
  const float a = at[lo], b = at[hi];
  at[lo] = a * c - b * s;
  at[hi] = a * s + b * c;
}

__global__ void rope_kernel(float* __restrict__ x, int heads, int head_dim, int dim, int neox,
                            const float* __restrict__ steps, const float* __restrict__ factors,
                            const int32_t* __restrict__ pos, int64_t row_stride) {
  const int t = blockIdx.x;
  const int pairs = dim >> 1;
  float* row = x + (int64_t)t * row_stride;
  for (int i = threadIdx.x; i < heads * pairs; i += blockDim.x)
    rotate_pair(row, head_dim, dim, neox, steps, factors, pos[t], i / pairs, i % pairs);
}

// Rotate q and k of a fused [q | k | v] row in place, then store k and v as
// halves at the token's slot (gpu_ops.mojo:1491, narrowing by a plain cast,
// i.e. round to nearest even).  The angle depends only on (position, pair),
// so the block computes each pair's cos/sin once, in float64 as the host
// does, into LDS; meanwhile every thread's pairs of q/k are already being
// loaded.  Rotation then runs from registers.
constexpr int kRopeThreads = 512;
constexpr int kRopePer = 8;  // pairs per thread held in registers per pass

// Q8: the cache is q8_0 (crow halves a position): the rotated keys go back
// into the row like q, and once the block has them all, each half-wave
// encodes 32-value blocks of k and v into the cache (no store launch).
template <bool Q8>
__global__ __launch_bounds__(kRopeThreads) void rope_store_kernel(
    float* __restrict__ qkv, int heads, int kv_heads, int head_dim, int dim, int neox,
    const float* __restrict__ steps, const float* __restrict__ factors, const int32_t* __restrict__ pos,
    int64_t row_stride,
    __half* __restrict__ kc, __half* __restrict__ vc, int64_t cache_stride, int crow,
    const int32_t* __restrict__ kv_index, int64_t index_stride) {
#pragma clang fp contract(off)
  extern __shared__ float trig[];  // [pairs][2]
  const int t = blockIdx.x;
  const int pairs = dim >> 1;
  const int p = pos[t];
  float* row = qkv + (int64_t)t * row_stride;
  const int kvw = kv_heads * head_dim;
  const int64_t at = kv_index ? (int64_t)kv_index[t * index_stride + p] * crow
                              : (int64_t)t * cache_stride + (int64_t)p * crow;
  __half* kd = kc + at;
  __half* vd = vc + at;
  const int total = (heads + kv_heads) * pairs;
  const int lo_step = neox ? 1 : 2, hi_off = neox ? pairs : 1;
  for (int base = 0; base < total; base += kRopeThreads * kRopePer) {
    float a[kRopePer], b[kRopePer];
#pragma unroll
    for (int k = 0; k < kRopePer; k++) {
      const int i = base + threadIdx.x + k * kRopeThreads;
      const int h = i / pairs, q = i - h * pairs;
      const int64_t lo = (int64_t)h * head_dim + q * lo_step;
      a[k] = i < total ? row[lo] : 0.0f;
      b[k] = i < total ? row[lo + hi_off] : 0.0f;
    }
    if (base == 0) {
      for (int q = threadIdx.x; q < pairs; q += kRopeThreads) {
        const float theta = rope_theta(p, steps, factors, q);
        trig[2 * q] = (float)cos((double)theta);
        trig[2 * q + 1] = (float)sin((double)theta);
      }
      __syncthreads();
    }
#pragma unroll
    for (int k = 0; k < kRopePer; k++) {
      const int i = base + threadIdx.x + k * kRopeThreads;
      if (i >= total) break;
      const int h = i / pairs, q = i - h * pairs;
      const float c = trig[2 * q], sn = trig[2 * q + 1];
      const float ra = a[k] * c - b[k] * sn;
      const float rb = a[k] * sn + b[k] * c;
      const int64_t lo = (int64_t)h * head_dim + q * lo_step;
      row[lo] = ra;
      row[lo + hi_off] = rb;
      if (!Q8 && h >= heads) {  // a key head: straight into the cache
        const int64_t kl = lo - (int64_t)heads * head_dim;
        kd[kl] = __float2half_rn(ra);
        kd[kl + hi_off] = __float2half_rn(rb);
      }
    }
  }
  const float* v = row + (int64_t)(heads + kv_heads) * head_dim;
  if constexpr (Q8) {
    __syncthreads();  // every rotated key is in the row
    const float* k = row + (int64_t)heads * head_dim;
    const int nb = kvw >> 5, lane32 = threadIdx.x & 31;
    for (int blk = threadIdx.x >> 5; blk < 2 * nb; blk += kRopeThreads >> 5) {
      const bool isv = blk >= nb;
      const int b = isv ? blk - nb : blk;
      q8_store_block((isv ? v : k)[b * 32 + lane32], isv ? vd : kd, b, kvw, lane32);
    }
    return;
  }
  // values, and any key elements past the rotary dimension
  for (int i = threadIdx.x; i < kvw; i += kRopeThreads) vd[i] = __float2half_rn(v[i]);
  if (dim < head_dim) {
    const float* k = row + (int64_t)heads * head_dim;
    const int tail = head_dim - dim;
    for (int i = threadIdx.x; i < kv_heads * tail; i += kRopeThreads) {
      const int h = i / tail, e = dim + (i - h * tail);
      kd[(int64_t)h * head_dim + e] = __float2half_rn(k[(int64_t)h * head_dim + e]);
    }
  }
}

__global__ void store_kv_kernel(const float* __restrict__ k, const float* __restrict__ v, int kvw,
                                __half* __restrict__ kc, __half* __restrict__ vc,
                                const int32_t* __restrict__ slot_dev, int slot_host, int64_t src_stride,
                                int64_t cache_stride) {
  const int t = blockIdx.y;
  const int slot = slot_dev ? slot_dev[t] : slot_host;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= kvw) return;
  // k null: the values only (the keys were stored, rotated, elsewhere)
  if (k) kc[(int64_t)t * cache_stride + (int64_t)slot * kvw + i] = __float2half_rn(k[(int64_t)t * src_stride + i]);
  vc[(int64_t)t * cache_stride + (int64_t)slot * kvw + i] = __float2half_rn(v[(int64_t)t * src_stride + i]);
}

// ---- attention -------------------------------------------------------------
// attention.mojo:144 attend, split over slices of keys like gpu_ops.mojo:929
// attend_split_kernel: a block takes one key head, one slice of keys and
// every query head that reads that key head (GQA), so each cached key and
// value is read once.  The slice's keys and values are staged into LDS with
// all loads in flight at once; lane k of a wave scores key k for one query
// head; the weighted sum of values reads them back from LDS.  Each slice
// writes its running maximum, its sum of exponentials and its unnormalised
// weighted values; the merge folds slices flash-style (gpu_ops.mojo:1104).
constexpr int kAttnThreads = 256;

// keys per slice: at most 64 (one per lane), fewer for wide heads so the
// block's LDS stays within 64 KB for any group of up to 8 query heads
__host__ __device__ __forceinline__ int attn_slice(int head_dim) {
  return head_dim <= 128 ? 64 : (head_dim <= 256 ? 32 : 16);
}
__host__ __device__ __forceinline__ size_t attn_q8_lds_bytes(int head_dim, int group) {
  const int kk = attn_slice(head_dim);
  return (size_t)kk * (head_dim + 16) + (size_t)kk * head_dim + (size_t)2 * kk * (head_dim / 32) * 4 +
         (size_t)group * head_dim * 4 + (size_t)group * kk * 4;
}
__host__ __device__ __forceinline__ size_t attn_lds_bytes(int head_dim, int group) {
  const int kk = attn_slice(head_dim);
  return (size_t)kk * (head_dim + 8) * 2 + (size_t)kk * head_dim * 2 + (size_t)group * head_dim * 4 +
         (size_t)group * kk * 4;
}

// Paged caches (gpu_ops.mojo:662 _row_of): with kv_index, position j of
// sequence t lives in cell kv_index[t * index_stride + j] of one shared pool
// (cells of one cache row each, cache_stride unused), and a negative cell is
// a position the sequence does not hold, masked like a key past the end;
// without it, position j of sequence t is row j of that sequence's own cache.
__device__ __forceinline__ int kv_cell(const int32_t* __restrict__ kv_index, int64_t index_stride, int t, int j) {
  return kv_index ? kv_index[t * index_stride + j] : j;
}

// tq > 1 (one sequence's chunk only: its tokens share the cache): the block
// stages the slice once and scores tq consecutive tokens against it, each
// with its own count, so a prefill chunk reads every slice once per tq
// tokens instead of once per token.
template <int GROUP>
__global__ __launch_bounds__(kAttnThreads) void attend_split_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc,
    const __half* __restrict__ vc, int64_t cache_stride, int heads, int kv_heads, int head_dim,
    float scale, const int32_t* __restrict__ pos_dev, int count_host, int max_chunks,
    float* __restrict__ part_acc, float* __restrict__ part_ml, const int32_t* __restrict__ kv_index,
    int64_t index_stride, int tokens, int tq) {
  const int c = blockIdx.x, kvh = blockIdx.y;
  const int t0 = blockIdx.z * tq, t1 = min(t0 + tq, tokens);
  // a position p attends over p + 1 slots; the block stages for its widest
  int count_max = 0;
  for (int t = t0; t < t1; t++) count_max = max(count_max, pos_dev ? pos_dev[t] + 1 : count_host);
  const int kk = attn_slice(head_dim);
  const int start = c * kk;
  if (start >= count_max) return;
  const int D = head_dim, KS = head_dim + 8;  // LDS key rows padded by 16 bytes
  const int nk_max = min(kk, count_max - start);
  const int kvw = kv_heads * D;
  extern __shared__ uint4 lds4[];
  __half* Ks = (__half*)lds4;
  __half* Vs = Ks + kk * KS;
  float* Qs = (float*)(Vs + kk * D);
  float* Ps = Qs + GROUP * D;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // stage keys, values (16-byte pieces; keys past the end repeat the last
  // live one and are masked below) and the group's queries
  const int64_t seq = kv_index ? 0 : (int64_t)t0 * cache_stride;
  const __half* kbase = kc + seq + (int64_t)kvh * D;
  const __half* vbase = vc + seq + (int64_t)kvh * D;
  // Every load of a batch is issued before any LDS store, with clamped
  // (always valid) addresses instead of guards: a guarded load becomes a
  // branch with its own wait, which serialised the staging.
  const int pieces = D >> 3;
  const int total = kk * pieces;
  constexpr int kBatch = 4;
  const int nq4 = GROUP * D / 4;
  auto q4_of = [&](int t) { return (const float4*)(q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * D); };
  const float4 qv = q4_of(t0)[min(tid, nq4 - 1)];
  for (int b0 = 0; b0 < total; b0 += kAttnThreads * kBatch) {
    uint4 kv[kBatch], vv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; j++) {
      const int i = min(b0 + tid + j * kAttnThreads, total - 1);
      const int key = min(i / pieces, nk_max - 1), pc = i % pieces;
      const int cell = max(kv_cell(kv_index, index_stride, t0, start + key), 0);
      const int64_t off = (int64_t)cell * kvw + pc * 8;
      kv[j] = *(const uint4*)(kbase + off);
      vv[j] = *(const uint4*)(vbase + off);
    }
#pragma unroll
    for (int j = 0; j < kBatch; j++) {
      const int i = b0 + tid + j * kAttnThreads;
      const int key = i / pieces, pc = i % pieces;
      if (i < total) {
        *(uint4*)(Ks + key * KS + pc * 8) = kv[j];
        *(uint4*)(Vs + key * D + pc * 8) = vv[j];
      }
    }
  }
  const int halfD = D >> 1;
  for (int t = t0; t < t1; t++) {
    const int count = pos_dev ? pos_dev[t] + 1 : count_host;
    if (start >= count) continue;  // uniform over the block: no keys of this slice for t
    const int nk = min(kk, count - start);
    if (t == t0) {
      if (tid < nq4) ((float4*)Qs)[tid] = qv;
      for (int i = tid + kAttnThreads; i < nq4; i += kAttnThreads) ((float4*)Qs)[i] = q4_of(t)[i];
    } else {
      for (int i = tid; i < nq4; i += kAttnThreads) ((float4*)Qs)[i] = q4_of(t)[i];
    }
    __syncthreads();

    const int64_t slot_base = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks + c;
    // scores and slice softmax: wave w takes query heads w, w+4, ...; lane = key
    for (int g = wave; g < GROUP; g += kAttnThreads / kWave) {
      float sdot = 0.0f;
      if (lane < kk) {
        const __half* kr = Ks + lane * KS;
        const float* qg = Qs + g * D;
        for (int d = 0; d < D; d += 8) {
          const uint4 raw = *(const uint4*)(kr + d);
          const __half2* h2 = (const __half2*)&raw;
          const float4 qa = *(const float4*)(qg + d), qb = *(const float4*)(qg + d + 4);
          const float2 k0 = __half22float2(h2[0]), k1 = __half22float2(h2[1]);
          const float2 k2 = __half22float2(h2[2]), k3 = __half22float2(h2[3]);
          sdot = fmaf(qa.x, k0.x, sdot);
          sdot = fmaf(qa.y, k0.y, sdot);
          sdot = fmaf(qa.z, k1.x, sdot);
          sdot = fmaf(qa.w, k1.y, sdot);
          sdot = fmaf(qb.x, k2.x, sdot);
          sdot = fmaf(qb.y, k2.y, sdot);
          sdot = fmaf(qb.z, k3.x, sdot);
          sdot = fmaf(qb.w, k3.y, sdot);
        }
      }
      const bool live = lane < nk && (!kv_index || kv_cell(kv_index, index_stride, t, start + lane) >= 0);
      const float sc = live ? sdot * scale : -INFINITY;
      float m = sc;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
      const float pr = live ? expf(sc - m) : 0.0f;
      float l = pr;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o);
      if (lane < kk) Ps[g * kk + lane] = pr;
      if (lane == 0) {
        part_ml[(slot_base + (int64_t)g * max_chunks) * 2 + 0] = m;
        part_ml[(slot_base + (int64_t)g * max_chunks) * 2 + 1] = l;
      }
    }
    __syncthreads();
    // unnormalised weighted values: thread o takes query head g, dims 2e, 2e+1
    for (int o = tid; o < GROUP * halfD; o += kAttnThreads) {
      const int g = o / halfD, e = o - g * halfD;
      const float* pg = Ps + g * kk;
      float a0 = 0.0f, a1 = 0.0f;
      // four keys per step: one float4 of weights, four value pairs (keys past
      // nk have weight 0 and a finite staged row, so they add exactly 0)
      for (int k = 0; k < nk; k += 4) {
        const float4 p4 = *(const float4*)(pg + k);
        const float2 v0 = __half22float2(*(const __half2*)(Vs + (k + 0) * D + 2 * e));
        const float2 v1 = __half22float2(*(const __half2*)(Vs + (k + 1) * D + 2 * e));
        const float2 v2 = __half22float2(*(const __half2*)(Vs + (k + 2) * D + 2 * e));
        const float2 v3 = __half22float2(*(const __half2*)(Vs + (k + 3) * D + 2 * e));
        a0 = fmaf(p4.x, v0.x, a0);
        a1 = fmaf(p4.x, v0.y, a1);
        a0 = fmaf(p4.y, v1.x, a0);
        a1 = fmaf(p4.y, v1.y, a1);
        a0 = fmaf(p4.z, v2.x, a0);
        a1 = fmaf(p4.z, v2.y, a1);
        a0 = fmaf(p4.w, v3.x, a0);
        a1 = fmaf(p4.w, v3.y, a1);
      }
      *(float2*)(part_acc + (slot_base + (int64_t)g * max_chunks) * D + 2 * e) = make_float2(a0, a1);
    }
    __syncthreads();  // Qs and Ps are rewritten for the next token
  }
}

// A prefill chunk's attention slice on the matrix cores
// (v_mfma_f32_16x16x32_f16): one block = one 64-key slice x one key head x
// 64 query rows, the rows being TQ = 64 / GROUP consecutive tokens times the
// GROUP query heads of that key head (row r = token r / GROUP, head r %
// GROUP).  One sequence's chunk only (its tokens share the cache).
//   S = Q K^T: queries as three halves (q1 = f16(q), q2 = f16(q - q1),
//   q3 = f16(q - q1 - q2): every bit of the f32 query), keys exact halves,
//   f32 accumulation.  Two halves (22 bits) were not enough: a softmax feels
//   a score's absolute error, and scores of a few hundred turned the last
//   bits of the query into 1e-4 of the output.
//   P = exp(S*scale - rowmax) per row over the slice's live keys (key <
//   pos[t] + 1, cell held), written as (m, l) like the VALU kernel.
//   O = P V with P as two halves and V (staged transposed) exact halves.
// The partial sums land where attend_split_kernel writes them, so
// attend_merge_kernel folds them unchanged.
// MFMA fragments (16x16x32): lane l holds row/column l % 16 and values
// 8 (l / 16) .. +8 of the 32; the result element i of lane l is row
// 4 (l / 16) + i, column l % 16.
typedef _Float16 att_h8 __attribute__((ext_vector_type(8)));
typedef float att_f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ att_f4 att_mfma(att_h8 a, att_h8 b, att_f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

constexpr int kChunkKeys = 64;
// The matrix-core slices split P (at most 1) into two halves after lifting
// it by 2^14, and scale the sums back: exact powers of two, which keep the
// low halves of weights down to ~1e-8 out of the f16 subnormals.
constexpr float kPLift = 16384.0f, kPDrop = 1.0f / 16384.0f;
__host__ __device__ __forceinline__ int attn_chunk_pad(int d) { return d + 8; }  // halves per LDS row
__host__ __device__ __forceinline__ size_t attn_chunk_lds_bytes(int head_dim) {
  const int dp = attn_chunk_pad(head_dim), kp = kChunkKeys + 8;
  return 2 * ((size_t)kChunkKeys * dp + (size_t)head_dim * kp + (size_t)2 * 4 * 16 * kp);
}

template <int GROUP, int D>
__global__ __launch_bounds__(256) void attend_chunk_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc, const __half* __restrict__ vc,
    int heads, int kv_heads, float scale, const int32_t* __restrict__ pos_dev, int max_chunks,
    float* __restrict__ part_acc, float* __restrict__ part_ml, const int32_t* __restrict__ kv_index, int tokens) {
  constexpr int TQ = 64 / GROUP;
  constexpr int DP = D + 8, KP = kChunkKeys + 8;
  const int c = blockIdx.x, kvh = blockIdx.y, t0 = blockIdx.z * TQ;
  const int t1 = min(t0 + TQ, tokens);
  int count_max = 0;
  for (int t = t0; t < t1; t++) count_max = max(count_max, pos_dev[t] + 1);
  const int start = c * kChunkKeys;
  if (start >= count_max) return;
  const int nk_max = min(kChunkKeys, count_max - start);
  const int kvw = kv_heads * D;
  extern __shared__ uint4 lds4[];
  _Float16* Ks = (_Float16*)lds4;
  _Float16* Vt = Ks + kChunkKeys * DP;
  _Float16* Ph = Vt + D * KP;
  _Float16* Pl = Ph + 4 * 16 * KP;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lm = lane & 15, lk = lane >> 4;

  // keys (rows) and values (transposed); keys past the end repeat the last
  // live one (masked below); every load issued before any LDS store
  const __half* kbase = kc + (int64_t)kvh * D;
  const __half* vbase = vc + (int64_t)kvh * D;
  constexpr int pieces = D / 8, total = kChunkKeys * pieces, per = total / 256;
  static_assert(total % 256 == 0, "whole pieces per thread");
  uint4 kv[per], vv[per];
#pragma unroll
  for (int j = 0; j < per; j++) {
    const int i = tid + j * 256;
    const int key = min(i / pieces, nk_max - 1), pc = i % pieces;
    const int cell = max(kv_cell(kv_index, 0, t0, start + key), 0);
    const int64_t off = (int64_t)cell * kvw + pc * 8;
    kv[j] = *(const uint4*)(kbase + off);
    vv[j] = *(const uint4*)(vbase + off);
  }
  // this wave's 16 query rows straight into A fragments (row r = token
  // t0 + r / GROUP, head kvh * GROUP + r % GROUP): lane row lm, values
  // 32 ks + 8 lk .. +8 of each 32-value step, as three halves
  const int row0 = wave * 16;
  float4 qraw[D / 32][2];
  {
    const int r = row0 + lm, t = t0 + r / GROUP;
    const float* qr = q + (int64_t)min(t, tokens - 1) * q_stride + (int64_t)(kvh * GROUP + r % GROUP) * D;
#pragma unroll
    for (int ks = 0; ks < D / 32; ks++) {
      qraw[ks][0] = t < tokens ? *(const float4*)(qr + 32 * ks + 8 * lk) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      qraw[ks][1] = t < tokens ? *(const float4*)(qr + 32 * ks + 8 * lk + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
#pragma unroll
  for (int j = 0; j < per; j++) {
    const int i = tid + j * 256;
    const int key = i / pieces, pc = i % pieces;
    *(uint4*)(Ks + key * DP + pc * 8) = kv[j];
    const _Float16* v8 = (const _Float16*)&vv[j];
#pragma unroll
    for (int d = 0; d < 8; d++) Vt[(pc * 8 + d) * KP + key] = v8[d];
  }
  __syncthreads();

  // S for this wave's 16 rows x 64 keys
  att_f4 sacc[4];
#pragma unroll
  for (int nt = 0; nt < 4; nt++) sacc[nt] = att_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ks = 0; ks < D / 32; ks++) {
    att_h8 ah, am, al;
    const float qf[8] = {qraw[ks][0].x, qraw[ks][0].y, qraw[ks][0].z, qraw[ks][0].w,
                         qraw[ks][1].x, qraw[ks][1].y, qraw[ks][1].z, qraw[ks][1].w};
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const _Float16 h = (_Float16)qf[u];
      const float r1 = qf[u] - (float)h;  // exact
      const _Float16 mid = (_Float16)r1;
      ah[u] = h;
      am[u] = mid;
      al[u] = (_Float16)(r1 - (float)mid);
    }
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const att_h8 b = *(const att_h8*)(Ks + (16 * nt + lm) * DP + 32 * ks + 8 * lk);
      sacc[nt] = att_mfma(ah, b, sacc[nt]);
      sacc[nt] = att_mfma(am, b, sacc[nt]);
      sacc[nt] = att_mfma(al, b, sacc[nt]);
    }
  }
  // rows 4 lk + i of this wave: token, its count, the slice's live keys
  float mrow[4], lrow[4];
  int cnt[4];
  bool rowlive[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = row0 + 4 * lk + i, t = t0 + r / GROUP;
    rowlive[i] = t < tokens;
    cnt[i] = rowlive[i] ? pos_dev[t] + 1 : 0;
    rowlive[i] = rowlive[i] && start < cnt[i];
  }
  float pv[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float m = -INFINITY;
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const int key = start + 16 * nt + lm;
      const bool live = key < cnt[i] && (!kv_index || kv_cell(kv_index, 0, t0, key) >= 0);
      pv[i][nt] = live ? sacc[nt][i] * scale : -INFINITY;
      m = fmaxf(m, pv[i][nt]);
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0.0f;
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      pv[i][nt] = pv[i][nt] == -INFINITY ? 0.0f : expf(pv[i][nt] - m);
      l += pv[i][nt];
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    mrow[i] = m;
    lrow[i] = l;
  }
  // P into this wave's LDS rows (hi and lo halves), read back as A fragments
  _Float16* ph = Ph + wave * 16 * KP;
  _Float16* pl = Pl + wave * 16 * KP;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
      const float p = pv[i][nt] * kPLift;  // see kPLift
      const _Float16 h = (_Float16)p;
      ph[(4 * lk + i) * KP + 16 * nt + lm] = h;
      pl[(4 * lk + i) * KP + 16 * nt + lm] = (_Float16)(p - (float)h);
    }
  // (a wave's LDS operations complete in order: its reads below see these stores)
  att_f4 oacc[D / 16];
#pragma unroll
  for (int nt = 0; nt < D / 16; nt++) oacc[nt] = att_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int ks = 0; ks < kChunkKeys / 32; ks++) {
    const att_h8 ah = *(const att_h8*)(ph + lm * KP + 32 * ks + 8 * lk);
    const att_h8 al = *(const att_h8*)(pl + lm * KP + 32 * ks + 8 * lk);
#pragma unroll
    for (int nt = 0; nt < D / 16; nt++) {
      const att_h8 b = *(const att_h8*)(Vt + (16 * nt + lm) * KP + 32 * ks + 8 * lk);
      oacc[nt] = att_mfma(ah, b, oacc[nt]);
      oacc[nt] = att_mfma(al, b, oacc[nt]);
    }
  }
  // the slot of (token, head): as attend_split_kernel
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (!rowlive[i]) continue;
    const int r = row0 + 4 * lk + i, t = t0 + r / GROUP, h = kvh * GROUP + r % GROUP;
    const int64_t slot = ((int64_t)t * heads + h) * max_chunks + c;
#pragma unroll
    for (int nt = 0; nt < D / 16; nt++) part_acc[slot * D + 16 * nt + lm] = oacc[nt][i] * kPDrop;
    if (lm == 0) {
      part_ml[slot * 2 + 0] = mrow[i];
      part_ml[slot * 2 + 1] = lrow[i];
    }
  }
}

// The same slice over a q8_0 cache (repack.mojo:181 CACHE_Q8): a position's
// row is kv_width signed bytes, then kv_width/32 float16 factors, `row`
// halves in all.  Quants and factors are staged in LDS as they are (half the
// bytes of the f16 form); a key or value element is read as float(q) *
// float(factor), which is gpu.mojo:1168 cache_load, and then used exactly
// as the f16 kernel uses a widened half.
template <int GROUP>
__global__ __launch_bounds__(kAttnThreads) void attend_split_q8_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc,
    const __half* __restrict__ vc, int64_t cache_stride, int row, int heads, int kv_heads, int head_dim,
    float scale, const int32_t* __restrict__ pos_dev, int count_host, int max_chunks,
    float* __restrict__ part_acc, float* __restrict__ part_ml, const int32_t* __restrict__ kv_index,
    int64_t index_stride) {
#pragma clang fp contract(off)
  const int c = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;
  const int kk = attn_slice(head_dim);
  const int start = c * kk;
  if (start >= count) return;
  const int D = head_dim, KQ = head_dim + 16, NB = head_dim >> 5;  // LDS key rows padded by 16 bytes
  const int nk = min(kk, count - start);
  const int kvw = kv_heads * D;
  extern __shared__ uint4 lds4[];
  int8_t* Kq = (int8_t*)lds4;
  int8_t* Vq = Kq + kk * KQ;
  float* Ksc = (float*)(Vq + kk * D);
  float* Vsc = Ksc + kk * NB;
  float* Qs = Vsc + kk * NB;
  float* Ps = Qs + GROUP * D;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  const int64_t seq = kv_index ? 0 : (int64_t)t * cache_stride;
  const __half* kseq = kc + seq;
  const __half* vseq = vc + seq;
  // quants in 16-byte pieces, every load of the slice issued before any
  // LDS store; keys past the end repeat the last live one (masked below)
  const int pieces = D >> 4;
  const int total = kk * pieces;
  const float4* q4 = (const float4*)(q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * D);
  const int nq4 = GROUP * D / 4;
  const float4 qv = q4[min(tid, nq4 - 1)];
  for (int b0 = 0; b0 < total; b0 += kAttnThreads * 2) {
    uint4 kv[2], vv[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = min(b0 + tid + j * kAttnThreads, total - 1);
      const int key = min(i / pieces, nk - 1), pc = i % pieces;
      const int cell = max(kv_cell(kv_index, index_stride, t, start + key), 0);
      const int64_t off = (int64_t)cell * row * 2 + (int64_t)kvh * D + pc * 16;  // bytes
      kv[j] = *(const uint4*)((const int8_t*)kseq + off);
      vv[j] = *(const uint4*)((const int8_t*)vseq + off);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = b0 + tid + j * kAttnThreads;
      const int key = i / pieces, pc = i % pieces;
      if (i < total) {
        *(uint4*)(Kq + key * KQ + pc * 16) = kv[j];
        *(uint4*)(Vq + key * D + pc * 16) = vv[j];
      }
    }
  }
  for (int i = tid; i < kk * NB; i += kAttnThreads) {
    const int key = min(i / NB, nk - 1), b = i % NB;
    const int cell = max(kv_cell(kv_index, index_stride, t, start + key), 0);
    const int64_t at = (int64_t)cell * row + (kvw >> 1) + (kvh * D >> 5) + b;  // halves
    Ksc[i] = __half2float(kseq[at]);
    Vsc[i] = __half2float(vseq[at]);
  }
  if (tid < nq4) ((float4*)Qs)[tid] = qv;
  for (int i = tid + kAttnThreads; i < nq4; i += kAttnThreads) ((float4*)Qs)[i] = q4[i];
  __syncthreads();

  const int64_t slot_base = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks + c;
  for (int g = wave; g < GROUP; g += kAttnThreads / kWave) {
    float sdot = 0.0f;
    if (lane < kk) {
      const int8_t* kr = Kq + lane * KQ;
      const float* qg = Qs + g * D;
      for (int d = 0; d < D; d += 16) {
        const uint4 raw = *(const uint4*)(kr + d);
        const int8_t* b = (const int8_t*)&raw;
        const float f = Ksc[lane * NB + (d >> 5)];
#pragma unroll
        for (int i = 0; i < 16; i++) sdot = fmaf(qg[d + i], (float)b[i] * f, sdot);
      }
    }
    const bool live = lane < nk && (!kv_index || kv_cell(kv_index, index_stride, t, start + lane) >= 0);
    const float sc = live ? sdot * scale : -INFINITY;
    float m = sc;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float pr = live ? expf(sc - m) : 0.0f;
    float l = pr;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    if (lane < kk) Ps[g * kk + lane] = pr;
    if (lane == 0) {
      part_ml[(slot_base + (int64_t)g * max_chunks) * 2 + 0] = m;
      part_ml[(slot_base + (int64_t)g * max_chunks) * 2 + 1] = l;
    }
  }
  __syncthreads();
  const int halfD = D >> 1;
  for (int o = tid; o < GROUP * halfD; o += kAttnThreads) {
    const int g = o / halfD, e = o - g * halfD;
    const float* pg = Ps + g * kk;
    const int b = (2 * e) >> 5;
    float a0 = 0.0f, a1 = 0.0f;
    for (int k = 0; k < nk; k += 4) {
      const float4 p4 = *(const float4*)(pg + k);
      const float pk[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const char2 v = *(const char2*)(Vq + (k + j) * D + 2 * e);
        const float f = Vsc[(k + j) * NB + b];
        a0 = fmaf(pk[j], (float)v.x * f, a0);
        a1 = fmaf(pk[j], (float)v.y * f, a1);
      }
    }
    *(float2*)(part_acc + (slot_base + (int64_t)g * max_chunks) * D + 2 * e) = make_float2(a0, a1);
  }
}

// f32 k / v rows -> q8_0 cache rows (gpu_ops.mojo:1531 store_kv_q8_kernel):
// each 32-lane half-wave encodes one block: factor amax / 127 stored as a
// half after the row's quants, quants round(v * 127 / amax) half away from
// zero, clamped to [-127, 127].  Grid: (blocks of 8 per 256 threads, tokens, 2
// for k then v).
__global__ __launch_bounds__(256) void store_kv_q8_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                          int kv_width, __half* __restrict__ kc,
                                                          __half* __restrict__ vc, const int32_t* __restrict__ slot_dev,
                                                          int slot_host, int64_t src_stride, int64_t cache_stride,
                                                          int row) {
  const int t = blockIdx.y;
  const bool isv = blockIdx.z == 1;
  const int lane32 = threadIdx.x & 31;
  const int b = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // block of the row
  if (b >= (kv_width >> 5)) return;  // whole half-waves leave together
  const int slot = slot_dev ? slot_dev[t] : slot_host;
  const float x = (isv ? v : k)[(int64_t)t * src_stride + b * 32 + lane32];
  q8_store_block(x, (isv ? vc : kc) + (int64_t)t * cache_stride + (int64_t)slot * row, b, kv_width, lane32);
}

// One block per (query head, token); thread d owns output dimension d (the
// block has max(64, head_dim) threads).  The first 64 slices' partial values
// and (max, sum) pairs are loaded before the position is known (slots past
// the live slices are read and then ignored), so the merge costs one memory
// latency, not a position load followed by one.  Each wave holds slice c's
// (max, sum) in lane c, derives the weights exp(m_c - M) there, and every
// thread takes the weights lane by lane (readlane) while it folds the values
// in slice order: no LDS and no barrier.  B, the slices a round takes, is
// the workspace's slice count rounded up to a multiple of 8 (at most 64,
// further rounds past it): each up-front load is an instruction of every
// thread, and 64 of them where 36 slices are live made a decode step
// 12-32 us slower (batch 1 to 8) than 40 or 48.
template <int B>
__global__ void attend_merge_kernel(const float* __restrict__ part_acc, const float* __restrict__ part_ml,
                                    int heads, int head_dim, const int32_t* __restrict__ pos_dev,
                                    int count_host, int max_chunks, float* __restrict__ out,
                                    uint8_t* __restrict__ xq, uint8_t* __restrict__ hx) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int64_t slot = ((int64_t)t * heads + h) * max_chunks;
  const int d = threadIdx.x, lane = d & 63;
  const bool live = d < head_dim;
  const float* pa = part_acc + slot * head_dim + min(d, head_dim - 1);
  const float2* pml = (const float2*)part_ml + slot;
  float a[B];
#pragma unroll
  for (int k = 0; k < B; k++) a[k] = pa[(int64_t)min(k, max_chunks - 1) * head_dim];
  float2 ml = pml[min(lane, max_chunks - 1)];
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;  // a position p attends over p + 1 slots
  const int kk = attn_slice(head_dim);
  const int chunks = min((count + kk - 1) / kk, max_chunks);
  // the largest slice max over every round
  float M = lane < chunks ? ml.x : -INFINITY;
  for (int c0 = B; c0 < chunks; c0 += B) {
    const int c = c0 + lane;
    if (c < chunks) M = fmaxf(M, pml[c].x);
  }
  M = lanes::reduce<64>(M, lanes::Max{});
  float o = 0.0f, L = 0.0f;
  for (int c0 = 0; c0 < chunks; c0 += B) {
    if (c0 > 0) {
#pragma unroll
      for (int k = 0; k < B; k++) a[k] = pa[(int64_t)min(c0 + k, chunks - 1) * head_dim];
      ml = pml[min(c0 + lane, chunks - 1)];
    }
    const int n = min(chunks - c0, B);
    const float w = lane < n ? expf(ml.x - M) : 0.0f;
    L += lane < n ? ml.y * w : 0.0f;
#pragma unroll
    for (int k = 0; k < B; k++) {
      if (k < n) o = fmaf(a[k], __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), k)), o);
    }
  }
  L = lanes::reduce<64>(L, lanes::Add{});
  o *= 1.0f / L;
  const int width = heads * head_dim;
  if (live && out) out[(int64_t)t * width + (int64_t)h * head_dim + d] = o;
  if (xq)
    quantize_group32(o, threadIdx.x & 31, (h * head_dim + d) >> 5, width >> 5,
                     xq + (int64_t)t * xq_token_bytes(width), live,
                     hx ? hx + (int64_t)t * xq_token_bytes(width) : nullptr);
}

// ---- decode attention slices ------------------------------------------------
// attend_wide_kernel: the slice half of attention.mojo:144 attend
// (gpu_ops.mojo:929 attend_split_kernel) for one query token per sequence
// over an f16 cache, head_dim 64 or 128.  A block takes one (64-key slice,
// key head, token) as attend_split_kernel does, with NT = 1024 threads (one
// token; 512 for a batch, so that two blocks share a CU) instead of 256, so
// every stage is spread over NT / 64 waves:
//   * the slice's keys and values go to LDS with one load per thread;
//   * each (query head, key) score is SPL threads of DPT dimensions each,
//     added by shuffles;
//   * the slice softmax is one wave per query head (lane = key);
//   * each weighted value pair (query head, 2 dims) is KQ threads over
//     interleaved keys, added by shuffles.
// It writes each slice's (max, sum) and unnormalised values exactly where
// attend_split_kernel does, and attend_merge_kernel folds them.
constexpr int kWideKeys = 64;

template <int GROUP, int D, int NT>
struct WideShape {
  static constexpr int KS = D + 8;   // K rows in halves (16-byte pad)
  static constexpr int VS = D + 32;  // V rows: 16 dwords of pad, so the KQ lanes
                                     // reading one dim pair hit distinct banks
  static constexpr int SPL0 = NT / (GROUP * kWideKeys);
  static constexpr int SPL = SPL0 < (D / 8) ? SPL0 : (D / 8);  // threads per score
  static constexpr int DPT = D / SPL;                           // dims per score thread
  static constexpr int KQ = 2 * NT / (GROUP * D);               // threads per output pair
};

template <int GROUP, int D, int NT>
__global__ __launch_bounds__(NT) void attend_wide_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc, const __half* __restrict__ vc,
    int64_t cache_stride, int heads, int kv_heads, float scale, const int32_t* __restrict__ pos_dev,
    int count_host, int max_chunks, float* __restrict__ part_acc, float* __restrict__ part_ml,
    const int32_t* __restrict__ kv_index, int64_t index_stride) {
  using S = WideShape<GROUP, D, NT>;
  constexpr int KK = kWideKeys, PIECES = D / 8, TOTAL = KK * PIECES, PAIRS = D / 2;
  constexpr int PER = (TOTAL + NT - 1) / NT;  // 16-byte pieces of K (and of V) per thread
  static_assert(GROUP * D / 4 <= NT && S::SPL >= 1 && S::KQ >= 1 && S::KQ <= 64, "shape");
  __shared__ __align__(16) __half Ks[KK * S::KS];
  __shared__ __align__(16) __half Vs[KK * S::VS];
  __shared__ __align__(16) float Qs[GROUP * D];
  __shared__ float Ss[GROUP * KK];
  const int c = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;  // a position p attends over p + 1 slots
  const int start = c * KK;
  if (start >= count) return;
  const int nk = min(KK, count - start);
  const int kvw = kv_heads * D;

  // stage: the group's queries, one 16-byte piece of a key and of a value
  // per thread (keys past the end repeat the last live one; masked below)
  const float* qg = q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * D;
  const bool has_q = tid < GROUP * D / 4;
  const float4 qv = ((const float4*)qg)[has_q ? tid : 0];
  const int64_t seq = kv_index ? 0 : (int64_t)t * cache_stride;
  uint4 kraw[PER], vraw[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = min(tid + j * NT, TOTAL - 1);
    const int skey = i / PIECES, pc = i % PIECES;
    const int cell = max(kv_cell(kv_index, index_stride, t, start + min(skey, nk - 1)), 0);
    const int64_t off = seq + (int64_t)cell * kvw + (int64_t)kvh * D + pc * 8;
    kraw[j] = *(const uint4*)(kc + off);
    vraw[j] = *(const uint4*)(vc + off);
  }
  if (has_q) ((float4*)Qs)[tid] = qv;
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * NT;
    const int skey = i / PIECES, pc = i % PIECES;
    if (i < TOTAL) {
      *(uint4*)(Ks + skey * S::KS + pc * 8) = kraw[j];
      *(uint4*)(Vs + skey * S::VS + pc * 8) = vraw[j];
    }
  }
  __syncthreads();

  // scores: thread = (query head g, key, part of DPT dims)
  {
    const int dot = tid / S::SPL, part = tid % S::SPL;
    const int g = dot / KK, key = dot % KK;
    float sdot = 0.0f;
    if (dot < GROUP * KK) {
      const __half* kr = Ks + key * S::KS + part * S::DPT;
      const float* qq = Qs + g * D + part * S::DPT;
#pragma unroll
      for (int d = 0; d < S::DPT; d += 8) {
        const uint4 raw = *(const uint4*)(kr + d);
        const __half2* h2 = (const __half2*)&raw;
        const float4 qa = *(const float4*)(qq + d), qb = *(const float4*)(qq + d + 4);
        const float2 k0 = __half22float2(h2[0]), k1 = __half22float2(h2[1]);
        const float2 k2 = __half22float2(h2[2]), k3 = __half22float2(h2[3]);
        sdot = fmaf(qa.x, k0.x, sdot);
        sdot = fmaf(qa.y, k0.y, sdot);
        sdot = fmaf(qa.z, k1.x, sdot);
        sdot = fmaf(qa.w, k1.y, sdot);
        sdot = fmaf(qb.x, k2.x, sdot);
        sdot = fmaf(qb.y, k2.y, sdot);
        sdot = fmaf(qb.z, k3.x, sdot);
        sdot = fmaf(qb.w, k3.y, sdot);
      }
    }
    sdot = lanes::reduce<S::SPL>(sdot, lanes::Add{});
    if (part == 0 && dot < GROUP * KK) {
      const bool live = key < nk && (!kv_index || kv_cell(kv_index, index_stride, t, start + key) >= 0);
      Ss[g * KK + key] = live ? sdot * scale : -INFINITY;
    }
  }
  __syncthreads();
  const int64_t slot0 = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks;
  // slice softmax: wave g takes query head g, lane = key
  if (wave < GROUP) {
    const float sc = Ss[wave * KK + lane];
    float m = sc;
    m = lanes::reduce<64>(m, lanes::Max{});
    const float pr = sc == -INFINITY ? 0.0f : expf(sc - m);
    float l = pr;
    l = lanes::reduce<64>(l, lanes::Add{});
    Ss[wave * KK + lane] = pr;
    if (lane == 0) *(float2*)(part_ml + (slot0 + (int64_t)wave * max_chunks + c) * 2) = make_float2(m, l);
  }
  __syncthreads();
  // unnormalised weighted values: thread = (query head, dim pair, key residue kq)
  const int kq = tid % S::KQ, oe = tid / S::KQ;
  const int g = oe / PAIRS, e = oe % PAIRS;
  float a0 = 0.0f, a1 = 0.0f;
  if (oe < GROUP * PAIRS) {
    const float* pg = Ss + g * KK;
#pragma unroll 4
    for (int k = kq; k < KK; k += S::KQ) {
      const float p = pg[k];
      const float2 v = __half22float2(*(const __half2*)(Vs + k * S::VS + 2 * e));
      a0 = fmaf(p, v.x, a0);
      a1 = fmaf(p, v.y, a1);
    }
  }
  a0 = lanes::reduce<S::KQ>(a0, lanes::Add{});
  a1 = lanes::reduce<S::KQ>(a1, lanes::Add{});
  if (kq == 0 && oe < GROUP * PAIRS)
    *(float2*)(part_acc + (slot0 + (int64_t)g * max_chunks + c) * D + 2 * e) = make_float2(a0, a1);
}

// attend_mfma_kernel: the same slice as attend_wide_kernel (one 64-key
// slice x one key head x one token, f16 cache, GROUP <= 4 query heads of
// head_dim D), with both products on the matrix cores
// (v_mfma_f32_16x16x32_f16), as attend_chunk_kernel computes them for a
// prefill chunk.  At 4 and 8 sequences the VALU dot loops of the wide
// kernel bound its time; here a block of 256 threads does
//   * S = K Q^T: wave w takes keys 16w..16w+15 as the A rows, read straight
//     from the cache into fragments; the N columns are the GROUP queries as
//     three halves each (q1 = f16(q), q2 = f16(q - q1), q3 = f16(q - q1 -
//     q2): every bit of the f32 query), staged once in LDS, so a score is
//     the sum of three columns;
//   * the slice softmax, one wave per query head (lane = key), as the wide
//     kernel;
//   * O = P V: P as two halves (rows h and GROUP + h), V staged by rows
//     (exact halves); wave w takes D / 64 of the D / 16 column tiles.
// MFMA fragments (16x16x32): lane l holds row / column l % 16 and values
// 8 (l / 16) .. +8 of the 32; result element i of lane l is row 4 (l / 16)
// + i, column l % 16.  The partial sums land where attend_wide_kernel
// writes them.
// PAGED: kv_index maps positions to cache cells; without it the cell is
// the position, and no index load sits under a branch (which would make the
// compiler wait for every load in flight at the join: the keys before the
// values went out).
template <int GROUP, int D, bool PAGED>
__global__ __launch_bounds__(256) void attend_mfma_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc, const __half* __restrict__ vc,
    int64_t cache_stride, int heads, int kv_heads, float scale, const int32_t* __restrict__ pos_dev,
    int count_host, int max_chunks, float* __restrict__ part_acc, float* __restrict__ part_ml,
    const int32_t* __restrict__ kv_index_arg, int64_t index_stride) {
  const int32_t* __restrict__ kv_index = PAGED ? kv_index_arg : nullptr;
  static_assert(GROUP == 1 || GROUP == 2 || GROUP == 4, "three halves of GROUP queries fill at most 12 columns");
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  constexpr int KK = kWideKeys, QP = D + 8, KP = KK + 8;
  constexpr int PIECES = D / 8, PER = KK * PIECES / 256;
  __shared__ __align__(16) _Float16 Qh[3 * GROUP * QP];
  __shared__ __align__(16) _Float16 Vr[KK * QP];
  __shared__ __align__(16) _Float16 Ph[2 * GROUP * KP];
  __shared__ float Ss[GROUP * KK];
  const int c = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lm = lane & 15, lk = lane >> 4;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;
  const int start = c * KK;
  if (start >= count) return;
  const int nk = min(KK, count - start);
  const int kvw = kv_heads * D;
  const int64_t seq = kv_index ? 0 : (int64_t)t * cache_stride;

  // this wave's 16 keys as A fragments (key 16 wave + lm, values 32 ks +
  // 8 lk .. +8), the block's share of the values, and the queries; keys past
  // the end repeat the last live one (masked below)
  const __half* kb = kc + seq + (int64_t)kvh * D;
  const __half* vb = vc + seq + (int64_t)kvh * D;
  // the queries first, then the keys, then the values: loads complete in
  // issue order, so the query halves wait only for the queries and the
  // scores only for the keys, while the values are still arriving
  constexpr int NQ4 = GROUP * D / 4;
  const float* qg = q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * D;
  const att_f4 qv = ((const att_f4*)qg)[tid < NQ4 ? tid : 0];
  __builtin_amdgcn_sched_barrier(0);
  att_h8 ka[D / 32];
  {
    const int cell = max(kv_cell(kv_index, index_stride, t, start + min(16 * wave + lm, nk - 1)), 0);
#pragma unroll
    for (int ks = 0; ks < D / 32; ks++) ka[ks] = *(const att_h8*)(kb + (int64_t)cell * kvw + 32 * ks + 8 * lk);
  }
  // (native vectors: an array of HIP's uint4 struct went to scratch)
  att_h8 vraw[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * 256;
    const int key = i / PIECES, pc = i % PIECES;
    const int cell = max(kv_cell(kv_index, index_stride, t, start + min(key, nk - 1)), 0);
    vraw[j] = *(const att_h8*)(vb + (int64_t)cell * kvw + pc * 8);
  }
  __builtin_amdgcn_sched_barrier(0);
  {
    // query h = tid / (D / 4), dims 4 (tid % (D / 4)) .. +4, as three halves
    // (computed by every thread, so the query load is not sunk into the
    // branch behind the keys and values; threads past NQ4 store nothing)
    const int h = (tid < NQ4 ? tid : 0) / (D / 4), d0 = 4 * ((tid < NQ4 ? tid : 0) % (D / 4));
    float qf[4] = {qv.x, qv.y, qv.z, qv.w};
    // here, not inside the branch below (where the compiler would sink the
    // query load, behind the keys and values)
    asm volatile("" : "+v"(qf[0]), "+v"(qf[1]), "+v"(qf[2]), "+v"(qf[3]));
    _Float16 hv[3][4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const _Float16 h1 = (_Float16)qf[u];
      const float r1 = qf[u] - (float)h1;  // exact
      const _Float16 h2 = (_Float16)r1;
      hv[0][u] = h1;
      hv[1][u] = h2;
      hv[2][u] = (_Float16)(r1 - (float)h2);
    }
    if (tid < NQ4) {
#pragma unroll
      for (int k = 0; k < 3; k++)
#pragma unroll
        for (int u = 0; u < 4; u++) Qh[(k * GROUP + h) * QP + d0 + u] = hv[k][u];
    }
  }
  __syncthreads();

  // S for keys 16 wave .. +15 against column lm = (half lm / GROUP, query
  // lm % GROUP); columns from 3 GROUP on are zero
  {
    att_f4 sacc = att_f4{0.0f, 0.0f, 0.0f, 0.0f};
    const bool qcol = lm < 3 * GROUP;
    const int qrow = qcol ? lm : 0;
#pragma unroll
    for (int ks = 0; ks < D / 32; ks++) {
      const att_h8 qb = *(const att_h8*)(Qh + qrow * QP + 32 * ks + 8 * lk);
      sacc = att_mfma(ka[ks], qcol ? qb : att_h8{0, 0, 0, 0, 0, 0, 0, 0}, sacc);
    }
    // lanes lm < GROUP: the score of query lm at keys 16 wave + 4 lk + i,
    // its three halves added in order
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // (row shifts within the lane's 16-lane row: lanes lm < GROUP read
      // lm + GROUP and lm + 2 GROUP)
      const float s2 = __uint_as_float(lanes::dpp<0x100 + GROUP>(__float_as_uint(sacc[i])));
      const float s3 = __uint_as_float(lanes::dpp<0x100 + 2 * GROUP>(__float_as_uint(sacc[i])));
      const float sc = (sacc[i] + s2) + s3;
      const int key = 16 * wave + 4 * lk + i;
      const bool live = key < nk && (!kv_index || kv_cell(kv_index, index_stride, t, start + key) >= 0);
      if (lm < GROUP) Ss[lm * KK + key] = live ? sc * scale : -INFINITY;
    }
  }
  // the values into LDS once the scores are out (they are read after the
  // softmax barrier)
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * 256;
    const int key = i / PIECES, pc = i % PIECES;
    *(att_h8*)(Vr + key * QP + pc * 8) = vraw[j];
  }
  __syncthreads();
  const int64_t slot0 = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks;
  // slice softmax: wave g takes query g, lane = key; P as two halves
  if (wave < GROUP) {
    const float sc = Ss[wave * KK + lane];
    const float m = lanes::reduce<64>(sc, lanes::Max{});
    const float pr = sc == -INFINITY ? 0.0f : expf(sc - m);
    const float l = lanes::reduce<64>(pr, lanes::Add{});
    // P lifted by 2^14 (exact; p <= 1 stays below the largest half) so that
    // the low halves of small weights are not f16 subnormals
    const float pl = pr * kPLift;
    const _Float16 ph = (_Float16)pl;
    Ph[wave * KP + lane] = ph;
    Ph[(GROUP + wave) * KP + lane] = (_Float16)(pl - (float)ph);
    if (lane == 0) *(float2*)(part_ml + (slot0 + (int64_t)wave * max_chunks + c) * 2) = make_float2(m, l);
  }
  __syncthreads();
  // O for column tiles nt = wave, wave + 4, ...: rows (half, query) =
  // 4 lk + i, column = dim 16 nt + lm; rows from 2 GROUP on are zero
  {
    const bool prow = lm < 2 * GROUP;
    const int arow = prow ? lm : 0;
    att_h8 pa[KK / 32];
#pragma unroll
    for (int ks = 0; ks < KK / 32; ks++) {
      const att_h8 a = *(const att_h8*)(Ph + arow * KP + 32 * ks + 8 * lk);
      pa[ks] = prow ? a : att_h8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int nt = wave; nt < D / 16; nt += 4) {
      att_f4 oacc = att_f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KK / 32; ks++)
      {
        // the B fragment (dim 16 nt + lm, keys 32 ks + 8 lk .. +8) gathered
        // from the row-major values: staging them transposed (a 2-byte
        // store per value, 8-way bank conflicts) took the kernel from 10.5
        // to 17.9 us at 4 sequences
        att_h8 vb;
#pragma unroll
        for (int e = 0; e < 8; e++) vb[e] = Vr[(32 * ks + 8 * lk + e) * QP + 16 * nt + lm];
        oacc = att_mfma(pa[ks], vb, oacc);
      }
      const int dim = 16 * nt + lm;
      // query g's output: row g (hi) plus row GROUP + g (lo)
      if constexpr (GROUP == 4) {
        // rows 0..3 in lanes lk = 0, rows 4..7 in lanes lk = 1
#pragma unroll
        for (int i = 0; i < 4; i++) {
          // row 0 (lk = 0) and row 1 swapped across: p[1] of a row-0 lane is
          // its row-1 partner's value
          const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(oacc[i]), __float_as_uint(oacc[i]), false,
                                                          false);
          const float hi = __uint_as_float(p[0]), lo = __uint_as_float(p[1]);
          if (lk == 0) part_acc[(slot0 + (int64_t)i * max_chunks + c) * D + dim] = (hi + lo) * kPDrop;
        }
      } else if constexpr (GROUP == 2) {
        if (lk == 0) {
          part_acc[(slot0 + 0 * (int64_t)max_chunks + c) * D + dim] = (oacc[0] + oacc[2]) * kPDrop;
          part_acc[(slot0 + 1 * (int64_t)max_chunks + c) * D + dim] = (oacc[1] + oacc[3]) * kPDrop;
        }
      } else {
        if (lk == 0) part_acc[(slot0 + c) * D + dim] = (oacc[0] + oacc[1]) * kPDrop;
      }
    }
  }
}

// attend_wide_q8_kernel: attend_wide_kernel over a q8_0 cache (the row's
// quants of every key head, then its factors: cache_row), the arithmetic of
// attend_split_q8_kernel (each key or value element float(quant) *
// float(factor) before it is used) spread the same way as the f16 form:
// a score is SPL threads of DPT dims (whole 32-value blocks, so one factor a
// block), a weighted value pair is KQ threads over interleaved keys, and the
// slice softmax is one wave per query head.
template <int GROUP, int D, int NT>
__global__ __launch_bounds__(NT) void attend_wide_q8_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc, const __half* __restrict__ vc,
    int64_t cache_stride, int row, int heads, int kv_heads, float scale, const int32_t* __restrict__ pos_dev,
    int count_host, int max_chunks, float* __restrict__ part_acc, float* __restrict__ part_ml,
    const int32_t* __restrict__ kv_index, int64_t index_stride) {
#pragma clang fp contract(off)
  using S = WideShape<GROUP, D, NT>;
  constexpr int KK = kWideKeys, NB = D / 32, PIECES = D / 16, TOTAL = KK * PIECES, PAIRS = D / 2;
  constexpr int PER = (TOTAL + NT - 1) / NT;  // 16-byte pieces of K (and of V) per thread
  constexpr int KQR = D + 16;                 // LDS key rows in bytes (16 bytes of pad)
  static_assert(GROUP * D / 4 <= NT && S::KQ >= 1 && S::KQ <= 64, "shape");
  if constexpr (S::DPT % 16 != 0) {
    return;  // never launched (wide_q8_fits): a score part is whole 16-byte pieces
  } else {
  __shared__ __align__(16) int8_t Kq[KK * KQR];
  __shared__ __align__(16) int8_t Vq[KK * D];
  __shared__ float Ksc[KK * NB], Vsc[KK * NB];
  __shared__ __align__(16) float Qs[GROUP * D];
  __shared__ float Ss[GROUP * KK];
  const int c = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;
  const int start = c * KK;
  if (start >= count) return;
  const int nk = min(KK, count - start);
  const int kvw = kv_heads * D;

  const float* qg = q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * D;
  const bool has_q = tid < GROUP * D / 4;
  const float4 qv = ((const float4*)qg)[has_q ? tid : 0];
  const int64_t seq = kv_index ? 0 : (int64_t)t * cache_stride;
  const int8_t* kseq = (const int8_t*)(kc + seq);
  const int8_t* vseq = (const int8_t*)(vc + seq);
  uint4 kraw[PER], vraw[PER];
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = min(tid + j * NT, TOTAL - 1);
    const int key = i / PIECES, pc = i % PIECES;
    const int cell = max(kv_cell(kv_index, index_stride, t, start + min(key, nk - 1)), 0);
    const int64_t off = (int64_t)cell * row * 2 + (int64_t)kvh * D + pc * 16;  // bytes
    kraw[j] = *(const uint4*)(kseq + off);
    vraw[j] = *(const uint4*)(vseq + off);
  }
  // the factors: KK * NB of each, at most one of each a thread
  const bool has_f = tid < KK * NB;
  float kf = 0.0f, vf = 0.0f;
  {
    const int i = has_f ? tid : 0, key = i / NB, b = i % NB;
    const int cell = max(kv_cell(kv_index, index_stride, t, start + min(key, nk - 1)), 0);
    const int64_t at = (int64_t)cell * row + (kvw >> 1) + (kvh * D >> 5) + b;  // halves
    kf = __half2float(kc[seq + at]);
    vf = __half2float(vc[seq + at]);
  }
  if (has_q) ((float4*)Qs)[tid] = qv;
  if (has_f) {
    Ksc[tid] = kf;
    Vsc[tid] = vf;
  }
#pragma unroll
  for (int j = 0; j < PER; j++) {
    const int i = tid + j * NT;
    const int key = i / PIECES, pc = i % PIECES;
    if (i < TOTAL) {
      *(uint4*)(Kq + key * KQR + pc * 16) = kraw[j];
      *(uint4*)(Vq + key * D + pc * 16) = vraw[j];
    }
  }
  __syncthreads();

  // scores: thread = (query head g, key, part of DPT dims)
  {
    const int dot = tid / S::SPL, part = tid % S::SPL;
    const int g = dot / KK, key = dot % KK;
    float sdot = 0.0f;
    if (dot < GROUP * KK) {
      const int8_t* kr = Kq + key * KQR + part * S::DPT;
      const float* qq = Qs + g * D + part * S::DPT;
#pragma unroll
      for (int d = 0; d < S::DPT; d += 16) {
        const float f = Ksc[key * NB + (part * S::DPT + d) / 32];
        const uint4 raw = *(const uint4*)(kr + d);
        const int8_t* b = (const int8_t*)&raw;
#pragma unroll
        for (int i = 0; i < 16; i++) sdot = fmaf(qq[d + i], (float)b[i] * f, sdot);
      }
    }
    sdot = lanes::reduce<S::SPL>(sdot, lanes::Add{});
    if (part == 0 && dot < GROUP * KK) {
      const bool live = key < nk && (!kv_index || kv_cell(kv_index, index_stride, t, start + key) >= 0);
      Ss[g * KK + key] = live ? sdot * scale : -INFINITY;
    }
  }
  __syncthreads();
  const int64_t slot0 = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks;
  if (wave < GROUP) {
    const float sc = Ss[wave * KK + lane];
    const float m = lanes::reduce<64>(sc, lanes::Max{});
    const float pr = sc == -INFINITY ? 0.0f : expf(sc - m);
    const float l = lanes::reduce<64>(pr, lanes::Add{});
    Ss[wave * KK + lane] = pr;
    if (lane == 0) *(float2*)(part_ml + (slot0 + (int64_t)wave * max_chunks + c) * 2) = make_float2(m, l);
  }
  __syncthreads();
  // unnormalised weighted values: thread = (query head, dim pair, key residue kq)
  const int kq = tid % S::KQ, oe = tid / S::KQ;
  const int g = oe / PAIRS, e = oe % PAIRS;
  float a0 = 0.0f, a1 = 0.0f;
  if (oe < GROUP * PAIRS) {
    const float* pg = Ss + g * KK;
    const int b = (2 * e) >> 5;
#pragma unroll 4
    for (int k = kq; k < KK; k += S::KQ) {
      const float p = pg[k];
      const char2 v = *(const char2*)(Vq + k * D + 2 * e);
      const float f = Vsc[k * NB + b];
      a0 = fmaf(p, (float)v.x * f, a0);
      a1 = fmaf(p, (float)v.y * f, a1);
    }
  }
  a0 = lanes::reduce<S::KQ>(a0, lanes::Add{});
  a1 = lanes::reduce<S::KQ>(a1, lanes::Add{});
  if (kq == 0 && oe < GROUP * PAIRS)
    *(float2*)(part_acc + (slot0 + (int64_t)g * max_chunks + c) * D + 2 * e) = make_float2(a0, a1);
  }
}

// whether attend_wide_q8_kernel takes a shape: each score thread's dims are
// whole 16-byte pieces
__host__ __device__ constexpr bool wide_q8_fits(int group, int d, int nt) {
  return d % (16 * (nt / (group * kWideKeys) < d / 8 ? nt / (group * kWideKeys) : d / 8)) == 0;
}

// ---- the optional layer parts of other families ----------------------------
// kernel.mojo:400 rms_norm_at over runs: every head of q (or k) in a row of
// the fused q|k|v, in place (gpu_block.mojo device_rms_norm_run, Qwen 3's
// per-head norms).  Block = one (head, token), 64 threads; float64 sum of
// squares, f32 scale, x * scale * gain as rms_norm_kernel.
__global__ __launch_bounds__(64) void head_norm_kernel(float* __restrict__ x, int64_t row_stride, int n,
                                                       const float* __restrict__ gain, float eps) {
#pragma clang fp contract(off)
  float* run = x + (int64_t)blockIdx.y * row_stride + (int64_t)blockIdx.x * n;
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += 64) acc += (double)run[i] * (double)run[i];
  acc = lanes::reduce_sum<64>(acc);
  const float scale = (float)(1.0 / sqrt(acc / (double)n + (double)eps));
  for (int i = threadIdx.x; i < n; i += 64) run[i] = run[i] * scale * gain[i];
}

// A sublayer's output normed on its way into the residual stream
// (gpu_block.mojo device_rms_norm_inplace then device_add_run, Gemma 2's post
// norms): resid[t] += rms_norm(y[t]) * gain.  Block = one token, 256 threads.
__global__ __launch_bounds__(256) void norm_add_kernel(float* __restrict__ resid, const float* __restrict__ y, int n,
                                                       const float* __restrict__ gain, float eps) {
#pragma clang fp contract(off)
  const float* yr = y + (int64_t)blockIdx.x * n;
  float* rr = resid + (int64_t)blockIdx.x * n;
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += 256) acc += (double)yr[i] * (double)yr[i];
  acc = lanes::reduce_sum<64>(acc);
  __shared__ double part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  const double sum = part[0] + part[1] + part[2] + part[3];
  const float scale = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
  for (int i = threadIdx.x; i < n; i += 256) rr[i] += yr[i] * scale * gain[i];
}

// The non-gated MLP's activation in place (gpu_block.mojo device_silu /
// device_gelu): x = act(x) over n values.
__global__ void act_kernel(float* __restrict__ x, int64_t n, int gelu_act) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    x[i] = gelu_act ? mv::gelu(x[i]) : mv::silu(x[i]);
}

// ---- argmax ----------------------------------------------------------------
// kernel.mojo:571: index of the maximum, ties to the lower index.
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

// Reduce (value, index) over the block; thread 0 writes the winner.
__device__ __forceinline__ void argmax_finish(float bv, int bi, int n, int32_t* __restrict__ out) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    better(bv, bi, ov, oi);
  }
  __shared__ float sv[16];
  __shared__ int si[16];
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) better(bv, bi, sv[w], si[w]);
    *out = bi < n ? bi : 0;
  }
}

// Rows of any length: strided scalar loop.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int n,
                                                      int32_t* __restrict__ out) {
  const int t = blockIdx.x;
  const float* xr = x + (int64_t)t * n;
  float bv = -INFINITY;
  int bi = n;  // sentinel: beaten by any real element
  for (int i = threadIdx.x; i < n; i += blockDim.x) better(bv, bi, xr[i], i);
  argmax_finish(bv, bi, n, out + t);
}

// Rows of a multiple of 4 floats, 16-byte aligned: each thread issues all of
// its PER float4 loads before comparing any, so the row costs one memory
// latency (a vocabulary of 128256 is 32 loads per thread).
template <int PER>
__global__ __launch_bounds__(1024) void argmax4_kernel(const float* __restrict__ x, int n,
                                                       int32_t* __restrict__ out) {
  const int t = blockIdx.x;
  const float4* xr = (const float4*)(x + (int64_t)t * n);
  const int n4 = n >> 2;
  // rounds of at most 16 loads a thread: 32 float4 are the 128 registers a
  // 1024-thread block has, and spilled
  constexpr int R = PER < 16 ? PER : 16;
  float bv = -INFINITY;
  int bi = n;
#pragma unroll
  for (int k0 = 0; k0 < PER; k0 += R) {
    float4 v[R];
#pragma unroll
    for (int k = 0; k < R; k++) {
      const int j = threadIdx.x + (k0 + k) * 1024;
      v[k] = j < n4 ? xr[j] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
#pragma unroll
    for (int k = 0; k < R; k++) {
      const int i = 4 * (threadIdx.x + (k0 + k) * 1024);
      if (i < n) {
        better(bv, bi, v[k].x, i);
        better(bv, bi, v[k].y, i + 1);
        better(bv, bi, v[k].z, i + 2);
        better(bv, bi, v[k].w, i + 3);
      }
    }
  }
  argmax_finish(bv, bi, n, out + t);
}

// Multi-block form (mi_argmax_ws): a row of n is cut into kArgParts chunks
// of whole float4s, one 256-thread block each, every thread issuing all of
// its loads before comparing; each block leaves its (value, index) in the
// workspace and argmax_pick_kernel folds the parts of a row in part order
// with the same tie rule.  One block streaming a 128256-logit row was bound
// by a single CU's bandwidth (about 16 us); the parts spread it over the chip.
constexpr int kArgParts = 64, kArgThreads = 256, kArgPer = 4;
__global__ __launch_bounds__(kArgThreads) void argmax_part_kernel(const float* __restrict__ x, int n, int chunk4,
                                                                  float2* __restrict__ part) {
  const int b = blockIdx.x, t = blockIdx.y;
  const float* xr = x + (int64_t)t * n;
  const int n4 = n >> 2, j0 = b * chunk4, j1 = min(j0 + chunk4, n4);
  float bv = -INFINITY;
  int bi = n;
  const bool vec = ((n & 3) == 0) && (((uintptr_t)xr & 15) == 0);
  if (vec) {
    const float4* xr4 = (const float4*)xr;
    for (int j = j0 + threadIdx.x; j < j1; j += kArgThreads * kArgPer) {
      float4 v[kArgPer];
#pragma unroll
      for (int k = 0; k < kArgPer; k++) {
        const int jj = j + k * kArgThreads;
        v[k] = jj < j1 ? xr4[jj] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      }
#pragma unroll
      for (int k = 0; k < kArgPer; k++) {
        const int i = 4 * (j + k * kArgThreads);
        if (j + k * kArgThreads < j1) {
          better(bv, bi, v[k].x, i);
          better(bv, bi, v[k].y, i + 1);
          better(bv, bi, v[k].z, i + 2);
          better(bv, bi, v[k].w, i + 3);
        }
      }
    }
  } else {
    // scalar chunks of 4 * chunk4 values (the last part also takes the tail)
    const int i1 = b == (int)gridDim.x - 1 ? n : min(4 * j1, n);
    for (int i = 4 * j0 + threadIdx.x; i < i1; i += kArgThreads) better(bv, bi, xr[i], i);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    better(bv, bi, ov, oi);
  }
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / 64; w++) better(bv, bi, sv[w], si[w]);
    part[(int64_t)t * gridDim.x + b] = make_float2(bv, __int_as_float(bi));
  }
}

// One wave per row: lane b holds part b; the winner goes to out[t], and
// optionally to next_ids[t] with next_pos[t] += 1 (the decode loop's
// bookkeeping, so it costs no launches of its own).
__global__ __launch_bounds__(64) void argmax_pick_kernel(const float2* __restrict__ part, int parts, int n,
                                                         int32_t* __restrict__ out, int32_t* __restrict__ next_ids,
                                                         int32_t* __restrict__ next_pos) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float bv = -INFINITY;
  int bi = n;
  for (int b = lane; b < parts; b += 64) {
    const float2 p = part[(int64_t)t * parts + b];
    better(bv, bi, p.x, __float_as_int(p.y));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    better(bv, bi, ov, oi);
  }
  if (lane == 0) {
    const int pick = bi < n ? bi : 0;
    out[t] = pick;
    if (next_ids) next_ids[t] = pick;
    if (next_pos) next_pos[t] += 1;
  }
}

// ---- embedding -------------------------------------------------------------
// model.mojo:102 embed for an f32 table: one row copy per token.
__global__ void embed_kernel(const float* __restrict__ emb, int vocab, int width,
                             const int32_t* __restrict__ ids, float* __restrict__ out) {
  const int t = blockIdx.y;
  int id = ids[t];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const float4* src = (const float4*)(emb + (int64_t)id * width);
  float4* dst = (float4*)(out + (int64_t)t * width);
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width / 4; i += gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace

static int norm_launch(hipStream_t s, const float* x, const float* gain, int32_t n, int32_t tokens, float eps,
                       float* out, void* xq, void* hx, const int32_t* pos, const float* steps, const float* factors,
                       int32_t pairs, float* trig) {
  const int per = (n + kNormThreads - 1) / kNormThreads;
  dim3 grid(per, tokens);
#define MI_NORM(P)                                                                                      \
  hipLaunchKernelGGL(rms_norm_kernel<P>, grid, dim3(kNormThreads), 0, s, x, gain, n, eps, out, (uint8_t*)xq, \
                     (uint8_t*)hx, pos, steps, factors, pairs, (float2*)trig, 0)
  if (per <= 4) MI_NORM(4);
  else if (per <= 8) MI_NORM(8);
  else if (per <= 16) MI_NORM(16);
  else if (per <= 32) MI_NORM(32);
  else if (per <= 64) MI_NORM(64);
  else return fail(MI_ERR_SHAPE, "rms_norm: %d values per row is more than %d", n, 64 * kNormThreads);
#undef MI_NORM
  return hip_check(hipGetLastError(), "rms_norm launch");
}

// 512 threads a block (8 values a thread of the whole-row sum, one block
// for each 512-value slice): 2.628 -> 2.599 ms a decode step at batch 4
// against 256 (16 loads a thread a part), 1024 no better than 256.
constexpr int kSplitNormThreads = 512;
int launch_split_add_norm(hipStream_t s, const float* part, int nsplit, float* resid, const float* gain, int32_t n,
                          int32_t tokens, float eps, void* xq, void* hx) {
  constexpr int kNt = kSplitNormThreads;
  const int per = (n + kNt - 1) / kNt;
  if (n % 32 || !xq || !hx) return fail(MI_ERR_SHAPE, "split norm: %d values a row, xq and hx forms", n);
  const int64_t ps = (int64_t)tokens * n;
  dim3 grid(per, tokens);
#define MI_SNORM(P, K)                                                                                         \
  hipLaunchKernelGGL((rms_norm_kernel<P, K, kNt>), grid, dim3(kNt), 0, s, part, gain, n, eps, resid,         \
                     (uint8_t*)xq, (uint8_t*)hx, nullptr, nullptr, nullptr, 0, nullptr, ps)
#define MI_SNORM_P(K)                                                                                          \
  if (per <= 4) MI_SNORM(4, K);                                                                                \
  else if (per <= 8) MI_SNORM(8, K);                                                                           \
  else if (per <= 16) MI_SNORM(16, K);                                                                         \
  else return fail(MI_ERR_SHAPE, "split norm: %d values per row is more than %d", n, 16 * kNt);
  switch (nsplit) {
    case 2: MI_SNORM_P(2) break;
    case 3: MI_SNORM_P(3) break;
    case 4: MI_SNORM_P(4) break;
    default: return fail(MI_ERR_ARG, "split norm: %d parts", nsplit);
  }
#undef MI_SNORM_P
#undef MI_SNORM
  return hip_check(hipGetLastError(), "split norm launch");
}

int launch_rms_norm(hipStream_t s, const float* x, const float* gain, int32_t n, int32_t tokens, float eps,
                    float* out, void* xq, void* hx) {
  return norm_launch(s, x, gain, n, tokens, eps, out, xq, hx, nullptr, nullptr, nullptr, 0, nullptr);
}

int launch_rms_norm_trig(hipStream_t s, const float* x, const float* gain, int32_t n, float eps, void* xq,
                         const int32_t* pos, const float* steps, const float* factors, int32_t pairs,
                         float* trig) {
  return norm_launch(s, x, gain, n, 1, eps, nullptr, xq, nullptr, pos, steps, factors, pairs, trig);
}

int launch_rope(hipStream_t s, float* x, int32_t heads, int32_t head_dim, int32_t dim, int32_t neox,
                const float* steps, const int32_t* pos, int32_t tokens, int64_t row_stride, const float* factors) {
  hipLaunchKernelGGL(rope_kernel, dim3(tokens), dim3(256), 0, s, x, heads, head_dim, dim, neox, steps, factors,
                     pos, row_stride);
  return hip_check(hipGetLastError(), "rope launch");
}

int launch_rope_store(hipStream_t s, float* qkv, int32_t heads, int32_t kv_heads, int32_t head_dim,
                      int32_t dim, int32_t neox, const float* steps, const int32_t* pos,
                      int32_t tokens, int64_t row_stride, uint16_t* k_cache, uint16_t* v_cache,
                      int64_t cache_stride, const float* factors, int32_t form, const int32_t* kv_index,
                      int64_t index_stride) {
  const int crow = cache_row(form, kv_heads * head_dim);
  if (form == MI_CACHE_Q8)
    hipLaunchKernelGGL(rope_store_kernel<true>, dim3(tokens), dim3(kRopeThreads), (size_t)dim * sizeof(float), s,
                       qkv, heads, kv_heads, head_dim, dim, neox, steps, factors, pos, row_stride, (__half*)k_cache,
                       (__half*)v_cache, cache_stride, crow, kv_index, index_stride);
  else
    hipLaunchKernelGGL(rope_store_kernel<false>, dim3(tokens), dim3(kRopeThreads), (size_t)dim * sizeof(float), s,
                       qkv, heads, kv_heads, head_dim, dim, neox, steps, factors, pos, row_stride, (__half*)k_cache,
                       (__half*)v_cache, cache_stride, crow, kv_index, index_stride);
  return hip_check(hipGetLastError(), "rope_store launch");
}

int launch_store_kv(hipStream_t s, const float* k, const float* v, int32_t kv_width,
                    uint16_t* k_cache, uint16_t* v_cache, const int32_t* slot_dev, int32_t slot_host,
                    int32_t tokens, int64_t src_stride, int64_t cache_stride, int32_t form) {
  if (form == MI_CACHE_Q8) {
    dim3 grid((kv_width / 32 + 7) / 8, tokens, 2);
    hipLaunchKernelGGL(store_kv_q8_kernel, grid, dim3(256), 0, s, k, v, kv_width, (__half*)k_cache,
                       (__half*)v_cache, slot_dev, slot_host, src_stride, cache_stride,
                       cache_row(MI_CACHE_Q8, kv_width));
    return hip_check(hipGetLastError(), "store_kv_q8 launch");
  }
  dim3 grid((kv_width + 255) / 256, tokens);
  hipLaunchKernelGGL(store_kv_kernel, grid, dim3(256), 0, s, k, v, kv_width, (__half*)k_cache,
                     (__half*)v_cache, slot_dev, slot_host, src_stride, cache_stride);
  return hip_check(hipGetLastError(), "store_kv launch");
}

// attend_merge_kernel with B the slice count rounded up to 8 (at most 64)
static int launch_merge(hipStream_t s, const float* part_acc, const float* part_ml, int heads, int head_dim,
                        const int32_t* pos_dev, int count_host, int chunks, int tokens, float* out, void* xq_out,
                        void* hx_out) {
  const dim3 grid(heads, tokens), block(head_dim < 64 ? 64 : head_dim);
#define MI_MERGE(B)                                                                                    \
  hipLaunchKernelGGL(attend_merge_kernel<B>, grid, block, 0, s, part_acc, part_ml, heads, head_dim, pos_dev, \
                     count_host, chunks, out, (uint8_t*)xq_out, (uint8_t*)hx_out)
  switch ((std::min(chunks, 64) + 7) / 8) {
    case 1: MI_MERGE(8); break;
    case 2: MI_MERGE(16); break;
    case 3: MI_MERGE(24); break;
    case 4: MI_MERGE(32); break;
    case 5: MI_MERGE(40); break;
    case 6: MI_MERGE(48); break;
    case 7: MI_MERGE(56); break;
    default: MI_MERGE(64); break;
  }
#undef MI_MERGE
  return hip_check(hipGetLastError(), "attend_merge launch");
}

size_t attend_workspace(int32_t heads, int32_t head_dim, int32_t max_count, int32_t tokens) {
  const int kk = attn_slice(head_dim);
  const int64_t chunks = (max_count + kk - 1) / kk;
  const int64_t slots = (int64_t)tokens * heads * chunks;
  const size_t acc = (size_t)slots * head_dim * sizeof(float);
  return ((acc + 255) & ~(size_t)255) + (size_t)slots * 2 * sizeof(float);
}

int launch_attend(hipStream_t s, const float* q, int64_t q_stride, const uint16_t* k_cache,
                  const uint16_t* v_cache, int64_t cache_stride, int32_t heads, int32_t kv_heads,
                  int32_t head_dim, float scale, const int32_t* pos_dev, int32_t count_host,
                  int32_t max_count, int32_t tokens, float* out, void* xq_out, void* work, int32_t form,
                  const int32_t* kv_index, int64_t index_stride, void* hx_out) {
  const int kk = attn_slice(head_dim);
  const int chunks = (max_count + kk - 1) / kk;
  const int64_t slots = (int64_t)tokens * heads * chunks;
  float* part_acc = (float*)work;
  const size_t acc_bytes = ((size_t)slots * head_dim * sizeof(float) + 255) & ~(size_t)255;
  float* part_ml = (float*)((char*)work + acc_bytes);
  const int group = heads / kv_heads;
  // decode (at most 8 tokens, one each per sequence): the matrix-core slice
  // kernel for an f16 cache and up to 4 query heads a key head, else the
  // wide VALU slice kernel (1024 threads at one token, 512 for a batch)
  if (tokens <= kMaxTokens && (head_dim == 64 || head_dim == 128) &&
      (form != MI_CACHE_Q8 || wide_q8_fits(group, head_dim, tokens == 1 ? 1024 : 512))) {
    dim3 grid(chunks, kv_heads, tokens);
    const int qrow = cache_row(MI_CACHE_Q8, kv_heads * head_dim);
#define MI_WIDE(G, DD)                                                                                       \
  if (form == MI_CACHE_Q8 && tokens == 1)                                                                    \
    hipLaunchKernelGGL((attend_wide_q8_kernel<G, DD, 1024>), grid, dim3(1024), 0, s, q, q_stride,            \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, qrow, heads, kv_heads,   \
                       scale, pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride);        \
  else if (form == MI_CACHE_Q8)                                                                              \
    hipLaunchKernelGGL((attend_wide_q8_kernel<G, DD, 512>), grid, dim3(512), 0, s, q, q_stride,              \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, qrow, heads, kv_heads,   \
                       scale, pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride);        \
  else if (G <= 4 && kv_index)                                                                               \
    hipLaunchKernelGGL((attend_mfma_kernel<(G <= 4 ? G : 4), DD, true>), grid, dim3(256), 0, s, q, q_stride,  \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, heads, kv_heads, scale,   \
                       pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride);               \
  else if (G <= 4)                                                                                           \
    hipLaunchKernelGGL((attend_mfma_kernel<(G <= 4 ? G : 4), DD, false>), grid, dim3(256), 0, s, q, q_stride, \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, heads, kv_heads, scale,   \
                       pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride);               \
  else if (tokens == 1)                                                                                      \
    hipLaunchKernelGGL((attend_wide_kernel<G, DD, 1024>), grid, dim3(1024), 0, s, q, q_stride,               \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, heads, kv_heads, scale,   \
                       pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride);               \
  else                                                                                                       \
    hipLaunchKernelGGL((attend_wide_kernel<G, DD, 512>), grid, dim3(512), 0, s, q, q_stride,                 \
                       (const __half*)k_cache, (const __half*)v_cache, cache_stride, heads, kv_heads, scale,   \
                       pos_dev, count_host, chunks, part_acc, part_ml, kv_index, index_stride)
#define MI_WIDE_D(G) \
  if (head_dim == 64) { MI_WIDE(G, 64); } else { MI_WIDE(G, 128); }
    switch (group) {
      case 1: MI_WIDE_D(1); break;
      case 2: MI_WIDE_D(2); break;
      case 4: MI_WIDE_D(4); break;
      case 8: MI_WIDE_D(8); break;
      default: return fail(MI_ERR_SHAPE, "attend: %d query heads per key head is not 1, 2, 4 or 8", group);
    }
#undef MI_WIDE_D
#undef MI_WIDE
    int rc = hip_check(hipGetLastError(), "attend_wide launch");
    if (rc) return rc;
    return launch_merge(s, part_acc, part_ml, heads, head_dim, pos_dev, count_host, chunks, tokens, out, xq_out,
                        hx_out);
  }
  // one sequence's chunk (its tokens share one cache): 16 tokens per block
  // over one staged slice (f16 form; the q8 kernel takes one token a block)
  const bool one_seq = kv_index ? index_stride == 0 : cache_stride == 0;
  if (one_seq && pos_dev && tokens > kMaxTokens && form != MI_CACHE_Q8 && kk == kChunkKeys &&
      (head_dim == 64 || head_dim == 128)) {
    // a prefill chunk: the matrix-core slice kernel, then the same merge
    dim3 cgrid(chunks, kv_heads, (tokens + 64 / group - 1) / (64 / group));
    const size_t lds = attn_chunk_lds_bytes(head_dim);
    // more than 64 KB of dynamic LDS has to be asked for, once per kernel and device
#define MI_CHUNK(G, DD)                                                                                        \
  {                                                                                                            \
    static bool done[kMaxDevices];                                                                            \
    if (int rc = allow_lds((const void*)attend_chunk_kernel<G, DD>, (int)attn_chunk_lds_bytes(DD), done,      \
                           "attend_chunk LDS size"))                                                          \
      return rc;                                                                                              \
    hipLaunchKernelGGL((attend_chunk_kernel<G, DD>), cgrid, dim3(256), lds, s, q, q_stride,                    \
                       (const __half*)k_cache, (const __half*)v_cache, heads, kv_heads, scale, pos_dev, chunks, \
                       part_acc, part_ml, kv_index, tokens);                                                   \
  }
#define MI_CHUNK_D(G) \
  if (head_dim == 64) MI_CHUNK(G, 64) else MI_CHUNK(G, 128)
    switch (group) {
      case 1: MI_CHUNK_D(1); break;
      case 2: MI_CHUNK_D(2); break;
      case 4: MI_CHUNK_D(4); break;
      case 8: MI_CHUNK_D(8); break;
      default: return fail(MI_ERR_SHAPE, "attend: %d query heads per key head is not 1, 2, 4 or 8", group);
    }
#undef MI_CHUNK_D
#undef MI_CHUNK
    int rc = hip_check(hipGetLastError(), "attend_chunk launch");
    if (rc) return rc;
    return launch_merge(s, part_acc, part_ml, heads, head_dim, pos_dev, count_host, chunks, tokens, out, xq_out,
                        hx_out);
  }
  const int tq = (one_seq && tokens > kMaxTokens && form != MI_CACHE_Q8) ? 16 : 1;
  dim3 grid(chunks, kv_heads, (tokens + tq - 1) / tq);
  const __half* kc = (const __half*)k_cache;
  const __half* vc = (const __half*)v_cache;
  const bool q8 = form == MI_CACHE_Q8;
  const int row = cache_row(form, kv_heads * head_dim);
  const size_t shmem = q8 ? attn_q8_lds_bytes(head_dim, group) : attn_lds_bytes(head_dim, group);
#define MI_ATTEND(G)                                                                                       \
  if (q8)                                                                                                  \
    hipLaunchKernelGGL(attend_split_q8_kernel<G>, grid, dim3(kAttnThreads), shmem, s, q, q_stride, kc, vc,  \
                       cache_stride, row, heads, kv_heads, head_dim, scale, pos_dev, count_host, chunks,    \
                       part_acc, part_ml, kv_index, index_stride);                                         \
  else                                                                                                     \
    hipLaunchKernelGGL(attend_split_kernel<G>, grid, dim3(kAttnThreads), shmem, s, q, q_stride, kc, vc,     \
                       cache_stride, heads, kv_heads, head_dim, scale, pos_dev, count_host, chunks,         \
                       part_acc, part_ml, kv_index, index_stride, tokens, tq)
  switch (group) {
    case 1: MI_ATTEND(1); break;
    case 2: MI_ATTEND(2); break;
    case 4: MI_ATTEND(4); break;
    case 8: MI_ATTEND(8); break;
    default: return fail(MI_ERR_SHAPE, "attend: %d query heads per key head is not 1, 2, 4 or 8", group);
  }
#undef MI_ATTEND
  int rc = hip_check(hipGetLastError(), "attend_split launch");
  if (rc) return rc;
  return launch_merge(s, part_acc, part_ml, heads, head_dim, pos_dev, count_host, chunks, tokens, out, xq_out,
                      hx_out);
}

int launch_argmax(hipStream_t s, const float* x, int32_t n, int32_t tokens, int32_t* out) {
  const int per = (n / 4 + 1023) / 1024;
  if (n % 4 == 0 && ((uintptr_t)x & 15) == 0 && per <= 32) {
#define MI_ARGMAX(P) hipLaunchKernelGGL(argmax4_kernel<P>, dim3(tokens), dim3(1024), 0, s, x, n, out)
    if (per <= 1) MI_ARGMAX(1);
    else if (per <= 4) MI_ARGMAX(4);
    else if (per <= 8) MI_ARGMAX(8);
    else if (per <= 16) MI_ARGMAX(16);
    else MI_ARGMAX(32);
#undef MI_ARGMAX
    return hip_check(hipGetLastError(), "argmax launch");
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(tokens), dim3(1024), 0, s, x, n, out);
  return hip_check(hipGetLastError(), "argmax launch");
}

size_t argmax_workspace(int32_t n, int32_t tokens) {
  (void)n;
  return (size_t)tokens * kArgParts * sizeof(float2);
}

int launch_argmax_ws(hipStream_t s, const float* x, int32_t n, int32_t tokens, int32_t* out, void* work,
                     int32_t* next_ids, int32_t* next_pos) {
  const int n4 = n >> 2;
  const int parts = n4 < kArgParts ? 1 : kArgParts;
  const int chunk4 = (n4 + parts - 1) / parts;
  hipLaunchKernelGGL(argmax_part_kernel, dim3(parts, tokens), dim3(kArgThreads), 0, s, x, n, chunk4, (float2*)work);
  int rc = hip_check(hipGetLastError(), "argmax launch");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_pick_kernel, dim3(tokens), dim3(64), 0, s, (const float2*)work, parts, n, out, next_ids,
                     next_pos);
  return hip_check(hipGetLastError(), "argmax launch");
}

int launch_embed(hipStream_t s, const float* emb, int32_t vocab, int32_t width, const int32_t* ids,
                 int32_t tokens, float* out) {
  dim3 grid((width / 4 + 255) / 256, tokens);
  hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, s, emb, vocab, width, ids, out);
  return hip_check(hipGetLastError(), "embed launch");
}

int launch_head_norm(hipStream_t s, float* x, int32_t heads, int32_t n, int32_t tokens, int64_t row_stride,
                     const float* gain, float eps) {
  hipLaunchKernelGGL(head_norm_kernel, dim3(heads, tokens), dim3(64), 0, s, x, row_stride, n, gain, eps);
  return hip_check(hipGetLastError(), "head_norm launch");
}

int launch_norm_add(hipStream_t s, float* resid, const float* y, int32_t n, int32_t tokens, const float* gain,
                    float eps) {
  hipLaunchKernelGGL(norm_add_kernel, dim3(tokens), dim3(256), 0, s, resid, y, n, gain, eps);
  return hip_check(hipGetLastError(), "norm_add launch");
}

int launch_act(hipStream_t s, float* x, int64_t n, int32_t act) {
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 2048);
  hipLaunchKernelGGL(act_kernel, dim3(blocks), dim3(256), 0, s, x, n, (act & MI_ACT_GELU) ? 1 : 0);
  return hip_check(hipGetLastError(), "act launch");
}

}  // namespace mi

// ops.hip -- the decoder layer's small kernels, gfx950.
//
// Replaces src/molla/nn/gpu_ops.mojo: rms_norm_kernel (:152), rope_kernel
// (:470), store_kv_kernel (:1491), attend_split_kernel / attend_merge_kernel
// (:929 / :1104), argmax_kernel (:408) and the embedding row copy (:320).
// Producers of a matvec input (norm, attention merge) also write the
// activation in the matvec's block fixed-point form (xq_device.h), so the
// next projection needs no separate quantize launch.
#include <math.h>

#include "mi_internal.h"
#include "xq_device.h"

namespace mi {
namespace {

// ---- RMSNorm ---------------------------------------------------------------
// kernel.mojo:432-467: float64 sum of squares, scale = f32(1/sqrt(sum/n+eps)),
// out = x * scale * gain.  One block per token.
constexpr int kNormThreads = 1024;

__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ gain, int n,
                                                                float eps, float* __restrict__ out,
                                                                uint8_t* __restrict__ xq) {
#pragma clang fp contract(off)
  const int t = blockIdx.x;
  const float* xr = x + (int64_t)t * n;
  double acc = 0.0;
  for (int i = threadIdx.x; i < n; i += kNormThreads) acc += (double)xr[i] * (double)xr[i];
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
  __shared__ double part[kNormThreads / kWave];
  __shared__ float scale_s;
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double sum = 0.0;
    for (int i = 0; i < kNormThreads / kWave; i++) sum += part[i];
    scale_s = (float)(1.0 / sqrt(sum / (double)n + (double)eps));
  }
  __syncthreads();
  const float scale = scale_s;
  const int G = n >> 5;
  uint8_t* xt = xq ? xq + (int64_t)t * xq_token_bytes(n) : nullptr;
  for (int base = 0; base < n; base += kNormThreads) {
    const int i = base + threadIdx.x;
    const bool live = i < n;
    const float v = live ? xr[i] * scale * gain[i] : 0.0f;
    if (out && live) out[(int64_t)t * n + i] = v;
    // A half-wave is one 32-value group; n is a multiple of 32, so a group is
    // either entirely live or entirely past the end.
    if (xt) quantize_group32(v, threadIdx.x & 31, i >> 5, G, xt, live);
  }
}

// ---- RoPE ------------------------------------------------------------------
// rope.mojo:253-338: theta = f32(pos) * step / freq (freq 1, scale 1),
// c = f32(cos(f64(theta))), s likewise, (a, b) <- (a*c - b*s, a*s + b*c).
// The trig is done in float64 on the device too, so the rotated values
// match the host's to float32 rounding at any position.
__device__ __forceinline__ void rotate_pair(float* __restrict__ row, int head_dim, int dim, int neox,
                                            const float* __restrict__ steps, int pos, int head, int pair) {
#pragma clang fp contract(off)
  const float theta = (float)pos * steps[pair];
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
                            const float* __restrict__ steps, const int32_t* __restrict__ pos,
                            int64_t row_stride) {
  const int t = blockIdx.x;
  const int pairs = dim >> 1;
  float* row = x + (int64_t)t * row_stride;
  for (int i = threadIdx.x; i < heads * pairs; i += blockDim.x)
    rotate_pair(row, head_dim, dim, neox, steps, pos[t], i / pairs, i % pairs);
}

// Rotate q and k of a fused [q | k | v] row in place, then store k and v as
// halves at the token's slot (gpu_ops.mojo:1491, narrowing by a plain cast,
// i.e. round to nearest even).
__global__ void rope_store_kernel(float* __restrict__ qkv, int heads, int kv_heads, int head_dim,
                                  int dim, int neox, const float* __restrict__ steps,
                                  const int32_t* __restrict__ pos, int64_t row_stride,
                                  __half* __restrict__ kc, __half* __restrict__ vc,
                                  int64_t cache_stride) {
  const int t = blockIdx.x;
  const int pairs = dim >> 1;
  const int p = pos[t];
  float* row = qkv + (int64_t)t * row_stride;
  for (int i = threadIdx.x; i < (heads + kv_heads) * pairs; i += blockDim.x)
    rotate_pair(row, head_dim, dim, neox, steps, p, i / pairs, i % pairs);
  __syncthreads();
  const int kvw = kv_heads * head_dim;
  const float* k = row + (int64_t)heads * head_dim;
  const float* v = k + kvw;
  __half* kd = kc + (int64_t)t * cache_stride + (int64_t)p * kvw;
  __half* vd = vc + (int64_t)t * cache_stride + (int64_t)p * kvw;
  for (int i = threadIdx.x; i < kvw; i += blockDim.x) {
    kd[i] = __float2half_rn(k[i]);
    vd[i] = __float2half_rn(v[i]);
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
  kc[(int64_t)t * cache_stride + (int64_t)slot * kvw + i] = __float2half_rn(k[(int64_t)t * src_stride + i]);
  vc[(int64_t)t * cache_stride + (int64_t)slot * kvw + i] = __float2half_rn(v[(int64_t)t * src_stride + i]);
}

// ---- attention -------------------------------------------------------------
// attention.mojo:144 attend, split over slices of kChunk keys like
// gpu_ops.mojo:929 attend_split_kernel: a block takes one key head, one
// slice and every query head that reads that key head (GQA), so each key and
// value is read once per slice.  It writes the slice's running maximum, its
// sum of exponentials and the unnormalised weighted values; the merge folds
// slices flash-style (gpu_ops.mojo:1104).
constexpr int kChunk = 128;

template <int GROUP>
__global__ __launch_bounds__(kChunk) void attend_split_kernel(
    const float* __restrict__ q, int64_t q_stride, const __half* __restrict__ kc,
    const __half* __restrict__ vc, int64_t cache_stride, int heads, int kv_heads, int head_dim,
    float scale, const int32_t* __restrict__ pos_dev, int count_host, int max_chunks,
    float* __restrict__ part_acc, float* __restrict__ part_ml) {
  const int c = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;  // a position p attends over p + 1 slots
  const int start = c * kChunk;
  if (start >= count) return;
  const int tid = threadIdx.x;
  const int kvw = kv_heads * head_dim;
  extern __shared__ float smem[];
  float* qs = smem;                      // [GROUP][head_dim]
  float* ps = smem + GROUP * head_dim;   // [GROUP][kChunk]
  __shared__ float red[GROUP][kChunk / kWave];
  const float* qrow = q + (int64_t)t * q_stride + (int64_t)kvh * GROUP * head_dim;
  for (int i = tid; i < GROUP * head_dim; i += kChunk) qs[i] = qrow[i];
  __syncthreads();

  const __half* kbase = kc + (int64_t)t * cache_stride + (int64_t)kvh * head_dim;
  const __half* vbase = vc + (int64_t)t * cache_stride + (int64_t)kvh * head_dim;
  const int key = start + tid;
  const bool live = key < count;
  float s[GROUP];
#pragma unroll
  for (int g = 0; g < GROUP; g++) s[g] = 0.0f;
  if (live) {
    const __half* kr = kbase + (int64_t)key * kvw;
    for (int d = 0; d < head_dim; d += 8) {
      const uint4 raw = *(const uint4*)(kr + d);
      const __half2* h2 = (const __half2*)&raw;
      float kf[8];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float2 f = __half22float2(h2[i]);
        kf[2 * i] = f.x;
        kf[2 * i + 1] = f.y;
      }
#pragma unroll
      for (int g = 0; g < GROUP; g++)
#pragma unroll
        for (int i = 0; i < 8; i++) s[g] = fmaf(qs[g * head_dim + d + i], kf[i], s[g]);
    }
  }
  // slice maximum per head
  float mx[GROUP];
#pragma unroll
  for (int g = 0; g < GROUP; g++) {
    s[g] = live ? s[g] * scale : -INFINITY;
    float m = s[g];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((tid & 63) == 0) red[g][tid >> 6] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GROUP; g++) {
    float m = red[g][0];
    for (int i = 1; i < kChunk / kWave; i++) m = fmaxf(m, red[g][i]);
    mx[g] = m;
  }
  __syncthreads();
#pragma unroll
  for (int g = 0; g < GROUP; g++) {
    const float p = live ? expf(s[g] - mx[g]) : 0.0f;
    ps[g * kChunk + tid] = p;
    float l = p;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o);
    if ((tid & 63) == 0) red[g][tid >> 6] = l;
  }
  __syncthreads();
  const int nkeys = min(kChunk, count - start);
  const int64_t slot_base = ((int64_t)t * heads + (int64_t)kvh * GROUP) * max_chunks + c;
  for (int d = tid; d < head_dim; d += kChunk) {
    float acc[GROUP];
#pragma unroll
    for (int g = 0; g < GROUP; g++) acc[g] = 0.0f;
    for (int k = 0; k < nkeys; k++) {
      const float vv = __half2float(vbase[(int64_t)(start + k) * kvw + d]);
#pragma unroll
      for (int g = 0; g < GROUP; g++) acc[g] = fmaf(ps[g * kChunk + k], vv, acc[g]);
    }
#pragma unroll
    for (int g = 0; g < GROUP; g++)
      part_acc[(slot_base + (int64_t)g * max_chunks) * head_dim + d] = acc[g];
  }
  if (tid < GROUP) {
    float l = 0.0f;
    for (int i = 0; i < kChunk / kWave; i++) l += red[tid][i];
    part_ml[(slot_base + (int64_t)tid * max_chunks) * 2 + 0] = mx[tid];
    part_ml[(slot_base + (int64_t)tid * max_chunks) * 2 + 1] = l;
  }
}

// One block per (query head, token); thread d owns output dimension d.
__global__ void attend_merge_kernel(const float* __restrict__ part_acc, const float* __restrict__ part_ml,
                                    int heads, int head_dim, const int32_t* __restrict__ pos_dev,
                                    int count_host, int max_chunks, float* __restrict__ out,
                                    uint8_t* __restrict__ xq) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int count = pos_dev ? pos_dev[t] + 1 : count_host;  // a position p attends over p + 1 slots
  const int chunks = (count + kChunk - 1) / kChunk;
  const int64_t slot = ((int64_t)t * heads + h) * max_chunks;
  float M = -INFINITY;
  for (int c = 0; c < chunks; c++) M = fmaxf(M, part_ml[(slot + c) * 2]);
  float L = 0.0f;
  for (int c = 0; c < chunks; c++) L += part_ml[(slot + c) * 2 + 1] * expf(part_ml[(slot + c) * 2] - M);
  const float inv = 1.0f / L;
  const int width = heads * head_dim;
  for (int base = 0; base < head_dim; base += blockDim.x) {
    const int d = base + threadIdx.x;
    const bool live = d < head_dim;
    float o = 0.0f;
    if (live) {
      for (int c = 0; c < chunks; c++)
        o = fmaf(part_acc[(slot + c) * head_dim + d], expf(part_ml[(slot + c) * 2] - M), o);
      o *= inv;
      if (out) out[(int64_t)t * width + (int64_t)h * head_dim + d] = o;
    }
    if (xq)
      quantize_group32(o, threadIdx.x & 31, (h * head_dim + d) >> 5, width >> 5,
                       xq + (int64_t)t * xq_token_bytes(width), live);
  }
}

// ---- argmax ----------------------------------------------------------------
// kernel.mojo:571: index of the maximum, ties to the lower index.
__device__ __forceinline__ void better(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) {
    v = ov;
    i = oi;
  }
}

__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int n,
                                                      int32_t* __restrict__ out) {
  const int t = blockIdx.x;
  const float* xr = x + (int64_t)t * n;
  float bv = -INFINITY;
  int bi = n;  // sentinel: beaten by any real element
  for (int i = threadIdx.x; i < n; i += blockDim.x) better(bv, bi, xr[i], i);
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
    out[t] = bi < n ? bi : 0;
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

int launch_rms_norm(hipStream_t s, const float* x, const float* gain, int32_t n, int32_t tokens,
                    float eps, float* out, void* xq) {
  hipLaunchKernelGGL(rms_norm_kernel, dim3(tokens), dim3(kNormThreads), 0, s, x, gain, n, eps, out,
                     (uint8_t*)xq);
  return hip_check(hipGetLastError(), "rms_norm launch");
}

int launch_rope(hipStream_t s, float* x, int32_t heads, int32_t head_dim, int32_t dim, int32_t neox,
                const float* steps, const int32_t* pos, int32_t tokens, int64_t row_stride) {
  hipLaunchKernelGGL(rope_kernel, dim3(tokens), dim3(256), 0, s, x, heads, head_dim, dim, neox, steps,
                     pos, row_stride);
  return hip_check(hipGetLastError(), "rope launch");
}

int launch_rope_store(hipStream_t s, float* qkv, int32_t heads, int32_t kv_heads, int32_t head_dim,
                      int32_t dim, int32_t neox, const float* steps, const int32_t* pos,
                      int32_t tokens, int64_t row_stride, uint16_t* k_cache, uint16_t* v_cache,
                      int64_t cache_stride) {
  hipLaunchKernelGGL(rope_store_kernel, dim3(tokens), dim3(512), 0, s, qkv, heads, kv_heads, head_dim,
                     dim, neox, steps, pos, row_stride, (__half*)k_cache, (__half*)v_cache,
                     cache_stride);
  return hip_check(hipGetLastError(), "rope_store launch");
}

int launch_store_kv(hipStream_t s, const float* k, const float* v, int32_t kv_width,
                    uint16_t* k_cache, uint16_t* v_cache, const int32_t* slot_dev, int32_t slot_host,
                    int32_t tokens, int64_t src_stride, int64_t cache_stride) {
  dim3 grid((kv_width + 255) / 256, tokens);
  hipLaunchKernelGGL(store_kv_kernel, grid, dim3(256), 0, s, k, v, kv_width, (__half*)k_cache,
                     (__half*)v_cache, slot_dev, slot_host, src_stride, cache_stride);
  return hip_check(hipGetLastError(), "store_kv launch");
}

size_t attend_workspace(int32_t heads, int32_t head_dim, int32_t max_count, int32_t tokens) {
  const int64_t chunks = (max_count + kChunk - 1) / kChunk;
  const int64_t slots = (int64_t)tokens * heads * chunks;
  const size_t acc = (size_t)slots * head_dim * sizeof(float);
  return ((acc + 255) & ~(size_t)255) + (size_t)slots * 2 * sizeof(float);
}

int launch_attend(hipStream_t s, const float* q, int64_t q_stride, const uint16_t* k_cache,
                  const uint16_t* v_cache, int64_t cache_stride, int32_t heads, int32_t kv_heads,
                  int32_t head_dim, float scale, const int32_t* pos_dev, int32_t count_host,
                  int32_t max_count, int32_t tokens, float* out, void* xq_out, void* work) {
  const int chunks = (max_count + kChunk - 1) / kChunk;
  const int64_t slots = (int64_t)tokens * heads * chunks;
  float* part_acc = (float*)work;
  const size_t acc_bytes = ((size_t)slots * head_dim * sizeof(float) + 255) & ~(size_t)255;
  float* part_ml = (float*)((char*)work + acc_bytes);
  const int group = heads / kv_heads;
  const size_t shmem = (size_t)group * (head_dim + kChunk) * sizeof(float);
  dim3 grid(chunks, kv_heads, tokens);
  const __half* kc = (const __half*)k_cache;
  const __half* vc = (const __half*)v_cache;
#define MI_ATTEND(G)                                                                                  \
  hipLaunchKernelGGL(attend_split_kernel<G>, grid, dim3(kChunk), shmem, s, q, q_stride, kc, vc,         \
                     cache_stride, heads, kv_heads, head_dim, scale, pos_dev, count_host, chunks,     \
                     part_acc, part_ml)
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
  hipLaunchKernelGGL(attend_merge_kernel, dim3(heads, tokens), dim3(head_dim < 64 ? 64 : head_dim), 0, s,
                     part_acc, part_ml, heads, head_dim, pos_dev, count_host, chunks, out,
                     (uint8_t*)xq_out);
  return hip_check(hipGetLastError(), "attend_merge launch");
}

int launch_argmax(hipStream_t s, const float* x, int32_t n, int32_t tokens, int32_t* out) {
  hipLaunchKernelGGL(argmax_kernel, dim3(tokens), dim3(1024), 0, s, x, n, out);
  return hip_check(hipGetLastError(), "argmax launch");
}

int launch_embed(hipStream_t s, const float* emb, int32_t vocab, int32_t width, const int32_t* ids,
                 int32_t tokens, float* out) {
  dim3 grid((width / 4 + 255) / 256, tokens);
  hipLaunchKernelGGL(embed_kernel, grid, dim3(256), 0, s, emb, vocab, width, ids, out);
  return hip_check(hipGetLastError(), "embed launch");
}

}  // namespace mi

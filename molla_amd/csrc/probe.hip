// probe.hip -- measurement helper for bench.py, not part of the decode path:
// a plain streaming read, so the bench line can report the read ceiling it
// measured on the same box next to the matvec's roofline fraction.
//
// probe_read: every thread of `blocks` x 256 reads float4s of the buffer
// in a grid-stride loop, four loads in flight per step, and folds them into
// a sum that is stored only if it hits an impossible value (so the loads
// are not dropped).  Built as its own library, libmolla_probe.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void read_kernel(const float4* __restrict__ p, int64_t n4,
                                                   float* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  float a = 0.0f;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    const float4 v0 = p[i], v1 = p[i + stride], v2 = p[i + 2 * stride], v3 = p[i + 3 * stride];
    a += (v0.x + v1.y) + (v2.z + v3.w);
  }
  for (; i < n4; i += stride) a += p[i].x;
  if (a == -1.2345e-30f) sink[0] = a;
}

}  // namespace

extern "C" int probe_read(void* stream, const void* p, int64_t bytes, int32_t blocks, float* sink) {
  if (!p || bytes < 16 || blocks <= 0 || ((uintptr_t)p & 15)) return -1;
  hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const float4*)p, bytes / 16,
                     sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

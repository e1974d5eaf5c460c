// Small device utilities of the runtime: tessery's elementwise `add` (kernels.metal:300-304),
// used by the runtime lifecycle tests, and a 16-byte copy that calibrates HBM traffic counters.
#include "common.h"
#include "kernels.h"

namespace tessery {

__global__ __launch_bounds__(256) void add_f32(const float* a, const float* b, float* out,
                                               uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) out[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void copy16(const uint4v* __restrict__ src, uint4v* __restrict__ dst,
                                              uint64_t n16) {
  for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n16; i += gridDim.x * 256ull)
    dst[i] = src[i];
}

hipError_t launch_add_f32(const float* a, const float* b, float* out, uint32_t n,
                          hipStream_t st) {
  if (!n) return hipSuccess;
  add_f32<<<(n + 255) / 256, 256, 0, st>>>(a, b, out, n);
  return hipGetLastError();
}

hipError_t launch_copy(const void* src, void* dst, uint64_t bytes, hipStream_t st) {
  if (bytes % 16) return hipErrorInvalidValue;
  const uint64_t n16 = bytes / 16;
  if (!n16) return hipSuccess;
  const uint64_t blocks = (n16 + 255) / 256;
  copy16<<<static_cast<unsigned>(blocks < 8192 ? blocks : 8192), 256, 0, st>>>(
      static_cast<const uint4v*>(src), static_cast<uint4v*>(dst), n16);
  return hipGetLastError();
}

}  // namespace tessery

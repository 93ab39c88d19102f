// Device-to-device copy used to measure the sustainable HBM rate of one GPU
// (read + write, 16-byte accesses, grid-stride with four independent vectors
// in flight per lane).
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const u32x4 a = src[i];
    const u32x4 b = src[i + stride];
    const u32x4 c = src[i + 2 * stride];
    const u32x4 d = src[i + 3 * stride];
    dst[i] = a;
    dst[i + stride] = b;
    dst[i + 2 * stride] = c;
    dst[i + 3 * stride] = d;
  }
  for (; i < n; i += stride) dst[i] = src[i];
}

}  // namespace

hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t s) {
  const int64_t n = bytes / 16;
  const int block = 256;
  // 256 CUs x 8 workgroups of 256 lanes keeps every SIMD busy; larger grids
  // only add scheduling overhead for a bandwidth-bound loop.
  int64_t grid = (n + block - 1) / block;
  if (grid > 2048 * 4) grid = 2048 * 4;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(block), 0, s,
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return hipGetLastError();
}

}  // namespace vbh

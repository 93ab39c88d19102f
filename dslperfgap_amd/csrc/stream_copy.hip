// Device-to-device copy used to measure the sustainable HBM rate of one GPU.
// Each 256-lane workgroup moves one contiguous 4 KiB tile (one 16-byte access
// per lane) with nontemporal hints, so reads and writes stream through the
// caches; the grid covers the buffer once.
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t s) {
  const int64_t n = bytes / 16;
  const int block = 256;
  const int64_t grid = (n + block - 1) / block;
  hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(block), 0, s,
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return hipGetLastError();
}

}  // namespace vbh

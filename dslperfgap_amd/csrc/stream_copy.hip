// The two yardstick kernels of the measured HBM rates of one GPU.
//
// copy_kernel: device-to-device copy (read + write).  Each 256-lane workgroup
// moves one contiguous 4 KiB tile (one 16-byte access per lane); the grid
// covers the buffer once.  Loads are nontemporal; stores are nontemporal and
// written through the L2 at device scope (the row kernels' kStoreThrough
// policy), the fastest store form measured on MI355X for a 4 GiB copy: 6657
// GB/s against 6467 with nontemporal stores kept in the L2.
//
// read_kernel: streaming read (the yardstick of kernels that read far more
// than they write: logsumexp, the cross-entropy forward, mean / max / argmax).
// A persistent grid of one 256-lane workgroup per CU walks the buffer in
// contiguous 32 KiB tiles (tile b, b + grid, ...), eight nontemporal 16-byte
// loads per lane per tile, folding every word by XOR into one 32-bit word per
// workgroup, so every load is used.  The workgroups move through memory
// together, a window of one tile per CU.  MI355X, 4 GiB: 7330-7353 GB/s,
// against 6909-6974 for one 16 KiB tile per workgroup over a grid that covers
// the buffer once; 24-32 KiB in flight per CU beat every larger or smaller
// amount tried (one workgroup per CU with 4 loads per lane: 5306-5349;
// 2 workgroups per CU with 4: 7220-7240; 3 with 2: 7230-7274).
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n) {
  const int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x;
  const int64_t i = first + threadIdx.x;
  // the workgroup's tile [first, first + tile) is the store window (its range
  // check also drops any store past the end of the buffer)
  const int64_t tile = n - first < blockDim.x ? n - first : blockDim.x;
  const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
      dst + first, static_cast<short>(0), static_cast<int>(tile * sizeof(u32x4)), kRawBufferWord3);
  const Span ss = VBH_SPAN(src, n), sd = VBH_SPAN(dst, n);
  if (i < n && VBH_IN_SPAN(ss, src + i, sizeof(u32x4)) && VBH_IN_SPAN(sd, dst + i, sizeof(u32x4)))
    __builtin_amdgcn_raw_buffer_store_b128(
        __builtin_bit_cast(i32x4, __builtin_nontemporal_load(src + i)), out,
        static_cast<int>(threadIdx.x * sizeof(u32x4)), 0, kCacheNtSc1);
}

constexpr int kReadBlock = 256;

template <int U>
__global__ __launch_bounds__(kReadBlock) void read_kernel(const u32x4* __restrict__ src,
                                                          uint32_t* __restrict__ partial,
                                                          int64_t n) {
  constexpr int64_t kTile = int64_t(kReadBlock) * U;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kTile;
  const Span ss = VBH_SPAN(src, n), sp = VBH_SPAN(partial, gridDim.x);
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t first = static_cast<int64_t>(blockIdx.x) * kTile; first < n; first += step) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = first + u * kReadBlock + threadIdx.x;
      v[u] = i < n && VBH_IN_SPAN(ss, src + i, sizeof(u32x4)) ? __builtin_nontemporal_load(src + i)
                                                           : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
  for (int m = kWave / 2; m >= 1; m /= 2) x ^= __shfl_xor(x, m, kWave);
  __shared__ uint32_t lds[kReadBlock / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kReadBlock / kWave; ++w) r ^= lds[w];
    if (VBH_IN_SPAN(sp, partial + blockIdx.x, sizeof(uint32_t))) partial[blockIdx.x] = r;
  }
}

}  // namespace

int64_t stream_read_tiles(int64_t bytes) {
  const int64_t tile = int64_t(kReadBlock) * kReadUnroll * 16;
  return (bytes + tile - 1) / tile;
}

hipError_t launch_stream_read(const void* src, void* partial, int64_t bytes, int grid,
                              hipStream_t s) {
  const int64_t n = bytes / 16;
  launch_kernel(read_kernel<kReadUnroll>, dim3(grid), dim3(kReadBlock), 0, s,
                static_cast<const u32x4*>(src), static_cast<uint32_t*>(partial), n);
  return hipGetLastError();
}

hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t s) {
  const int64_t n = bytes / 16;
  const int block = 256;
  const int64_t grid = (n + block - 1) / block;
  launch_kernel(copy_kernel, dim3(grid), dim3(block), 0, s,
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return hipGetLastError();
}

}  // namespace vbh

// LayerNorm and RMSNorm forward for gfx950.
//
// Register-resident path (rows of up to 64 * tpr values per lane group):
//   `tpr` lanes own one row; each lane loads its share of the row with 16-byte
//   loads into fp32 registers exactly once, the row statistics are all-reduced
//   across the group (DPP / permlane inside a wave, LDS across waves), and the
//   normalized row is written once in the input dtype.
// Streaming path (wider rows): one 1024-thread workgroup per row, a statistics
//   pass (Welford/Chan moments for LayerNorm) and an output pass that reads the
//   row again.
//
// Semantics follow ViperBench/layer_norm/pytorch_impl.py:5-12 (F.layer_norm,
// biased variance, y = (x - mean) * rstd * w + b) and
// ViperBench/rms_norm/pytorch_impl.py:8-10 (rms = sqrt(mean(x^2) + eps),
// y = (x / rms) * w, rounded to x's dtype).
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

template <typename T, int V, int MAXIT>
__device__ __forceinline__ void load_row(const T* __restrict__ xr, int nvec, int g, int tpr,
                                         float (&v)[MAXIT][V]) {
#pragma unroll
  for (int i = 0; i < MAXIT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v[i]);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) v[i][k] = 0.f;
    }
  }
}

template <int V>
__device__ __forceinline__ float tree_sum(const float (&a)[V]) {
  float t[V];
#pragma unroll
  for (int k = 0; k < V; ++k) t[k] = a[k];
#pragma unroll
  for (int w = V / 2; w >= 1; w /= 2)
#pragma unroll
    for (int k = 0; k < w; ++k) t[k] += t[k + w];
  return t[0];
}

// ---------------------------------------------------------------------------
// register-resident kernels
// ---------------------------------------------------------------------------

template <typename T, typename TW, int V, int MAXIT>
__global__ __launch_bounds__(kMaxBlock) void layer_norm_rows(
    const T* __restrict__ x, const TW* __restrict__ w, const TW* __restrict__ b,
    T* __restrict__ y, int64_t rows, int cols, int tpr, float eps) {
  __shared__ float lds[2][kMaxWaves];
  const int nvec = cols / V;
  const int g = threadIdx.x & (tpr - 1);
  int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / tpr) + threadIdx.x / tpr;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const T* xr = x + row * cols;

  float v[MAXIT][V];
  load_row<T, V, MAXIT>(xr, nvec, g, tpr, v);

  // exact two-pass moments over the register-resident row
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < MAXIT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] += v[i][k];
  const float sum = group_allreduce<Sum>(tree_sum<V>(acc), tpr, lds[0]);
  const float mean = sum / static_cast<float>(cols);

#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < MAXIT; ++i) {
    if (i * tpr + g < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const float d = v[i][k] - mean;
        acc[k] = fmaf(d, d, acc[k]);
      }
    }
  }
  const float m2 = group_allreduce<Sum>(tree_sum<V>(acc), tpr, lds[1]);
  const float rstd = 1.0f / sqrtf(m2 / static_cast<float>(cols) + eps);
  if (!live) return;

  T* yr = y + row * cols;
#pragma unroll
  for (int i = 0; i < MAXIT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      float wv[V], bv[V], o[V];
      load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv);
      if (b != nullptr) {
        load_f32<TW, V>(b + static_cast<int64_t>(j) * V, bv);
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k) bv[k] = 0.f;
      }
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = (v[i][k] - mean) * rstd * wv[k] + bv[k];
      store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o);
    }
  }
}

template <typename T, typename TW, int V, int MAXIT>
__global__ __launch_bounds__(kMaxBlock) void rms_norm_rows(
    const T* __restrict__ x, const TW* __restrict__ w, T* __restrict__ y, int64_t rows,
    int cols, int tpr, float eps) {
  __shared__ float lds[kMaxWaves];
  const int nvec = cols / V;
  const int g = threadIdx.x & (tpr - 1);
  int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / tpr) + threadIdx.x / tpr;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const T* xr = x + row * cols;

  float v[MAXIT][V];
  load_row<T, V, MAXIT>(xr, nvec, g, tpr, v);

  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < MAXIT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] = fmaf(v[i][k], v[i][k], acc[k]);
  const float ss = group_allreduce<Sum>(tree_sum<V>(acc), tpr, lds);
  const float rinv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
  if (!live) return;

  T* yr = y + row * cols;
#pragma unroll
  for (int i = 0; i < MAXIT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      float wv[V], o[V];
      load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv);
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = (v[i][k] * rinv) * wv[k];
      store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o);
    }
  }
}

// ---------------------------------------------------------------------------
// streaming kernels (one 1024-thread workgroup per row, chunked two passes)
// ---------------------------------------------------------------------------

template <typename T, typename TW, int V>
__global__ __launch_bounds__(kMaxBlock) void layer_norm_stream(
    const T* __restrict__ x, const TW* __restrict__ w, const TW* __restrict__ b,
    T* __restrict__ y, int cols, float eps) {
  __shared__ float lds[3 * kMaxWaves];
  const int tpr = blockDim.x;
  const int nvec = cols / V;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  Moments m{0.f, 0.f, 0.f};
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) s += v[k];
    const float cm = s / static_cast<float>(V);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) q = fmaf(v[k] - cm, v[k] - cm, q);
    m = merge_moments(m, Moments{static_cast<float>(V), cm, q});
  }
  m = group_allreduce_moments(m, tpr, lds);
  const float mean = m.mean;
  const float rstd = 1.0f / sqrtf(m.m2 / static_cast<float>(cols) + eps);
  T* yr = y + row * cols;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V], wv[V], bv[V], o[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v);
    load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv);
    if (b != nullptr) {
      load_f32<TW, V>(b + static_cast<int64_t>(j) * V, bv);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) bv[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = (v[k] - mean) * rstd * wv[k] + bv[k];
    store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o);
  }
}

template <typename T, typename TW, int V>
__global__ __launch_bounds__(kMaxBlock) void rms_norm_stream(
    const T* __restrict__ x, const TW* __restrict__ w, T* __restrict__ y, int cols,
    float eps) {
  __shared__ float lds[kMaxWaves];
  const int tpr = blockDim.x;
  const int nvec = cols / V;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * cols;
  float acc = 0.f;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v);
#pragma unroll
    for (int k = 0; k < V; ++k) acc = fmaf(v[k], v[k], acc);
  }
  const float ss = group_allreduce<Sum>(acc, tpr, lds);
  const float rinv = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
  T* yr = y + row * cols;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V], wv[V], o[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v);
    load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv);
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = (v[k] * rinv) * wv[k];
    store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o);
  }
}

// weight dtype: either the activation dtype or fp32
template <typename T, typename Fn>
bool dispatch_weight_type(int dt, int wdt, Fn&& fn) {
  if (wdt == dt) {
    fn(TypeTag<T>{});
    return true;
  }
  if (wdt == kF32) {
    fn(TypeTag<float>{});
    return true;
  }
  return false;
}

}  // namespace

hipError_t launch_layer_norm(const void* x, const void* w, const void* b, void* y,
                             int64_t rows, int cols, float eps, int dt, int wdt,
                             const Geometry& g, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_float_type(dt, [&](auto tt) {
    using T = typename decltype(tt)::type;
    dispatch_weight_type<T>(dt, wdt, [&](auto wt) {
      using TW = typename decltype(wt)::type;
      constexpr int VN = Vec<T>::n;
      auto go = [&](auto vc) {
        constexpr int V = decltype(vc)::value;
        if (g.stream) {
          hipLaunchKernelGGL((layer_norm_stream<T, TW, V>), dim3(rows), dim3(g.block), 0, s,
                             static_cast<const T*>(x), static_cast<const TW*>(w),
                             static_cast<const TW*>(b), static_cast<T*>(y), cols, eps);
          err = hipGetLastError();
          return;
        }
        dispatch_maxit(g.maxit, [&](auto mc) {
          constexpr int M = decltype(mc)::value;
          if constexpr (M <= lane_cap(V)) {
            hipLaunchKernelGGL((layer_norm_rows<T, TW, V, M>), dim3(grid_for(rows, g)),
                               dim3(g.block), 0, s, static_cast<const T*>(x),
                               static_cast<const TW*>(w), static_cast<const TW*>(b),
                               static_cast<T*>(y), rows, cols, g.tpr, eps);
            err = hipGetLastError();
          }
        });
      };
      if (g.v == 1) go(std::integral_constant<int, 1>{});
      else go(std::integral_constant<int, VN>{});
    });
  });
  return err;
}

hipError_t launch_rms_norm(const void* x, const void* w, void* y, int64_t rows, int cols,
                           float eps, int dt, int wdt, const Geometry& g, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_float_type(dt, [&](auto tt) {
    using T = typename decltype(tt)::type;
    dispatch_weight_type<T>(dt, wdt, [&](auto wt) {
      using TW = typename decltype(wt)::type;
      constexpr int VN = Vec<T>::n;
      auto go = [&](auto vc) {
        constexpr int V = decltype(vc)::value;
        if (g.stream) {
          hipLaunchKernelGGL((rms_norm_stream<T, TW, V>), dim3(rows), dim3(g.block), 0, s,
                             static_cast<const T*>(x), static_cast<const TW*>(w),
                             static_cast<T*>(y), cols, eps);
          err = hipGetLastError();
          return;
        }
        dispatch_maxit(g.maxit, [&](auto mc) {
          constexpr int M = decltype(mc)::value;
          if constexpr (M <= lane_cap(V)) {
            hipLaunchKernelGGL((rms_norm_rows<T, TW, V, M>), dim3(grid_for(rows, g)),
                               dim3(g.block), 0, s, static_cast<const T*>(x),
                               static_cast<const TW*>(w), static_cast<T*>(y), rows, cols,
                               g.tpr, eps);
            err = hipGetLastError();
          }
        });
      };
      if (g.v == 1) go(std::integral_constant<int, 1>{});
      else go(std::integral_constant<int, VN>{});
    });
  });
  return err;
}

}  // namespace vbh

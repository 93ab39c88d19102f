// LayerNorm and RMSNorm forward for gfx950.
//
// Register-resident path: `tpr` lanes own one row (a power of two up to 64, or
// any multiple of 64 up to 1024).  Each lane loads its share of the row once,
// with 16-byte loads, into registers that keep the storage type (two bf16/fp16
// values per VGPR), widens to fp32 where a value is used, and the row
// statistics are all-reduced across the group (DPP / permlane inside a wave, an
// LDS exchange across waves).  The normalized row is
// written once in the input dtype.
//   LayerNorm statistics are the exact two-pass ones over the register-resident
//   row: the row sum gives the mean, then the sum of squared deviations from it
//   gives the biased variance (two all-reduces of plain sums); fp32 rows are
//   first shifted by their first element (kShiftLN).
//   Weight / bias slices are loaded together with the row when the registers
//   allow, so a row costs one memory round trip.
// Persistent pipelined path (vbh_tune_override / heuristic): the grid holds as
//   many workgroups as are resident at once; each row group loops over rows,
//   keeps its weight / bias slice in registers for the whole kernel, and loads
//   its next row before reducing the current one.
// Streaming path (rows wider than the register budget): one 1024-lane
//   workgroup per row; a Welford/Chan statistics pass, then an output pass that
//   reads the row again, both on the row shifted by its first element.
//
// Semantics: ViperBench/layer_norm/pytorch_impl.py:5-12 (F.layer_norm, biased
// variance, y = (x - mean) * rstd * w + b) and ViperBench/rms_norm/pytorch_impl.py:8-10
// (rms = sqrt(mean(x^2) + eps), y = (x / rms) * w, rounded to x's dtype).
#include <algorithm>

#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

template <typename T, int V, int IT, bool NT, bool FULL = false>
__device__ __forceinline__ void load_raw_row(const T* __restrict__ xr, int nvec, int g, int tpr,
                                             typename Raw<T, V>::type (&dst)[IT],
                                             const Span& s) {
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (FULL || j < nvec) dst[i] = load_raw<T, V, NT>(xr + static_cast<int64_t>(j) * V, s);
    else dst[i] = typename Raw<T, V>::type{};
  }
}

template <typename T, int V, int IT>
__device__ __forceinline__ void zero_row(typename Raw<T, V>::type (&dst)[IT]) {
#pragma unroll
  for (int i = 0; i < IT; ++i) dst[i] = typename Raw<T, V>::type{};
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

// Products of 16-bit pairs on the packed dot-product unit: a.lo * b.lo +
// a.hi * b.hi + c (v_dot2c_f32_bf16 / v_dot2c_f32_f16; the products of 16-bit
// values are exact in fp32), two values per instruction and no widening.
template <typename T> struct Pair;
template <> struct Pair<__bf16> {
  typedef __bf16 type __attribute__((ext_vector_type(2)));
  __device__ static float dot(type a, type b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <> struct Pair<_Float16> {
  typedef _Float16 type __attribute__((ext_vector_type(2)));
  __device__ static float dot(type a, type b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
};

// sum over the lane's 16-bit values of x * (SQ ? x : 1), V / 2 accumulators
template <typename T, int V, int IT, bool SQ>
__device__ __forceinline__ float lane_dot2_sum(const typename Raw<T, V>::type (&xr)[IT]) {
  typedef typename Pair<T>::type P;
  float acc[V / 2];
#pragma unroll
  for (int k = 0; k < V / 2; ++k) acc[k] = 0.f;
  P one;
  one[0] = static_cast<T>(1.0f);
  one[1] = static_cast<T>(1.0f);
#pragma unroll
  for (int i = 0; i < IT; ++i) {
#pragma unroll
    for (int k = 0; k < V / 2; ++k) {
      P x;
      x[0] = xr[i][2 * k];
      x[1] = xr[i][2 * k + 1];
      acc[k] = Pair<T>::dot(x, SQ ? x : one, acc[k]);
    }
  }
  return tree_sum<V / 2>(acc);
}

// Sum of the lane's values (padding vectors are zero).
template <typename T, int V, int IT>
__device__ __forceinline__ float lane_sum(const typename Raw<T, V>::type (&xr)[IT]) {
  if constexpr (sizeof(T) == 2 && V >= 2) return lane_dot2_sum<T, V, IT, false>(xr);
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] += raw_at<T, V>(xr[i], k);
  return tree_sum<V>(acc);
}

// Sum of squared deviations from `mean` over the lane's valid values
// (vectors i with i * tpr + g < nvec).
template <typename T, int V, int IT, bool FULL = false>
__device__ __forceinline__ float lane_centered_sumsq(const typename Raw<T, V>::type (&xr)[IT],
                                                     float mean, int nvec, int g, int tpr) {
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    if (FULL || i * tpr + g < nvec) {
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const float d = raw_at<T, V>(xr[i], k) - mean;
        acc[k] = fmaf(d, d, acc[k]);
      }
    }
  }
  return tree_sum<V>(acc);
}

template <typename T, int V, int IT>
__device__ __forceinline__ float lane_sumsq(const typename Raw<T, V>::type (&xr)[IT]) {
  if constexpr (sizeof(T) == 2 && V >= 2) return lane_dot2_sum<T, V, IT, true>(xr);
  float acc[V];
#pragma unroll
  for (int k = 0; k < V; ++k) acc[k] = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float v = raw_at<T, V>(xr[i], k);  // padding vectors are zero
      acc[k] = fmaf(v, v, acc[k]);
    }
  return tree_sum<V>(acc);
}

// Row statistics on the hardware units: 1 / cols by v_rcp_f32 and 1 / sqrt(v)
// by v_rsq_f32 (1 ulp each; torch's rsqrt is the latter), where IEEE division
// and square root take about ten instructions each, paid per lane and row.
__device__ __forceinline__ float inv_count(int cols) {
  return __builtin_amdgcn_rcpf(static_cast<float>(cols));
}
__device__ __forceinline__ float rsqrt_hw(float v) { return __builtin_amdgcn_rsqf(v); }

// sum / cols for the row mean: the v_rcp_f32 quotient refined by one residual
// step (the residual sum - q * cols is exact in the FMA).  It matched the
// correctly rounded quotient in all of 66,000 emulated cases, with the
// reciprocal also taken 1 ulp off either way; a row of equal values thus gets
// its value back exactly and centres to 0, as under IEEE division.
__device__ __forceinline__ float mean_of(float sum, int cols) {
  const float n = static_cast<float>(cols);
  const float inv = __builtin_amdgcn_rcpf(n);
  const float q = sum * inv;
  return fmaf(fmaf(-q, n, sum), inv, q);
}

// fp32 LayerNorm rows are shifted by their first element x0 before their
// statistics, in the row's registers, and normalized in that shifted form:
// y = ((x - x0) - mean') * rstd * w + b with mean' = mean(x - x0).  The row
// mean as an fp32 number carries a rounding of up to half an ulp of |mean|,
// which x - mean divides by the row's deviation: at |mean| / std = 1000 that
// is 1e-4 of every output, in torch's fp32 LayerNorm too.  Shifted, the mean
// is that of x - x0, within a few deviations of 0, and x - x0 itself is exact
// where it matters (Sterbenz: x within a factor 2 of x0), so the error stays
// near 1e-6 at any |mean| / std.  One subtract per element; 16-bit rows keep
// their raw values (their output rounding, 2^-8 or 2^-11, dwarfs the mean's).
template <typename T>
constexpr bool kShiftLN = sizeof(T) == 4;

template <typename T, int V, int IT, bool FULL = false>
__device__ __forceinline__ void shift_row(typename Raw<T, V>::type (&xr)[IT], float x0, int nvec,
                                          int g, int tpr) {
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    if (FULL || i * tpr + g < nvec) {  // padding vectors stay 0
      if constexpr (V == 1) {
        xr[i] -= x0;
      } else {
#pragma unroll
        for (int k = 0; k < V; ++k) xr[i][k] -= x0;
      }
    }
  }
}

// The shift of a row starting at `xr`: its first element for fp32 rows, else 0.
template <typename T>
__device__ __forceinline__ float row_shift(const T* __restrict__ xr, const Span& s) {
  if constexpr (!kShiftLN<T>) return 0.f;
  float x0;
  load_f32<T, 1>(xr, &x0, s);
  return x0;
}

// Weight / bias slices ride along with the row when they take at most 32
// VGPRs in raw storage; otherwise they are read after the reduction.
template <typename TW, int V, int IT> constexpr bool kEarlyLN = 2 * raw_vgprs<TW>(V, IT) <= 32;
template <typename TW, int V, int IT> constexpr bool kEarlyRMS = raw_vgprs<TW>(V, IT) <= 32;

// Deepest row slice (vectors per lane) of the persistent kernels: current and
// next row plus the per-column vectors must stay within about 64 VGPRs of raw
// storage.
template <typename T, typename TW, int V, int NVEC_COL>
constexpr int pipe_cap() {
  int it = kPipeMaxIt;
  while (it > 1 && 2 * raw_vgprs<T>(V, it) + NVEC_COL * raw_vgprs<TW>(V, it) > 64)
    it /= 2;
  return it;
}

// ---------------------------------------------------------------------------
// register-resident kernels: one row group per row
// ---------------------------------------------------------------------------

template <typename T, typename TW, int V, int IT, int SP>
__global__ __launch_bounds__(kMaxBlock) void layer_norm_rows(
    const T* __restrict__ x, const TW* __restrict__ w, const TW* __restrict__ b,
    T* __restrict__ y, int64_t rows, int cols, int tpr, float eps) {
  typedef typename Raw<T, V>::type RT;
  typedef typename Raw<TW, V>::type RW;
  __shared__ float lds[2][kMaxWaves];
  const int nvec = cols / V;
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * rpb;
  int64_t row = first + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const Span sw = VBH_SPAN(w, cols), sb = VBH_SPAN(b, cols);

  const float x0 = row_shift<T>(x + row * cols, sx);
  RT xr[IT];
  load_raw_row<T, V, IT, SP != kStoreCached>(x + row * cols, nvec, g, tpr, xr, sx);
  constexpr bool kEarly = kEarlyLN<TW, V, IT>;
  RW wr[kEarly ? IT : 1], br[kEarly ? IT : 1];
  if constexpr (kEarly) {
    load_raw_row<TW, V, IT, false>(w, nvec, g, tpr, wr, sw);
    if (b != nullptr) load_raw_row<TW, V, IT, false>(b, nvec, g, tpr, br, sb);
  }
  if constexpr (kShiftLN<T>) shift_row<T, V, IT>(xr, x0, nvec, g, tpr);

  const float mean =
      mean_of(group_allreduce<Sum>(lane_sum<T, V, IT>(xr), tpr, lds[0]), cols);
  reload_barrier<T, V, IT>(xr);
  const float m2 = group_allreduce<Sum>(lane_centered_sumsq<T, V, IT>(xr, mean, nvec, g, tpr),
                                        tpr, lds[1]);
  const float rstd = rsqrt_hw(m2 * inv_count(cols) + eps);
  if (!live) return;
  reload_barrier<T, V, IT>(xr);

  const OutWindow<T, SP> out(y + first * cols, std::min<int64_t>(rpb, rows - first) * cols);
  T* yr = y + row * cols;
  const int yoff = static_cast<int>(row - first) * cols;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      RW wv, bv{};
      if constexpr (kEarly) {
        wv = wr[i];
        if (b != nullptr) bv = br[i];
      } else {
        wv = load_raw<TW, V, false>(w + static_cast<int64_t>(j) * V, sw);
        if (b != nullptr) bv = load_raw<TW, V, false>(b + static_cast<int64_t>(j) * V, sb);
      }
      float o[V];
#pragma unroll
      for (int k = 0; k < V; ++k)
        o[k] = (raw_at<T, V>(xr[i], k) - mean) * rstd * raw_at<TW, V>(wv, k) +
               raw_at<TW, V>(bv, k);
      out.template store<V>(yr + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
    }
  }
}

template <typename T, typename TW, int V, int IT, int SP>
__global__ __launch_bounds__(kMaxBlock) void rms_norm_rows(
    const T* __restrict__ x, const TW* __restrict__ w, T* __restrict__ y, int64_t rows,
    int cols, int tpr, float eps) {
  typedef typename Raw<T, V>::type RT;
  typedef typename Raw<TW, V>::type RW;
  __shared__ float lds[kMaxWaves];
  const int nvec = cols / V;
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * rpb;
  int64_t row = first + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const Span sw = VBH_SPAN(w, cols);

  RT xr[IT];
  load_raw_row<T, V, IT, SP != kStoreCached>(x + row * cols, nvec, g, tpr, xr, sx);
  constexpr bool kEarly = kEarlyRMS<TW, V, IT>;
  RW wr[kEarly ? IT : 1];
  if constexpr (kEarly) load_raw_row<TW, V, IT, false>(w, nvec, g, tpr, wr, sw);

  const float ss = group_allreduce<Sum>(lane_sumsq<T, V, IT>(xr), tpr, lds);
  const float rinv = rsqrt_hw(ss * inv_count(cols) + eps);
  if (!live) return;
  reload_barrier<T, V, IT>(xr);

  const OutWindow<T, SP> out(y + first * cols, std::min<int64_t>(rpb, rows - first) * cols);
  T* yr = y + row * cols;
  const int yoff = static_cast<int>(row - first) * cols;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      RW wv;
      if constexpr (kEarly) wv = wr[i];
      else wv = load_raw<TW, V, false>(w + static_cast<int64_t>(j) * V, sw);
      float o[V];
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = (raw_at<T, V>(xr[i], k) * rinv) * raw_at<TW, V>(wv, k);
      out.template store<V>(yr + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
    }
  }
}

// ---------------------------------------------------------------------------
// rows not a multiple of V long (MIS): each row, starting at element `start`
// of a 16-byte aligned buffer, is a scalar head up to the first 16-byte
// boundary (lanes g < head hold element g), whole aligned vectors and a
// scalar tail (lanes g < tail); the launcher makes tpr >= V.  The weight and
// bias of body vector j are elements [head + j V, head + j V + V), read as
// vectors at the nearest dword boundary (row_weights).  Nothing outside the
// row or the weights is read or written.
// ---------------------------------------------------------------------------

struct NormMisRow {
  int head, nvec, tail;
};

template <int V>
__device__ __forceinline__ NormMisRow norm_mis_row(int64_t start, int cols) {
  int head = static_cast<int>((V - start % V) % V);
  if (head > cols) head = cols;
  const int nvec = (cols - head) / V;
  return NormMisRow{head, nvec, cols - head - nvec * V};
}

// Global loads of several dwords need only dword alignment on gfx9, so the
// weights of body vector j come from one vector load at a dword boundary:
// elements [head + jV, head + jV + V) themselves for 4-byte weights and for
// 16-bit weights at an even head; at an odd head, 16-bit weights load the V
// elements from one element earlier plus element head + jV + V - 1 (inside
// the body) and take each element from its upper neighbour.  No branch on
// `head`, so a wave holding rows of different heads does not diverge.
template <typename TW, int V>
__device__ __forceinline__ void row_weights(const TW* __restrict__ w, int j, int head,
                                            float (&out)[V], const Span& s) {
  typedef typename Raw<TW, V>::type RW;
  const TW* p = w + head + static_cast<int64_t>(j) * V;
  RW a;
  if constexpr (sizeof(TW) == 4) {
    if (!VBH_IN_SPAN(s, p, sizeof(a))) a = RW{};
    else __builtin_memcpy(&a, __builtin_assume_aligned(p, 4), sizeof(a));
#pragma unroll
    for (int k = 0; k < V; ++k) out[k] = raw_at<TW, V>(a, k);
  } else {
    static_assert(sizeof(TW) == 2, "16-bit or 4-byte weights");
    const int odd = head & 1;
    if (!VBH_IN_SPAN(s, p - odd, sizeof(a))) a = RW{};
    else __builtin_memcpy(&a, __builtin_assume_aligned(p - odd, 4), sizeof(a));
    const float last = odd && VBH_IN_SPAN(s, p + V - 1, sizeof(TW)) ? static_cast<float>(p[V - 1])
                                                                 : 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float up = k + 1 < V ? raw_at<TW, V>(a, k + 1) : last;
      out[k] = odd ? up : raw_at<TW, V>(a, k);
    }
  }
}

template <typename T, typename TW, int V, int IT, int SP, bool RMS>
__global__ __launch_bounds__(kMaxBlock) void norm_rows_mis(
    const T* __restrict__ x, const TW* __restrict__ w, const TW* __restrict__ b,
    T* __restrict__ y, int64_t rows, int cols, int tpr, float eps) {
  typedef typename Raw<T, V>::type RT;
  __shared__ float lds[2][kMaxWaves];
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * rpb;
  int64_t row = first + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const Span sw = VBH_SPAN(w, cols), sb = VBH_SPAN(b, cols);
  const int64_t start = row * cols;
  const NormMisRow mr = norm_mis_row<V>(start, cols);
  const int nvec = mr.nvec;
  const T* xb = x + start + mr.head;

  RT xr[IT];
  load_raw_row<T, V, IT, SP != kStoreCached>(xb, nvec, g, tpr, xr, sx);
  const bool hv = g < mr.head, tv = g < mr.tail;
  const int tcol = mr.head + nvec * V + g;  // this lane's tail column
  float hx = hv && VBH_IN_SPAN(sx, x + start + g, sizeof(T)) ? static_cast<float>(x[start + g])
                                                        : 0.f;
  float tx =
      tv && VBH_IN_SPAN(sx, x + start + tcol, sizeof(T)) ? static_cast<float>(x[start + tcol]) : 0.f;
  float mean = 0.f, scale;
  if constexpr (!RMS && kShiftLN<T>) {  // shifted by the row's first element
    const float x0 = row_shift<T>(x + start, sx);
    shift_row<T, V, IT>(xr, x0, nvec, g, tpr);
    if (hv) hx -= x0;
    if (tv) tx -= x0;
  }
  if constexpr (RMS) {
    const float ss = group_allreduce<Sum>(lane_sumsq<T, V, IT>(xr) + hx * hx + tx * tx, tpr,
                                          lds[0]);
    scale = rsqrt_hw(ss * inv_count(cols) + eps);
  } else {
    mean = mean_of(group_allreduce<Sum>(lane_sum<T, V, IT>(xr) + hx + tx, tpr, lds[0]), cols);
    reload_barrier<T, V, IT>(xr);
    float c2 = lane_centered_sumsq<T, V, IT>(xr, mean, nvec, g, tpr);
    if (hv) c2 = fmaf(hx - mean, hx - mean, c2);
    if (tv) c2 = fmaf(tx - mean, tx - mean, c2);
    const float m2 = group_allreduce<Sum>(c2, tpr, lds[1]);
    scale = rsqrt_hw(m2 * inv_count(cols) + eps);
  }
  if (!live) return;
  reload_barrier<T, V, IT>(xr);

  // element c of this row's output, from its value v
  auto out_at = [&](float v, int c) {
    const float wv = VBH_IN_SPAN(sw, w + c, sizeof(TW)) ? static_cast<float>(w[c]) : 0.f;
    if constexpr (RMS) return (v * scale) * wv;
    const float bv =
        b != nullptr && VBH_IN_SPAN(sb, b + c, sizeof(TW)) ? static_cast<float>(b[c]) : 0.f;
    return (v - mean) * scale * wv + bv;
  };
  const OutWindow<T, SP> out(y + first * cols, std::min<int64_t>(rpb, rows - first) * cols);
  T* yb = y + start + mr.head;
  const int yoff = static_cast<int>(row - first) * cols + mr.head;
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) {
      float wv[V], bv[V], o[V];
      row_weights<TW, V>(w, j, mr.head, wv, sw);
      if (!RMS && b != nullptr) row_weights<TW, V>(b, j, mr.head, bv, sb);
#pragma unroll
      for (int k = 0; k < V; ++k) {
        const float v = raw_at<T, V>(xr[i], k);
        if constexpr (RMS) o[k] = (v * scale) * wv[k];
        else o[k] = (v - mean) * scale * wv[k] + (b != nullptr ? bv[k] : 0.f);
      }
      out.template store<V>(yb + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
    }
  }
  if (hv) {
    const float o = out_at(hx, g);
    store_from_f32<T, 1>(y + start + g, &o, sy);
  }
  if (tv) {
    const float o = out_at(tx, tcol);
    store_from_f32<T, 1>(y + start + tcol, &o, sy);
  }
}

// ---------------------------------------------------------------------------
// persistent pipelined kernels
//
// Row group `grp` of workgroup `blk` handles rows blk*rpb + grp, then
// + gridDim.x*rpb, ...  The row loop is uniform across the workgroup (groups
// past the last row still take part in the barriers), and the LDS reduction
// buffers alternate between two parities, which makes one barrier per
// reduction sufficient: a thread can only overwrite a parity after passing the
// next iteration's barrier, which every thread reaches only after reading it.
//
// FULL drops every per-vector and per-row guard around the loads and stores
// (the host checks the preconditions: pipe_full).  The vector-memory counter of
// gfx9-family GPUs counts stores as well as loads, in order; with guarded
// (divergent) stores the compiler cannot count how many follow the next-row
// loads, so before using the prefetched row it waits for everything, this
// row's stores included.  Unguarded, the wait can leave the stores in flight.
// ---------------------------------------------------------------------------

template <typename T, typename TW, int V, int IT, int SP, bool FULL>
__global__ __launch_bounds__(kMaxBlock) void layer_norm_pipe(
    const T* __restrict__ x, const TW* __restrict__ w, const TW* __restrict__ b,
    T* __restrict__ y, int64_t rows, int cols, int tpr, float eps) {
  typedef typename Raw<T, V>::type RT;
  typedef typename Raw<TW, V>::type RW;
  __shared__ float lds[2][2][kMaxWaves];
  const int nvec = cols / V;
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int grp = gs.sub;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * rpb;
  constexpr bool kNT = SP != kStoreCached;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const Span sw = VBH_SPAN(w, cols), sb = VBH_SPAN(b, cols);

  RW wr[IT], br[IT];
  load_raw_row<TW, V, IT, false, FULL>(w, nvec, g, tpr, wr, sw);
  if (b != nullptr) load_raw_row<TW, V, IT, false, FULL>(b, nvec, g, tpr, br, sb);
  else
#pragma unroll
    for (int i = 0; i < IT; ++i) br[i] = RW{};

  RT cur[IT], nxt[IT];
  int64_t base = static_cast<int64_t>(blockIdx.x) * rpb;
  // Rows past the end: zero registers.  The guarded kernels get them from a
  // load helper whose guards are all false (which schedules better for fp32
  // rows than plain register zeroing); FULL never reaches the first branch.
  float x0 = 0.f, x0n = 0.f;  // the rows' shifts (kShiftLN)
  if (base + grp < rows) {
    x0 = row_shift<T>(x + (base + grp) * cols, sx);
    load_raw_row<T, V, IT, kNT, FULL>(x + (base + grp) * cols, nvec, g, tpr, cur, sx);
  } else {
    if constexpr (FULL) zero_row<T, V, IT>(cur);
    else load_raw_row<T, V, IT, kNT>(x, 0, g, tpr, cur, sx);
  }
  int par = 0;
  for (; base < rows; base += stride) {
    const int64_t row = base + grp;
    const int64_t next = row + stride;
    if (next < rows) {
      x0n = row_shift<T>(x + next * cols, sx);
      load_raw_row<T, V, IT, kNT, FULL>(x + next * cols, nvec, g, tpr, nxt, sx);
    } else {
      if constexpr (FULL) zero_row<T, V, IT>(nxt);
      else load_raw_row<T, V, IT, kNT>(x, 0, g, tpr, nxt, sx);
    }
    if constexpr (kShiftLN<T>) shift_row<T, V, IT, FULL>(cur, x0, nvec, g, tpr);

    const float mean =
        mean_of(group_allreduce<Sum>(lane_sum<T, V, IT>(cur), tpr, lds[par][0]), cols);
    reload_barrier<T, V, IT>(cur);
    const float m2 = group_allreduce<Sum>(
        lane_centered_sumsq<T, V, IT, FULL>(cur, mean, nvec, g, tpr), tpr, lds[par][1]);
    const float rstd = rsqrt_hw(m2 * inv_count(cols) + eps);
    reload_barrier<T, V, IT>(cur);
    if (FULL || row < rows) {
      const OutWindow<T, SP> out(y + base * cols, std::min<int64_t>(rpb, rows - base) * cols);
      T* yr = y + row * cols;
      const int yoff = grp * cols;
#pragma unroll
      for (int i = 0; i < IT; ++i) {
        const int j = i * tpr + g;
        if (FULL || j < nvec) {
          float o[V];
#pragma unroll
          for (int k = 0; k < V; ++k)
            o[k] = (raw_at<T, V>(cur[i], k) - mean) * rstd * raw_at<TW, V>(wr[i], k) +
                   raw_at<TW, V>(br[i], k);
          out.template store<V>(yr + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) cur[i] = nxt[i];
    x0 = x0n;
    par ^= 1;
  }
}

template <typename T, typename TW, int V, int IT, int SP, bool FULL>
__global__ __launch_bounds__(kMaxBlock) void rms_norm_pipe(
    const T* __restrict__ x, const TW* __restrict__ w, T* __restrict__ y, int64_t rows,
    int cols, int tpr, float eps) {
  typedef typename Raw<T, V>::type RT;
  typedef typename Raw<TW, V>::type RW;
  __shared__ float lds[2][kMaxWaves];
  const int nvec = cols / V;
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int grp = gs.sub;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * rpb;
  constexpr bool kNT = SP != kStoreCached;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const Span sw = VBH_SPAN(w, cols);

  RW wr[IT];
  load_raw_row<TW, V, IT, false, FULL>(w, nvec, g, tpr, wr, sw);
  RT cur[IT], nxt[IT];
  int64_t base = static_cast<int64_t>(blockIdx.x) * rpb;
  // Rows past the end: zero registers.  The guarded kernels get them from a
  // load helper whose guards are all false (which schedules better for fp32
  // rows than plain register zeroing); FULL never reaches the first branch.
  if (base + grp < rows) {
    load_raw_row<T, V, IT, kNT, FULL>(x + (base + grp) * cols, nvec, g, tpr, cur, sx);
  } else {
    if constexpr (FULL) zero_row<T, V, IT>(cur);
    else load_raw_row<T, V, IT, kNT>(x, 0, g, tpr, cur, sx);
  }
  int par = 0;
  for (; base < rows; base += stride) {
    const int64_t row = base + grp;
    const int64_t next = row + stride;
    if (next < rows) {
      load_raw_row<T, V, IT, kNT, FULL>(x + next * cols, nvec, g, tpr, nxt, sx);
    } else {
      if constexpr (FULL) zero_row<T, V, IT>(nxt);
      else load_raw_row<T, V, IT, kNT>(x, 0, g, tpr, nxt, sx);
    }

    const float ss = group_allreduce<Sum>(lane_sumsq<T, V, IT>(cur), tpr, lds[par]);
    const float rinv = rsqrt_hw(ss * inv_count(cols) + eps);
    reload_barrier<T, V, IT>(cur);
    if (FULL || row < rows) {
      const OutWindow<T, SP> out(y + base * cols, std::min<int64_t>(rpb, rows - base) * cols);
      T* yr = y + row * cols;
      const int yoff = grp * cols;
#pragma unroll
      for (int i = 0; i < IT; ++i) {
        const int j = i * tpr + g;
        if (FULL || j < nvec) {
          float o[V];
#pragma unroll
          for (int k = 0; k < V; ++k)
            o[k] = (raw_at<T, V>(cur[i], k) * rinv) * raw_at<TW, V>(wr[i], k);
          out.template store<V>(yr + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < IT; ++i) cur[i] = nxt[i];
    par ^= 1;
  }
}

// ---------------------------------------------------------------------------
// streaming kernels (one 1024-lane workgroup per row, chunked two passes)
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
  // one workgroup per row: the grid is the row count
  const Span sx = VBH_SPAN(x, static_cast<int64_t>(gridDim.x) * cols);
  const Span sy = VBH_SPAN(y, static_cast<int64_t>(gridDim.x) * cols);
  const Span sw = VBH_SPAN(w, cols), sb = VBH_SPAN(b, cols);
  // both passes work on x - x0 (x0 the row's first element; see kShiftLN),
  // in fp32 whatever the storage type
  float x0;
  load_f32<T, 1>(xr, &x0, sx);
  Moments m{0.f, 0.f, 0.f};
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v, sx);
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] -= x0;
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
  const float rstd = rsqrt_hw(m.m2 * inv_count(cols) + eps);
  T* yr = y + row * cols;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V], wv[V], bv[V], o[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v, sx);
    load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv, sw);
    if (b != nullptr) {
      load_f32<TW, V>(b + static_cast<int64_t>(j) * V, bv, sb);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) bv[k] = 0.f;
    }
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = ((v[k] - x0) - mean) * rstd * wv[k] + bv[k];
    store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o, sy);
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
  // one workgroup per row: the grid is the row count
  const Span sx = VBH_SPAN(x, static_cast<int64_t>(gridDim.x) * cols);
  const Span sy = VBH_SPAN(y, static_cast<int64_t>(gridDim.x) * cols);
  const Span sw = VBH_SPAN(w, cols);
  float acc = 0.f;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v, sx);
#pragma unroll
    for (int k = 0; k < V; ++k) acc = fmaf(v[k], v[k], acc);
  }
  const float ss = group_allreduce<Sum>(acc, tpr, lds);
  const float rinv = rsqrt_hw(ss * inv_count(cols) + eps);
  T* yr = y + row * cols;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V], wv[V], o[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v, sx);
    load_f32<TW, V>(w + static_cast<int64_t>(j) * V, wv, sw);
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = (v[k] * rinv) * wv[k];
    store_from_f32<T, V>(yr + static_cast<int64_t>(j) * V, o, sy);
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

// The unguarded (FULL) persistent kernel: 16-bit rows in which every lane
// holds exactly `it` vectors and a workgroup is one row group (then the grid,
// capped at the row count, gives every workgroup a row, and row == base <
// rows inside the loop).  Measured on MI355X against the guarded kernel:
// bf16 LayerNorm 2048 x 20480 5116 -> 5256 GB/s, 8192 x 8192 5638 -> 5730,
// fp16 RMSNorm 8192 x 8192 5851 -> 6014; fp32 rows lose 1-6%, so they keep
// the guarded kernel.
template <typename T>
constexpr bool kPipeFullType = sizeof(T) == 2;

// The guarded persistent kernels (rows that do not fill every lane) keep
// their output stores in the L2: the 16-bit LayerNorm one sits at the
// 128-VGPR cap of a 1024-lane workgroup and the write-through addressing
// would make it spill.
template <int SP>
constexpr int kGuardedPipeSP = SP == kStoreThrough ? kStoreStream : SP;

template <typename T>
bool pipe_full(const Geometry& g, int64_t nvec, int it) {
  return kPipeFullType<T> && g.v > 1 && g.block == g.tpr &&
         nvec == static_cast<int64_t>(it) * g.tpr;
}

// Launch the register-resident kernel (one row group per row) or the
// persistent one (grid capped at the resident capacity, and at the input
// bytes a CU may hold in flight: pipe_grid) through `launch`.
template <class RowsK, class PipeK, class Launch>
hipError_t launch_rows_or_pipe(RowsK rows_k, PipeK pipe_k, bool persist, int64_t rows,
                               const Geometry& g, Launch&& launch, int64_t row_bytes) {
  if (persist) launch(pipe_k, pipe_grid(reinterpret_cast<const void*>(pipe_k), g, rows, row_bytes));
  else launch(rows_k, grid_for(rows, g));
  return hipGetLastError();
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
          launch_kernel((layer_norm_stream<T, TW, V>), dim3(rows), dim3(g.block), 0, s,
                             static_cast<const T*>(x), static_cast<const TW*>(w),
                             static_cast<const TW*>(b), static_cast<T*>(y), cols, eps);
          err = hipGetLastError();
          return;
        }
        dispatch_maxit(g.maxit, [&](auto mc) {
          constexpr int M = decltype(mc)::value;
          if constexpr (M <= lane_cap(V)) {
            dispatch_store_policy<V>(g, [&](auto sp) {
              constexpr int SP = decltype(sp)::value;
              if constexpr (V > 1) {
                if (g.mis) {
                  launch_kernel((norm_rows_mis<T, TW, V, M, SP, false>),
                                     dim3(grid_for(rows, g)), dim3(g.block), 0, s,
                                     static_cast<const T*>(x), static_cast<const TW*>(w),
                                     static_cast<const TW*>(b), static_cast<T*>(y), rows, cols,
                                     g.tpr, eps);
                  err = hipGetLastError();
                  return;
                }
              }
              constexpr int PC = pipe_cap<T, TW, V, 2>();
              constexpr int MP = M <= PC ? M : PC;
              auto pipe_k = pipe_full<T>(g, cols / V, MP)
                                ? layer_norm_pipe<T, TW, V, MP, SP, V != 1 && kPipeFullType<T>>
                                : layer_norm_pipe<T, TW, V, MP, kGuardedPipeSP<SP>, false>;
              err = launch_rows_or_pipe(
                  layer_norm_rows<T, TW, V, M, SP>, pipe_k,
                  g.persist && M <= PC, rows, g, [&](auto kern, int64_t grid) {
                    launch_kernel(kern, dim3(grid), dim3(g.block), 0, s,
                                       static_cast<const T*>(x), static_cast<const TW*>(w),
                                       static_cast<const TW*>(b), static_cast<T*>(y), rows,
                                       cols, g.tpr, eps);
                  }, static_cast<int64_t>(cols) * sizeof(T));
            });
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
          launch_kernel((rms_norm_stream<T, TW, V>), dim3(rows), dim3(g.block), 0, s,
                             static_cast<const T*>(x), static_cast<const TW*>(w),
                             static_cast<T*>(y), cols, eps);
          err = hipGetLastError();
          return;
        }
        dispatch_maxit(g.maxit, [&](auto mc) {
          constexpr int M = decltype(mc)::value;
          if constexpr (M <= lane_cap(V)) {
            dispatch_store_policy<V>(g, [&](auto sp) {
              constexpr int SP = decltype(sp)::value;
              if constexpr (V > 1) {
                if (g.mis) {
                  launch_kernel((norm_rows_mis<T, TW, V, M, SP, true>),
                                     dim3(grid_for(rows, g)), dim3(g.block), 0, s,
                                     static_cast<const T*>(x), static_cast<const TW*>(w),
                                     static_cast<const TW*>(nullptr), static_cast<T*>(y), rows,
                                     cols, g.tpr, eps);
                  err = hipGetLastError();
                  return;
                }
              }
              constexpr int PC = pipe_cap<T, TW, V, 1>();
              constexpr int MP = M <= PC ? M : PC;
              auto pipe_k = pipe_full<T>(g, cols / V, MP)
                                ? rms_norm_pipe<T, TW, V, MP, SP, V != 1 && kPipeFullType<T>>
                                : rms_norm_pipe<T, TW, V, MP, kGuardedPipeSP<SP>, false>;
              err = launch_rows_or_pipe(
                  rms_norm_rows<T, TW, V, M, SP>, pipe_k,
                  g.persist && M <= PC, rows, g, [&](auto kern, int64_t grid) {
                    launch_kernel(kern, dim3(grid), dim3(g.block), 0, s,
                                       static_cast<const T*>(x), static_cast<const TW*>(w),
                                       static_cast<T*>(y), rows, cols, g.tpr, eps);
                  }, static_cast<int64_t>(cols) * sizeof(T));
            });
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

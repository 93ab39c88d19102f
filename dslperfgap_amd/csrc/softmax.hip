// Softmax, log-softmax and logsumexp forward for gfx950.
//
// Register-resident path: `tpr` lanes own one row (a power of two up to 64 or a
// multiple of 64 up to 1024) and load it once into registers that keep the
// storage type; the group all-reduces the row max, then the sum of
// exp(x - max), and writes the row once.
// Streaming path (rows wider than the register budget): one workgroup per row,
// online (max, rescaled sum) statistics pass, then an output pass.
// Middle-axis path: contiguous [outer, n, inner] reduced over n; one thread per
// (outer, inner) column, consecutive threads on consecutive inner indices so
// every access is coalesced.
//
// Semantics: ViperBench/softmax/pytorch_impl.py:4-6 (F.softmax, dim=-1),
// ViperBench/log_softmax/pytorch_impl.py:4-8 (F.log_softmax(x, dim, dtype)),
// ViperBench/logsumexp/pytorch_impl.py:3-5 (torch.logsumexp, dim=-1: the max
// used for the shift is replaced by 0 when it is infinite).
#include <algorithm>
#include <type_traits>

#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// fp16 values stay within 65504 < 2^24, so a row of fp16 inputs always takes
// the one-FMA exp form (shift_fma_ok): the kernels leave the other one out.
template <typename T>
constexpr bool kFarShiftFree = std::is_same<T, _Float16>::value;

// The lane's vectors of the row; those past the row's end hold -inf, which
// the row max ignores and exp maps to 0, so lane_max and lane_sum_exp need no
// mask.  (With a mask there, and 0 as the filler, the compiler kept a second,
// -inf filled copy of each loaded vector, and filling it waited for each load
// on the spot, one row load at a time.)
template <typename T, int V, int IT, bool NT>
__device__ __forceinline__ void load_raw_row(const T* __restrict__ xr, int nvec, int g, int tpr,
                                             typename Raw<T, V>::type (&dst)[IT],
                                             const Span& s) {
  typedef typename Raw<T, V>::type RT;
  const RT fill = RT(static_cast<T>(kNegInf));
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) dst[i] = load_raw<T, V, NT>(xr + static_cast<int64_t>(j) * V, s);
    else dst[i] = fill;
  }
}

// max over the lane's values (-inf when it holds none; NaN when one is NaN)
template <typename T, int V, int IT>
__device__ __forceinline__ float lane_max(const typename Raw<T, V>::type (&xr)[IT]) {
  float m[V];
#pragma unroll
  for (int k = 0; k < V; ++k) m[k] = kNegInf;
#pragma unroll
  for (int i = 0; i < IT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) m[k] = max_nan(m[k], raw_at<T, V>(xr[i], k));
  float r = m[0];
#pragma unroll
  for (int k = 1; k < V; ++k) r = max_nan(r, m[k]);
  return r;
}

// sum over the lane's values of exp(v - m), in the row's form `ex` (ExpFma or
// ExpSub; the -inf filler adds 0).  KEEP (fp32 rows only) leaves each
// exp(v - m) in place of v, for a softmax output pass that then only multiplies.
template <typename T, int V, int IT, bool KEEP = false, class Ex>
__device__ __forceinline__ float lane_sum_exp(typename Raw<T, V>::type (&xr)[IT], Ex ex) {
  static_assert(!KEEP || sizeof(T) == 4, "exp values are kept in fp32 registers only");
  float a[V];
#pragma unroll
  for (int k = 0; k < V; ++k) a[k] = 0.f;
#pragma unroll
  for (int i = 0; i < IT; ++i)
#pragma unroll
    for (int k = 0; k < V; ++k) {
      const float e = ex(raw_at<T, V>(xr[i], k));
      if constexpr (KEEP) {
        if constexpr (V == 1) xr[i] = e;
        else xr[i][k] = e;
      }
      a[k] += e;
    }
#pragma unroll
  for (int w = V / 2; w >= 1; w /= 2)
#pragma unroll
    for (int k = 0; k < w; ++k) a[k] += a[k + w];
  return a[0];
}

// Rows whose length is not a multiple of the vector width start at varying
// offsets within a 16-byte vector.  MIS kernels split such a row (element
// `start` of a 16-byte aligned buffer, `cols` long) into a head of up to V - 1
// elements before the first 16-byte boundary, a body of whole aligned vectors
// and a tail of up to V - 1 elements; lanes g < head and g < tail each hold one
// head / tail element as an extra scalar (the launcher makes tpr >= V).
// Nothing outside the row is read or written.
struct MisRow {
  int head, nvec, tail;
};

template <int V>
__device__ __forceinline__ MisRow mis_row(int64_t start, int cols) {
  int head = static_cast<int>((V - start % V) % V);
  if (head > cols) head = cols;
  const int nvec = (cols - head) / V;
  return MisRow{head, nvec, cols - head - nvec * V};
}

template <typename Ti, typename To, int V, int IT, bool LOG, int SP, bool MIS>
__global__ __launch_bounds__(kMaxBlock) void softmax_rows(const Ti* __restrict__ x,
                                                          To* __restrict__ y, int64_t rows,
                                                          int cols, int tpr) {
  typedef typename Raw<Ti, V>::type RT;
  __shared__ float lds[2][kMaxWaves];
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int rpb = gs.per_block;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * rpb;
  int64_t row = first + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const Span sx = VBH_SPAN(x, rows * cols), sy = VBH_SPAN(y, rows * cols);
  const int64_t start = row * cols;
  const MisRow mr = MIS ? mis_row<V>(start, cols) : MisRow{0, cols / V, 0};
  const int nvec = mr.nvec;
  const Ti* xb = x + start + mr.head;  // 16-byte aligned body

  RT xr[IT];
  load_raw_row<Ti, V, IT, SP != kStoreCached>(xb, nvec, g, tpr, xr, sx);
  const bool hv = MIS && g < mr.head, tv = MIS && g < mr.tail;
  float hx = 0.f, tx = 0.f;
  if (hv) load_f32<Ti, 1>(x + start + g, &hx, sx);
  if (tv) load_f32<Ti, 1>(xb + static_cast<int64_t>(nvec) * V + g, &tx, sx);
  float lm = lane_max<Ti, V, IT>(xr);
  if (hv) lm = max_nan(lm, hx);
  if (tv) lm = max_nan(lm, tx);
  const float m = group_allreduce<Max>(lm, tpr, lds[0]);
  reload_barrier<Ti, V, IT>(xr);
  // fp32 softmax keeps each exp(x - m) for the output pass
  constexpr bool KEEP = !LOG && sizeof(Ti) == 4;
  const bool fma_ok = kFarShiftFree<Ti> || shift_fma_ok(m);
  const float mb = m * kLog2e;
  const ExpFma efma{mb};
  const ExpSub esub{m};
  float le = fma_ok ? lane_sum_exp<Ti, V, IT, KEEP>(xr, efma)
                    : lane_sum_exp<Ti, V, IT, KEEP>(xr, esub);
  if (hv) le += fma_ok ? efma(hx) : esub(hx);
  if (tv) le += fma_ok ? efma(tx) : esub(tx);
  const float s = group_allreduce<Sum>(le, tpr, lds[1]);
  if (!live) return;
  reload_barrier<Ti, V, IT>(xr);

  const OutWindow<To, SP> out(y + first * cols, std::min<int64_t>(rpb, rows - first) * cols);
  To* yr = y + start + mr.head;
  const int yoff = static_cast<int>(row - first) * cols + mr.head;
  const float ls = LOG ? fast_log(s) - (fma_ok ? shift_residual(m, mb) : 0.f) * kLn2 : 0.f;
  const float r = LOG ? 0.f : __builtin_amdgcn_rcpf(s);  // v_rcp_f32, 1 ulp
  auto emit = [&](auto ex) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int j = i * tpr + g;
      if (j < nvec) {
        float o[V];
#pragma unroll
        for (int k = 0; k < V; ++k) {
          const float v = raw_at<Ti, V>(xr[i], k);
          if constexpr (LOG) o[k] = (v - m) - ls;
          else if constexpr (KEEP) o[k] = v * r;
          else o[k] = ex(v) * r;
        }
        out.template store<V>(yr + static_cast<int64_t>(j) * V, yoff + j * V, o, sy);
      }
    }
  };
  // only a 16-bit softmax recomputes its exps here
  if constexpr (LOG || KEEP) emit(efma);
  else if (fma_ok) emit(efma);
  else emit(esub);
  if (hv) {
    const float o = LOG ? (hx - m) - ls : (fma_ok ? efma(hx) : esub(hx)) * r;
    store_from_f32<To, 1>(y + start + g, &o, sy);
  }
  if (tv) {
    const float o = LOG ? (tx - m) - ls : (fma_ok ? efma(tx) : esub(tx)) * r;
    store_from_f32<To, 1>(yr + static_cast<int64_t>(nvec) * V + g, &o, sy);
  }
}

// `rows` units of `cols` columns.  MIS launches may instead split each row of
// `cols` columns into `segs` segments of `seg_cols` columns (the last one
// shorter): unit u is then segment u % segs of row u / segs, and y[u] its
// logsumexp.  PAIR (first stage of a split row; To is float): y[2u], y[2u+1]
// get the unit's SegPair -- its max and its sum of exp(x - max) -- instead.
template <typename Ti, typename To, int V, int IT, bool NT, bool MIS, bool PAIR = false>
__global__ __launch_bounds__(kMaxBlock) void logsumexp_rows(const Ti* __restrict__ x,
                                                            To* __restrict__ y, int64_t rows,
                                                            int cols, int tpr, int segs,
                                                            int seg_cols) {
  typedef typename Raw<Ti, V>::type RT;
  __shared__ float lds[2][kMaxWaves];
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  int64_t row = static_cast<int64_t>(blockIdx.x) * gs.per_block + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  // x holds rows / segs rows of `cols` in the MIS segment mode
  const Span sx = VBH_SPAN(x, (MIS && segs > 1 ? rows / segs : rows) * cols);
  const Span sy = VBH_SPAN(y, PAIR ? 2 * rows : rows);
  int64_t start = row * cols;
  int len = cols;
  if (MIS && segs > 1) {
    const int64_t r = row / segs;
    const int k = static_cast<int>(row - r * segs);
    start = r * cols + static_cast<int64_t>(k) * seg_cols;
    len = min(seg_cols, cols - k * seg_cols);
  }
  const MisRow mr = MIS ? mis_row<V>(start, len) : MisRow{0, cols / V, 0};
  const int nvec = mr.nvec;
  const Ti* xb = x + start + mr.head;

  RT xr[IT];
  load_raw_row<Ti, V, IT, NT>(xb, nvec, g, tpr, xr, sx);
  const bool hv = MIS && g < mr.head, tv = MIS && g < mr.tail;
  float hx = 0.f, tx = 0.f;
  if (hv) load_f32<Ti, 1>(x + start + g, &hx, sx);
  if (tv) load_f32<Ti, 1>(xb + static_cast<int64_t>(nvec) * V + g, &tx, sx);
  float lm = lane_max<Ti, V, IT>(xr);
  if (hv) lm = max_nan(lm, hx);
  if (tv) lm = max_nan(lm, tx);
  const float m_raw = group_allreduce<Max>(lm, tpr, lds[0]);
  reload_barrier<Ti, V, IT>(xr);
  const float m = __builtin_isinf(m_raw) ? 0.f : m_raw;
  const bool fma_ok = kFarShiftFree<Ti> || shift_fma_ok(m);
  const float mb = m * kLog2e;
  const ExpFma efma{mb};
  const ExpSub esub{m};
  float le = fma_ok ? lane_sum_exp<Ti, V, IT>(xr, efma) : lane_sum_exp<Ti, V, IT>(xr, esub);
  if (hv) le += fma_ok ? efma(hx) : esub(hx);
  if (tv) le += fma_ok ? efma(tx) : esub(tx);
  const float s = group_allreduce<Sum>(le, tpr, lds[1]);
  if (live && g == 0) {
    if constexpr (PAIR) {
      // the sum relative to m itself (2^residual taken back out); an all -inf
      // segment sums to 0
      const float t = m_raw == kNegInf
                          ? 0.f
                          : (fma_ok ? s * __builtin_amdgcn_exp2f(-shift_residual(m, mb)) : s);
      const float pair[2] = {m_raw, t};
      store_from_f32<float, 2>(reinterpret_cast<float*>(y) + 2 * row, pair, sy);
    } else {
      const float r = (fast_log(s) - (fma_ok ? shift_residual(m, mb) : 0.f) * kLn2) + m;
      store_from_f32<To, 1>(y + row, &r, sy);
    }
  }
}

// Second stage of a split logsumexp: one wave per row, lane k holding the
// row's segment k (segs <= 64), merges the row's `segs` SegPairs
// (pairs[2 * (row * segs + k)]) under torch's rules (NaN anywhere: NaN; a +inf
// max: +inf; all -inf: -inf).
constexpr int kCombineRowsPerBlock = 4;  // waves of a 256-lane workgroup

template <typename To>
__global__ __launch_bounds__(256) void logsumexp_pairs_combine(const float* __restrict__ pairs,
                                                               To* __restrict__ y, int64_t rows,
                                                               int segs) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kCombineRowsPerBlock +
                      static_cast<int>(threadIdx.x >> 6);
  if (row >= rows) return;  // a whole wave
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const Span sp = VBH_SPAN(pairs, 2 * rows * segs), sy = VBH_SPAN(y, rows);
  const bool has = lane < segs;
  float mt[2] = {0.f, 0.f};
  if (has) load_f32<float, 2>(pairs + 2 * (row * segs + lane), mt, sp);
  const RowPairs rp = wave_combine_seg_pairs(has, mt[0], mt[1]);
  if (lane != 0) return;
  float r;
  if (rp.nan) r = __builtin_nanf("");
  else if (__builtin_isinf(rp.m)) r = rp.m;
  else r = fast_log(rp.s) + rp.m;
  store_from_f32<To, 1>(y + row, &r, sy);
}

// ---------------------------------------------------------------------------
// second stage of a split softmax / log_softmax (rows of whole vectors)
//
// The first stage writes the SegPair (max m_k, sum t_k of exp(x - m_k)) of
// each of a row's `segs` segments (logsumexp_rows<PAIR> over the
// [rows * segs, cols / segs] view).  Here one kApplyLanes-lane workgroup owns
// one tile of kApplyLanes vectors of a row, one 16-byte vector per lane (the
// copy kernel's shape).  Every wave combines the row's pairs itself
// (segs <= 64: one per lane): M = max m_k, the row max, and
// S = sum t_k exp(m_k - M), and writes (x - M) - log S or its exp.  (A
// logsumexp per segment would not do: where |M| is large, m_k + log t_k rounds
// the log away.)  A row with a NaN, a +inf element or only -inf elements is all
// NaN, as torch's softmax / log_softmax give.
// MIS rows (not whole vectors; the first stage ran the MIS segment mode): the
// tiles cover each row's aligned body, and tile 0 also writes the row's scalar
// head and tail (lanes t < head, t < tail).
// ---------------------------------------------------------------------------

template <typename Ti, typename To, int V, bool LOG, int SP, bool MIS>
__global__ __launch_bounds__(kApplyLanes) void softmax_apply_tiles(
    const Ti* __restrict__ x, To* __restrict__ y, const float* __restrict__ seg_pairs, int cols,
    int segs, uint32_t tiles_per_row) {
  const uint32_t row32 = blockIdx.x / tiles_per_row;
  const int tix = static_cast<int>(blockIdx.x - row32 * tiles_per_row);
  const int64_t row = row32;
  // the grid is the row count times tiles_per_row
  const Span sx = VBH_SPAN(x, static_cast<int64_t>(gridDim.x / tiles_per_row) * cols);
  const Span sy = VBH_SPAN(y, static_cast<int64_t>(gridDim.x / tiles_per_row) * cols);
  const Span sl =
      VBH_SPAN(seg_pairs, static_cast<int64_t>(gridDim.x / tiles_per_row) * segs * 2);
  const int64_t start = row * cols;
  const MisRow mr = MIS ? mis_row<V>(start, cols) : MisRow{0, cols / V, 0};
  const int nvec = mr.nvec;
  const Ti* xb = x + start + mr.head;  // 16-byte aligned body
  const int j0 = tix * kApplyLanes;
  const int j = j0 + static_cast<int>(threadIdx.x);
  typename Raw<Ti, V>::type r{};
  if (j < nvec) r = load_raw<Ti, V, SP != kStoreCached>(xb + static_cast<int64_t>(j) * V, sx);

  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const bool has = lane < segs;
  float mt[2] = {kNegInf, 0.f};
  if (has) load_f32<float, 2>(seg_pairs + 2 * (row * segs + lane), mt, sl);
  const float m = wave_allreduce<Max>(mt[0], kWave);
  const float nan = wave_allreduce<Max>(mt[0] != mt[0] || mt[1] != mt[1] ? 1.f : 0.f, kWave);
  const bool bad = nan > 0.f || __builtin_isinf(m);
  const float sum = wave_allreduce<Sum>(
      has && !bad && mt[0] != kNegInf ? mt[1] * fast_exp(mt[0] - m) : 0.f, kWave);
  const float ls = fast_log(sum);

  auto value = [&](float v) {
    const float d = (v - m) - ls;
    return bad ? __builtin_nanf("") : (LOG ? d : fast_exp(d));
  };
  const int tile = nvec - j0 < kApplyLanes ? nvec - j0 : kApplyLanes;  // <= 0: no body here
  To* yb = y + start + mr.head;
  const OutWindow<To, SP> out(yb + static_cast<int64_t>(j0) * V,
                              static_cast<int64_t>(tile > 0 ? tile : 0) * V);
  if (j < nvec) {
    float o[V];
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = value(raw_at<Ti, V>(r, k));
    out.template store<V>(yb + static_cast<int64_t>(j) * V, static_cast<int>(threadIdx.x) * V, o,
                          sy);
  }
  if (MIS && tix == 0) {
    const int t = static_cast<int>(threadIdx.x);
    if (t < mr.head) {
      float v;
      load_f32<Ti, 1>(x + start + t, &v, sx);
      const float o = value(v);
      store_from_f32<To, 1>(y + start + t, &o, sy);
    }
    if (t < mr.tail) {
      const int64_t k = static_cast<int64_t>(nvec) * V + t;
      float v;
      load_f32<Ti, 1>(xb + k, &v, sx);
      const float o = value(v);
      store_from_f32<To, 1>(yb + k, &o, sy);
    }
  }
}

// ---------------------------------------------------------------------------
// streaming (one workgroup per row)
// ---------------------------------------------------------------------------

// Online row statistics for the streaming path: running max `m` (NaN ignored),
// sum `s` of exp(x - m) rescaled whenever m grows, and a NaN flag.  The final
// outputs reproduce torch's special values explicitly:
//   softmax / log_softmax: a row holding NaN or +inf, or only -inf, is all NaN;
//   logsumexp: NaN row -> NaN, a +inf max -> +inf, an all -inf row -> -inf.
struct RowStats {
  float m, s, nan;
};

template <typename T, int V>
__device__ __forceinline__ RowStats stream_stats(const T* __restrict__ xr, int nvec,
                                                 float* lds, const Span& sx) {
  float m = kNegInf, s = 0.f, nan = 0.f;
  for (int j = threadIdx.x; j < nvec; j += blockDim.x) {
    float v[V];
    load_f32<T, V>(xr + static_cast<int64_t>(j) * V, v, sx);
    float cm = kNegInf;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      cm = fmaxf(cm, v[k]);
      if (v[k] != v[k]) nan = 1.f;
    }
    if (cm > m) {
      s = (m == kNegInf) ? 0.f : s * fast_exp(m - cm);
      m = cm;
    }
    if (m != kNegInf && m != -kNegInf) {
#pragma unroll
      for (int k = 0; k < V; ++k) s += (v[k] != v[k]) ? 0.f : fast_exp(v[k] - m);
    }
  }
  const int tpr = blockDim.x;
  const float gm = group_allreduce<Max>(m, tpr, lds);
  const bool finite = gm != kNegInf && gm != -kNegInf;
  const float t = (finite && m != kNegInf) ? s * fast_exp(m - gm) : 0.f;
  const float gs = group_allreduce<Sum>(t, tpr, lds + kMaxWaves);
  const float gn = group_allreduce<Max>(nan, tpr, lds + 2 * kMaxWaves);
  return RowStats{gm, gs, gn};
}

template <typename Ti, typename To, int V, bool LOG>
__global__ __launch_bounds__(kMaxBlock) void softmax_stream(const Ti* __restrict__ x,
                                                            To* __restrict__ y, int cols) {
  __shared__ float lds[3 * kMaxWaves];
  const int nvec = cols / V;
  const int64_t row = blockIdx.x;
  const Ti* xr = x + row * cols;
  // one workgroup per row: the grid is the row count
  const Span sx = VBH_SPAN(x, static_cast<int64_t>(gridDim.x) * cols);
  const Span sy = VBH_SPAN(y, static_cast<int64_t>(gridDim.x) * cols);
  const RowStats st = stream_stats<Ti, V>(xr, nvec, lds, sx);
  const bool special = st.nan != 0.f || st.m == kNegInf || st.m == -kNegInf;
  const float qnan = __builtin_nanf("");
  const float m = st.m;
  To* yr = y + row * cols;
  if constexpr (LOG) {
    const float ls = special ? qnan : fast_log(st.s);
    for (int j = threadIdx.x; j < nvec; j += blockDim.x) {
      float v[V], o[V];
      load_f32<Ti, V>(xr + static_cast<int64_t>(j) * V, v, sx);
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = (v[k] - m) - ls;
      store_from_f32<To, V>(yr + static_cast<int64_t>(j) * V, o, sy);
    }
  } else {
    const float r = special ? qnan : 1.0f / st.s;
    for (int j = threadIdx.x; j < nvec; j += blockDim.x) {
      float v[V], o[V];
      load_f32<Ti, V>(xr + static_cast<int64_t>(j) * V, v, sx);
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = fast_exp(v[k] - m) * r;
      store_from_f32<To, V>(yr + static_cast<int64_t>(j) * V, o, sy);
    }
  }
}

// PAIR: as logsumexp_rows<PAIR>, the row's SegPair into y[2 row], y[2 row + 1].
template <typename Ti, typename To, int V, bool PAIR = false>
__global__ __launch_bounds__(kMaxBlock) void logsumexp_stream(const Ti* __restrict__ x,
                                                              To* __restrict__ y, int cols) {
  __shared__ float lds[3 * kMaxWaves];
  const int nvec = cols / V;
  const int64_t row = blockIdx.x;
  // one workgroup per row: the grid is the row count
  const Span sx = VBH_SPAN(x, static_cast<int64_t>(gridDim.x) * cols);
  const Span sy = VBH_SPAN(y, static_cast<int64_t>(gridDim.x) * (PAIR ? 2 : 1));
  const RowStats st = stream_stats<Ti, V>(x + row * cols, nvec, lds, sx);
  if (threadIdx.x == 0) {
    const bool inf = st.m == kNegInf || st.m == -kNegInf;
    if constexpr (PAIR) {
      const float pair[2] = {st.nan != 0.f ? __builtin_nanf("") : st.m, inf ? 0.f : st.s};
      store_from_f32<float, 2>(reinterpret_cast<float*>(y) + 2 * row, pair, sy);
    } else {
      float r;
      if (st.nan != 0.f) r = __builtin_nanf("");
      else if (inf) r = st.m;
      else r = fast_log(st.s) + st.m;
      store_from_f32<To, 1>(y + row, &r, sy);
    }
  }
}

// ---------------------------------------------------------------------------
// middle axis: [outer, n, inner], reduce over n
// ---------------------------------------------------------------------------
template <typename Ti, typename To, bool LOG>
__global__ __launch_bounds__(256) void softmax_mid(const Ti* __restrict__ x,
                                                   To* __restrict__ y, int64_t outer, int n,
                                                   int64_t inner) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (col >= outer * inner) return;
  const int64_t o = col / inner;
  const int64_t i = col - o * inner;
  const Ti* xc = x + o * n * inner + i;
  To* yc = y + o * n * inner + i;
  const Span sx = VBH_SPAN(x, outer * n * inner), sy = VBH_SPAN(y, outer * n * inner);
  auto xat = [&](int r) {
    const Ti* p = xc + r * inner;
    return VBH_IN_SPAN(sx, p, sizeof(Ti)) ? static_cast<float>(*p) : 0.f;
  };
  float m = kNegInf;
  for (int r = 0; r < n; ++r) m = fmaxf(m, xat(r));
  float s = 0.f;
  for (int r = 0; r < n; ++r) s += fast_exp(xat(r) - m);
  if constexpr (LOG) {
    const float ls = fast_log(s);
    for (int r = 0; r < n; ++r) {
      const float out = (xat(r) - m) - ls;
      store_from_f32<To, 1>(yc + r * inner, &out, sy);
    }
  } else {
    const float rs = 1.0f / s;
    for (int r = 0; r < n; ++r) {
      const float out = fast_exp(xat(r) - m) * rs;
      store_from_f32<To, 1>(yc + r * inner, &out, sy);
    }
  }
}

// (in, out) dtype pairs: same type, or fp16/bf16 in with fp32 out
template <typename Fn>
bool dispatch_in_out(int idt, int odt, Fn&& fn) {
  if (idt == odt) {
    return dispatch_float_type(idt, [&](auto t) { fn(t, t); });
  }
  if (odt == kF32 && (idt == kF16 || idt == kBF16)) {
    return dispatch_float_type(idt, [&](auto t) { fn(t, TypeTag<float>{}); });
  }
  return false;
}

}  // namespace

hipError_t launch_softmax(const void* x, void* y, int64_t rows, int cols, int idt, int odt,
                          int log_mode, const Geometry& g, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_in_out(idt, odt, [&](auto ti, auto to) {
    using Ti = typename decltype(ti)::type;
    using To = typename decltype(to)::type;
    constexpr int VN = Vec<Ti>::n;
    auto go = [&](auto vc, auto lc) {
      constexpr int V = decltype(vc)::value;
      constexpr bool LOG = decltype(lc)::value;
      if (g.stream) {
        launch_kernel((softmax_stream<Ti, To, V, LOG>), dim3(rows), dim3(g.block), 0, s,
                           static_cast<const Ti*>(x), static_cast<To*>(y), cols);
        err = hipGetLastError();
        return;
      }
      dispatch_maxit(g.maxit, [&](auto mc) {
        constexpr int M = decltype(mc)::value;
        if constexpr (M <= lane_cap(V)) {
          dispatch_store_policy<V>(g, [&](auto sp) {
            constexpr int SP = decltype(sp)::value;
            if (V > 1 && g.mis)
              launch_kernel((softmax_rows<Ti, To, V, M, LOG, SP, V != 1>),
                                 dim3(grid_for(rows, g)), dim3(g.block), 0, s,
                                 static_cast<const Ti*>(x), static_cast<To*>(y), rows, cols,
                                 g.tpr);
            else
              launch_kernel((softmax_rows<Ti, To, V, M, LOG, SP, false>),
                                 dim3(grid_for(rows, g)), dim3(g.block), 0, s,
                                 static_cast<const Ti*>(x), static_cast<To*>(y), rows, cols,
                                 g.tpr);
          });
          err = hipGetLastError();
        }
      });
    };
    auto with_log = [&](auto vc) {
      if (log_mode) go(vc, std::true_type{});
      else go(vc, std::false_type{});
    };
    if (g.v == 1) with_log(std::integral_constant<int, 1>{});
    else with_log(std::integral_constant<int, VN>{});
  });
  return err;
}

namespace {

// logsumexp_rows / logsumexp_stream over `rows` units (PAIR: their SegPairs,
// fp32, into y)
template <bool PAIR, class Ti, class To>
hipError_t launch_logsumexp_units(const void* x, void* y, int64_t rows, int cols,
                                  const Geometry& g, hipStream_t s, int segs, int seg_cols) {
  hipError_t err = hipErrorInvalidValue;
  constexpr int VN = Vec<Ti>::n;
  auto go = [&](auto vc) {
    constexpr int V = decltype(vc)::value;
    if (g.stream) {
      launch_kernel((logsumexp_stream<Ti, To, V, PAIR>), dim3(rows), dim3(g.block), 0, s,
                    static_cast<const Ti*>(x), static_cast<To*>(y), cols);
      err = hipGetLastError();
      return;
    }
    dispatch_maxit(g.maxit, [&](auto mc) {
      constexpr int M = decltype(mc)::value;
      if constexpr (M <= lane_cap(V)) {
        auto launch = [&](auto kern) {
          launch_kernel(kern, dim3(grid_for(rows, g)), dim3(g.block), 0, s,
                        static_cast<const Ti*>(x), static_cast<To*>(y), rows, cols, g.tpr, segs,
                        seg_cols);
        };
        if (V > 1 && g.mis) launch(logsumexp_rows<Ti, To, V, M, true, V != 1, PAIR>);
        else if (g.nt) launch(logsumexp_rows<Ti, To, V, M, true, false, PAIR>);
        else launch(logsumexp_rows<Ti, To, V, M, false, false, PAIR>);
        err = hipGetLastError();
      }
    });
  };
  if (g.v == 1) go(std::integral_constant<int, 1>{});
  else go(std::integral_constant<int, VN>{});
  return err;
}

}  // namespace

hipError_t launch_logsumexp(const void* x, void* y, int64_t rows, int cols, int idt, int odt,
                            const Geometry& g, hipStream_t s, int segs, int seg_cols) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_in_out(idt, odt, [&](auto ti, auto to) {
    using Ti = typename decltype(ti)::type;
    using To = typename decltype(to)::type;
    err = launch_logsumexp_units<false, Ti, To>(x, y, rows, cols, g, s, segs, seg_cols);
  });
  return err;
}

hipError_t launch_logsumexp_pairs(const void* x, float* pairs, int64_t units, int cols, int idt,
                                  const Geometry& g, hipStream_t s, int segs, int seg_cols) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_float_type(idt, [&](auto ti) {
    using Ti = typename decltype(ti)::type;
    err = launch_logsumexp_units<true, Ti, float>(x, pairs, units, cols, g, s, segs, seg_cols);
  });
  return err;
}

hipError_t launch_logsumexp_combine(const float* pairs, void* y, int64_t rows, int segs,
                                    int odt, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  dispatch_float_type(odt, [&](auto to) {
    using To = typename decltype(to)::type;
    launch_kernel(logsumexp_pairs_combine<To>,
                  dim3((rows + kCombineRowsPerBlock - 1) / kCombineRowsPerBlock),
                  dim3(kCombineRowsPerBlock * kWave), 0, s, pairs, static_cast<To*>(y), rows,
                  segs);
    err = hipGetLastError();
  });
  return err;
}

hipError_t launch_softmax_apply(const void* x, void* y, const float* seg_pairs, int64_t rows,
                                int cols, int segs, int idt, int odt, int log_mode,
                                const Geometry& g, hipStream_t s) {
  // MIS rows: the tiles cover at most cols / V body vectors per row
  hipError_t err = hipErrorInvalidValue;
  dispatch_in_out(idt, odt, [&](auto ti, auto to) {
    using Ti = typename decltype(ti)::type;
    using To = typename decltype(to)::type;
    constexpr int V = Vec<Ti>::n;
    const int64_t tiles = (cols / V + kApplyLanes - 1) / kApplyLanes;
    dispatch_store_policy<V>(g, [&](auto sp) {
      constexpr int SP = decltype(sp)::value;
      auto launch = [&](auto kern) {
        launch_kernel(kern, dim3(rows * tiles), dim3(kApplyLanes), 0, s,
                           static_cast<const Ti*>(x), static_cast<To*>(y), seg_pairs, cols, segs,
                           static_cast<uint32_t>(tiles));
      };
      if (g.mis) {
        if (log_mode) launch(softmax_apply_tiles<Ti, To, V, true, SP, true>);
        else launch(softmax_apply_tiles<Ti, To, V, false, SP, true>);
      } else {
        if (log_mode) launch(softmax_apply_tiles<Ti, To, V, true, SP, false>);
        else launch(softmax_apply_tiles<Ti, To, V, false, SP, false>);
      }
    });
    err = hipGetLastError();
  });
  return err;
}

hipError_t launch_softmax_dim(const void* x, void* y, int64_t outer, int n, int64_t inner,
                              int idt, int odt, int log_mode, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  const int64_t cols = outer * inner;
  const int block = 256;
  const int64_t grid = (cols + block - 1) / block;
  dispatch_in_out(idt, odt, [&](auto ti, auto to) {
    using Ti = typename decltype(ti)::type;
    using To = typename decltype(to)::type;
    if (log_mode)
      launch_kernel((softmax_mid<Ti, To, true>), dim3(grid), dim3(block), 0, s,
                         static_cast<const Ti*>(x), static_cast<To*>(y), outer, n, inner);
    else
      launch_kernel((softmax_mid<Ti, To, false>), dim3(grid), dim3(block), 0, s,
                         static_cast<const Ti*>(x), static_cast<To*>(y), outer, n, inner);
    err = hipGetLastError();
  });
  return err;
}

}  // namespace vbh

// Mean, max (value + index) and argmax over one axis, for gfx950.
//
// The tensor is viewed as contiguous [outer, n, inner] and reduced over n.
//   inner == 1 (last axis): `tpr` lanes own one row and stream it with 16-byte
//   loads (nothing per element is written, so the row is never held in
//   registers and any n works), then all-reduce across the group.
//   inner > 1: one lane per (outer, inner) column loops over n; consecutive
//   lanes read consecutive inner indices, so every access is coalesced.
// Each input element is read once; one value (and/or index) per output is
// written.
//
// Semantics (torch): mean accumulates in fp32 and divides by n
// (ViperBench/mean_reduction/pytorch_impl.py:4-8); max returns (values, int64
// indices) (ViperBench/max_reduction/pytorch_impl.py:4-11); argmax returns
// int64 indices (ViperBench/argmax/pytorch_impl.py:4-8).  NaN counts as the
// largest value and ties resolve to the smallest index, so the first maximal
// (or first NaN) position is returned.
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// true when (av, ai) should win over (bv, bi): a total order, so every lane of
// a butterfly picks the same pair.
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

struct ValIdx {
  float v;
  int i;
};

__device__ __forceinline__ ValIdx pick(ValIdx a, ValIdx b) {
  return better(a.v, a.i, b.v, b.i) ? a : b;
}

template <int Ctrl>
__device__ __forceinline__ ValIdx dpp_vi(ValIdx a) {
  return ValIdx{dpp<Ctrl>(a.v),
                __builtin_amdgcn_update_dpp(0, a.i, Ctrl, 0xF, 0xF, false)};
}

__device__ __forceinline__ int swap16_partner_i(int v) {
  auto p = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(v), static_cast<unsigned>(v),
                                            false, false);
  return static_cast<int>((threadIdx.x & 16) ? p[0] : p[1]);
}
__device__ __forceinline__ int swap32_partner_i(int v) {
  auto p = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(v), static_cast<unsigned>(v),
                                            false, false);
  return static_cast<int>((threadIdx.x & 32) ? p[0] : p[1]);
}

// All-reduce of (value, index) pairs over the tpr lanes of one row (see
// group_allreduce for the lane layout and the LDS contract; `lds` holds
// 2 * kMaxWaves words).
__device__ __forceinline__ ValIdx group_allreduce_vi(ValIdx a, int tpr, float* lds) {
  const int width = tpr < kWave ? tpr : kWave;
  if (width >= 2) a = pick(a, dpp_vi<0xB1>(a));
  if (width >= 4) a = pick(a, dpp_vi<0x4E>(a));
  if (width >= 8) a = pick(a, dpp_vi<0x141>(a));
  if (width >= 16) a = pick(a, dpp_vi<0x140>(a));
  if (width >= 32) a = pick(a, ValIdx{swap16_partner(a.v), swap16_partner_i(a.i)});
  if (width >= 64) a = pick(a, ValIdx{swap32_partner(a.v), swap32_partner_i(a.i)});
  if (tpr <= kWave) return a;
  const int wave = threadIdx.x / kWave;
  const int nwaves = tpr / kWave;
  const int first = (wave / nwaves) * nwaves;
  int* ldsi = reinterpret_cast<int*>(lds + kMaxWaves);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    lds[wave] = a.v;
    ldsi[wave] = a.i;
  }
  __syncthreads();
  ValIdx r{lds[first], ldsi[first]};
  for (int w = first + 1; w < first + nwaves; ++w) r = pick(r, ValIdx{lds[w], ldsi[w]});
  return r;
}

// IEEE maximum of a 16-byte vector's values: NaN if one of them is NaN
// (fp16 pairs go to v_pk_maximum3_f16, fp32 values to v_maximum3_f32).
template <typename T, int V>
__device__ __forceinline__ float vec_max_nan(const typename Raw<T, V>::type& r) {
  float m = raw_at<T, V>(r, 0);
#pragma unroll
  for (int k = 1; k < V; ++k) m = max_nan(m, raw_at<T, V>(r, k));
  return m;
}

// The first element of `r` equal to `m` (the vector's maximum, so one
// exists), or its first NaN when `m` is NaN: (its value, its position in `r`).
// A NaN comes back as the canonical quiet NaN.
template <typename T, int V>
__device__ __forceinline__ ValIdx first_max_at(const typename Raw<T, V>::type& r, float m) {
  const bool nan = m != m;
  ValIdx f{m, V - 1};
#pragma unroll
  for (int k = V - 1; k >= 0; --k) {
    const float v = raw_at<T, V>(r, k);
    if (nan ? v != v : v == m) f = ValIdx{v, k};
  }
  if (nan) f.v = __builtin_nanf("");
  return f;
}

// An element as a (value, position) candidate, a NaN as the canonical one.
__device__ __forceinline__ ValIdx candidate(float v, int i) {
  return ValIdx{v != v ? __builtin_nanf("") : v, i};
}

template <typename T, int V, int OP>
__device__ __forceinline__ void write_result(void* vals, int64_t* idx, int64_t o, float sum_or_v,
                                             int i, int n, const Span& sv, const Span& si) {
  if constexpr (OP == 0) {
    const float m = sum_or_v / static_cast<float>(n);
    store_from_f32<T, 1>(static_cast<T*>(vals) + o, &m, sv);
  } else {
    if constexpr (OP == 1) store_from_f32<T, 1>(static_cast<T*>(vals) + o, &sum_or_v, sv);
    if (VBH_IN_SPAN(si, idx + o, sizeof(int64_t))) idx[o] = i;
  }
}

// OP: 0 = mean (To = output type), 1 = max values + indices, 2 = argmax.
// MIS: rows not a multiple of V long start at varying offsets within a
// 16-byte vector; each row is read as a scalar head up to the first 16-byte
// boundary (lanes g < head, element g), whole aligned vectors, and a scalar
// tail (lanes g < tail); the launcher makes tpr >= V.  A lane visits its head
// element first and its tail element last, so its positions still increase.
template <typename Ti, typename To, int V, int OP, bool MIS>
__global__ __launch_bounds__(kMaxBlock) void reduce_rows(const Ti* __restrict__ x,
                                                         void* __restrict__ vals,
                                                         int64_t* __restrict__ idx,
                                                         int64_t rows, int n, int tpr) {
  __shared__ float lds[2 * kMaxWaves];
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  int64_t row = static_cast<int64_t>(blockIdx.x) * gs.per_block + gs.sub;
  const bool live = row < rows;
  if (!live) row = rows - 1;
  const Span sx = VBH_SPAN(x, rows * n);
  const Span sv = VBH_SPAN(static_cast<To*>(vals), rows), si = VBH_SPAN(idx, rows);
  const int64_t start = row * n;
  int head = 0, nvec = n / V, tail = 0;
  if constexpr (MIS) {
    head = static_cast<int>((V - start % V) % V);
    if (head > n) head = n;
    nvec = (n - head) / V;
    tail = n - head - nvec * V;
  }
  const Ti* xr = x + start + head;  // 16-byte aligned body; element j * V + k is head + j * V + k
  const bool hv = MIS && g < head, tv = MIS && g < tail;
  const int tail0 = head + nvec * V;  // row index of the first tail element
  typedef typename Raw<Ti, V>::type RT;
  // Each lane loads kChunk vectors (kChunk * tpr apart... j, j + tpr, ...) before
  // processing any of them, so a chunk's loads are in flight together whatever
  // the data-dependent branches below do.
  constexpr int kChunk = 4;
  if constexpr (OP == 0) {
    float acc[V];
#pragma unroll
    for (int k = 0; k < V; ++k) acc[k] = 0.f;
    for (int base = g; base < nvec; base += kChunk * tpr) {
      RT r[kChunk];
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int j = base + c * tpr;
        r[c] = j < nvec ? load_raw<Ti, V, true>(xr + static_cast<int64_t>(j) * V, sx) : RT{};
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c)
#pragma unroll
        for (int k = 0; k < V; ++k) acc[k] += raw_at<Ti, V>(r[c], k);  // padding is zero
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < V; ++k) s += acc[k];
    if (hv) {
      float v;
      load_f32<Ti, 1>(x + start + g, &v, sx);
      s += v;
    }
    if (tv) {
      float v;
      load_f32<Ti, 1>(x + start + tail0 + g, &v, sx);
      s += v;
    }
    s = group_allreduce<Sum>(s, tpr, lds);
    if (live && g == 0) write_result<To, V, OP>(vals, idx, row, s, 0, n, sv, si);
  } else {
    ValIdx best;
    if (nvec >= kChunk * tpr) {  // uniform: every lane holds a chunk of vectors or more
      // The lane's vectors are visited in increasing position order.  Per vector
      // only its IEEE maximum (NaN if it holds one) is formed and compared with
      // the lane's best; the winning vector is kept raw, and the position of its
      // first maximal (or first NaN) element is looked up once, after the loop.
      // A later vector wins only with a strictly larger maximum, or with the
      // first NaN, so the lane's result is its first maximal position.
      float bv = kNegInf;  // best vector's maximum
      int bj = -1;         // its vector index (-1: none yet)
      RT braw = RT{};
      for (int base = g; base < nvec; base += kChunk * tpr) {
        RT r[kChunk];
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int j = base + c * tpr;
          r[c] = j < nvec ? load_raw<Ti, V, true>(xr + static_cast<int64_t>(j) * V, sx) : RT{};
        }
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int j = base + c * tpr;
          if (j >= nvec) break;  // the lane's later vectors are past the row too
          const float m = vec_max_nan<Ti, V>(r[c]);
          const bool win = bj < 0 || m > bv || (m != m && bv == bv);
          bv = win ? m : bv;
          bj = win ? j : bj;
          braw = win ? r[c] : braw;
        }
      }
      best = ValIdx{kNegInf, n};  // an empty lane loses to any element
      if (bj >= 0) {
        const ValIdx f = first_max_at<Ti, V>(braw, bv);
        best = ValIdx{f.v, head + bj * V + f.i};
      }
      // the head element precedes every body position and the tail element
      // follows them; pick() orders by value (NaN largest), then position
      if (hv) {
        float v;
        load_f32<Ti, 1>(x + start + g, &v, sx);
        best = pick(candidate(v, g), best);
      }
      if (tv) {
        float v;
        load_f32<Ti, 1>(x + start + tail0 + g, &v, sx);
        best = pick(best, candidate(v, tail0 + g));
      }
    } else {
      // Short rows (fewer than kChunk vectors per lane), visited in
      // increasing position order: head element, body vectors, tail element.
      // Per vector an fmax tree and a NaN test; the index search runs where
      // the vector beats the lane's best (a later value only wins when it is
      // strictly larger, or the first NaN).  With one or two vectors per lane
      // this is 3-8% faster than the search after the loop (fp16, 64, 100 and
      // 255 columns).
      best = ValIdx{kNegInf, n};  // an empty lane loses to any element
      bool done = false;        // a NaN was found: nothing later can win
      if (hv) {
        float v;
        load_f32<Ti, 1>(x + start + g, &v, sx);
        if (v != v) {
          best = ValIdx{__builtin_nanf(""), g};
          done = true;
        } else {
          best = ValIdx{v, g};
        }
      }
      for (int base = g; base < nvec; base += kChunk * tpr) {
        RT r[kChunk];
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int j = base + c * tpr;
          r[c] = j < nvec ? load_raw<Ti, V, true>(xr + static_cast<int64_t>(j) * V, sx) : RT{};
        }
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int j = base + c * tpr;
          if (done || j >= nvec) continue;
          float v[V];
#pragma unroll
          for (int k = 0; k < V; ++k) v[k] = raw_at<Ti, V>(r[c], k);
          float m = v[0];
          bool nan = v[0] != v[0];
#pragma unroll
          for (int k = 1; k < V; ++k) {
            m = fmaxf(m, v[k]);
            nan |= v[k] != v[k];
          }
          if (nan) {  // first NaN of the vector (unrolled selects, no indexed registers)
            int kk = V - 1;
#pragma unroll
            for (int k = V - 1; k >= 0; --k)
              if (v[k] != v[k]) kk = k;
            best = ValIdx{__builtin_nanf(""), head + j * V + kk};
            done = true;
          } else if (m > best.v || best.i == n) {  // first position of the vector max
            int kk = V - 1;
#pragma unroll
            for (int k = V - 1; k >= 0; --k)
              if (v[k] == m) kk = k;
            best = ValIdx{m, head + j * V + kk};
          }
        }
      }
      if (tv && !done) {
        float v;
        load_f32<Ti, 1>(x + start + tail0 + g, &v, sx);
        if (v != v) best = ValIdx{__builtin_nanf(""), tail0 + g};
        else if (v > best.v || best.i == n) best = ValIdx{v, tail0 + g};
      }
    }
    best = group_allreduce_vi(best, tpr, lds);
    if (live && g == 0) write_result<To, V, OP>(vals, idx, row, best.v, best.i, n, sv, si);
  }
}

// Second stage of a row reduction split into `segs` segments of `segn`
// elements (max / argmax): one lane per row picks the winner of the segments'
// (value, index) results, which the first stage wrote as values of type T and
// int64 segment-local indices, under the same order as the row kernel (NaN
// largest, then the smaller global index).
template <typename T, int OP>
__global__ __launch_bounds__(256) void reduce_combine_vi(const T* __restrict__ pvals,
                                                         const int64_t* __restrict__ pidx,
                                                         void* __restrict__ vals,
                                                         int64_t* __restrict__ idx, int64_t rows,
                                                         int segs, int segn) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int64_t base = row * segs;
  const Span spv = VBH_SPAN(pvals, rows * segs), spi = VBH_SPAN(pidx, rows * segs);
  const Span sv = VBH_SPAN(static_cast<T*>(vals), rows), si = VBH_SPAN(idx, rows);
  ValIdx best{VBH_IN_SPAN(spv, pvals + base, sizeof(T)) ? static_cast<float>(pvals[base]) : 0.f,
              VBH_IN_SPAN(spi, pidx + base, sizeof(int64_t)) ? static_cast<int>(pidx[base]) : 0};
  for (int s = 1; s < segs; ++s) {
    const ValIdx c{
        VBH_IN_SPAN(spv, pvals + base + s, sizeof(T)) ? static_cast<float>(pvals[base + s]) : 0.f,
        s * segn + (VBH_IN_SPAN(spi, pidx + base + s, sizeof(int64_t))
                        ? static_cast<int>(pidx[base + s])
                        : 0)};
    best = pick(best, c);
  }
  if constexpr (OP == 1) store_from_f32<T, 1>(static_cast<T*>(vals) + row, &best.v, sv);
  if (VBH_IN_SPAN(si, idx + row, sizeof(int64_t))) idx[row] = best.i;
}

template <typename Ti, typename To, int OP>
__global__ __launch_bounds__(256) void reduce_cols(const Ti* __restrict__ x,
                                                   void* __restrict__ vals,
                                                   int64_t* __restrict__ idx, int64_t outer,
                                                   int n, int64_t inner) {
  const int64_t col = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (col >= outer * inner) return;
  const int64_t o = col / inner;
  const int64_t c = col - o * inner;
  const Ti* xc = x + o * n * inner + c;
  const Span sx = VBH_SPAN(x, outer * n * inner);
  const Span sv = VBH_SPAN(static_cast<To*>(vals), outer * inner), si = VBH_SPAN(idx, outer * inner);
  auto xat = [&](int r) {
    float v;
    load_f32<Ti, 1>(xc + r * inner, &v, sx);
    return v;
  };
  if constexpr (OP == 0) {
    float s = 0.f;
    for (int r = 0; r < n; ++r) s += xat(r);
    write_result<To, 1, OP>(vals, idx, col, s, 0, n, sv, si);
  } else {
    ValIdx best{kNegInf, n};
    for (int r = 0; r < n; ++r) {
      const float v = xat(r);
      if (better(v, r, best.v, best.i)) best = ValIdx{v, r};
    }
    write_result<To, 1, OP>(vals, idx, col, best.v, best.i, n, sv, si);
  }
}

}  // namespace

hipError_t launch_reduce(const void* x, void* vals, int64_t* idx, int64_t outer, int n,
                         int64_t inner, int idt, int odt, int op, const Geometry& g,
                         hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  auto body = [&](auto ti, auto to) {
    using Ti = typename decltype(ti)::type;
    using To = typename decltype(to)::type;
    constexpr int VN = Vec<Ti>::n;
    auto go = [&](auto opc) {
      constexpr int OP = decltype(opc)::value;
      if (inner == 1) {
        auto launch = [&](auto kern) {
          launch_kernel(kern, dim3(grid_for(outer, g)), dim3(g.block), 0, s,
                             static_cast<const Ti*>(x), vals, idx, outer, n, g.tpr);
        };
        if (g.v == 1) launch(reduce_rows<Ti, To, 1, OP, false>);
        else if (g.mis) launch(reduce_rows<Ti, To, VN, OP, true>);
        else launch(reduce_rows<Ti, To, VN, OP, false>);
      } else {
        const int64_t cols = outer * inner;
        launch_kernel((reduce_cols<Ti, To, OP>), dim3((cols + 255) / 256), dim3(256), 0, s,
                           static_cast<const Ti*>(x), vals, idx, outer, n, inner);
      }
      err = hipGetLastError();
    };
    if (op == 0) go(std::integral_constant<int, 0>{});
    else if (op == 1) go(std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, 2>{});
  };
  if (idt == odt) {
    dispatch_float_type(idt, [&](auto t) { body(t, t); });
  } else if (op == 0 && odt == kF32 && (idt == kF16 || idt == kBF16)) {
    dispatch_float_type(idt, [&](auto t) { body(t, TypeTag<float>{}); });
  } else if (op == 0 && idt == kF32 && (odt == kF16 || odt == kBF16) && inner == 1) {
    // second stage of a split mean: fp32 segment means in, the output type out
    dispatch_float_type(odt, [&](auto t) { body(TypeTag<float>{}, t); });
  }
  return err;
}

hipError_t launch_reduce_combine(const void* pvals, const int64_t* pidx, void* vals, int64_t* idx,
                                 int64_t rows, int segs, int segn, int dt, int op,
                                 hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  const int64_t grid = (rows + 255) / 256;
  dispatch_float_type(dt, [&](auto t) {
    using T = typename decltype(t)::type;
    if (op == 1)
      launch_kernel((reduce_combine_vi<T, 1>), dim3(grid), dim3(256), 0, s,
                         static_cast<const T*>(pvals), pidx, vals, idx, rows, segs, segn);
    else
      launch_kernel((reduce_combine_vi<T, 2>), dim3(grid), dim3(256), 0, s,
                         static_cast<const T*>(pvals), pidx, vals, idx, rows, segs, segn);
    err = hipGetLastError();
  });
  return err;
}

}  // namespace vbh

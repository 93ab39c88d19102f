// Device building blocks shared by every row kernel of libvbhip (gfx950 / CDNA4).
//
//  * 16-byte global loads/stores with conversion to and from fp32 registers
//    (fp32 x4, fp16 x8, bf16 x8; scalar variants for unaligned rows).
//  * Group all-reduce over `tpr` consecutive lanes (tpr a power of two):
//    DPP quad_perm / row_half_mirror / row_mirror inside a 16-lane row,
//    v_permlane16_swap and v_permlane32_swap across rows of one wave64,
//    and an LDS exchange across the waves of a workgroup when tpr > 64.
//    Every step combines a value with its partner through a commutative
//    operation, so all lanes of a group end with bit-identical results.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vbh {

constexpr int kWave = 64;
constexpr int kMaxBlock = 1024;
constexpr int kMaxWaves = kMaxBlock / kWave;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Elements per 16-byte vector for each storage type.
template <typename T> struct Vec;
template <> struct Vec<float> { static constexpr int n = 4; };
template <> struct Vec<_Float16> { static constexpr int n = 8; };
template <> struct Vec<__bf16> { static constexpr int n = 8; };

// ---------------------------------------------------------------------------
// debug bounds checks
//
// A build with VBH_DEBUG_BOUNDS defined (libvbhip_debug.so, `python -m
// dslperfgap_amd.build` makes it next to the release library) checks every
// global-memory access of every kernel before making it: the accessed bytes
// must lie inside the buffer the access belongs to.  Each kernel describes its
// buffers as Spans made from its own size arguments (VBH_SPAN(pointer,
// elements)), and every load / store helper below takes the Span of its
// buffer.  A failing access is not made (a load yields zeros, a store is
// dropped); it is counted in this translation unit's record together with the
// source line of the Span's VBH_SPAN, and the host reads the records through
// vbh_debug_bounds.  In a release build a Span is an empty struct and every
// check the constant true, so the generated code is the code without them.
// ---------------------------------------------------------------------------

struct Span {
#ifdef VBH_DEBUG_BOUNDS
  uintptr_t lo, hi;  // the buffer's bytes [lo, hi)
  int line;          // source line of the VBH_SPAN that made it
#endif
};

#ifdef VBH_DEBUG_BOUNDS
// This translation unit's record: [0] failed checks, [1] the Span line of the
// first failure (0: none).
static __device__ unsigned g_bounds_record[2];
// Bytes taken off the end of every Span (vbh_debug_bounds_slack): a test sets
// it to watch the checks fail on accesses near a buffer's end, which are then
// skipped, never made out of bounds.
static __device__ long long g_bounds_slack;

template <typename T>
__device__ __forceinline__ Span make_span(const T* p, int64_t elems, int line) {
  const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
  return Span{lo, lo + static_cast<uintptr_t>(elems > 0 ? elems : 0) * sizeof(T), line};
}

// The `bytes` at `p` lie inside `s` (less the slack); otherwise count the
// failure (vector atomics on the record) and return false.
__device__ __forceinline__ bool in_span(const Span& s, const void* p, int bytes) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  const long long room = static_cast<long long>(s.hi - s.lo) - g_bounds_slack;
  if (a >= s.lo && static_cast<long long>(a - s.lo) + bytes <= room) return true;
  atomicAdd(&g_bounds_record[0], 1u);
  atomicCAS(&g_bounds_record[1], 0u, static_cast<unsigned>(s.line));
  return false;
}

#define VBH_SPAN(p, elems) ::vbh::make_span((p), static_cast<int64_t>(elems), __LINE__)
#define VBH_IN_SPAN(s, p, bytes) ::vbh::in_span((s), (p), static_cast<int>(bytes))
#else
// the constant true: the access is made as if unchecked (the pointer and size
// are not evaluated; naming the empty Span keeps it a used variable)
#define VBH_SPAN(p, elems) ::vbh::Span{}
#define VBH_IN_SPAN(s, p, bytes) (static_cast<void>(s), true)
#endif

// Elements a [rows, cols] matrix with row stride `ld` spans (for Spans).
__device__ __forceinline__ int64_t strided_extent(int64_t rows, int64_t ld, int64_t cols) {
  return rows > 0 ? (rows - 1) * ld + cols : 0;
}

// ---------------------------------------------------------------------------
// loads / stores (each takes the Span of the buffer it accesses)
// ---------------------------------------------------------------------------

// Read V consecutive elements at p (V == Vec<T>::n: one 16-byte load, p 16-byte
// aligned; V == 1: one element) and widen them to fp32.
template <typename T, int V>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float* o, const Span& s) {
  if (!VBH_IN_SPAN(s, p, V * sizeof(T))) {
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = 0.f;
    return;
  }
  if constexpr (V == 1) {
    o[0] = static_cast<float>(p[0]);
  } else {
    typedef T vec_t __attribute__((ext_vector_type(V)));
    const vec_t v = *reinterpret_cast<const vec_t*>(p);
#pragma unroll
    for (int k = 0; k < V; ++k) o[k] = static_cast<float>(v[k]);
  }
}

// Round V fp32 values to T (round-to-nearest-even, NaN preserved) and store.
template <typename T, int V>
__device__ __forceinline__ void store_from_f32(T* __restrict__ p, const float* o, const Span& s) {
  if (!VBH_IN_SPAN(s, p, V * sizeof(T))) return;
  if constexpr (V == 1) {
    p[0] = static_cast<T>(o[0]);
  } else {
    typedef T vec_t __attribute__((ext_vector_type(V)));
    vec_t v;
#pragma unroll
    for (int k = 0; k < V; ++k) v[k] = static_cast<T>(o[k]);
    *reinterpret_cast<vec_t*>(p) = v;
  }
}

// Raw storage vectors: a row kept in registers in its storage type (4 VGPRs
// per 16-byte vector whatever the dtype) and widened to fp32 where used.
template <typename T, int V> struct Raw { typedef T type __attribute__((ext_vector_type(V))); };
template <typename T> struct Raw<T, 1> { typedef T type; };

// 16-byte (or scalar) load; NT marks the access nontemporal (streamed data
// that is touched once), which keeps it from displacing reused lines.
template <typename T, int V, bool NT>
__device__ __forceinline__ typename Raw<T, V>::type load_raw(const T* __restrict__ p,
                                                             const Span& s) {
  typedef typename Raw<T, V>::type R;
  if (!VBH_IN_SPAN(s, p, sizeof(R))) return R{};
  const R* q = reinterpret_cast<const R*>(p);
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}

template <typename T, int V>
__device__ __forceinline__ float raw_at(const typename Raw<T, V>::type& r, int k) {
  if constexpr (V == 1) return static_cast<float>(r);
  else return static_cast<float>(r[k]);
}

// Register barrier for a row held in a 16-bit storage type: after this point
// the compiler must assume the raw registers changed, so it re-widens values
// from them instead of keeping a widened fp32 copy of the whole row live across
// a reduction (which would double the VGPRs of the row and halve occupancy).
// fp32 rows need no barrier (raw and widened are the same registers).
template <typename T, int V, int IT>
__device__ __forceinline__ void reload_barrier(typename Raw<T, V>::type (&r)[IT]) {
  if constexpr (sizeof(T) == 2 && V > 1) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    static_assert(sizeof(typename Raw<T, V>::type) == 16, "16-byte vectors expected");
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      u32x4 u = __builtin_bit_cast(u32x4, r[i]);
      asm volatile("" : "+v"(u));
      r[i] = __builtin_bit_cast(typename Raw<T, V>::type, u);
    }
  }
}

template <typename T, int V, bool NT>
__device__ __forceinline__ void store_raw(T* __restrict__ p, const float* o, const Span& s) {
  typedef typename Raw<T, V>::type R;
  if (!VBH_IN_SPAN(s, p, sizeof(R))) return;
  R r;
  if constexpr (V == 1) {
    r = static_cast<T>(o[0]);
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k) r[k] = static_cast<T>(o[k]);
  }
  R* q = reinterpret_cast<R*>(p);
  if constexpr (NT) __builtin_nontemporal_store(r, q);
  else *q = r;
}

// ---------------------------------------------------------------------------
// output store policies of the row kernels
// ---------------------------------------------------------------------------

// kStoreCached:  plain loads and stores.
// kStoreStream:  nontemporal row loads and output stores (data touched once).
// kStoreThrough: as kStoreStream, and the 16-byte output stores are also
//   written through the L2 at device scope (buffer stores with the sc1 and nt
//   cache-policy bits).  The L2 then holds no dirty output lines when the
//   kernel ends, so the end-of-kernel write-back has nothing to flush; on
//   MI355X a 134 MB copy runs about 4% faster this way (the gap between
//   back-to-back kernels drops from about 1.4 to 1.0 us).
enum StorePolicy : int { kStoreCached = 0, kStoreStream = 1, kStoreThrough = 2 };

// Cache-policy operand of the buffer intrinsics on gfx940+: bit 0 sc0,
// bit 1 nt, bit 4 sc1.
constexpr int kCacheNtSc1 = (1 << 4) | (1 << 1);
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9-family GPUs.
constexpr int kRawBufferWord3 = 0x00020000;

// A workgroup's window of output elements [base, base + elems).  `base` and
// `elems` must be uniform across the workgroup (they form a scalar buffer
// resource) and the window must span less than 2^31 bytes.  Under
// kStoreThrough, 16-byte stores go through the buffer resource (whose range
// check also drops any store outside the window); every other store is a
// plain or nontemporal global store to its address, and the window is unused
// (the compiler drops it, so those kernels keep their register allocation).
template <typename T, int SP>
struct OutWindow {
  __amdgpu_buffer_rsrc_t rsrc;

  // The byte count goes through readfirstlane: a uniform clamp such as
  // max(min(n, lanes), 0) is selected as v_med3_i32, a VGPR, and a resource
  // with a field in a VGPR makes the compiler wrap every store in a loop over
  // the distinct values of the lanes.
  __device__ __forceinline__ OutWindow(T* base, int64_t elems) {
    if constexpr (SP == kStoreThrough)
      rsrc = __builtin_amdgcn_make_buffer_rsrc(
          base, static_cast<short>(0),
          __builtin_amdgcn_readfirstlane(static_cast<int>(elems * sizeof(T))), kRawBufferWord3);
  }

  // Round V fp32 values to T and store them at `p`, which is element `off` of
  // the window; `s` is the Span of the output buffer.
  template <int V>
  __device__ __forceinline__ void store(T* p, int off, const float* o, const Span& s) const {
    if constexpr (SP == kStoreThrough && V * sizeof(T) == 16) {
      if (!VBH_IN_SPAN(s, p, 16)) return;
      typedef typename Raw<T, V>::type R;
      typedef int i32x4 __attribute__((ext_vector_type(4)));
      R r;
#pragma unroll
      for (int k = 0; k < V; ++k) r[k] = static_cast<T>(o[k]);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, r), rsrc,
                                             off * static_cast<int>(sizeof(T)), 0,
                                             kCacheNtSc1);
    } else {
      store_raw<T, V, SP != kStoreCached>(p, o, s);
    }
  }
};

// ---------------------------------------------------------------------------
// reductions
// ---------------------------------------------------------------------------

struct Sum {
  __device__ static float apply(float a, float b) { return a + b; }
};
// Max of two floats for the row maxima of the exp-sum kernels: IEEE maximum,
// NaN if either operand is NaN.  It compiles to one v_maximum3_f32 per two
// values.  fmaxf (which drops a NaN operand) costs up to three instructions per
// value here: in the kernels' IEEE mode the compiler first quiets every operand
// it cannot prove canonical (v_max_f32 v, x, x), which includes every loaded
// value.  No output depends on which of the two a NaN row gets: every output
// that depends on the max also depends on exp(x - max) summed over the row,
// which a NaN element (or a NaN max) makes NaN.
__device__ __forceinline__ float max_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

struct Max {
  __device__ static float apply(float a, float b) { return max_nan(a, b); }
};

template <int Ctrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// All-reduce across aligned groups of `width` lanes of one wave64
// (width a power of two in [1, 64], uniform across the wave).
template <class Op>
__device__ __forceinline__ float wave_allreduce(float v, int width) {
  if (width >= 2) v = Op::apply(v, dpp<0xB1>(v));   // quad_perm [1,0,3,2]: lane ^ 1
  if (width >= 4) v = Op::apply(v, dpp<0x4E>(v));   // quad_perm [2,3,0,1]: lane ^ 2
  if (width >= 8) v = Op::apply(v, dpp<0x141>(v));  // row_half_mirror: other quad of 8
  if (width >= 16) v = Op::apply(v, dpp<0x140>(v)); // row_mirror: other half of 16
  if (width >= 32) {
    // rows (0,1) and (2,3) exchange: lo = even row, hi = odd row in every lane
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                              false, false);
    v = Op::apply(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  if (width >= 64) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                              false, false);
    v = Op::apply(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  return v;
}

// ---------------------------------------------------------------------------
// row groups without integer division
//
// The launchers make the lanes per row group, tpr, a power of two up to 64 or
// a multiple of 64 up to 1024 that divides the workgroup size.  Integer
// division by a run-time value costs about a dozen VALU instructions per lane
// here; for these shapes shifts do the work, and several multi-wave groups in
// one workgroup take one float multiply.
// ---------------------------------------------------------------------------

// a / b for 0 <= a <= 64 and 1 <= b <= 64, exact: (a + 1/2) / b lies at least
// 1 / (2b) >= 1/128 from an integer, far beyond the error of v_rcp_f32 (1 ulp).
__device__ __forceinline__ int small_quotient(int a, int b) {
  return static_cast<int>((static_cast<float>(a) + 0.5f) *
                          __builtin_amdgcn_rcpf(static_cast<float>(b)));
}

// A lane's place in the workgroup's row groups: lane `g` of its group, group
// `sub` of the workgroup, `per_block` groups per workgroup.
struct GroupShape {
  int g, sub, per_block;
};

__device__ __forceinline__ GroupShape group_shape(int tpr) {
  const int t = static_cast<int>(threadIdx.x);
  const int block = static_cast<int>(blockDim.x);
  if (tpr == block) return GroupShape{t, 0, 1};
  if ((tpr & (tpr - 1)) == 0) {  // every tpr <= 64 is one
    const int sh = __builtin_ctz(static_cast<unsigned>(tpr));
    return GroupShape{t & (tpr - 1), t >> sh, block >> sh};
  }
  const int k = tpr >> 6;  // waves per group
  const int sub = small_quotient(t >> 6, k);
  return GroupShape{t - sub * tpr, sub, small_quotient(block >> 6, k)};
}

// First wave of the row group that wave `wave` belongs to, for groups of
// nwaves = tpr / 64 > 1 waves: 0 when the group is the workgroup, a mask when
// nwaves is a power of two, else the float quotient (whose v_rcp_f32 runs at
// the transcendental rate, on the reduction's path).
__device__ __forceinline__ int first_wave_of_group(int wave, int nwaves, int tpr) {
  if (tpr == static_cast<int>(blockDim.x)) return 0;
  if ((nwaves & (nwaves - 1)) == 0) return wave & -nwaves;
  return small_quotient(wave, nwaves) * nwaves;
}

// All-reduce across the `tpr` threads that own one row.  For tpr <= 64 (a
// power of two) the group lives inside one wave; for tpr > 64 (any multiple of
// 64) a row spans tpr / 64 consecutive waves of the workgroup and wave partials
// are exchanged through `lds` (kMaxWaves floats, one slot per wave of the
// workgroup).  When tpr > 64 every thread of the workgroup must reach the call
// (it contains a barrier), and each `lds` buffer may serve only one reduction
// per kernel instance (there is no trailing barrier).
template <class Op>
__device__ __forceinline__ float group_allreduce(float v, int tpr, float* lds) {
  if (tpr <= kWave) return wave_allreduce<Op>(v, tpr);
  v = wave_allreduce<Op>(v, kWave);
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int nwaves = tpr >> 6;
  const int first = first_wave_of_group(wave, nwaves, tpr);
  if ((threadIdx.x & (kWave - 1)) == 0) lds[wave] = v;
  __syncthreads();
  float r = lds[first];
  for (int w = 1; w < nwaves; ++w) r = Op::apply(r, lds[first + w]);
  return r;
}

// Welford / Chan partial statistics (count, mean, sum of squared deviations).
struct Moments {
  float n, mean, m2;
};

// Chan et al. pairwise merge in a form that is symmetric in (a, b), so both
// partners of a butterfly step compute bit-identical results:
//   mean = (ma + mb) / 2 + (mb - ma) * (nb - na) / (2 n)
// (= (na ma + nb mb) / n), which is exact when the two means are equal, and
//   m2   = m2a + m2b + (mb - ma)^2 * na nb / n.
// Swapping a and b negates both factors of the correction term, which leaves
// every rounded intermediate unchanged.
__device__ __forceinline__ Moments merge_moments(Moments a, Moments b) {
  if (a.n == 0.f) return b;
  if (b.n == 0.f) return a;
  const float n = a.n + b.n;
  const float inv = 1.0f / n;
  const float d = b.mean - a.mean;
  Moments r;
  r.n = n;
  r.mean = 0.5f * (a.mean + b.mean) + (0.5f * d) * ((b.n - a.n) * inv);
  r.m2 = (a.m2 + b.m2) + d * d * (a.n * b.n * inv);
  return r;
}

template <int Ctrl>
__device__ __forceinline__ Moments dpp_moments(Moments m) {
  return Moments{dpp<Ctrl>(m.n), dpp<Ctrl>(m.mean), dpp<Ctrl>(m.m2)};
}

__device__ __forceinline__ float swap16_partner(float v) {
  // lane i receives lane i ^ 16
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                            false);
  const bool odd_row = (threadIdx.x & 16) != 0;
  return __uint_as_float(odd_row ? p[0] : p[1]);
}
__device__ __forceinline__ float swap32_partner(float v) {
  // lane i receives lane i ^ 32
  auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                            false);
  const bool hi = (threadIdx.x & 32) != 0;
  return __uint_as_float(hi ? p[0] : p[1]);
}

// All-reduce of Moments over the `tpr` threads of one row (see group_allreduce;
// `lds` must hold 3 * kMaxWaves floats).
__device__ __forceinline__ Moments group_allreduce_moments(Moments m, int tpr, float* lds) {
  const int width = tpr < kWave ? tpr : kWave;
  if (width >= 2) m = merge_moments(m, dpp_moments<0xB1>(m));
  if (width >= 4) m = merge_moments(m, dpp_moments<0x4E>(m));
  if (width >= 8) m = merge_moments(m, dpp_moments<0x141>(m));
  if (width >= 16) m = merge_moments(m, dpp_moments<0x140>(m));
  if (width >= 32)
    m = merge_moments(m, Moments{swap16_partner(m.n), swap16_partner(m.mean),
                                 swap16_partner(m.m2)});
  if (width >= 64)
    m = merge_moments(m, Moments{swap32_partner(m.n), swap32_partner(m.mean),
                                 swap32_partner(m.m2)});
  if (tpr <= kWave) return m;
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int nwaves = tpr >> 6;
  const int first = first_wave_of_group(wave, nwaves, tpr);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    lds[wave] = m.n;
    lds[kMaxWaves + wave] = m.mean;
    lds[2 * kMaxWaves + wave] = m.m2;
  }
  __syncthreads();
  Moments r{lds[first], lds[kMaxWaves + first], lds[2 * kMaxWaves + first]};
  for (int w = first + 1; w < first + nwaves; ++w)
    r = merge_moments(r, Moments{lds[w], lds[kMaxWaves + w], lds[2 * kMaxWaves + w]});
  return r;
}

// x * y rounded to fp32 by itself, never fused with a following add or
// subtract into one FMA.  exp(x * scale - m) where m is the rounded product of
// the row's max needs it: fused, x * scale - m is the product's rounding error
// for the max element itself, up to half an ulp of the product (1e31 at 2e38),
// not 0.
__device__ __forceinline__ float mul_rn(float x, float y) {
#pragma clang fp contract(off)
  return x * y;
}

// Fast exp / log on the hardware transcendental unit (v_exp_f32 / v_log_f32,
// 1 ulp in the base-2 domain).  exp(x) = 2^(x * log2 e); log(x) = log2(x) * ln 2.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * kLog2e);
}
__device__ __forceinline__ float fast_log(float x) {
  return __builtin_amdgcn_logf(x) * kLn2;
}

// exp(x - m) for many x against one row shift m, given mb = m * log2 e once per
// row: 2^(x * log2 e - mb), one FMA ahead of v_exp_f32 where fast_exp(x - m)
// takes a subtract and a multiply.  The rounding of mb moves every exponent of
// the row by the same amount, shift_residual(m, mb): it cancels in a softmax
// normalisation, and a log of the row sum subtracts it (times ln 2) -- at
// |m| = 3e4 it is 2e-3.  Special values follow x - m: -inf - (-inf) and
// +inf - (+inf) give NaN (as fma(x, log2 e, -mb) does), -inf against a finite m
// gives 0.
__device__ __forceinline__ float exp_shifted(float x, float mb) {
  return __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -mb));
}

// m * log2 e - mb, exactly (one FMA): sum of exp_shifted(x, mb) over a row =
// 2^shift_residual * the sum of exp(x - m).
__device__ __forceinline__ float shift_residual(float m, float mb) {
  return fmaf(m, kLog2e, -mb);
}

// The residual is up to half an ulp of m * log2 e, so it grows with |m|: at
// |m| = 1e9 it reaches 18 (every exp scaled by 2^-18), at 1e10 it is 440 and
// every exp of the row underflows, and above FLT_MAX / log2 e = 2.36e38 mb
// itself overflows.  Up to |m| = 2^24 it stays within +-1 (m * log2 e < 2^25,
// whose ulp is 2), which no row sum can turn into an overflow or a lost term.
// Rows whose finite shift is larger take exp(x - m) on a subtract instead; the
// choice is made once per row (shift_fma_ok), outside any barrier.  Infinite
// and NaN shifts keep the FMA form, whose special values follow x - m.
constexpr float kShiftFmaMax = 16777216.0f;  // 2^24

__device__ __forceinline__ bool shift_fma_ok(float m) {
  return !(__builtin_fabsf(m) > kShiftFmaMax) || __builtin_isinf(m);
}

// exp(x - m) of one row's values, in the form shift_fma_ok picked for the row:
struct ExpFma {  // 2^(x * log2 e - mb), mb = m * log2 e
  float mb;
  __device__ __forceinline__ float operator()(float x) const { return exp_shifted(x, mb); }
};
struct ExpSub {  // exp(x - m) on a subtract
  float m;
  __device__ __forceinline__ float operator()(float x) const { return fast_exp(x - m); }
};

// The first stage of a split row writes one SegPair per segment: its max m
// (NaN if it holds a NaN, -inf if it holds only -inf) and t, the sum over it of
// exp(x - m) (0 for an all -inf segment).  A second stage merges a row's pairs
// (wave_combine_seg_pairs): M = max m_k, S = sum t_k * exp(m_k - M) over the
// segments whose m_k > -inf, and `nan` if any m_k or t_k is NaN (S is then
// meaningless, as it is when M is infinite).  The row's logsumexp M + log S is
// then rounded once, as in a single pass; a logsumexp per segment would round
// m_k + log t_k first, which loses the log entirely where |m_k| is large.
struct RowPairs {
  float m, s;
  bool nan;
};

// The merge of one row's SegPairs by one wave: lane k < segs (`has`) holds
// segment k's (m_k, t_k), the other lanes nothing, and every lane gets the
// row's M, S and `nan`.  The segments' values arrive in one round of loads
// (one per lane) instead of a loop over them in one lane, whose dependent
// loads made the second stage of a split row several microseconds long.
__device__ __forceinline__ RowPairs wave_combine_seg_pairs(bool has, float mk, float tk) {
  const float neg_inf = -__builtin_huge_valf();
  if (!has) {
    mk = neg_inf;
    tk = 0.f;
  }
  const bool nan = wave_allreduce<Max>(mk != mk || tk != tk ? 1.f : 0.f, kWave) > 0.f;
  const float mx = wave_allreduce<Max>(mk, kWave);  // NaN where `nan` (then unused)
  const bool use = !nan && !__builtin_isinf(mx) && mk != neg_inf;
  const float s = wave_allreduce<Sum>(use ? tk * fast_exp(mk - mx) : 0.f, kWave);
  return RowPairs{mx, s, nan};
}

#ifdef VBH_DEBUG_BOUNDS
// Host side of the records: every translation unit that includes this header
// registers a reader of its own record (and setter of its slack) with the
// library (capi.hip), which combines them in vbh_debug_bounds.
typedef hipError_t (*BoundsRecordFn)(unsigned* failed, unsigned* line, const long long* slack,
                                     bool clear);
int register_bounds_record(const char* file, BoundsRecordFn fn);

// Read this translation unit's record on the current device into *failed /
// *line; with `clear` zero it, with `slack` non-null set the slack.
static hipError_t bounds_record_here(unsigned* failed, unsigned* line, const long long* slack,
                                     bool clear) {
  unsigned rec[2] = {0u, 0u};
  hipError_t e = hipMemcpyFromSymbol(rec, HIP_SYMBOL(g_bounds_record), sizeof(rec), 0,
                                     hipMemcpyDeviceToHost);
  if (e != hipSuccess) return e;
  *failed = rec[0];
  *line = rec[1];
  if (clear) {
    const unsigned zero[2] = {0u, 0u};
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_bounds_record), zero, sizeof(zero), 0,
                          hipMemcpyHostToDevice);
    if (e != hipSuccess) return e;
  }
  if (slack != nullptr)
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_bounds_slack), slack, sizeof(*slack), 0,
                          hipMemcpyHostToDevice);
  return e;
}
[[maybe_unused]] static const int g_bounds_registered =
    register_bounds_record(__BASE_FILE__, &bounds_record_here);
#endif

}  // namespace vbh

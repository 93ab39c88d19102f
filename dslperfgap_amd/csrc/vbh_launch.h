// Host-side contract between the C ABI (capi.hip) and the kernel translation
// units.  Argument checking happens in capi.hip; the launchers below assume
// valid sizes, dtype codes and a geometry produced by pick_geometry().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <tuple>
#include <type_traits>
#include <utility>

#include "vbh_device.h"

namespace vbh {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2, kI32 = 3, kI64 = 4 };

// Launch geometry of a row kernel.
//   v      elements per lane access (16-byte vector width, or 1 for rows that
//          are not 16-byte aligned)
//   tpr    threads per row (power of two, 1..1024)
//   block  workgroup size (a multiple of 64 and of tpr)
//   maxit  vectors held in registers per lane (power of two)
//   stream row too wide for registers: chunked two-pass kernel instead
//   persist  persistent pipelined kernel: grid sized to the resident
//          capacity, each row group loops over rows, keeps per-column vectors
//          (weight, bias) in registers and prefetches its next row
//   nt     nontemporal hints on the streamed row loads / output stores
//   wt     16-byte output stores also written through the L2 (kStoreThrough;
//          only with nt, and only where the kernel has 16-byte output rows)
struct Geometry {
  int v = 1;
  int tpr = 64;
  int block = 256;
  int maxit = 1;
  bool stream = false;
  bool persist = false;
  bool nt = false;
  bool wt = false;
  // rows not a multiple of V long: head / aligned body / tail per row (MIS
  // kernels; v is the vector width, tpr >= v)
  bool mis = false;
  // persistent grid: input bytes of current and next rows a CU may hold in
  // flight (0: pipe_grid's rule by workgroup size), where that leaves every
  // row group at least pipe_min_rows rows (0: always)
  int64_t pipe_bytes = 0;
  int pipe_min_rows = 0;
};

// The current device's hipFunction_t of `kernel` (a __global__ function of
// this library), looked up once per device with hipGetFuncBySymbol and cached;
// null where the lookup fails (no device, or a device index beyond the cache).
hipFunction_t function_for(const void* kernel);

// Launch `kernel` with `args` converted to its parameter types.  The launch
// goes through hipModuleLaunchKernel with the cached hipFunction_t, which skips
// the runtime's per-launch lookup of the host stub hipLaunchKernel does
// (MI355X, back-to-back launches of a small kernel from a C loop: 2.7 us per
// launch against 3.0-3.4 us).  Where no hipFunction_t is available it falls
// back to hipLaunchKernel, whose error the caller then reads with
// hipGetLastError as after any launch.
template <typename... P, typename... A>
void launch_kernel(void (*kernel)(P...), dim3 grid, dim3 block, unsigned shmem, hipStream_t s,
                   A&&... args) {
  static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
  std::tuple<std::decay_t<P>...> params(static_cast<std::decay_t<P>>(std::forward<A>(args))...);
  hipFunction_t f = function_for(reinterpret_cast<const void*>(kernel));
  std::apply(
      [&](auto&... p) {
        void* ptrs[] = {static_cast<void*>(&p)...};
        if (f != nullptr)
          (void)hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, shmem,
                                      s, ptrs, nullptr);
        else
          (void)hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, shmem,
                                s);
      },
      params);
}

// vbh_tune_override flag bits
constexpr int kFlagPersist = 1;
constexpr int kFlagNoPersist = 2;
constexpr int kFlagNontemporal = 4;
constexpr int kFlagTemporal = 8;
constexpr int kFlagWriteThrough = 16;
constexpr int kFlagNoWriteThrough = 32;
constexpr int kFlagAll = 63;

// The persistent kernels keep up to this many 16-byte vectors per lane for each
// of: current row, next row, and every per-column vector (their register cap
// per instantiation is pipe_cap in rownorm.hip).
constexpr int kPipeMaxIt = 4;

// Number of workgroups of `block` lanes of `kernel` that are resident on the
// whole current device at once (occupancy, at most max_per_cu, x compute
// units); the occupancy is cached.
int64_t resident_blocks(const void* kernel, int block, int max_per_cu = 1 << 30);

// Grid of a persistent row kernel over `rows` rows of `row_bytes` input
// bytes each: as many workgroups as are resident at once (capped by the input
// bytes a CU may hold in flight, current and next rows), at most one per row
// group.
int64_t pipe_grid(const void* kernel, const Geometry& g, int64_t rows, int64_t row_bytes);

// Register budget per lane for a register-resident row: 64 values (the
// compiler widens every 16-bit value it reuses to an fp32 register), i.e. 16
// fp32 or 8 bf16/fp16 vectors of 16 bytes, or 16 scalar elements for rows that
// are not 16-byte aligned (each scalar access also holds its own address).
constexpr int lane_cap(int vec) { return vec > 1 ? 64 / vec : 16; }

// VGPRs that IT vectors of V elements of type T occupy in raw storage.
template <typename T>
constexpr int raw_vgprs(int v, int it) {
  return static_cast<int>((it * v * sizeof(T) + 3) / 4);
}

// Choose the geometry for rows of `cols` elements.  `vec` is the 16-byte vector
// width when every row start is 16-byte aligned and cols % vec == 0, else 1;
// `it_target` the preferred vectors per lane.  `tpr_override` /
// `block_override` come from vbh_tune_override (0 = none), `flags` are the
// resolved kFlagPersist / kFlagNontemporal bits.
Geometry pick_geometry(int64_t cols, int vec, int it_target, int tpr_override,
                       int block_override, int flags);

// ---------------------------------------------------------------------------
// compile-time dispatch helpers
// ---------------------------------------------------------------------------
template <typename T> struct TypeTag { using type = T; };

template <typename Fn>
bool dispatch_float_type(int dt, Fn&& fn) {
  switch (dt) {
    case kF32: fn(TypeTag<float>{}); return true;
    case kF16: fn(TypeTag<_Float16>{}); return true;
    case kBF16: fn(TypeTag<__bf16>{}); return true;
    default: return false;
  }
}

// maxit buckets for the register-resident path (1..lane_cap(v))
template <typename Fn>
bool dispatch_maxit(int maxit, Fn&& fn) {
  switch (maxit) {
    case 1: fn(std::integral_constant<int, 1>{}); return true;
    case 2: fn(std::integral_constant<int, 2>{}); return true;
    case 4: fn(std::integral_constant<int, 4>{}); return true;
    case 8: fn(std::integral_constant<int, 8>{}); return true;
    case 16: fn(std::integral_constant<int, 16>{}); return true;
    case 32: fn(std::integral_constant<int, 32>{}); return true;
    default: return false;
  }
}

// Store policy of a launch with V-element accesses (StorePolicy in
// vbh_device.h): write-through needs 16-byte vector rows.
template <int V, typename Fn>
void dispatch_store_policy(const Geometry& g, Fn&& fn) {
  if (!g.nt) fn(std::integral_constant<int, kStoreCached>{});
  else if (V > 1 && g.wt) fn(std::integral_constant<int, kStoreThrough>{});
  else fn(std::integral_constant<int, kStoreStream>{});
}

inline int64_t grid_for(int64_t rows, const Geometry& g) {
  const int64_t rpb = g.block / g.tpr;
  return (rows + rpb - 1) / rpb;
}

// ---------------------------------------------------------------------------
// launchers (return hipError_t of the launch)
// ---------------------------------------------------------------------------
hipError_t launch_layer_norm(const void* x, const void* w, const void* b, void* y,
                             int64_t rows, int cols, float eps, int dt, int wdt,
                             const Geometry& g, hipStream_t s);
hipError_t launch_rms_norm(const void* x, const void* w, void* y, int64_t rows,
                           int cols, float eps, int dt, int wdt, const Geometry& g,
                           hipStream_t s);
hipError_t launch_softmax(const void* x, void* y, int64_t rows, int cols, int idt,
                          int odt, int log_mode, const Geometry& g, hipStream_t s);
hipError_t launch_softmax_dim(const void* x, void* y, int64_t outer, int n,
                              int64_t inner, int idt, int odt, int log_mode,
                              hipStream_t s);
// Second stage of a split softmax / log_softmax: y from x and each row's
// `segs` (<= 64) segment SegPairs (seg_pairs[2 * (row * segs + k)], written by
// launch_logsumexp_pairs), one kApplyLanes-lane workgroup per tile of
// kApplyLanes vectors; g.nt / g.wt select the store policy.
constexpr int kApplyLanes = 256;
hipError_t launch_softmax_apply(const void* x, void* y, const float* seg_pairs, int64_t rows,
                                int cols, int segs, int idt, int odt, int log_mode,
                                const Geometry& g, hipStream_t s);
// segs > 1 (MIS geometry only): each of rows / segs rows of `cols` columns is
// split into segs segments of seg_cols columns, the last one shorter.
hipError_t launch_logsumexp(const void* x, void* y, int64_t rows, int cols, int idt,
                            int odt, const Geometry& g, hipStream_t s, int segs = 1,
                            int seg_cols = 0);
// First stage of a split row: launch_logsumexp's units (same segs / seg_cols
// rule), each writing its SegPair (max, sum of exp(x - max)) as two fp32 values
// into pairs[2 * unit].
hipError_t launch_logsumexp_pairs(const void* x, float* pairs, int64_t units, int cols, int idt,
                                  const Geometry& g, hipStream_t s, int segs = 1,
                                  int seg_cols = 0);
// Second stage of a split logsumexp: y[row] (dtype odt) from the row's `segs`
// SegPairs at pairs[2 * (row * segs + k)].
hipError_t launch_logsumexp_combine(const float* pairs, void* y, int64_t rows, int segs,
                                    int odt, hipStream_t s);

struct CeArgs {
  const void* logits;
  const void* labels;
  int logits_dt;
  int label_i64;
  float* loss;
  float* lse;
  float* z_loss;
  int64_t n_rows;
  int n_cols;
  int64_t ld;
  int block_size;
  int ncb;
  float smoothing;
  float logit_scale;
  float lse_square_scale;
  int64_t ignored_index;
  float total_classes;
  int64_t class_start;
  int has_smoothing;
  int split;
  int empty_neg_inf = 0;  // first stage of a split row (see ce_combine)
  int pair_out = 0;       // first stage of a split row: SegPairs to z_loss (max), lse (sum)
};
hipError_t launch_cross_entropy_fwd(const CeArgs& a, const Geometry& g, hipStream_t s);
// The persistent forward (ce_fwd_persist): fp32 logits whose rows (one
// column block per row) hold at least one chunk of
// cross_entropy_fwd_persist_chunk_cols() columns, under 1 GiB, in
// 16-byte-aligned rows.  Its grid is one workgroup per CU, at most `max_grid`
// (0: no limit), of `lanes` lanes: 256 or 512, or 0 for the launcher's choice
// by the launch's chunks per CU.
bool cross_entropy_fwd_persist_fits(int logits_dtype, int64_t n_cols);
int64_t cross_entropy_fwd_persist_chunk_cols();
hipError_t launch_cross_entropy_fwd_persist(const CeArgs& a, int64_t max_grid, int lanes,
                                            hipStream_t s);
// Second stage of a split row: `a` describes the caller's launch (one column
// block per row); seg_loss / seg_lse hold the first stage's `segs` segments
// per row at flat index k * n_rows + row.
hipError_t launch_cross_entropy_combine(const CeArgs& a, const float* seg_loss,
                                        const float* seg_sum, const float* seg_max, int segs,
                                        hipStream_t s);

struct CeBwdArgs {
  const float* dloss;
  const void* logits;
  const float* lse;
  const void* labels;
  void* dlogits;
  int logits_dt;
  int label_i64;
  int64_t n_rows;
  int n_cols;
  int64_t ld_logits;
  int64_t ld_dlogits;
  int64_t dloss_stride;
  float smoothing;
  float logit_scale;
  float lse_square_scale;
  int64_t ignored_index;
  float total_classes;
  int64_t class_start;
  int has_smoothing;
  int vec;
  int nt;  // nontemporal logits loads / dlogits stores
  int wt;  // dlogits stores also written through the L2 (with nt, 16-byte rows)
  int mis = 0;  // rows not a multiple of vec long: head / aligned body / tail
};
// One workgroup of this many lanes per tile of as many vectors of one row.
constexpr int kCeBwdLanes = 256;
hipError_t launch_cross_entropy_bwd(const CeBwdArgs& a, hipStream_t s);

hipError_t launch_reduce(const void* x, void* vals, int64_t* idx, int64_t outer, int n,
                         int64_t inner, int idt, int odt, int op, const Geometry& g,
                         hipStream_t s);
// Second stage of a split max (op 1) / argmax (op 2): per row, the winner of
// `segs` segment results (values of type `dt`, int64 segment-local indices).
hipError_t launch_reduce_combine(const void* pvals, const int64_t* pidx, void* vals, int64_t* idx,
                                 int64_t rows, int segs, int segn, int dt, int op,
                                 hipStream_t s);

hipError_t launch_stream_copy(const void* src, void* dst, int64_t bytes, hipStream_t s);

// streaming-read yardstick: 16-byte vectors per lane per workgroup tile
constexpr int kReadUnroll = 8;
// workgroup tiles of a read of `bytes`
int64_t stream_read_tiles(int64_t bytes);
// `grid` persistent workgroups (at most the tile count), one 32-bit partial
// word each
hipError_t launch_stream_read(const void* src, void* partial, int64_t bytes, int grid,
                              hipStream_t s);

}  // namespace vbh

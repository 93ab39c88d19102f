// C ABI of libvbhip.so: argument validation, launch-geometry selection and
// error reporting around the kernel launchers.  Declarations and the reference
// interface each entry point stands in for are in include/vbhip.h.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "../../include/vbhip.h"
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err[0] = '\0';
    return 0;
  }
  return fail(static_cast<int>(e), "%s: %s (%s)", what, hipGetErrorName(e),
              hipGetErrorString(e));
}

int elt_size(int dt) {
  switch (dt) {
    case kF32: return 4;
    case kF16: return 2;
    case kBF16: return 2;
    case kI32: return 4;
    case kI64: return 8;
    default: return 0;
  }
}

bool is_float(int dt) { return dt == kF32 || dt == kF16 || dt == kBF16; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// process-wide launch-geometry overrides (vbh_tune_override)
constexpr int kNumOps = 6;
std::atomic<int> g_tpr[kNumOps];
std::atomic<int> g_block[kNumOps];
std::atomic<int> g_flags[kNumOps];

// Built-in choices per op, from launch-shape sweeps on MI355X:
//   vectors per lane before more lanes are added (pick_geometry): 2 for RMSNorm
//   and fp32 softmax, 4 for 16-bit softmax (bf16 8192 columns: +8% over 2),
//   4 for LayerNorm (its two reductions per row favour fewer waves per row) and
//   for the reductions that write one value per row (logsumexp, cross entropy,
//   mean / max / argmax), 8 for logsumexp and mean / max / argmax rows of more
//   than 2048 vectors (1024 lanes x 4 -- one batch of loads per lane -- is the
//   slow spot: fp32 16384-column logsumexp 6.1 TB/s, 512 x 8 6.9 TB/s) and
//   earlier still on 16-byte rows (it_target);
//   nontemporal row loads / stores for every op (rows are touched once);
//   the persistent pipelined kernel for LayerNorm rows that span 128 or more
//   lanes and RMSNorm rows that span 512 or more (it keeps every CU streaming
//   instead of running the grid in rounds: on MI355X, LayerNorm gains 3-9% at
//   128 and 256 lanes -- bf16 4096 / 8192 and fp32 2048 / 4096 columns -- and
//   loses 3-13% at 64 lanes); narrower rows run one row group per workgroup.
constexpr int kItTarget[kNumOps][2] = {{4, 4}, {2, 2}, {2, 4}, {4, 4}, {4, 4}, {4, 4}};
constexpr int64_t kLongRowVecs = 2048;
constexpr int64_t kMidRowVecs = 256;

// [op][0] for 4-byte (or unaligned scalar) access, [op][1] for 16-bit vectors.
// The read-only row reductions take 8 vectors per lane earlier on 16-byte rows
// (MI355X sweep over 512-16384 columns, 256 MB per launch): cross entropy at
// every width (fp32 +6 to +18%, bf16 +12 to +22% over 4), 16-bit logsumexp
// above 256 vectors (+7% at 500, +12% at 2048), fp32 mean / max / argmax above
// 256 vectors (+2 to +4%) and their 16-bit rows above 1024 vectors (+13% at
// 2048).  fp32 logsumexp takes 8 above 256 vectors as well: within 1% of 4
// at 256 MB per launch (C3's 16384 x 4096: 6296-6385 GB/s either way) and
// ahead at 64 MB (3072 columns 4689 -> 5164 GB/s, 8192 4673 -> 5088).
// Short rows (at most kShortRowVecs vectors) want several lanes per row: one
// or two lanes per row serialise each row's loads and leave the reductions
// nothing to share.  There each op takes kItShort vectors per lane, halved
// until the row has kMinLanesShort lanes.  MI355X, bf16 at 64 MB per call,
// default -> rule: 64 columns (8 vectors) LayerNorm 2068 -> 4794 GB/s,
// RMSNorm 5006 -> 5841, softmax 1969 -> 5546, cross entropy 2170 -> 3073,
// argmax 3139 -> 4645; 128 columns LayerNorm 4503 -> 5698, softmax 4532 ->
// 5768, cross entropy 2786 -> 3970; 256 columns +0 to +4%.
constexpr int64_t kShortRowVecs = 32;
constexpr int kItShort[kNumOps] = {2, 2, 2, 2, 4, 4};
constexpr int kMinLanesShort[kNumOps] = {4, 8, 8, 8, 2, 4};

int it_target(int op, int64_t nvec, int vec, bool column_blocks) {
  if (vec > 1 && nvec <= kShortRowVecs) {
    int it = kItShort[op];
    while (it > 1 && nvec / it < kMinLanesShort[op]) it /= 2;
    return it;
  }
  // fp32 softmax rows of 33-64 vectors: one wave per row (log_softmax fp32,
  // 64 MB per call: 256 columns 5730 -> 5849 GB/s, 255 columns 4843 -> 5241;
  // 512 columns and more keep 2 vectors per lane, within 1% of the best)
  if (op == VBH_OP_SOFTMAX && vec == 4 && nvec <= kWave) return 1;
  // 16-bit LayerNorm rows of 1025-1536 vectors: 2 vectors per lane, 9-12 waves
  // per row (bf16 at 64 MB per call, 4 -> 2: 9216 columns 4298 -> 5247 GB/s,
  // 10240 4501 -> 5194, 11264 4855 -> 5199, 12288 5126 -> 5290; at 768 and
  // 896 vectors 2 per lane loses 1-8%, from 1664 vectors on 13 or more waves
  // per row lose 6%)
  if (op == VBH_OP_LAYER_NORM && vec == 8 && nvec > 1024 && nvec <= 1536) return 2;
  // 16-bit LayerNorm rows that 4 vectors per lane would leave short of whole
  // waves (so the guarded persistent kernel runs) but 2 per lane fill exactly
  // (the unguarded one): 2 vectors per lane.  MI355X, 8192 rows, 4 -> 2: bf16
  // 3072 columns 4188 -> 5303 GB/s, 5120 4891 -> 5501, fp16 7168 5369 -> 5667;
  // bf16 2048 x 7168 3779 -> 4916, 4096 x 5120 4292 -> 5044.  Rows that 4 per
  // lane already fill keep 4 (bf16 6144 columns: 5539 at 4, 5453 at 2).
  if (op == VBH_OP_LAYER_NORM && vec == 8 && nvec > 4 * kWave && nvec <= 2 * kMaxBlock &&
      nvec % (4 * kWave) != 0 && nvec % (2 * kWave) == 0)
    return 2;
  // fp32 LayerNorm rows of 128 or 256 vectors (512 / 1024 columns): 2 vectors
  // per lane, so 1024 columns take a 2-wave row group, persistent in 512-lane
  // workgroups (below).  MI355X, 4 -> 2 per lane: 1024 columns 4575 -> 4720
  // GB/s at 33.6 MB per call (C1), 5282 -> 5497 at 134 MB; 512 columns +1 to
  // +2%.  Rows that do not fill whole 2-vector lanes lose (768 columns -1 to -6%).
  if (op == VBH_OP_LAYER_NORM && vec == 4 && nvec > kWave && nvec <= 256 &&
      (nvec & (nvec - 1)) == 0)
    return 2;
  if (vec > 1) {
    // cross entropy: 8 where a segment is a whole row (the sweep above); 4
    // where rows are cut into column blocks (BLOCK_SIZE < n_cols).  MI355X, 8
    // -> 4 at 512 MB per launch: fp32 4096 x 32768 at BLOCK_SIZE 512 / 1024 /
    // 2048 / 4096 +10.5 / +11.0 / +6.7 / +4.2%, fp32 16384 x 4096 at 1024
    // +13.0%, bf16 4096 x 32768 at 1024 / 2048 +7.7 / +3.7%; whole rows of
    // 512-2048 columns lose 2-7% at 4.
    if (op == VBH_OP_CROSS_ENTROPY) return column_blocks ? 4 : 8;
    if (op == VBH_OP_LOGSUMEXP && nvec > kMidRowVecs) return 8;
    if (op == VBH_OP_REDUCE && nvec > (vec == 8 ? int64_t(1024) : kMidRowVecs)) return 8;
  }
  if ((op == VBH_OP_LOGSUMEXP || op == VBH_OP_REDUCE) && nvec > kLongRowVecs) return 8;
  return kItTarget[op][vec == 8 ? 1 : 0];
}
constexpr int kPersistMinTpr[kNumOps] = {128, 512, 0, 0, 0, 0};

// Small launches are bound by latency, not bandwidth: with too few lanes the
// grid leaves CUs idle and each lane's chain of loads is long.  While a launch
// would have fewer than kFillLanes lanes (256 per CU), the vectors per lane
// are halved, down to 2 and as long as a row still fits one wave (a row group
// over several waves adds an LDS exchange and a barrier).  MI355X, kernel time
// per launch from HIP-graph replays at the reference's small shapes: LayerNorm
// bf16 512 x 1024 3.26 -> 2.76 us, softmax fp16 512 x 1024 3.23 -> 2.62,
// log_softmax 3.06 -> 2.51, cross entropy fp32 256 x 1024 (256-column blocks)
// 3.63 -> 2.93, argmax fp16 1024 x 1024 3.07 -> 2.85.
constexpr int64_t kFillLanes = 65536;

int pow2ceil(int64_t n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// a * b for sizes (a, b >= 0), saturated at INT64_MAX: products of caller
// sizes are formed before the range checks that reject them.
int64_t mul_sat(int64_t a, int64_t b) {
  int64_t r;
  return __builtin_mul_overflow(a, b, &r) ? INT64_MAX : r;
}

int row_group_lanes(int64_t nvec, int it) {
  const int64_t lanes = (nvec + it - 1) / it;
  if (lanes <= kWave) return pow2ceil(lanes < 1 ? 1 : lanes);
  return static_cast<int>((lanes + kWave - 1) / kWave) * kWave;
}

// `units`: row groups one launch runs (rows, or row x column-block segments).
int fill_it(int it, int64_t nvec, int64_t units) {
  while (it > 2 && mul_sat(units, row_group_lanes(nvec, it)) < kFillLanes &&
         (nvec + it / 2 - 1) / (it / 2) <= kWave)
    it /= 2;
  return it;
}

// Write-through output stores (kStoreThrough) by default for the kernels that
// write a full-size output (LayerNorm, RMSNorm, softmax / log_softmax) once
// one launch writes at least this much.  Measured on MI355X against
// nontemporal stores kept in the L2: RMSNorm bf16 8192 x 4096 +0.9%, softmax
// fp32 16384 x 4096 +1.6%, softmax fp16 4096 x 32768 +4.3%, LayerNorm fp32
// 4096 x 1024 (16 MiB out) -0.2%, RMSNorm bf16 1024 x 4096 (8 MiB out) -2.5%.
// Only rows that are whole 128-byte L2 lines: where a line holds the end of
// one row and the start of the next, the two halves are written through
// separately, and the launch is slower than with L2 stores (softmax fp16
// 50256 columns -5%, log_softmax fp16 -7%; rows of 50257 or 4097 columns
// -7 to -24%).
constexpr int64_t kWriteThroughMinBytes = int64_t(32) << 20;
constexpr int64_t kLineBytes = 128;

// Write-through suits a launch of `units` output rows, `out_bytes` in all.
bool write_through_ok(int64_t out_bytes, int64_t units) {
  return out_bytes >= kWriteThroughMinBytes && units > 0 && out_bytes % units == 0 &&
         (out_bytes / units) % kLineBytes == 0;
}

// Few wide rows leave CUs idle when each row has one row group (128 fp32 rows
// of 131072 columns: 128 workgroups on 256 CUs), and one workgroup streams a
// long row at about 20 GB/s.  The read-only row reductions (logsumexp, cross
// entropy with one column block per row, mean / max / argmax) then split every
// row into `segs` equal segments: a first launch reduces the
// [rows * segs, cols / segs] view into a caller-provided workspace, a second
// combines each row's segments.  On MI355X, time per call of both launches:
// fp32 logsumexp 128 x 131072 27.7 -> 15.5 us, 32 x 262144 33.8 -> 10.8;
// cross entropy fp32 64 x 128256 26.8 -> 16.4, 1 x 128256 24.8 -> 15.7.  The
// split costs a second launch and, in Python, a workspace allocation, so
// shorter rows stay unsplit: cross entropy fp32 64 x 50304 (200 KB rows)
// 11.6 us unsplit, 14.9 split.  The register-resident logsumexp and cross
// entropy row kernels also gain at 256-511 rows of at least 12288 vectors,
// (fp32, interleaved: logsumexp 256 x 65536 3778 -> 4377 GB/s, 335 x 50000
// 3126 -> 4202, 400 x 65536 3780 -> 4923; cross entropy 335 x 50000 2965 ->
// 3650, 400 x 65536 3695 -> 4387, but 256 x 65536 3734 -> 3584, so cross
// entropy starts above 256 rows; 384 x 32768 logsumexp: 3929 unsplit,
// 3569-3848 split); the streaming mean does not (fp32 256 x 65536: 5217
// unsplit, 4840-5004 split).
// Default launches of the persistent cross-entropy forward (ce_fwd_persist):
// at least this many rows, of at least this many of its chunks.
constexpr int64_t kCePersistMinRows = 1024;
constexpr int64_t kCePersistMinChunks = 2;
constexpr int64_t kSplitMaxRows = 256;      // split launches of fewer rows ...
constexpr int64_t kSplitRowVecs = 16384;    // ... of 16-byte vectors per row, at least
constexpr int64_t kSplitMaxRowsLong = 512;  // two-round launches (logsumexp, CE) ...
constexpr int64_t kSplitLongVecs = 12288;   // ... of rows of at least this many vectors
constexpr int64_t kSplitTarget = 1024;      // segments per launch to aim for
constexpr int64_t kSplitMinVecs = 512;      // 16-byte vectors per segment, at least
constexpr int kSplitMaxSegs = 64;
static_assert(kSplitMaxSegs <= kWave, "the second stages combine one segment per lane of a wave");

// Segments per row (a power of two dividing the row's vectors unless `even` is
// false), or 1.  `long_from`: the op also splits launches of long_from to 511
// rows of long rows (0: it does not).
int split_segments(int64_t rows, int64_t nvec, int64_t long_from = 0, bool even = true,
                   int64_t min_vecs = kSplitRowVecs) {
  const bool few = rows > 0 && rows < kSplitMaxRows && nvec >= min_vecs;
  const bool two_rounds = long_from > 0 && rows >= long_from && rows < kSplitMaxRowsLong &&
                          nvec >= kSplitLongVecs;
  if (!few && !two_rounds) return 1;
  int segs = 1;
  while (segs < kSplitMaxSegs && rows * segs < kSplitTarget &&
         (!even || nvec % (2 * segs) == 0) && nvec / (2 * segs) >= kSplitMinVecs)
    segs *= 2;
  return segs;
}

// A split of rows of `cols` columns: `segs` segments of `seg_cols` columns.
// Rows of whole vectors split evenly (split_segments); other rows (run by the
// MIS kernels, each segment with its own head and tail) into segments of a
// whole number of vectors, the last one shorter.
struct RowSplit {
  int segs;
  int64_t seg_cols;
};

RowSplit split_row(int64_t rows, int64_t cols, int vn, int64_t long_from) {
  if (cols % vn == 0) {
    const int segs = split_segments(rows, cols / vn, long_from);
    return RowSplit{segs, cols / segs};
  }
  const int segs = split_segments(rows, cols / vn, long_from, false);
  if (segs == 1) return RowSplit{1, cols};
  const int64_t seg_cols = ((cols + segs - 1) / segs + vn - 1) / vn * vn;
  return RowSplit{static_cast<int>((cols + seg_cols - 1) / seg_cols), seg_cols};
}

// Rows whose length is not a multiple of the 16-byte vector (GPT-2's 50257
// columns) run the MIS row kernels -- scalar head and tail, aligned vector
// body -- instead of one scalar access per element, when every row of input
// and output starts at the same offset within a vector (both buffers 16-byte
// aligned, same row length) and the row fits the register-resident kernel.
// MI355X, 50257 columns: fp32 log_softmax 2407 GB/s scalar, 4811 at 50256.
constexpr int64_t kMisMinVecs = 4;  // shorter rows keep the scalar kernel

// logsumexp rows of 512 lanes at 8 vectors per lane (4096-vector rows: fp32
// 16384, 16-bit 32768 columns) run two to a 1024-lane workgroup in launches of
// at least kLseTwoRowsMin rows.  MI355X, one -> two per workgroup: fp32 4096 /
// 8192 / 16384 x 16384 +7.0 / +6.1 / +5.4%, fp16 2048 / 4096 / 8192 x 32768
// +4.7 / +8.7 / +8.2%, but fp32 1024 x 16384 -4%.  Not bf16: its kernel
// keeps the row widened to fp32 as well (105 VGPRs against 58 for fp16), so
// two 16-wave workgroups do not fit a CU (bf16 8192 x 32768 -26%).
constexpr int64_t kLseTwoRowsMin = 2048;

bool lse_two_rows_per_block(const Geometry& g, int dtype, int64_t rows) {
  return !g.stream && g.tpr == 8 * kWave && g.maxit == 8 && dtype >= 0 && dtype != kBF16 &&
         rows >= kLseTwoRowsMin;
}

// 16-bit LayerNorm rows of exactly 2 waves: launches of up to this many rows
// run one row group per workgroup (geometry_for)
constexpr int64_t kLn2WaveRows = 16384;
// Input bytes of current and next rows a CU may hold in flight in the
// unguarded persistent LayerNorm / RMSNorm kernels (16-bit rows that fill
// their row group, one row group per workgroup), at least 2 workgroups per CU,
// where every workgroup still gets kPipeFullMinRows rows.  MI355X, interleaved
// against pipe_grid's 96 KiB rule: LayerNorm bf16 8192 x 8192 5837 -> 5966
// GB/s, 4096 x 8192 5382 -> 5540, 8192 x 5120 5481 -> 5579, fp16 16384 x 8192
// 5956 -> 6118; RMSNorm fp16 8192 x 8192 6091 -> 6167, bf16 4096 x 8192 5768
// -> 5816; but LayerNorm bf16 2048 x 8192 (4 rows per workgroup under the cap)
// 5050 -> 4943, so launches of fewer rows keep the 96 KiB rule.  bf16
// LayerNorm rows of 2 waves take the cap whatever their row count: 4
// workgroups per CU instead of every resident one, +2 to +10% at 2048-16384
// rows.
constexpr int64_t kPipeFullBytesPerCu = int64_t(64) << 10;
constexpr int kPipeFullMinRows = 8;

// `units`: row groups of the launch (see fill_it); `out_bytes`: bytes it
// writes; `column_blocks`: the units are column blocks of longer rows (cross
// entropy with BLOCK_SIZE < n_cols); `dtype`: the input type where a rule
// depends on it (-1: not given).
Geometry geometry_for(int op, int64_t cols, int vec, int64_t units, int64_t out_bytes = 0,
                      bool column_blocks = false, int dtype = -1) {
  const int over = g_flags[op].load();
  int flags = kFlagNontemporal;
  if (over & kFlagNontemporal) flags |= kFlagNontemporal;
  if (over & kFlagTemporal) flags &= ~kFlagNontemporal;
  const bool norm = op == VBH_OP_LAYER_NORM || op == VBH_OP_RMS_NORM;
  if (norm && !(over & kFlagNoPersist)) flags |= kFlagPersist;
  const int64_t nvec = cols / vec;
  Geometry g =
      pick_geometry(cols, vec, fill_it(it_target(op, nvec, vec, column_blocks), nvec, units),
                    g_tpr[op].load(), g_block[op].load(), flags);
  if (g.persist && !(over & kFlagPersist) && g.tpr < kPersistMinTpr[op]) g.persist = false;
  // LayerNorm row groups of exactly 2 waves run 4 to a 512-lane workgroup
  // instead of one per 128-lane workgroup.  MI355X, persistent kernel, default
  // -> 512 lanes: fp32 2048 columns 5314 -> 5558 GB/s at 134 MB per call, bf16
  // 4096 5207 -> 5303, fp32 1536 4161 -> 4414 at 33.6 MB (5416 -> 5386 at 134 MB).
  // Except 16-bit rows that fill the 2 waves exactly, in launches of up to
  // kLn2WaveRows rows: one row group per 128-lane workgroup, where the
  // unguarded persistent kernel runs (it needs a workgroup of one row group),
  // with its cap of rows in flight per CU (kPipeFullBytesPerCu).  MI355X, bf16 4096
  // columns, 512-lane workgroups -> this: 1024 rows 2348 -> 3183 GB/s, 2048
  // 2985 -> 4603, 4096 3982 -> 4934, 8192 4734 -> 5545, 16384 5334 -> 5753;
  // larger launches keep 512 lanes (65536 rows: 5813 against 5118).
  const bool ln_2wave = op == VBH_OP_LAYER_NORM && !g.stream && g.tpr == 2 * kWave &&
                        g_block[op].load() <= 0;
  if (ln_2wave && !(vec == 8 && cols % vec == 0 && cols / vec == int64_t(g.maxit) * g.tpr &&
                    units <= kLn2WaveRows))
    g.block = 8 * kWave;
  // the unguarded persistent kernels (16-bit rows filling a row group that is
  // the whole workgroup: pipe_full in rownorm.hip)
  if (norm && g.persist && vec == 8 && cols % vec == 0 && g.block == g.tpr &&
      cols / vec == int64_t(g.maxit) * g.tpr) {
    g.pipe_bytes = kPipeFullBytesPerCu;
    g.pipe_min_rows = ln_2wave ? 0 : kPipeFullMinRows;
  }
  if (op == VBH_OP_LOGSUMEXP && lse_two_rows_per_block(g, dtype, units) &&
      g_block[op].load() <= 0)
    g.block = 16 * kWave;
  const bool full_output =
      op == VBH_OP_LAYER_NORM || op == VBH_OP_RMS_NORM || op == VBH_OP_SOFTMAX;
  bool wt = full_output && write_through_ok(out_bytes, units);
  if (over & kFlagWriteThrough) wt = true;
  if (over & kFlagNoWriteThrough) wt = false;
  g.wt = g.nt && wt;
  return g;
}

constexpr int64_t kMaxCols = (int64_t(1) << 31) - 1;
constexpr int64_t kMaxWorkItems = (int64_t(1) << 32) - 1;

int check_grid(int64_t units, const Geometry& g) {
  // the row kernels place a lane in its row group with shifts (group_shape),
  // which holds for these shapes only
  const bool shape_ok = g.tpr >= 1 && g.block >= g.tpr && g.block <= kMaxBlock &&
                        g.block % g.tpr == 0 &&
                        (g.tpr <= kWave ? (g.tpr & (g.tpr - 1)) == 0 : g.tpr % kWave == 0);
  if (!shape_ok)
    return fail(VBH_E_INVALID, "internal: launch shape of %d lanes per row, %d per workgroup",
                g.tpr, g.block);
  // every unit takes at least one lane
  if (units > kMaxWorkItems)
    return fail(VBH_E_RANGE, "launch of %lld rows exceeds 2^32 work-items",
                static_cast<long long>(units));
  const int64_t grid = g.stream ? units : grid_for(units, g);
  if (grid * g.block > kMaxWorkItems)
    return fail(VBH_E_RANGE, "launch of %lld workgroups x %d lanes exceeds 2^32 work-items",
                static_cast<long long>(grid), g.block);
  return 0;
}

// A workgroup holds whole row groups: a requested size is rounded down to a
// multiple of tpr (and is at least tpr).  A tpr alone may come from the
// heuristic while the size comes from vbh_tune_override.
int fit_block(int block, int tpr) { return block < tpr ? tpr : block / tpr * tpr; }

// Switch `g` (computed for `vn`-wide vectors) to the MIS kernel, or return
// false when the launch must take the scalar kernel instead.
bool use_mis(Geometry& g, int vn) {
  if (g.stream || g.v != vn || vn == 1) return false;
  g.mis = true;
  if (g.tpr < vn) {  // every head / tail element needs its own lane
    g.tpr = vn;
    g.block = fit_block(g.block, vn);
  }
  return true;
}

// The reduction row kernel streams its row whatever the vectors per lane, so
// its geometry has no register cap: it_target vectors per lane, with more
// lanes per row (a power of two up to 64, then whole waves up to 1024) as the
// row grows (fp16 rows of 4096 vectors: 1024 lanes x 4 at 4.8 TB/s, 512 x 8
// at 6.5 TB/s).
Geometry reduce_geometry(int64_t n, int vec, int64_t units) {
  Geometry g;
  g.v = vec;
  g.nt = true;
  const int64_t nvec = n / vec;
  int tpr = g_tpr[VBH_OP_REDUCE].load();
  if (tpr <= 0) {
    const int per_lane = fill_it(it_target(VBH_OP_REDUCE, nvec, vec, false), nvec, units);
    const int64_t lanes = (nvec + per_lane - 1) / per_lane;
    if (lanes <= kWave) {
      tpr = pow2ceil(lanes < 1 ? 1 : lanes);
    } else {
      const int64_t waves = (lanes + kWave - 1) / kWave;
      tpr = static_cast<int>(waves < kMaxWaves ? waves : kMaxWaves) * kWave;
    }
    // rows of 4097-8192 vectors: 512 lanes at up to 16 vectors each, not 1024
    // at 8 (MI355X, 512 MB per launch: mean fp32 8192 x 32768 +2.9%, argmax
    // fp16 2048 x 65536 +5.4%, max fp32 4096 x 32768 +0.2%; 16384-vector rows
    // keep 1024 lanes, mean fp32 4096 x 65536 -1.7% at 512)
    if (tpr == 16 * kWave && nvec <= 8192) tpr = 8 * kWave;
  }
  int block = g_block[VBH_OP_REDUCE].load();
  // rows of at most 4096 vectors over 512 lanes (8 vectors per lane) run two to
  // a 1024-lane workgroup, as logsumexp's: argmax fp16 4096 / 8192 x 32768
  // +4.4 / +5.1%, fp32 8192 x 16384 +5.3%, bf16 8192 x 32768 +4.4%; mean fp32
  // 16384 x 16384 +3.1%, fp16 8192 x 32768 +2.8%
  if (block <= 0) block = tpr < 128 ? 256 : (tpr == 8 * kWave && nvec <= 4096 ? 16 * kWave : tpr);
  g.tpr = tpr;
  g.block = fit_block(block, tpr);
  return g;
}

}  // namespace

// function_for's cache: per device, an open-addressing table from kernel
// address to hipFunction_t.  Readers probe without a lock (a slot's function is
// stored before its key, with release / acquire ordering); inserts take the mutex.
namespace {
constexpr int kFnDevices = 16;
constexpr int kFnSlots = 2048;  // a power of two, well above the library's kernel count
struct FnSlot {
  std::atomic<const void*> key{nullptr};
  std::atomic<hipFunction_t> fn{nullptr};
};
FnSlot g_fn[kFnDevices][kFnSlots];
std::mutex g_fn_mu;

inline uint64_t fn_hash(const void* k) {
  return (static_cast<uint64_t>(reinterpret_cast<uintptr_t>(k)) >> 4) * 0x9E3779B97F4A7C15ull;
}
}  // namespace

hipFunction_t function_for(const void* kernel) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kFnDevices) return nullptr;
  FnSlot* table = g_fn[dev];
  const uint64_t h = fn_hash(kernel);
  for (int i = 0; i < kFnSlots; ++i) {
    FnSlot& sl = table[(h + i) & (kFnSlots - 1)];
    const void* k = sl.key.load(std::memory_order_acquire);
    if (k == kernel) return sl.fn.load(std::memory_order_relaxed);
    if (k == nullptr) break;
  }
  std::lock_guard<std::mutex> lock(g_fn_mu);
  for (int i = 0; i < kFnSlots; ++i) {
    FnSlot& sl = table[(h + i) & (kFnSlots - 1)];
    const void* k = sl.key.load(std::memory_order_relaxed);
    if (k == kernel) return sl.fn.load(std::memory_order_relaxed);
    if (k == nullptr) {
      hipFunction_t f = nullptr;
      if (hipGetFuncBySymbol(&f, kernel) != hipSuccess || f == nullptr) {
        (void)hipGetLastError();  // the fallback launch reports its own status
        return nullptr;
      }
      sl.fn.store(f, std::memory_order_relaxed);
      sl.key.store(kernel, std::memory_order_release);
      return f;
    }
  }
  return nullptr;  // table full: the runtime's own lookup
}

int64_t resident_blocks(const void* kernel, int block, int max_per_cu) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> per_cu;  // (kernel, block) -> blocks per CU
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cus[dev] = n;
  }
  const uint64_t key = reinterpret_cast<uint64_t>(kernel) ^ (static_cast<uint64_t>(block) << 52);
  auto it = per_cu.find(key);
  int nb;
  if (it != per_cu.end()) {
    nb = it->second;
  } else {
    nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, block, 0) != hipSuccess ||
        nb <= 0)
      nb = 1;
    per_cu.emplace(key, nb);
  }
  return static_cast<int64_t>(std::min(nb, max_per_cu)) * cus[dev];
}

// Input bytes a CU's resident persistent workgroups may hold in flight (each
// row group loads its next row while it reduces the current one), but never
// fewer than 2 workgroups per CU (bf16 LayerNorm 16384 columns, 64 KiB per
// workgroup: 1 lost 4.6% at 2048 rows; fp32 LayerNorm 4608 columns, 36 KiB:
// 3 lost the 13% that 2 gain).  Uncapped,
// small fp32 kernels put 3 workgroups on a CU; capped (MI355X, 64 MB per
// call): fp32 RMSNorm 5120 columns +17.6%, LayerNorm 4608 / 5120 +13%, bf16
// RMSNorm 10240 +10%, bf16 LayerNorm 8192 columns +0.8%, C1 / C5 and the other
// shapes within 0.4%.  A 64 KiB cap starved fp32 LayerNorm (-12%).
constexpr int64_t kPipeBytesPerCu = int64_t(96) << 10;
// Workgroups of fewer lanes keep their full occupancy: at 2 waves each, the
// cap left 12 waves per CU (bf16 LayerNorm 4096 columns -2.7%).
constexpr int kPipeCapMinBlock = 256;

int64_t pipe_grid(const void* kernel, const Geometry& g, int64_t rows, int64_t row_bytes) {
  const int64_t per_block = 2 * (g.block / g.tpr) * row_bytes;  // current + next rows
  const int64_t pb = std::max<int64_t>(per_block, 1);
  if (g.pipe_bytes > 0) {
    const int per_cu = static_cast<int>(std::max<int64_t>(2, g.pipe_bytes / pb));
    const int64_t grid = std::min<int64_t>(grid_for(rows, g),
                                           std::max<int64_t>(resident_blocks(kernel, g.block, per_cu), 1));
    if (rows >= mul_sat(mul_sat(g.pipe_min_rows, grid), g.block / g.tpr)) return grid;
  }
  const int max_per_cu = g.block < kPipeCapMinBlock
                             ? 1 << 30
                             : static_cast<int>(std::max<int64_t>(2, kPipeBytesPerCu / pb));
  const int64_t cap = resident_blocks(kernel, g.block, max_per_cu);
  return std::min<int64_t>(grid_for(rows, g), std::max<int64_t>(cap, 1));
}

Geometry pick_geometry(int64_t cols, int vec, int it_target, int tpr_override,
                       int block_override, int flags) {
  // Rows are held in registers at about `it_target` 16-byte vectors per lane:
  // short rows take a power-of-two slice of one wave, longer ones as many waves
  // as needed (any multiple of 64 lanes, up to 1024), with twice, four times...
  // as many vectors per lane only when 16 waves are not enough.  Beyond the
  // per-lane register budget (lane_cap) the streaming kernels take over.
  Geometry g;
  g.v = vec;
  const int64_t nvec = cols / vec;
  const int cap = lane_cap(vec);
  int tpr = 0;
  if (tpr_override > 0) {
    tpr = tpr_override;
  } else if (nvec <= int64_t(it_target) * kWave) {
    const int64_t lanes = (nvec + it_target - 1) / it_target;
    tpr = pow2ceil(lanes < 1 ? 1 : lanes);
  } else {
    for (int it = it_target; it <= cap; it *= 2) {
      const int64_t waves = (nvec + int64_t(kWave) * it - 1) / (int64_t(kWave) * it);
      if (waves <= kMaxWaves) {
        tpr = static_cast<int>(waves) * kWave;
        break;
      }
    }
  }
  // the store policy follows the op's flags whether or not the row streams
  // (the streaming kernels ignore it; the split softmax's second stage, which
  // takes its policy from the full row's geometry, does not)
  g.nt = (flags & kFlagNontemporal) != 0;
  const int64_t it = tpr > 0 ? (nvec + tpr - 1) / tpr : cap + 1;
  if (it > cap) {
    g.stream = true;
    g.tpr = kMaxBlock;
    g.block = kMaxBlock;
    g.maxit = 1;
    return g;
  }
  g.tpr = tpr;
  g.maxit = pow2ceil(it < 1 ? 1 : it);
  int block;
  if (block_override > 0) block = fit_block(block_override, tpr);
  else block = tpr < 128 ? 256 : tpr;
  g.block = block;
  g.persist = (flags & kFlagPersist) != 0 && g.maxit <= kPipeMaxIt;
  return g;
}

// ---------------------------------------------------------------------------
// Static scratch of vbh_cross_entropy_fwd_noalloc: the split cross entropy's
// segment results (loss, lse, z_loss per segment) for callers that cannot
// allocate device memory.  Each GPU holds its own copy of `scratch` from the
// first use until the process ends.  Host code never passes `scratch` itself
// (in host code the name is a host-side stand-in, not a device address): it
// passes the device address hipGetSymbolAddress returned for the current GPU,
// looked up once per device with that device current.  Calls that overlap on
// one GPU share this memory and race; calls on one stream do not overlap.
// Every call writes the segment results it reads, so nothing must start at zero.
// ---------------------------------------------------------------------------
constexpr int64_t kNoAllocScratchBytes = int64_t(32) << 10;
static_assert(kNoAllocScratchBytes >= 3 * 2 * kSplitTarget * int64_t(sizeof(float)),
              "a split launch has fewer than 2 * kSplitTarget segments of 3 floats");
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {nullptr};

// The current GPU's copy of `scratch` (looked up on first use per device).
static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "noalloc scratch: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(VBH_E_RANGE, "noalloc scratch: device %d beyond the %d the library tracks", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "noalloc scratch: hipGetSymbolAddress");
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) & 255u) != 0)
      return fail(VBH_E_INVALID, "noalloc scratch: symbol address %p not 256-byte aligned", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

#ifdef VBH_DEBUG_BOUNDS
// The debug bounds records of the library's translation units (each registers
// its reader at load time, from its static initialisation; vbh_device.h).
struct BoundsTu {
  const char* file;
  BoundsRecordFn fn;
};
static std::mutex& bounds_mu() {
  static std::mutex mu;
  return mu;
}
static std::vector<BoundsTu>& bounds_tus() {
  static std::vector<BoundsTu> tus;
  return tus;
}
int register_bounds_record(const char* file, BoundsRecordFn fn) {
  std::lock_guard<std::mutex> lock(bounds_mu());
  bounds_tus().push_back(BoundsTu{file, fn});
  return 1;
}
#endif

}  // namespace vbh

using namespace vbh;

extern "C" {

int vbh_abi_version(void) { return VBH_ABI_VERSION; }

const char* vbh_last_error(void) { return g_err; }

int vbh_tune_override(int op, int tpr, int block, int flags) {
  if (op < 0 || op >= kNumOps) return fail(VBH_E_INVALID, "tune_override: bad op %d", op);
  if (tpr != 0 && (tpr < 1 || tpr > kMaxBlock ||
                   (tpr <= kWave ? (tpr & (tpr - 1)) != 0 : tpr % kWave != 0)))
    return fail(VBH_E_INVALID,
                "tune_override: tpr %d is neither a power of two <= 64 nor a multiple of 64 "
                "<= 1024",
                tpr);
  if (block != 0 && (block < kWave || block > kMaxBlock || block % kWave != 0))
    return fail(VBH_E_INVALID, "tune_override: block %d is not a multiple of 64 in [64, 1024]",
                block);
  if (tpr != 0 && block != 0 && block % tpr != 0)
    return fail(VBH_E_INVALID, "tune_override: block %d is not a multiple of tpr %d", block,
                tpr);
  if (flags < 0 || flags > kFlagAll)
    return fail(VBH_E_INVALID, "tune_override: unknown flag bits 0x%x", flags);
  g_tpr[op].store(tpr);
  g_block[op].store(block);
  g_flags[op].store(flags);
  g_err[0] = '\0';
  return 0;
}

int vbh_layer_norm_fwd(const void* x, const void* w, const void* b, void* y, int64_t rows,
                       int64_t cols, float eps, int dtype, int w_dtype, void* stream) {
  if (!is_float(dtype)) return fail(VBH_E_DTYPE, "layer_norm: unsupported dtype %d", dtype);
  if (w_dtype != dtype && w_dtype != kF32)
    return fail(VBH_E_DTYPE, "layer_norm: weight dtype %d must equal x dtype %d or be fp32",
                w_dtype, dtype);
  if (rows < 0 || cols < 0) return fail(VBH_E_INVALID, "layer_norm: negative size");
  if (cols > kMaxCols) return fail(VBH_E_RANGE, "layer_norm: cols %lld too large",
                                   static_cast<long long>(cols));
  if (rows == 0 || cols == 0) return 0;  // empty output
  if (!x || !w || !y) return fail(VBH_E_INVALID, "layer_norm: null pointer");
  const int vn = 16 / elt_size(dtype);
  const bool vec_ok = cols % vn == 0 && aligned16(x) && aligned16(y) && aligned16(w) &&
                      (b == nullptr || aligned16(b));
  // MIS: rows not whole vectors, x / y rows at the same offsets, weights read
  // as aligned vectors and shifted to each row's offset
  const bool mis_ok = cols % vn != 0 && aligned16(x) && aligned16(y) && aligned16(w) &&
                      (b == nullptr || aligned16(b)) && cols >= kMisMinVecs * vn;
  const int64_t out_bytes = mul_sat(mul_sat(rows, cols), elt_size(dtype));
  Geometry g = geometry_for(VBH_OP_LAYER_NORM, cols, vec_ok || mis_ok ? vn : 1, rows, out_bytes);
  if (mis_ok && use_mis(g, vn)) g.persist = false;  // the MIS kernel is one row group per row
  else if (mis_ok) g = geometry_for(VBH_OP_LAYER_NORM, cols, 1, rows, out_bytes);
  if (int rc = check_grid(rows, g)) return rc;
  return hip_status(launch_layer_norm(x, w, b, y, rows, static_cast<int>(cols), eps, dtype,
                                      w_dtype, g, static_cast<hipStream_t>(stream)),
                    "layer_norm launch");
}

int vbh_rms_norm_fwd(const void* x, const void* w, void* y, int64_t rows, int64_t cols,
                     float eps, int dtype, int w_dtype, void* stream) {
  if (!is_float(dtype)) return fail(VBH_E_DTYPE, "rms_norm: unsupported dtype %d", dtype);
  if (w_dtype != dtype && w_dtype != kF32)
    return fail(VBH_E_DTYPE, "rms_norm: weight dtype %d must equal x dtype %d or be fp32",
                w_dtype, dtype);
  if (rows < 0 || cols < 0) return fail(VBH_E_INVALID, "rms_norm: negative size");
  if (cols > kMaxCols) return fail(VBH_E_RANGE, "rms_norm: cols %lld too large",
                                   static_cast<long long>(cols));
  if (rows == 0 || cols == 0) return 0;  // empty output
  if (!x || !w || !y) return fail(VBH_E_INVALID, "rms_norm: null pointer");
  const int vn = 16 / elt_size(dtype);
  const bool vec_ok = cols % vn == 0 && aligned16(x) && aligned16(y) && aligned16(w);
  const bool mis_ok = cols % vn != 0 && aligned16(x) && aligned16(y) && aligned16(w) &&
                      cols >= kMisMinVecs * vn;
  const int64_t out_bytes = mul_sat(mul_sat(rows, cols), elt_size(dtype));
  Geometry g = geometry_for(VBH_OP_RMS_NORM, cols, vec_ok || mis_ok ? vn : 1, rows, out_bytes);
  if (mis_ok && use_mis(g, vn)) g.persist = false;  // the MIS kernel is one row group per row
  else if (mis_ok) g = geometry_for(VBH_OP_RMS_NORM, cols, 1, rows, out_bytes);
  if (int rc = check_grid(rows, g)) return rc;
  return hip_status(launch_rms_norm(x, w, y, rows, static_cast<int>(cols), eps, dtype,
                                    w_dtype, g, static_cast<hipStream_t>(stream)),
                    "rms_norm launch");
}

static bool softmax_pair_ok(int idt, int odt) {
  if (!is_float(idt) || !is_float(odt)) return false;
  return idt == odt || (odt == kF32 && idt != kF32);
}

// The split softmax reads x twice and adds a launch (about 6.5 us for both
// launches of a small split), so it pays only where the unsplit kernel, one
// workgroup per row, is bound by the time one workgroup takes to stream its
// row: few rows, long enough.  MI355X, softmax, unsplit / split time:
//   fp32 8192 columns (2048 vectors) 0.60-0.73 at every row count, 16384
//   columns 0.74-0.91, 32000 1.09-1.18 up to 32 rows and 0.69-0.91 at 64-128,
//   50304 1.38-1.72 up to 32 rows, 1.00 at 64, 0.79 at 128; 65536 1.46-1.75
//   up to 32, 0.99 at 64, 0.91 at 128; 131072 at 128 rows 1.28, 8 rows 3.5;
//   bf16 32000 columns (4000 vectors) 0.93-1.05, 50304 1.36-1.51 up to 32
//   rows, 1.12 at 64, 0.81 at 128; 65536 1.39-1.62 up to 32, 1.19 at 64,
//   0.77 at 128; fp32 200 x 65536 0.77.
bool softmax_split_pays(int64_t rows, int64_t nvec, bool half) {
  if (rows <= 32) return nvec >= 6144;
  if (rows <= 64) return nvec >= (half ? 6144 : 32768);
  if (rows <= 128) return nvec >= 32768;
  return false;
}

// Segments of a split softmax: equal ones for rows of whole vectors, else
// segments of a whole number of vectors with the last one shorter (the MIS
// kernels run them); segs == 1: no split.
RowSplit softmax_split(int64_t rows, int64_t cols, int vn) {
  const int64_t nvec = cols / vn;
  if (!softmax_split_pays(rows, nvec, vn == 8)) return RowSplit{1, cols};
  const bool even = cols % vn == 0;
  const int segs = split_segments(rows, nvec, 0, even, 0);
  if (segs == 1 || even) return RowSplit{segs, cols / segs};
  const int64_t seg_cols = ((cols + segs - 1) / segs + vn - 1) / vn * vn;
  return RowSplit{static_cast<int>((cols + seg_cols - 1) / seg_cols), seg_cols};
}

int64_t vbh_softmax_workspace_bytes(int64_t rows, int64_t cols, int in_dtype) {
  if (!is_float(in_dtype) || rows <= 0 || cols <= 0 || cols > kMaxCols) return 0;
  const int vn = 16 / elt_size(in_dtype);
  if (g_tpr[VBH_OP_SOFTMAX].load() || g_block[VBH_OP_SOFTMAX].load()) return 0;
  const RowSplit sp = softmax_split(rows, cols, vn);
  // one SegPair (two fp32 values) per segment
  return sp.segs > 1 ? rows * sp.segs * 2 * static_cast<int64_t>(sizeof(float)) : 0;
}

int vbh_softmax_fwd_ws(const void* x, void* y, int64_t rows, int64_t cols, int in_dtype,
                       int out_dtype, int log_mode, void* workspace, int64_t workspace_bytes,
                       void* stream) {
  if (!softmax_pair_ok(in_dtype, out_dtype))
    return fail(VBH_E_DTYPE, "softmax: unsupported (in, out) dtype pair (%d, %d)", in_dtype,
                out_dtype);
  if (log_mode != 0 && log_mode != 1)
    return fail(VBH_E_INVALID, "softmax: log_mode must be 0 or 1");
  if (rows < 0 || cols < 0) return fail(VBH_E_INVALID, "softmax: negative size");
  if (cols > kMaxCols) return fail(VBH_E_RANGE, "softmax: cols %lld too large",
                                   static_cast<long long>(cols));
  if (workspace_bytes < 0) return fail(VBH_E_INVALID, "softmax: negative workspace size");
  if (rows == 0 || cols == 0) return 0;
  if (!x || !y) return fail(VBH_E_INVALID, "softmax: null pointer");
  const int vn = 16 / elt_size(in_dtype);
  const bool aligned = aligned16(x) && aligned16(y);
  const bool vec_ok = cols % vn == 0 && aligned;
  const bool mis_ok = !vec_ok && aligned && cols >= kMisMinVecs * vn;
  const int64_t out_bytes = mul_sat(mul_sat(rows, cols), elt_size(out_dtype));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t need = vbh_softmax_workspace_bytes(rows, cols, in_dtype);
  if (need > 0 && (vec_ok || mis_ok) && workspace != nullptr && workspace_bytes >= need &&
      aligned16(workspace)) {
    // segment SegPairs (fp32 max, sum of exp): the [rows * segs, cols / segs]
    // view, or the MIS kernel's segment mode; then one pass over x that
    // combines each row's segments and writes y
    const RowSplit sp = softmax_split(rows, cols, vn);
    const int segs = sp.segs;
    const int64_t units = rows * segs;
    const int seg_cols = static_cast<int>(sp.seg_cols);
    Geometry g1 = geometry_for(VBH_OP_LOGSUMEXP, seg_cols, vn, units);
    Geometry g2 = geometry_for(VBH_OP_SOFTMAX, cols, vn, rows, out_bytes);  // nt / wt
    g2.mis = !vec_ok;
    if (vec_ok || use_mis(g1, vn)) {
      if (int rc = check_grid(units, g1)) return rc;
      float* seg_pairs = static_cast<float*>(workspace);
      hipError_t e =
          vec_ok ? launch_logsumexp_pairs(x, seg_pairs, units, seg_cols, in_dtype, g1, s)
                 : launch_logsumexp_pairs(x, seg_pairs, units, static_cast<int>(cols), in_dtype,
                                          g1, s, segs, seg_cols);
      if (e == hipSuccess)
        e = launch_softmax_apply(x, y, seg_pairs, rows, static_cast<int>(cols), segs, in_dtype,
                                 out_dtype, log_mode, g2, s);
      return hip_status(e, "softmax launch");
    }
  }
  Geometry g = geometry_for(VBH_OP_SOFTMAX, cols, vec_ok || mis_ok ? vn : 1, rows, out_bytes);
  if (mis_ok && !use_mis(g, vn)) g = geometry_for(VBH_OP_SOFTMAX, cols, 1, rows, out_bytes);
  if (int rc = check_grid(rows, g)) return rc;
  return hip_status(launch_softmax(x, y, rows, static_cast<int>(cols), in_dtype, out_dtype,
                                   log_mode, g, s),
                    "softmax launch");
}

int vbh_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols, int in_dtype,
                    int out_dtype, int log_mode, void* stream) {
  return vbh_softmax_fwd_ws(x, y, rows, cols, in_dtype, out_dtype, log_mode, nullptr, 0,
                            stream);
}

int vbh_softmax_dim_fwd(const void* x, void* y, int64_t outer, int64_t n, int64_t inner,
                        int in_dtype, int out_dtype, int log_mode, void* stream) {
  if (!softmax_pair_ok(in_dtype, out_dtype))
    return fail(VBH_E_DTYPE, "softmax_dim: unsupported (in, out) dtype pair (%d, %d)",
                in_dtype, out_dtype);
  if (log_mode != 0 && log_mode != 1)
    return fail(VBH_E_INVALID, "softmax_dim: log_mode must be 0 or 1");
  if (outer < 0 || n < 0 || inner < 0) return fail(VBH_E_INVALID, "softmax_dim: negative size");
  if (n > kMaxCols) return fail(VBH_E_RANGE, "softmax_dim: n too large");
  if (outer == 0 || n == 0 || inner == 0) return 0;
  if (!x || !y) return fail(VBH_E_INVALID, "softmax_dim: null pointer");
  if (mul_sat(outer, inner) > kMaxWorkItems / 256 * 256)
    return fail(VBH_E_RANGE, "softmax_dim: outer * inner too large");
  return hip_status(launch_softmax_dim(x, y, outer, static_cast<int>(n), inner, in_dtype,
                                       out_dtype, log_mode, static_cast<hipStream_t>(stream)),
                    "softmax_dim launch");
}

int64_t vbh_logsumexp_workspace_bytes(int64_t rows, int64_t cols, int in_dtype) {
  if (!is_float(in_dtype) || rows <= 0 || cols <= 0 || cols > kMaxCols) return 0;
  const int vn = 16 / elt_size(in_dtype);
  if (g_tpr[VBH_OP_LOGSUMEXP].load() || g_block[VBH_OP_LOGSUMEXP].load()) return 0;
  const RowSplit sp = split_row(rows, cols, vn, kSplitMaxRows);
  // one SegPair (two fp32 values) per segment
  return sp.segs > 1 ? rows * sp.segs * 2 * static_cast<int64_t>(sizeof(float)) : 0;
}

int vbh_logsumexp_fwd_ws(const void* x, void* y, int64_t rows, int64_t cols, int in_dtype,
                         int out_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!softmax_pair_ok(in_dtype, out_dtype))
    return fail(VBH_E_DTYPE, "logsumexp: unsupported (in, out) dtype pair (%d, %d)", in_dtype,
                out_dtype);
  if (rows < 0 || cols < 0) return fail(VBH_E_INVALID, "logsumexp: negative size");
  if (workspace_bytes < 0) return fail(VBH_E_INVALID, "logsumexp: negative workspace size");
  if (cols > kMaxCols) return fail(VBH_E_RANGE, "logsumexp: cols %lld too large",
                                   static_cast<long long>(cols));
  if (rows == 0) return 0;
  // cols == 0 is valid: every row reduces an empty set and gets -inf (x unread)
  if ((!x && cols > 0) || !y) return fail(VBH_E_INVALID, "logsumexp: null pointer");
  const int vn = 16 / elt_size(in_dtype);
  const bool vec_ok = cols % vn == 0 && aligned16(x);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t need = vbh_logsumexp_workspace_bytes(rows, cols, in_dtype);
  if (need > 0 && aligned16(x) && workspace != nullptr && workspace_bytes >= need &&
      aligned16(workspace)) {
    // segment SegPairs in fp32, then each row's combined from them; rows of
    // whole vectors as a [rows * segs, seg_cols] view, other rows through the
    // MIS kernel's segment mode
    const RowSplit sp = split_row(rows, cols, vn, kSplitMaxRows);
    const int segs = sp.segs;
    const int64_t units = rows * segs;
    const int seg_cols = static_cast<int>(sp.seg_cols);
    Geometry g1 = geometry_for(VBH_OP_LOGSUMEXP, seg_cols, vn, units);
    if (vec_ok || use_mis(g1, vn)) {
      if (int rc = check_grid(units, g1)) return rc;
      float* pairs = static_cast<float*>(workspace);
      hipError_t e =
          vec_ok ? launch_logsumexp_pairs(x, pairs, units, seg_cols, in_dtype, g1, s)
                 : launch_logsumexp_pairs(x, pairs, units, static_cast<int>(cols), in_dtype, g1,
                                          s, segs, seg_cols);
      if (e == hipSuccess) e = launch_logsumexp_combine(pairs, y, rows, segs, out_dtype, s);
      return hip_status(e, "logsumexp launch");
    }
  }
  const bool mis_ok = !vec_ok && aligned16(x) && cols >= kMisMinVecs * vn;
  Geometry g =
      geometry_for(VBH_OP_LOGSUMEXP, cols, vec_ok || mis_ok ? vn : 1, rows, 0, false, in_dtype);
  if (mis_ok && !use_mis(g, vn)) g = geometry_for(VBH_OP_LOGSUMEXP, cols, 1, rows);
  if (int rc = check_grid(rows, g)) return rc;
  return hip_status(launch_logsumexp(x, y, rows, static_cast<int>(cols), in_dtype, out_dtype,
                                     g, s),
                    "logsumexp launch");
}

int vbh_logsumexp_fwd(const void* x, void* y, int64_t rows, int64_t cols, int in_dtype,
                      int out_dtype, void* stream) {
  return vbh_logsumexp_fwd_ws(x, y, rows, cols, in_dtype, out_dtype, nullptr, 0, stream);
}

int64_t vbh_cross_entropy_workspace_bytes(int64_t n_rows, int64_t n_cols, int64_t block_size,
                                          int logits_dtype) {
  if (!is_float(logits_dtype) || n_rows <= 0 || n_cols <= 0 || n_cols > (int64_t(1) << 30) ||
      block_size < n_cols)  // one column block per row only
    return 0;
  const int vn = 16 / elt_size(logits_dtype);
  if (g_tpr[VBH_OP_CROSS_ENTROPY].load() || g_block[VBH_OP_CROSS_ENTROPY].load()) return 0;
  const RowSplit sp = split_row(n_rows, n_cols, vn, kSplitMaxRows + 1);
  // segment loss, lse and (unused) z_loss
  return sp.segs > 1 ? 3 * n_rows * sp.segs * static_cast<int64_t>(sizeof(float)) : 0;
}

int vbh_cross_entropy_fwd_ws(const void* logits, const void* labels, int logits_dtype,
                             int label_dtype, void* loss, void* lse, void* z_loss,
                             int64_t n_rows, int64_t n_cols, int64_t row_stride, float smoothing,
                             float logit_scale, float lse_square_scale, int64_t ignored_index,
                             int64_t total_classes, int64_t class_start_idx, int64_t block_size,
                             int has_smoothing, int split, void* workspace,
                             int64_t workspace_bytes, void* stream) {
  if (!is_float(logits_dtype))
    return fail(VBH_E_DTYPE, "cross_entropy_fwd: unsupported logits dtype %d", logits_dtype);
  if (label_dtype != kI32 && label_dtype != kI64)
    return fail(VBH_E_DTYPE, "cross_entropy_fwd: labels must be int32 or int64");
  if (n_rows < 0 || n_cols < 0) return fail(VBH_E_INVALID, "cross_entropy_fwd: negative size");
  if (block_size <= 0) return fail(VBH_E_INVALID, "cross_entropy_fwd: BLOCK_SIZE must be > 0");
  if (workspace_bytes < 0)
    return fail(VBH_E_INVALID, "cross_entropy_fwd: negative workspace size");
  if (n_cols > (int64_t(1) << 30))
    return fail(VBH_E_RANGE, "cross_entropy_fwd: n_cols too large");
  if (row_stride < n_cols) return fail(VBH_E_INVALID, "cross_entropy_fwd: row_stride < n_cols");
  if (n_rows == 0 || n_cols == 0) return 0;
  if (!logits || !labels || !loss || !lse || !z_loss)
    return fail(VBH_E_INVALID, "cross_entropy_fwd: null pointer");
  const int64_t bs = block_size < n_cols ? block_size : n_cols;
  const int64_t ncb = (n_cols + block_size - 1) / block_size;
  const int vn = 16 / elt_size(logits_dtype);
  const bool vec_ok =
      n_cols % vn == 0 && bs % vn == 0 && row_stride % vn == 0 && aligned16(logits);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  CeArgs a;
  a.logits = logits;
  a.labels = labels;
  a.logits_dt = logits_dtype;
  a.label_i64 = label_dtype == kI64;
  a.loss = static_cast<float*>(loss);
  a.lse = static_cast<float*>(lse);
  a.z_loss = static_cast<float*>(z_loss);
  a.n_rows = n_rows;
  a.n_cols = static_cast<int>(n_cols);
  a.ld = row_stride;
  a.block_size = static_cast<int>(bs);
  a.ncb = static_cast<int>(ncb);
  a.smoothing = smoothing;
  a.logit_scale = logit_scale;
  a.lse_square_scale = lse_square_scale;
  a.ignored_index = ignored_index;
  a.total_classes = static_cast<float>(total_classes);
  a.class_start = class_start_idx;
  a.has_smoothing = has_smoothing != 0;
  a.split = split != 0;
  const int64_t need =
      vbh_cross_entropy_workspace_bytes(n_rows, n_cols, block_size, logits_dtype);
  if (need > 0 && aligned16(logits) && workspace != nullptr && workspace_bytes >= need &&
      aligned16(workspace)) {
    // first stage: the row's segments as column blocks with SPLIT semantics
    // (the MIS kernel where a segment does not start at a vector boundary)
    const RowSplit sp = split_row(n_rows, n_cols, vn, kSplitMaxRows + 1);
    const int segs = sp.segs;
    const int64_t units = n_rows * segs;
    Geometry g1 = geometry_for(VBH_OP_CROSS_ENTROPY, sp.seg_cols, vn, units);
    if (vec_ok || use_mis(g1, vn)) {
      if (int rc = check_grid(units, g1)) return rc;
      CeArgs p = a;
      p.loss = static_cast<float*>(workspace);
      p.lse = p.loss + units;
      p.z_loss = p.lse + units;
      p.block_size = static_cast<int>(sp.seg_cols);
      p.ncb = segs;
      p.split = 1;
      p.empty_neg_inf = 1;
      p.pair_out = 1;
      hipError_t e = launch_cross_entropy_fwd(p, g1, s);
      if (e == hipSuccess) e = launch_cross_entropy_combine(a, p.loss, p.lse, p.z_loss, segs, s);
      return hip_status(e, "cross_entropy_fwd launch");
    }
  }
  const int64_t segments = mul_sat(n_rows, ncb);
  // the persistent forward (one workgroup per CU walking the rows chunk by
  // chunk): fp32 rows of one column block and at least one chunk; by default
  // in launches of at least kCePersistMinRows rows of kCePersistMinChunks
  // chunks or more, its workgroup size the launcher's choice.  kFlagPersist
  // lifts those two limits, and with it a block override of 256 or 512 sets
  // the workgroup size; kFlagNoPersist, a tpr override or another block
  // override keeps ce_fwd_rows.
  const int over = g_flags[VBH_OP_CROSS_ENTROPY].load();
  const int ce_block = g_block[VBH_OP_CROSS_ENTROPY].load();
  const bool ce_lanes_ok =
      ce_block <= 0 || ((over & kFlagPersist) && (ce_block == 256 || ce_block == 512));
  if (vec_ok && ncb == 1 && cross_entropy_fwd_persist_fits(logits_dtype, n_cols) &&
      g_tpr[VBH_OP_CROSS_ENTROPY].load() <= 0 && ce_lanes_ok && !(over & kFlagNoPersist) &&
      ((over & kFlagPersist) ||
       (n_rows >= kCePersistMinRows &&
        n_cols >= kCePersistMinChunks * cross_entropy_fwd_persist_chunk_cols())))
    return hip_status(launch_cross_entropy_fwd_persist(a, 0, ce_block > 0 ? ce_block : 0, s),
                      "cross_entropy_fwd launch");
  const bool mis_ok = !vec_ok && aligned16(logits) && bs >= kMisMinVecs * vn;
  Geometry g = geometry_for(VBH_OP_CROSS_ENTROPY, bs, vec_ok || mis_ok ? vn : 1, segments, 0,
                            ncb > 1);
  if (mis_ok && !use_mis(g, vn))
    g = geometry_for(VBH_OP_CROSS_ENTROPY, bs, 1, segments, 0, ncb > 1);
  if (int rc = check_grid(segments, g)) return rc;
  return hip_status(launch_cross_entropy_fwd(a, g, s), "cross_entropy_fwd launch");
}

int vbh_cross_entropy_fwd(const void* logits, const void* labels, int logits_dtype,
                          int label_dtype, void* loss, void* lse, void* z_loss,
                          int64_t n_rows, int64_t n_cols, int64_t row_stride, float smoothing,
                          float logit_scale, float lse_square_scale, int64_t ignored_index,
                          int64_t total_classes, int64_t class_start_idx, int64_t block_size,
                          int has_smoothing, int split, void* stream) {
  return vbh_cross_entropy_fwd_ws(logits, labels, logits_dtype, label_dtype, loss, lse, z_loss,
                                  n_rows, n_cols, row_stride, smoothing, logit_scale,
                                  lse_square_scale, ignored_index, total_classes,
                                  class_start_idx, block_size, has_smoothing, split, nullptr, 0,
                                  stream);
}

int vbh_cross_entropy_fwd_noalloc(const void* logits, const void* labels, int logits_dtype,
                                  int label_dtype, void* loss, void* lse, void* z_loss,
                                  int64_t n_rows, int64_t n_cols, int64_t row_stride,
                                  float smoothing, float logit_scale, float lse_square_scale,
                                  int64_t ignored_index, int64_t total_classes,
                                  int64_t class_start_idx, int64_t block_size, int has_smoothing,
                                  int split, void* stream) {
  const int64_t need =
      vbh_cross_entropy_workspace_bytes(n_rows, n_cols, block_size, logits_dtype);
  if (need > kNoAllocScratchBytes)
    return fail(VBH_E_RANGE,
                "cross_entropy_fwd_noalloc: the row split needs %lld bytes of scratch, more than "
                "the %lld bytes of the library's static scratch",
                static_cast<long long>(need), static_cast<long long>(kNoAllocScratchBytes));
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = noalloc_scratch(&ws)) return rc;
  }
  return vbh_cross_entropy_fwd_ws(logits, labels, logits_dtype, label_dtype, loss, lse, z_loss,
                                  n_rows, n_cols, row_stride, smoothing, logit_scale,
                                  lse_square_scale, ignored_index, total_classes,
                                  class_start_idx, block_size, has_smoothing, split, ws, need,
                                  stream);
}

int vbh_cross_entropy_bwd(const void* dloss, const void* logits, const void* lse,
                          const void* labels, void* dlogits, int logits_dtype,
                          int label_dtype, int64_t n_rows, int64_t n_cols,
                          int64_t logits_row_stride, int64_t dlogits_row_stride,
                          int64_t dloss_stride, float smoothing, float logit_scale,
                          float lse_square_scale, int64_t ignored_index, int64_t total_classes,
                          int64_t class_start_idx, int has_smoothing, void* stream) {
  if (!is_float(logits_dtype))
    return fail(VBH_E_DTYPE, "cross_entropy_bwd: unsupported logits dtype %d", logits_dtype);
  if (label_dtype != kI32 && label_dtype != kI64)
    return fail(VBH_E_DTYPE, "cross_entropy_bwd: labels must be int32 or int64");
  if (n_rows < 0 || n_cols < 0) return fail(VBH_E_INVALID, "cross_entropy_bwd: negative size");
  if (n_cols > kMaxCols) return fail(VBH_E_RANGE, "cross_entropy_bwd: n_cols too large");
  if (logits_row_stride < n_cols || dlogits_row_stride < n_cols || dloss_stride < 0)
    return fail(VBH_E_INVALID, "cross_entropy_bwd: bad stride");
  if (n_rows == 0 || n_cols == 0) return 0;
  if (!dloss || !logits || !lse || !labels || !dlogits)
    return fail(VBH_E_INVALID, "cross_entropy_bwd: null pointer");
  const int vn = 16 / elt_size(logits_dtype);
  const bool vec_ok = n_cols % vn == 0 && logits_row_stride % vn == 0 &&
                      dlogits_row_stride % vn == 0 && aligned16(logits) && aligned16(dlogits);
  // MIS: every logits and dlogits row starts at the same offset within a vector
  const bool mis_ok = !vec_ok && aligned16(logits) && aligned16(dlogits) &&
                      logits_row_stride == dlogits_row_stride && n_cols >= kMisMinVecs * vn;
  const int64_t tiles =
      (n_cols / (vec_ok || mis_ok ? vn : 1) + kCeBwdLanes - 1) / kCeBwdLanes;
  if (n_rows > kMaxWorkItems / (tiles * kCeBwdLanes))
    return fail(VBH_E_RANGE, "cross_entropy_bwd: %lld x %lld elements exceed one launch",
                static_cast<long long>(n_rows), static_cast<long long>(n_cols));
  CeBwdArgs a;
  a.dloss = static_cast<const float*>(dloss);
  a.logits = logits;
  a.lse = static_cast<const float*>(lse);
  a.labels = labels;
  a.dlogits = dlogits;
  a.logits_dt = logits_dtype;
  a.label_i64 = label_dtype == kI64;
  a.n_rows = n_rows;
  a.n_cols = static_cast<int>(n_cols);
  a.ld_logits = logits_row_stride;
  a.ld_dlogits = dlogits_row_stride;
  a.dloss_stride = dloss_stride;
  a.smoothing = smoothing;
  a.logit_scale = logit_scale;
  a.lse_square_scale = lse_square_scale;
  a.ignored_index = ignored_index;
  a.total_classes = static_cast<float>(total_classes);
  a.class_start = class_start_idx;
  a.has_smoothing = has_smoothing != 0;
  a.vec = vec_ok || mis_ok ? vn : 1;
  a.mis = mis_ok;
  // store policy: the cross-entropy op's tune flags, else nontemporal, and
  // written through the L2 from kWriteThroughMinBytes of dlogits in whole lines
  const int over = g_flags[VBH_OP_CROSS_ENTROPY].load();
  a.nt = !(over & kFlagTemporal);
  bool wt = write_through_ok(mul_sat(mul_sat(n_rows, n_cols), elt_size(logits_dtype)), n_rows) &&
            dlogits_row_stride == n_cols;
  if (over & kFlagWriteThrough) wt = true;
  if (over & kFlagNoWriteThrough) wt = false;
  a.wt = a.nt && wt;
  return hip_status(launch_cross_entropy_bwd(a, static_cast<hipStream_t>(stream)),
                    "cross_entropy_bwd launch");
}

// Split reductions keep, per segment, an fp32 mean, or an int64 index followed
// (after all indices) by a value of the input type.
int64_t split_entry_bytes(int op, int in_dtype) {
  return op == 0 ? static_cast<int64_t>(sizeof(float)) : 8 + elt_size(in_dtype);
}

int64_t vbh_reduce_workspace_bytes(int64_t outer, int64_t n, int64_t inner, int in_dtype,
                                   int op) {
  if (op < 0 || op > 2 || !is_float(in_dtype) || inner != 1 || outer <= 0 || n <= 0 ||
      n > kMaxCols)
    return 0;
  const int vn = 16 / elt_size(in_dtype);
  if (n % vn != 0 || g_tpr[VBH_OP_REDUCE].load() || g_block[VBH_OP_REDUCE].load()) return 0;
  const int segs = split_segments(outer, n / vn);
  return segs > 1 ? outer * segs * split_entry_bytes(op, in_dtype) : 0;
}

int vbh_reduce_fwd_ws(const void* x, void* values, void* indices, int64_t outer, int64_t n,
                      int64_t inner, int in_dtype, int out_dtype, int op, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  if (op < 0 || op > 2) return fail(VBH_E_INVALID, "reduce: unknown op %d", op);
  if (!is_float(in_dtype)) return fail(VBH_E_DTYPE, "reduce: unsupported dtype %d", in_dtype);
  if (op == 0 ? !(out_dtype == in_dtype || (out_dtype == kF32 && in_dtype != kF32))
              : out_dtype != in_dtype)
    return fail(VBH_E_DTYPE, "reduce: unsupported (in, out) dtype pair (%d, %d)", in_dtype,
                out_dtype);
  if (outer < 0 || n < 0 || inner < 0) return fail(VBH_E_INVALID, "reduce: negative size");
  if (workspace_bytes < 0) return fail(VBH_E_INVALID, "reduce: negative workspace size");
  if (n > kMaxCols) return fail(VBH_E_RANGE, "reduce: n too large");
  if (outer == 0 || inner == 0) return 0;
  if (n == 0 && op != 0) return fail(VBH_E_INVALID, "reduce: max / argmax of an empty axis");
  if ((!x && n > 0) || (op != 2 && !values) || (op != 0 && !indices))
    return fail(VBH_E_INVALID, "reduce: null pointer");
  const hipStream_t s = static_cast<hipStream_t>(stream);
  int64_t* idx = static_cast<int64_t*>(indices);
  Geometry g;
  if (inner == 1) {
    const int vn = 16 / elt_size(in_dtype);
    const bool vec_ok = n % vn == 0 && aligned16(x);
    const int64_t need = vbh_reduce_workspace_bytes(outer, n, inner, in_dtype, op);
    if (need > 0 && vec_ok && workspace != nullptr && workspace_bytes >= need &&
        aligned16(workspace)) {
      const int segs = split_segments(outer, n / vn);
      const int64_t units = outer * segs;
      const int seg_n = static_cast<int>(n / segs);
      const Geometry g1 = reduce_geometry(seg_n, vn, units);
      if (int rc = check_grid(units, g1)) return rc;
      hipError_t e;
      if (op == 0) {
        // segment means in fp32 (equal segments: their mean is the row's mean)
        float* means = static_cast<float*>(workspace);
        const Geometry g2 = reduce_geometry(segs, segs % 4 == 0 ? 4 : 1, outer);
        if (int rc = check_grid(outer, g2)) return rc;
        e = launch_reduce(x, means, nullptr, units, seg_n, 1, in_dtype, kF32, 0, g1, s);
        if (e == hipSuccess)
          e = launch_reduce(means, values, nullptr, outer, segs, 1, kF32, out_dtype, 0, g2, s);
      } else {
        // segment (value, index) results, then the first maximal one per row
        int64_t* pidx = static_cast<int64_t*>(workspace);
        void* pvals = pidx + units;
        e = launch_reduce(x, pvals, pidx, units, seg_n, 1, in_dtype, in_dtype, 1, g1, s);
        if (e == hipSuccess)
          e = launch_reduce_combine(pvals, pidx, values, idx, outer, segs, seg_n, in_dtype, op,
                                    s);
      }
      return hip_status(e, "reduce launch");
    }
    const bool mis_ok = !vec_ok && aligned16(x) && n >= kMisMinVecs * vn;
    g = reduce_geometry(n, vec_ok || mis_ok ? vn : 1, outer);
    if (mis_ok && !use_mis(g, vn)) g = reduce_geometry(n, 1, outer);
    if (int rc = check_grid(outer, g)) return rc;
  } else if (mul_sat(outer, inner) > kMaxWorkItems / 256 * 256) {
    return fail(VBH_E_RANGE, "reduce: outer * inner too large");
  }
  return hip_status(launch_reduce(x, values, idx, outer, static_cast<int>(n), inner, in_dtype,
                                  out_dtype, op, g, s),
                    "reduce launch");
}

int vbh_reduce_fwd(const void* x, void* values, void* indices, int64_t outer, int64_t n,
                   int64_t inner, int in_dtype, int out_dtype, int op, void* stream) {
  return vbh_reduce_fwd_ws(x, values, indices, outer, n, inner, in_dtype, out_dtype, op, nullptr,
                           0, stream);
}

int vbh_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes < 0 || bytes % 16 != 0)
    return fail(VBH_E_INVALID, "stream_copy: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return 0;
  if (bytes / 16 > kMaxWorkItems) return fail(VBH_E_RANGE, "stream_copy: more than 64 GiB");
  if (!src || !dst || !aligned16(src) || !aligned16(dst))
    return fail(VBH_E_INVALID, "stream_copy: pointers must be non-null and 16-byte aligned");
  return hip_status(launch_stream_copy(src, dst, bytes, static_cast<hipStream_t>(stream)),
                    "stream_copy launch");
}

// The read yardstick's persistent grid: one workgroup per CU, never more than
// the read has tiles, and at most kReadMaxGrid (the partial buffer's size does
// not depend on the device).
constexpr int64_t kReadMaxGrid = 4096;

int64_t vbh_stream_read_partial_bytes(int64_t bytes) {
  if (bytes <= 0 || bytes % 16 != 0 || bytes / 16 > kMaxWorkItems) return 0;
  return 4 * std::min(stream_read_tiles(bytes), kReadMaxGrid);
}

int vbh_stream_read(const void* src, int64_t bytes, void* partial, int64_t partial_bytes,
                    void* stream) {
  if (bytes < 0 || bytes % 16 != 0)
    return fail(VBH_E_INVALID, "stream_read: bytes must be a non-negative multiple of 16");
  if (bytes == 0) return 0;
  if (bytes / 16 > kMaxWorkItems) return fail(VBH_E_RANGE, "stream_read: more than 64 GiB");
  if (!src || !aligned16(src) || !partial || (reinterpret_cast<uintptr_t>(partial) & 3u) != 0)
    return fail(VBH_E_INVALID,
                "stream_read: src must be non-null and 16-byte aligned, partial non-null and "
                "4-byte aligned");
  const int64_t need = vbh_stream_read_partial_bytes(bytes);
  if (partial_bytes < need)
    return fail(VBH_E_INVALID, "stream_read: partial holds %lld bytes, %lld needed",
                static_cast<long long>(partial_bytes), static_cast<long long>(need));
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int grid = static_cast<int>(std::min<int64_t>(
      {static_cast<int64_t>(cus), stream_read_tiles(bytes), kReadMaxGrid}));
  return hip_status(
      launch_stream_read(src, partial, bytes, grid, static_cast<hipStream_t>(stream)),
      "stream_read launch");
}

int vbh_debug_bounds(int64_t* failed, char* where, int64_t where_len, int clear) {
#ifndef VBH_DEBUG_BOUNDS
  (void)failed, (void)where, (void)where_len, (void)clear;
  return fail(VBH_E_UNSUPPORTED,
              "debug_bounds: this library was built without VBH_DEBUG_BOUNDS "
              "(libvbhip_debug.so is the bounds-checked build)");
#else
  if (failed == nullptr) return fail(VBH_E_INVALID, "debug_bounds: null count pointer");
  if (where != nullptr && where_len > 0) where[0] = '\0';
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_status(e, "debug_bounds: hipDeviceSynchronize");
  std::lock_guard<std::mutex> lock(bounds_mu());
  int64_t total = 0;
  for (const BoundsTu& tu : bounds_tus()) {
    unsigned n = 0, line = 0;
    e = tu.fn(&n, &line, nullptr, clear != 0);
    if (e != hipSuccess) return hip_status(e, "debug_bounds: reading a record");
    if (n != 0 && total == 0 && where != nullptr && where_len > 0) {
      const char* base = strrchr(tu.file, '/');
      snprintf(where, static_cast<size_t>(std::min<int64_t>(where_len, 1 << 20)), "%s:%u",
               base != nullptr ? base + 1 : tu.file, line);
    }
    total += n;
  }
  *failed = total;
  return hip_status(hipSuccess, "");
#endif
}

int vbh_debug_bounds_slack(int64_t bytes) {
#ifndef VBH_DEBUG_BOUNDS
  (void)bytes;
  return fail(VBH_E_UNSUPPORTED,
              "debug_bounds_slack: this library was built without VBH_DEBUG_BOUNDS");
#else
  if (bytes < 0) return fail(VBH_E_INVALID, "debug_bounds_slack: negative byte count");
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_status(e, "debug_bounds_slack: hipDeviceSynchronize");
  std::lock_guard<std::mutex> lock(bounds_mu());
  const long long slack = static_cast<long long>(bytes);
  for (const BoundsTu& tu : bounds_tus()) {
    unsigned n = 0, line = 0;
    e = tu.fn(&n, &line, &slack, false);
    if (e != hipSuccess) return hip_status(e, "debug_bounds_slack: setting a slack");
  }
  return hip_status(hipSuccess, "");
#endif
}

}  // extern "C"

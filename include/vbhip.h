/*
 * vbhip.h - C ABI of libvbhip.so, the MI355X (gfx950) HIP backend for ViperBench's
 * normalization / row-reduction family.
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are caller-owned device pointers; the library never
 *     allocates device memory and never synchronizes the host.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the default stream).
 *   - Return value 0 = success.  A negative value is an argument error
 *     (VBH_E_*); a positive value is the hipError_t reported by the runtime.
 *     In both cases vbh_last_error() returns a thread-local message.
 *   - Tensors are row-major with unit stride along the reduced (last) axis.
 *     `rows` is the product of all leading dimensions, `cols` the reduced length.
 *   - Element types are selected by VBH_DTYPE_* codes.  Arithmetic is fp32.
 *
 * Each function below names the reference interface it stands in for
 * (paths relative to the tingxi-li/DSLPerfGap checkout).
 */
#ifndef VBHIP_H
#define VBHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VBH_ABI_VERSION 1

/* element type codes */
#define VBH_DTYPE_F32 0
#define VBH_DTYPE_F16 1
#define VBH_DTYPE_BF16 2
#define VBH_DTYPE_I32 3
#define VBH_DTYPE_I64 4

/* argument-error codes (negative) */
#define VBH_E_INVALID (-1)   /* bad size, null pointer, bad flag            */
#define VBH_E_DTYPE (-2)     /* unsupported dtype or dtype combination       */
#define VBH_E_RANGE (-3)     /* size beyond what the kernels index (2^31-1)  */
#define VBH_E_UNSUPPORTED (-4) /* not available in this build of the library */

/* operation codes for vbh_tune_override */
#define VBH_OP_LAYER_NORM 0
#define VBH_OP_RMS_NORM 1
#define VBH_OP_SOFTMAX 2
#define VBH_OP_LOGSUMEXP 3
#define VBH_OP_CROSS_ENTROPY 4
#define VBH_OP_REDUCE 5

/* reduction codes for vbh_reduce_fwd */
#define VBH_REDUCE_MEAN 0
#define VBH_REDUCE_MAX 1
#define VBH_REDUCE_ARGMAX 2

int vbh_abi_version(void);
const char* vbh_last_error(void);

/* LayerNorm forward over the last axis: y = (x - mean) / sqrt(var + eps) * w + b,
 * biased variance.  x, y: [rows, cols] of `dtype`; w, b: [cols] of `w_dtype`
 * (either `dtype` or F32); b may be NULL (no bias).
 * Replaces: ViperBench/layer_norm/pytorch_impl.py:5-12 (F.layer_norm golden),
 *           ViperBench/layer_norm/triton_impl.py:101-137,
 *           ViperBench/layer_norm/tilelang_impl.py:64-80. */
int vbh_layer_norm_fwd(const void* x, const void* w, const void* b, void* y,
                       int64_t rows, int64_t cols, float eps,
                       int dtype, int w_dtype, void* stream);

/* RMSNorm forward: y = (x / sqrt(mean(x^2) + eps)) * w, computed in fp32 and
 * rounded to `dtype`.  x, y: [rows, cols] of `dtype`; w: [cols] of `w_dtype`.
 * Replaces: ViperBench/rms_norm/pytorch_impl.py:3-10,
 *           ViperBench/rms_norm/triton_impl.py:43-61,
 *           ViperBench/rms_norm/tilelang_impl.py:53-70. */
int vbh_rms_norm_fwd(const void* x, const void* w, void* y,
                     int64_t rows, int64_t cols, float eps,
                     int dtype, int w_dtype, void* stream);

/* Softmax (log_mode = 0) or log-softmax (log_mode = 1) over the last axis.
 * x: [rows, cols] of `in_dtype`; y: [rows, cols] of `out_dtype`.
 * Supported (in, out): (F32,F32) (F16,F16) (BF16,BF16) (F16,F32) (BF16,F32).
 * Replaces: ViperBench/softmax/pytorch_impl.py:4-6 (F.softmax, dim=-1),
 *           ViperBench/log_softmax/pytorch_impl.py:4-8 (F.log_softmax),
 *           ViperBench/softmax/triton_impl.py:28-47,
 *           ViperBench/log_softmax/triton_impl.py:70-101. */
int vbh_softmax_fwd(const void* x, void* y, int64_t rows, int64_t cols,
                    int in_dtype, int out_dtype, int log_mode, void* stream);

/* vbh_softmax_fwd with a caller-provided workspace (16-byte aligned).  Few
 * long rows split into segments (of whole 16-byte vectors, the last one
 * shorter where rows are not whole vectors): a first launch writes each row
 * segment's max and sum of exp(x - max) into the workspace (the two-stage
 * shape of ViperBench/logsumexp/triton_impl.py:48-71), a second reads x again
 * and writes y from each row's segments.  The workspace must hold
 * vbh_softmax_workspace_bytes(rows, cols, in_dtype) bytes; when that is 0, or
 * the workspace is null or smaller, this is vbh_softmax_fwd.  The workspace is
 * scratch of this call (stream-ordered, as for vbh_logsumexp_fwd_ws). */
int vbh_softmax_fwd_ws(const void* x, void* y, int64_t rows, int64_t cols,
                       int in_dtype, int out_dtype, int log_mode, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* Workspace bytes vbh_softmax_fwd_ws splits such a launch with (0: it does
 * not split).  A pure function of its arguments and of vbh_tune_override's
 * state (an overridden softmax geometry disables the split). */
int64_t vbh_softmax_workspace_bytes(int64_t rows, int64_t cols, int in_dtype);

/* Softmax / log-softmax over the middle axis of a contiguous [outer, n, inner]
 * tensor (the `dim` argument of log_softmax when dim is not the last axis).
 * Replaces: the (M, N, K) stride handling of
 *           ViperBench/log_softmax/triton_impl.py:44-67, 72-90. */
int vbh_softmax_dim_fwd(const void* x, void* y, int64_t outer, int64_t n,
                        int64_t inner, int in_dtype, int out_dtype,
                        int log_mode, void* stream);

/* logsumexp over the last axis: y[r] = log(sum_c exp(x[r, c])), with the
 * max-shift of torch.logsumexp (an infinite row max shifts by 0).
 * x: [rows, cols] of `in_dtype`; y: [rows] of `out_dtype` (F32 or in_dtype).
 * Replaces: ViperBench/logsumexp/pytorch_impl.py:3-5 (torch.logsumexp),
 *           ViperBench/logsumexp/triton_impl.py:48-71,
 *           ViperBench/logsumexp/tilelang_impl.py:44-72. */
int vbh_logsumexp_fwd(const void* x, void* y, int64_t rows, int64_t cols,
                      int in_dtype, int out_dtype, void* stream);

/* vbh_logsumexp_fwd with a caller-provided device workspace (16-byte aligned).
 * When a launch has few rows (fewer than 256) of many 16-byte vectors, each
 * row is split into segments reduced in parallel into the workspace (each
 * segment's max and sum of exp(x - max)), then combined per row -- the
 * two-stage shape of ViperBench/logsumexp/triton_impl.py:48-71 (block partials,
 * then a logsumexp over them), with the second stage on the GPU.  The workspace must
 * hold vbh_logsumexp_workspace_bytes(rows, cols, in_dtype) bytes; when that is
 * 0, or the workspace is null or smaller, this is vbh_logsumexp_fwd.  The
 * workspace is scratch of this call (stream-ordered: reuse it after the call's
 * work on `stream`, not concurrently on another stream). */
int vbh_logsumexp_fwd_ws(const void* x, void* y, int64_t rows, int64_t cols,
                         int in_dtype, int out_dtype, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* Workspace bytes vbh_logsumexp_fwd_ws splits such a launch with (0: it does
 * not split).  A pure function of its arguments and of vbh_tune_override's
 * state (an overridden logsumexp geometry disables the split). */
int64_t vbh_logsumexp_workspace_bytes(int64_t rows, int64_t cols, int in_dtype);

/* Column-blocked cross-entropy forward.  For every (row, column block cb) with
 * cb < ceil(n_cols / block_size) it writes loss, lse and z_loss (fp32) at flat
 * index cb * n_rows + row of the three output buffers.  Positions past
 * n_rows * ceil(n_cols / block_size) are not written.
 * logits: [n_rows, row_stride] of `logits_dtype` (unit column stride);
 * labels: [n_rows] of `label_dtype` (I32 or I64).
 * Replaces: ViperBench/cross_entropy/pytorch_impl.py:4-90,
 *           ViperBench/cross_entropy/triton_impl.py:13-75, 123-140,
 *           ViperBench/cross_entropy/tilelang_impl.py:213-260. */
int vbh_cross_entropy_fwd(const void* logits, const void* labels, int logits_dtype,
                          int label_dtype, void* loss, void* lse, void* z_loss,
                          int64_t n_rows, int64_t n_cols, int64_t row_stride,
                          float smoothing, float logit_scale, float lse_square_scale,
                          int64_t ignored_index, int64_t total_classes,
                          int64_t class_start_idx, int64_t block_size,
                          int has_smoothing, int split, void* stream);

/* vbh_cross_entropy_fwd with a caller-provided device workspace (16-byte
 * aligned).  When each row is one column block (block_size >= n_cols) and the
 * launch has few long rows, each row is cut into segments reduced in parallel
 * as column blocks with SPLIT semantics -- the vocab-parallel form of the
 * golden (pytorch_impl.py:38-52: a row's loss is the logsumexp of its blocks'
 * lse plus the sum of their SPLIT losses; each segment's lse is kept as its
 * max and sum of exp(x - max), so the row's lse is rounded once) -- then one
 * lane per row combines them into the caller's outputs, with the golden's NaN
 * rule for the whole row.  Workspace size from vbh_cross_entropy_workspace_bytes; fallback and
 * reuse as for vbh_logsumexp_fwd_ws. */
int vbh_cross_entropy_fwd_ws(const void* logits, const void* labels, int logits_dtype,
                             int label_dtype, void* loss, void* lse, void* z_loss,
                             int64_t n_rows, int64_t n_cols, int64_t row_stride,
                             float smoothing, float logit_scale, float lse_square_scale,
                             int64_t ignored_index, int64_t total_classes,
                             int64_t class_start_idx, int64_t block_size,
                             int has_smoothing, int split, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* Workspace bytes vbh_cross_entropy_fwd_ws splits such a launch with (0: no
 * split). */
int64_t vbh_cross_entropy_workspace_bytes(int64_t n_rows, int64_t n_cols, int64_t block_size,
                                          int logits_dtype);

/* vbh_cross_entropy_fwd for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No reference counterpart: the reference's implementations
 * allocate their outputs and temporaries through torch.  Same arguments and
 * results as vbh_cross_entropy_fwd_ws with the split taken whenever it pays,
 * but the split's segment results go to a static scratch buffer of the library
 * (32 KiB per GPU, held from the first call on a GPU until the process ends),
 * so the call allocates nothing.  A launch whose split would need more than
 * that returns VBH_E_RANGE (none does under the current split rule: at most
 * 24 KiB).  Every call on one GPU shares that GPU's scratch: calls that overlap
 * on one GPU (different streams, or different host threads without ordering)
 * race and must not be issued; calls on one stream are ordered and safe. */
int vbh_cross_entropy_fwd_noalloc(const void* logits, const void* labels, int logits_dtype,
                                  int label_dtype, void* loss, void* lse, void* z_loss,
                                  int64_t n_rows, int64_t n_cols, int64_t row_stride,
                                  float smoothing, float logit_scale, float lse_square_scale,
                                  int64_t ignored_index, int64_t total_classes,
                                  int64_t class_start_idx, int64_t block_size,
                                  int has_smoothing, int split, void* stream);

/* Cross-entropy backward: dlogits[r, c] = dloss[r] * logit_scale *
 * (p + 2 * lse_square_scale * lse[r] * p - target), p = exp(logit_scale * x - lse[r]).
 * dloss is read at dloss[r * dloss_stride]; ignored rows get dlogits = 0 * (...).
 * logits / dlogits: [n_rows, *_row_stride] of `logits_dtype`; lse: [n_rows] fp32.
 * Replaces: ViperBench/cross_entropy/pytorch_impl.py:93-141,
 *           ViperBench/cross_entropy/triton_impl.py:78-120, 143-158. */
int vbh_cross_entropy_bwd(const void* dloss, const void* logits, const void* lse,
                          const void* labels, void* dlogits, int logits_dtype,
                          int label_dtype, int64_t n_rows, int64_t n_cols,
                          int64_t logits_row_stride, int64_t dlogits_row_stride,
                          int64_t dloss_stride, float smoothing, float logit_scale,
                          float lse_square_scale, int64_t ignored_index,
                          int64_t total_classes, int64_t class_start_idx,
                          int has_smoothing, void* stream);

/* Mean, max or argmax over the middle axis of a contiguous [outer, n, inner]
 * tensor x of `in_dtype` (inner == 1 is the last axis).
 *   VBH_REDUCE_MEAN:   values[outer * inner] of `out_dtype` (in_dtype, or F32
 *                      for F16/BF16 input) = fp32 sum / n; indices unused.
 *   VBH_REDUCE_MAX:    values (in_dtype) and int64 indices of the maximum.
 *   VBH_REDUCE_ARGMAX: int64 indices only; values unused.
 * NaN counts as the largest value; ties give the smallest index.  n == 0 is
 * allowed for the mean only (every output is 0/0 = NaN, as torch.mean gives).
 * Replaces: ViperBench/mean_reduction/pytorch_impl.py:4-8 (torch.mean),
 *           ViperBench/max_reduction/pytorch_impl.py:4-11 (torch.max with dim),
 *           ViperBench/argmax/pytorch_impl.py:4-8 (torch.argmax). */
int vbh_reduce_fwd(const void* x, void* values, void* indices, int64_t outer, int64_t n,
                   int64_t inner, int in_dtype, int out_dtype, int op, void* stream);

/* vbh_reduce_fwd with a caller-provided device workspace (16-byte aligned):
 * last-axis reductions (inner == 1) of few long rows are split into segments
 * reduced in parallel, then combined per row (the mean of the equal segments'
 * fp32 means; the first maximal segment result, NaN largest).  Workspace
 * size, fallback and reuse as for vbh_logsumexp_fwd_ws, with
 * vbh_reduce_workspace_bytes.  No reference counterpart: torch.mean / max /
 * argmax (the goldens above) choose their own split internally. */
int vbh_reduce_fwd_ws(const void* x, void* values, void* indices, int64_t outer, int64_t n,
                      int64_t inner, int in_dtype, int out_dtype, int op, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* Workspace bytes vbh_reduce_fwd_ws splits such a launch with (0: no split). */
int64_t vbh_reduce_workspace_bytes(int64_t outer, int64_t n, int64_t inner, int in_dtype,
                                   int op);

/* Device-to-device stream copy of `bytes` (16-byte aligned pointers and size),
 * the kernel whose sustained rate is the measured HBM peak.
 * Replaces: the vendor-spec PEAKS table of experiments/exp_cliff_roofline.py:192-218
 *           (no AMD entry there) with a measured figure. */
int vbh_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* Streaming read of `bytes` (16-byte aligned pointer, multiple of 16): every
 * 16-byte vector is loaded once, by a persistent grid of one workgroup per CU
 * walking 32 KiB tiles, and folded by XOR into one 32-bit word per workgroup,
 * written to `partial` (4-byte aligned, at least
 * vbh_stream_read_partial_bytes(bytes) bytes; the XOR of the words written is
 * the XOR of every 32-bit word read).  Its sustained rate is the
 * measured read peak that read-dominated kernels (logsumexp, cross-entropy
 * forward, mean / max / argmax) are quoted against.
 * Replaces: the vendor-spec PEAKS table of experiments/exp_cliff_roofline.py:192-218,
 *           as vbh_stream_copy does, for kernels that write almost nothing. */
int vbh_stream_read(const void* src, int64_t bytes, void* partial, int64_t partial_bytes,
                    void* stream);

/* Bytes of `partial` vbh_stream_read needs for a read of `bytes` (0 for an
 * invalid or empty size). */
int64_t vbh_stream_read_partial_bytes(int64_t bytes);

/* Launch-geometry override for sweeps: threads per row `tpr` (a power of two
 * up to 64, or a multiple of 64 up to 1024) and workgroup size `block`
 * (64..1024, a multiple of 64 and of tpr)
 * for op `op`; `flags` ORs VBH_TUNE_* bits.  tpr = 0 keeps the built-in shape
 * heuristic, block = 0 its workgroup size, flags = 0 its kernel choice.
 * Process-wide setting.
 * Replaces: the import-time config injection of ViperBench/tuning/cache.py:31-36. */
#define VBH_TUNE_PERSIST 1      /* force the persistent pipelined row kernel
                                   (cross entropy: the persistent forward for
                                   fp32 rows of one column block of at least
                                   8192 columns; a block of 256 or 512 with
                                   it sets that kernel's workgroup size)     */
#define VBH_TUNE_NO_PERSIST 2   /* force one row group per workgroup            */
#define VBH_TUNE_NONTEMPORAL 4  /* force nontemporal row loads / output stores  */
#define VBH_TUNE_TEMPORAL 8     /* force plain row loads / output stores        */
#define VBH_TUNE_WRITE_THROUGH 16    /* nontemporal 16-byte output stores also
                                        written through the L2 (device scope) */
#define VBH_TUNE_NO_WRITE_THROUGH 32 /* keep output stores in the L2            */
int vbh_tune_override(int op, int tpr, int block, int flags);

/* Debug bounds checks.  libvbhip_debug.so is the library built with
 * VBH_DEBUG_BOUNDS: there every global-memory access of every kernel first
 * checks that its bytes lie inside the buffer it belongs to (each kernel's
 * extent of that buffer, from the entry point's sizes); an access that fails
 * is not made (a load yields zeros, a store is dropped) and is counted.
 * vbh_debug_bounds waits for the device, writes the number of failed checks
 * since the last clear to *failed and, when there were any, "<file>:<line>" of
 * the first failing buffer's description to `where` (when non-null), and with
 * clear != 0 resets the count.  vbh_debug_bounds_slack takes `bytes` off the
 * end of every buffer's allowed extent (0 restores), so that a test can watch
 * checks fail, on accesses that are then skipped rather than made.  Both act
 * on the current device.  The release library returns VBH_E_UNSUPPORTED.
 * No counterpart in the reference (its kernels are Python DSL code); this is
 * the debug-build bounds check for the library's own kernels. */
int vbh_debug_bounds(int64_t* failed, char* where, int64_t where_len, int clear);
int vbh_debug_bounds_slack(int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* VBHIP_H */

// Column-blocked cross-entropy forward and backward for gfx950.
//
// Forward: a "segment" is one (row, column block) pair, i.e. up to block_size
// consecutive logits of one row.  `tpr` lanes own one segment, load it once
// into registers in the storage type (scaled by logit_scale where used),
// all-reduce max, sum of exp(x - max) and, with smoothing, the plain sum of the
// logits, and one lane writes loss / lse / z_loss at flat index
// cb * n_rows + row.  The label logit is fetched by that lane at kernel start;
// only the storing lane's wave waits for it before issuing its segment loads,
// the segment's other waves load at once (a version without the fetch ran
// 0.1% faster on MI355X).  Segments wider than the register budget use a
// streaming online (max, rescaled sum) pass.
//
// Semantics: ViperBench/cross_entropy/pytorch_impl.py:22-90 (golden) and
// ViperBench/cross_entropy/triton_impl.py:33-75 (per-(row, block) program).
// Backward: ViperBench/cross_entropy/pytorch_impl.py:93-141 and
// ViperBench/cross_entropy/triton_impl.py:98-120.
#include "vbh_device.h"
#include "vbh_launch.h"

namespace vbh {

namespace {

constexpr float kNegInf = -__builtin_huge_valf();

// Scalar parameters.  The golden evaluates `1 - smoothing`,
// `smoothing / total_classes` and `2.0 * lse_square_scale` in Python double
// precision before they meet an fp32 tensor, so the host precomputes them in
// double and rounds once.
struct CeScalars {
  float smoothing, logit_scale, lse_square_scale, total_classes;
  float one_minus_smoothing, smooth_negative, two_lse_square_scale;
  int64_t ignored_index, class_start;
  int has_smoothing, split;
  // first stage of a split row: an all -inf segment (no NaN) gets lse = -inf,
  // as a logsumexp would, not the golden's NaN; the second stage applies the
  // golden's rule to the whole row
  int empty_neg_inf;
  // first stage of a split row: each segment's SegPair (max of the scaled
  // logits, sum of exp(x * scale - max)) goes to z_out (max) and lse_out (sum),
  // both otherwise unused there; ce_combine merges them
  int pair_out;
  // logit_scale * log2(e): exp(x * scale - m) = 2^(x * exp_scale - m * log2(e)),
  // one FMA per logit ahead of v_exp_f32
  float exp_scale;
  // logit_scale > 0: the row max of the scaled logits is scale * the max of the
  // raw ones (rounding is monotone), one multiply per row instead of per logit
  int scale_pos;
};

CeScalars make_scalars(float smoothing, float logit_scale, float lse_square_scale,
                       float total_classes, int64_t ignored_index, int64_t class_start,
                       int has_smoothing, int split) {
  CeScalars c;
  c.smoothing = smoothing;
  c.logit_scale = logit_scale;
  c.lse_square_scale = lse_square_scale;
  c.total_classes = total_classes;
  c.one_minus_smoothing = static_cast<float>(1.0 - static_cast<double>(smoothing));
  c.smooth_negative =
      static_cast<float>(static_cast<double>(smoothing) / static_cast<double>(total_classes));
  c.two_lse_square_scale = static_cast<float>(2.0 * static_cast<double>(lse_square_scale));
  c.ignored_index = ignored_index;
  c.class_start = class_start;
  c.has_smoothing = has_smoothing;
  c.split = split;
  c.empty_neg_inf = 0;
  c.pair_out = 0;
  c.exp_scale = static_cast<float>(static_cast<double>(logit_scale) * 1.4426950408889634);
  c.scale_pos = logit_scale > 0.f && logit_scale <= 3.4028234663852886e38f;
  return c;
}

__device__ __forceinline__ int64_t read_label(const void* labels, int label_i64, int64_t row,
                                              const Span& s) {
  if (!VBH_IN_SPAN(s, static_cast<const char*>(labels) + row * (label_i64 ? 8 : 4),
                   label_i64 ? 8 : 4))
    return 0;
  return label_i64 ? static_cast<const int64_t*>(labels)[row]
                   : static_cast<int64_t>(static_cast<const int32_t*>(labels)[row]);
}

// The labels buffer: n_rows int32 or int64 values.
#define VBH_LABEL_SPAN(labels, label_i64, n_rows) \
  VBH_SPAN(static_cast<const char*>(labels), (n_rows) * ((label_i64) ? 8 : 4))

// The three per-segment outputs (loss, lse, z_loss) have one extent.
struct CeOutSpans {
  Span loss, lse, z;
};

// Per-segment outputs (pytorch_impl.py:37-76): loss and z_loss from the lse.
struct CeOut {
  float loss, z;
};

__device__ __forceinline__ CeOut ce_outputs(float lse, float sum_logits, bool in_block,
                                            float logit_label, bool ignored,
                                            const CeScalars& c) {
  if (ignored) return CeOut{0.f, 0.f};
  float l, z;
  const float lse_term = c.split ? 0.f : lse;
  if (c.has_smoothing) {
    if (in_block)
      l = lse_term - c.smoothing * sum_logits / c.total_classes -
          c.one_minus_smoothing * logit_label;
    else
      l = c.smoothing * (lse_term - sum_logits / c.total_classes);
  } else {
    l = in_block ? lse_term - logit_label : 0.f;
  }
  if (!c.split) {
    z = c.lse_square_scale * lse * lse;
    l = l + z;
  } else {
    z = 0.f;
  }
  return CeOut{l, z};
}

// The per-segment epilogue, executed by one lane.
__device__ __forceinline__ void ce_store(float lse, float sum_logits, bool in_block,
                                         float logit_label, bool ignored,
                                         const CeScalars& c, float* loss, float* lse_out,
                                         float* z_out, int64_t idx, const CeOutSpans& so) {
  if (VBH_IN_SPAN(so.lse, lse_out + idx, sizeof(float))) lse_out[idx] = lse;
  const CeOut o = ce_outputs(lse, sum_logits, in_block, logit_label, ignored, c);
  if (VBH_IN_SPAN(so.loss, loss + idx, sizeof(float))) loss[idx] = o.loss;
  if (VBH_IN_SPAN(so.z, z_out + idx, sizeof(float))) z_out[idx] = o.z;
}

// A split row's first stage: the segment's SegPair (max m, sum t of
// exp(x * scale - m)) over its lse and z_loss slots.
__device__ __forceinline__ void ce_store_pair(float m, float t, float* lse_out, float* z_out,
                                              int64_t idx, const CeOutSpans& so) {
  if (VBH_IN_SPAN(so.lse, lse_out + idx, sizeof(float))) lse_out[idx] = t;
  if (VBH_IN_SPAN(so.z, z_out + idx, sizeof(float))) z_out[idx] = m;
}

// Segments whose start is not on a 16-byte boundary (rows not a multiple of
// the vector width long): MIS kernels read a scalar head up to the first
// boundary, whole aligned vectors and a scalar tail, one head and one tail
// element per lane (the launcher makes tpr >= V); nothing outside the
// segment is read.
struct MisSeg {
  int head, nvec, tail;
};

template <int V>
__device__ __forceinline__ MisSeg mis_seg(int64_t start, int len) {
  int head = static_cast<int>((V - start % V) % V);
  if (head > len) head = len;
  const int nvec = (len - head) / V;
  return MisSeg{head, nvec, len - head - nvec * V};
}

// SL: the segment's sum of logits is needed (smoothing, or the first stage of
// a split row); without it that accumulation is left out.
template <typename T, int V, int IT, bool NT, bool MIS, bool SL>
__global__ __launch_bounds__(kMaxBlock) void ce_fwd_rows(
    const T* __restrict__ logits, const void* __restrict__ labels, int label_i64,
    float* __restrict__ loss, float* __restrict__ lse_out, float* __restrict__ z_out,
    int64_t n_rows, int n_cols, int64_t ld, int bs, int ncb, int tpr, CeScalars c) {
  typedef typename Raw<T, V>::type RT;
  __shared__ float lds[3][kMaxWaves];
  const GroupShape gs = group_shape(tpr);
  const int g = gs.g;
  const int64_t nseg = n_rows * ncb;
  int64_t seg = static_cast<int64_t>(blockIdx.x) * gs.per_block + gs.sub;
  const bool live = seg < nseg;
  if (!live) seg = nseg - 1;
  const int64_t row = seg / ncb;
  const int cb = static_cast<int>(seg - row * ncb);
  const int col0 = cb * bs;
  const int col_end = min(n_cols, col0 + bs);
  const Span sx = VBH_SPAN(logits, strided_extent(n_rows, ld, n_cols));
  const Span sb = VBH_LABEL_SPAN(labels, label_i64, n_rows);
  const CeOutSpans so{VBH_SPAN(loss, nseg), VBH_SPAN(lse_out, nseg), VBH_SPAN(z_out, nseg)};
  const T* lr = logits + row * ld;
  const int64_t sstart = row * ld + col0;
  const MisSeg ms = MIS ? mis_seg<V>(sstart, col_end - col0) : MisSeg{0, (col_end - col0) / V, 0};
  const int nvec = ms.nvec;
  const T* lb = logits + sstart + ms.head;  // 16-byte aligned body

  // label logit, fetched early by the storing lane
  bool ignored = false, in_block = false;
  float logit_label = 0.f;
  if (live && g == 0) {
    const int64_t label = read_label(labels, label_i64, row, sb);
    ignored = label == c.ignored_index;
    const int64_t adj = label - c.class_start;
    in_block = adj >= col0 && adj < col_end;
    if (!ignored && in_block && VBH_IN_SPAN(sx, lr + adj, sizeof(T)))
      logit_label = mul_rn(static_cast<float>(lr[adj]), c.logit_scale);
  }

  RT xr[IT];
#pragma unroll
  for (int i = 0; i < IT; ++i) {
    const int j = i * tpr + g;
    if (j < nvec) xr[i] = load_raw<T, V, NT>(lb + static_cast<int64_t>(j) * V, sx);
    else xr[i] = RT{};
  }
  const float scale = c.logit_scale;
  const bool hv = MIS && g < ms.head, tv = MIS && g < ms.tail;
  float hr = 0.f, tr = 0.f;  // raw head / tail logits
  if (hv) load_f32<T, 1>(logits + sstart + g, &hr, sx);
  if (tv) load_f32<T, 1>(lb + static_cast<int64_t>(nvec) * V + g, &tr, sx);
  const float hx = hr * scale, tx = tr * scale;

  float mx[V];
#pragma unroll
  for (int k = 0; k < V; ++k) mx[k] = kNegInf;
  if (c.scale_pos) {  // max of the raw logits, scaled once
#pragma unroll
    for (int i = 0; i < IT; ++i)
      if (i * tpr + g < nvec)
#pragma unroll
        for (int k = 0; k < V; ++k) mx[k] = max_nan(mx[k], raw_at<T, V>(xr[i], k));
#pragma unroll
    for (int k = 0; k < V; ++k) mx[k] *= scale;
  } else {
#pragma unroll
    for (int i = 0; i < IT; ++i)
      if (i * tpr + g < nvec)
#pragma unroll
        for (int k = 0; k < V; ++k) mx[k] = max_nan(mx[k], raw_at<T, V>(xr[i], k) * scale);
  }
  float lm = mx[0];
#pragma unroll
  for (int k = 1; k < V; ++k) lm = max_nan(lm, mx[k]);
  if (hv) lm = max_nan(lm, hx);
  if (tv) lm = max_nan(lm, tx);
  const float m = group_allreduce<Max>(lm, tpr, lds[0]);
  reload_barrier<T, V, IT>(xr);

  float se[V], sl[V];
#pragma unroll
  for (int k = 0; k < V; ++k) se[k] = sl[k] = 0.f;
  // exp(x * scale - m) of a raw logit x: one FMA ahead of v_exp_f32
  // (2^(x * scale * log2 e - m * log2 e)), or on a multiply and a subtract
  // where m is too large for that form (shift_fma_ok)
  const bool fma_ok = shift_fma_ok(m);
  const float mb = m * kLog2e;
  const float es = c.exp_scale;
  auto efma = [=](float x) { return __builtin_amdgcn_exp2f(fmaf(x, es, -mb)); };
  // a scale other than 1: the product rounded first, as the golden rounds
  // x * scale before it subtracts the max (x * exp_scale would carry
  // exp_scale's own rounding, up to |x * scale| * 2^-24 in the exponent)
  auto efms = [=](float x) {
    return __builtin_amdgcn_exp2f(fmaf(mul_rn(x, scale), kLog2e, -mb));
  };
  auto esub = [=](float x) { return fast_exp(mul_rn(x, scale) - m); };
  const bool one = scale == 1.f;
  auto ex1 = [&](float x) { return fma_ok ? (one ? efma(x) : efms(x)) : esub(x); };
  auto sum_exp = [&](auto ex) {
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      if (i * tpr + g < nvec) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
          const float x = raw_at<T, V>(xr[i], k);
          se[k] += ex(x);
          if constexpr (SL) sl[k] += x * scale;
        }
      }
    }
  };
  if (!fma_ok) sum_exp(esub);
  else if (one) sum_exp(efma);
  else sum_exp(efms);
#pragma unroll
  for (int w = V / 2; w >= 1; w /= 2)
#pragma unroll
    for (int k = 0; k < w; ++k) {
      se[k] += se[k + w];
      sl[k] += sl[k + w];
    }
  if (hv) {
    se[0] += ex1(hr);
    sl[0] += hx;
  }
  if (tv) {
    se[0] += ex1(tr);
    sl[0] += tx;
  }
  const float s = group_allreduce<Sum>(se[0], tpr, lds[1]);
  float sum_logits = 0.f;
  if constexpr (SL) sum_logits = group_allreduce<Sum>(sl[0], tpr, lds[2]);

  if (live && g == 0) {
    float lse = (fast_log(s) - (fma_ok ? shift_residual(m, mb) : 0.f) * kLn2) + m;
    // all -inf (the sum of logits is -inf, not NaN): -inf in a first stage
    if (c.empty_neg_inf && m == kNegInf && sum_logits == sum_logits) lse = kNegInf;
    const int64_t idx = static_cast<int64_t>(cb) * n_rows + row;
    ce_store(lse, sum_logits, in_block, logit_label, ignored, c, loss, lse_out, z_out, idx, so);
    if (c.pair_out) {
      const float t = m == kNegInf
                          ? 0.f
                          : (fma_ok ? s * __builtin_amdgcn_exp2f(-shift_residual(m, mb)) : s);
      ce_store_pair(m, t, lse_out, z_out, idx, so);
    }
  }
}

// Segments wider than the register budget: one workgroup per segment,
// online (max, rescaled sum) over 16-byte chunks.
template <typename T, int V>
__global__ __launch_bounds__(kMaxBlock) void ce_fwd_stream(
    const T* __restrict__ logits, const void* __restrict__ labels, int label_i64,
    float* __restrict__ loss, float* __restrict__ lse_out, float* __restrict__ z_out,
    int64_t n_rows, int n_cols, int64_t ld, int bs, int ncb, CeScalars c) {
  __shared__ float lds[3][kMaxWaves];
  const int tpr = blockDim.x;
  const int64_t seg = blockIdx.x;
  const int64_t row = seg / ncb;
  const int cb = static_cast<int>(seg - row * ncb);
  const int col0 = cb * bs;
  const int col_end = min(n_cols, col0 + bs);
  const int nvec = (col_end - col0) / V;
  const T* lr = logits + row * ld + col0;
  const Span sx = VBH_SPAN(logits, strided_extent(n_rows, ld, n_cols));
  const Span sb = VBH_LABEL_SPAN(labels, label_i64, n_rows);
  const CeOutSpans so{VBH_SPAN(loss, n_rows * ncb), VBH_SPAN(lse_out, n_rows * ncb),
                      VBH_SPAN(z_out, n_rows * ncb)};

  // per-thread running max (NaN ignored), rescaled sum, NaN-propagating sum of logits
  float m = kNegInf, s = 0.f, sl = 0.f, nan = 0.f;
  for (int j = threadIdx.x; j < nvec; j += tpr) {
    float v[V];
    load_f32<T, V>(lr + static_cast<int64_t>(j) * V, v, sx);
    float cm = kNegInf;
#pragma unroll
    for (int k = 0; k < V; ++k) {
      v[k] = mul_rn(v[k], c.logit_scale);
      cm = fmaxf(cm, v[k]);
      sl += v[k];
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
  const float gm = group_allreduce<Max>(m, tpr, lds[0]);
  const bool finite = gm != kNegInf && gm != -kNegInf;
  const float t = (finite && m != kNegInf) ? s * fast_exp(m - gm) : 0.f;
  const float gs = group_allreduce<Sum>(t, tpr, lds[1]);
  // The NaN flag rides on the sum of logits: a NaN logit makes that sum NaN in
  // the golden as well (pytorch_impl.py:56).
  const float gl = group_allreduce<Sum>(nan != 0.f ? __builtin_nanf("") : sl, tpr, lds[2]);
  if (threadIdx.x != 0) return;
  // Golden lse = log(sum(exp(L - max))) + max with a NaN-propagating max: a NaN
  // logit, a +inf max (inf - inf) or an all -inf segment (-inf - -inf) give NaN.
  const bool has_nan = nan != 0.f || (gl != gl);
  float lse = (has_nan || !finite) ? __builtin_nanf("") : fast_log(gs) + gm;
  if (c.empty_neg_inf && !has_nan && gm == kNegInf) lse = kNegInf;  // as in ce_fwd_rows
  const int64_t label = read_label(labels, label_i64, row, sb);
  const bool ignored = label == c.ignored_index;
  const int64_t adj = label - c.class_start;
  const bool in_block = adj >= col0 && adj < col_end;
  float logit_label = 0.f;
  if (!ignored && in_block && VBH_IN_SPAN(sx, logits + row * ld + adj, sizeof(T)))
    logit_label = mul_rn(static_cast<float>(logits[row * ld + adj]), c.logit_scale);
  const int64_t idx = static_cast<int64_t>(cb) * n_rows + row;
  ce_store(lse, gl, in_block, logit_label, ignored, c, loss, lse_out, z_out, idx, so);
  if (c.pair_out) ce_store_pair(has_nan ? __builtin_nanf("") : gm, finite ? gs : 0.f, lse_out,
                                z_out, idx, so);
}

// Persistent forward for fp32 rows of one column block (the whole row is the
// segment): a grid of one workgroup per CU, workgroup b taking rows b, b + G,
// b + 2G, ... (G the grid) in chunks of kCePersistChunk 16-byte vectors (32
// KiB), the next chunk's loads in flight while the current one is folded.  All
// workgroups move through the logits together, the waves of a workgroup in
// step (a barrier after every chunk); ce_fwd_rows (one row per 1024-lane
// workgroup) leaves a CU's loads idle while a finished workgroup reduces its
// row and the next one starts.  MI355X, fp32, 512-lane workgroups against
// ce_fwd_rows on the same box: 32000 columns, 1024 rows +14%, 2048 +7%, 4096
// +4%, 8192 (C4) +2.2%, 16384 +0.8%; 1024 x 50304 +32%, 2048 x 65536 +25%,
// 8192 x 16384 (two chunks per row) +2.4%; rows of one chunk lose (8192 x
// 8192: -12%), hence the launcher's default of at least two chunks per row.
// Chunks of 16 KiB with two or three in flight, 8 KiB with three or four and
// three of 32 KiB all measured slower at C4 (-0.1 to -20%).  256-lane
// workgroups (8 vectors per lane per chunk) stream faster and start and drain
// slower: against 512 lanes, 64 chunks per CU or more +0.9 to +2.0% (C4
// +0.9%, 4096 x 32000 and 8192 x 16384 +1.0%, 16384 x 32000 +1.5%, 2048 x
// 65536 +2.0%), 48 or fewer -1.7 to -2.8% (4096 x 24576, 2048 x 32000,
// 1024 x 50304, 1024 x 32000), so the launcher takes 256 lanes from 64
// chunks per CU up.  At C4, 1024 lanes x 2 vectors -0.9%, 128 x 16 -10%,
// 256 x 4 (16 KiB chunks) -15%, global instead of buffer loads +-0.1%.
//
// Each lane folds its share of a row into an online pair: m, the max of its
// scaled logits (NaN if any is NaN), and s, the sum of exp(x - m) over its
// scaled logits x, held relative to 2^nb with nb = m * log2 e rounded -- the
// FMA form of ce_fwd_rows, 2^(x * log2 e - nb) per logit -- and rescaled by
// 2^(nb_old - nb) when m grows.  A lane whose max lies beyond that form's
// range (shift_fma_ok) holds s relative to e^m and takes exp(x - m) on a
// subtract; a wave takes that path only when one of its lanes needs it.  At
// the row's end each lane's pair becomes a SegPair (t = s * 2^-shift_residual
// in the FMA form), and the workgroup merges them as the second stage of a
// split row merges segments: M = max m, S = sum t * exp(m - M) over the lanes
// with m > -inf; a NaN anywhere, an infinite M or an all -inf row give the
// golden's NaN lse (pytorch_impl.py:37-47): each wave merges its lanes' pairs,
// and wave 0 the waves' pairs, one per lane of a group of W.  Lanes 0, 1 and 2
// then store the row's loss, lse and z_loss.  The label comes from a scalar
// load one row ahead, its logit from a scalar load at the row's first chunk.
// Buffer loads with a range of one row: vectors past its end (the last
// chunk's spare lanes, the loads past a workgroup's last row) read nothing.
constexpr int kCePersistChunk = 2048;  // 16-byte vectors per chunk (32 KiB)
constexpr int kCePersistBufs = 2;      // chunks in rotation (loads NB - 1 ahead)

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int U>
struct CeChunk {
  f32x4 v[U];
};

// SL: the row's sum of scaled logits is needed (smoothing); ONE: logit_scale
// is 1 (else each logit's product with it is rounded once, as the golden
// rounds it, and used for the max, the exps and the sum).  L: lanes per
// workgroup (256 or 512), each loading kCePersistChunk / L vectors per chunk.
template <bool SL, typename LabelT, bool ONE, int L>
__global__ __launch_bounds__(L) void ce_fwd_persist(
    const float* __restrict__ logits, const LabelT* __restrict__ labels,
    float* __restrict__ loss, float* __restrict__ lse_out, float* __restrict__ z_out,
    int64_t n_rows, int n_cols, int64_t ld, CeScalars c) {
  constexpr int CH = kCePersistChunk, U = CH / L;
  constexpr int W = L / kWave;
  static_assert(U * L == CH && (W & (W - 1)) == 0 && W <= kWave, "a chunk's shape");
  using Chunk = CeChunk<U>;
  // per wave, by row parity: the wave's max, its sum of t * exp(m - max) and
  // its sum of logits
  __shared__ float lds_pair[2][3][W];
  const int lane = static_cast<int>(threadIdx.x);
  const int wave = lane >> 6;
  const int64_t b = blockIdx.x;
  if (b >= n_rows) return;  // the whole workgroup
  const int64_t grid = gridDim.x;
  const int nvec = n_cols / 4;
  const int cpr = (nvec + CH - 1) / CH;
  const int64_t chunks = ((n_rows - 1 - b) / grid + 1) * cpr;
  const Span sx = VBH_SPAN(logits, strided_extent(n_rows, ld, n_cols));
  const Span sb = VBH_SPAN(labels, n_rows);
  const Span sloss = VBH_SPAN(loss, n_rows), slse = VBH_SPAN(lse_out, n_rows),
             sz = VBH_SPAN(z_out, n_rows);
  const float scale = c.logit_scale;

  // the load cursor: row lrow, chunk lc
  int64_t lrow = b;
  int lc = 0;
  // (every lambda is inlined: a call would put the captured cursors in memory)
  auto load = [&](Chunk& ch, bool real) __attribute__((always_inline)) {
    const float* base = logits + (real ? lrow * ld : 0);
    const bool ok = real && VBH_IN_SPAN(sx, base, static_cast<int64_t>(nvec) * 16);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(base), static_cast<short>(0), ok ? nvec * 16 : 0, kRawBufferWord3);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = lc * CH + u * L + lane;
      ch.v[u] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, j * 16, 0, 2));
    }
    if (++lc == cpr) {
      lc = 0;
      lrow += grid;
    }
  };

  // the fold cursor and this lane's pair for the fold's row
  int64_t frow = b;
  int fc = 0;
  float m = kNegInf, nb = kNegInf, s = 0.f, sl = 0.f;
  // the row's label facts; the next row's label (loaded one row ahead)
  LabelT label_next = VBH_IN_SPAN(sb, labels + b, sizeof(LabelT)) ? labels[b] : LabelT(0);
  bool ignored = false, in_row = false;
  int parity = 0;  // of the fold's row: its LDS slots
  float logit_raw = 0.f;  // the label's logit, scaled where used (at the row's end)

  auto fold_values = [&](const Chunk& ch, auto mask) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(mask)::value;
    const int c0 = fc * CH;
    float xv[U][4];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int k = 0; k < 4; ++k) xv[u][k] = ONE ? ch.v[u][k] : mul_rn(ch.v[u][k], scale);
    float cm = kNegInf;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = !MASK || c0 + u * L + lane < nvec;
#pragma unroll
      for (int k = 0; k < 4; ++k) cm = max_nan(cm, ok ? xv[u][k] : kNegInf);
    }
    const float nm = max_nan(m, cm);
    const float nnb = nm * kLog2e;
    float xs = 0.f;
    const bool lane_fma = shift_fma_ok(m) && shift_fma_ok(nm);
    if (__builtin_amdgcn_ballot_w64(!lane_fma) == 0) {
      // every lane in the FMA form: s relative to 2^nb
      float e = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = !MASK || c0 + u * L + lane < nvec;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float v = __builtin_amdgcn_exp2f(fmaf(xv[u][k], kLog2e, -nnb));
          e += ok ? v : 0.f;
          if constexpr (SL) xs += ok ? xv[u][k] : 0.f;
        }
      }
      // an all -inf share so far holds nothing (its exps would be NaN)
      s = nm == kNegInf ? 0.f : fmaf(s, __builtin_amdgcn_exp2f(nb - nnb), e);
    } else {
      // some lane beyond the FMA form: each lane through the sum relative to
      // e^m (t), the exps on a subtract, back to its new form
      float e = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool ok = !MASK || c0 + u * L + lane < nvec;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float v = fast_exp(xv[u][k] - nm);
          e += ok ? v : 0.f;
          if constexpr (SL) xs += ok ? xv[u][k] : 0.f;
        }
      }
      float t = m == kNegInf ? 0.f
                             : (shift_fma_ok(m) ? s * __builtin_amdgcn_exp2f(-shift_residual(m, nb))
                                                : s);
      t = nm == kNegInf ? 0.f : t * fast_exp(m - nm) + e;
      s = shift_fma_ok(nm) && nm != kNegInf
              ? t * __builtin_amdgcn_exp2f(shift_residual(nm, nnb))
              : t;
    }
    m = nm;
    nb = nnb;
    if constexpr (SL) sl += xs;
    // every path has waited for the whole chunk here, so the loads that reuse
    // its registers need no wait of their own
#pragma unroll
    for (int u = 0; u < U; ++u) asm volatile("" ::"v"(ch.v[u]));
  };

  auto fold = [&](const Chunk& ch) __attribute__((always_inline)) {
    if (fc == 0) {  // a new row: its label facts and logit, the next row's label
      const int64_t label = static_cast<int64_t>(label_next);
      ignored = label == c.ignored_index;
      const int64_t adj = label - c.class_start;
      in_row = adj >= 0 && adj < n_cols;
      logit_raw = 0.f;
      if (!ignored && in_row && VBH_IN_SPAN(sx, logits + frow * ld + adj, sizeof(float)))
        logit_raw = logits[frow * ld + adj];
      const int64_t nrow = frow + grid < n_rows ? frow + grid : n_rows - 1;
      label_next = VBH_IN_SPAN(sb, labels + nrow, sizeof(LabelT)) ? labels[nrow] : LabelT(0);
    }
    if (fc == cpr - 1) fold_values(ch, std::true_type{});
    else fold_values(ch, std::false_type{});
    // the waves issue each chunk's loads together: a barrier after every
    // chunk (the row's last one has the merge's) kept them in step, +1% at C4
    // on MI355X against a barrier per row only
    if (fc != cpr - 1) __syncthreads();
    if (fc == cpr - 1) {
      // each wave merges its lanes' pairs into one (a NaN max or sum
      // propagates into it), one LDS exchange and one barrier per row, and
      // wave 0 merges the waves' pairs: reads of row k's slots end before the
      // barrier of row k + 1, writes of row k + 2 come after it
      const float wm = wave_allreduce<Max>(m, kWave);
      // this lane's SegPair sum, relative to e^m
      const float t = shift_fma_ok(m) ? s * __builtin_amdgcn_exp2f(-shift_residual(m, nb)) : s;
      const bool use = m != kNegInf && !__builtin_isinf(wm);
      const float ws = wave_allreduce<Sum>(use ? t * fast_exp(m - wm) : 0.f, kWave);
      const float wl = SL ? wave_allreduce<Sum>(sl, kWave) : 0.f;
      if ((lane & (kWave - 1)) == 0) {
        lds_pair[parity][0][wave] = wm;
        lds_pair[parity][1][wave] = ws;
        if constexpr (SL) lds_pair[parity][2][wave] = wl;
      }
      __syncthreads();
      if (wave == 0) {
        // lane k of each group of W holds wave k's pair: the merge in
        // log2(W) DPP steps per reduction instead of a loop over the waves
        const int k = lane & (W - 1);
        const float mw = lds_pair[parity][0][k], sw = lds_pair[parity][1][k];
        const float mx = wave_allreduce<Max>(mw, W);
        const bool nan = wave_allreduce<Max>(mw != mw || sw != sw ? 1.f : 0.f, W) > 0.f;
        const float sum = wave_allreduce<Sum>(mw != kNegInf ? sw * fast_exp(mw - mx) : 0.f, W);
        const float sum_logits = SL ? wave_allreduce<Sum>(lds_pair[parity][2][k], W) : 0.f;
        const float lse = nan || __builtin_isinf(mx) ? __builtin_nanf("") : fast_log(sum) + mx;
        const float logit_label = ONE ? logit_raw : mul_rn(logit_raw, scale);
        const CeOut o = ce_outputs(lse, sum_logits, in_row, logit_label, ignored, c);
        // (one pointer chosen per lane would put the kernel's locals in scratch)
        if (lane == 0 && VBH_IN_SPAN(sloss, loss + frow, sizeof(float))) loss[frow] = o.loss;
        if (lane == 1 && VBH_IN_SPAN(slse, lse_out + frow, sizeof(float))) lse_out[frow] = lse;
        if (lane == 2 && VBH_IN_SPAN(sz, z_out + frow, sizeof(float))) z_out[frow] = o.z;
      }
      parity ^= 1;
      m = kNegInf;
      nb = kNegInf;
      s = 0.f;
      sl = 0.f;
    }
    if (++fc == cpr) {
      fc = 0;
      frow += grid;
    }
  };

  constexpr int NB = kCePersistBufs;
  Chunk buf[NB];
#pragma unroll
  for (int i = 0; i < NB - 1; ++i) load(buf[i], i < chunks);
  const int64_t rounds = chunks / NB;
  for (int64_t q = 0; q < rounds; ++q) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      load(buf[(i + NB - 1) % NB], q * NB + i + NB - 1 < chunks);
      fold(buf[i]);
    }
  }
  const int64_t rest = chunks - NB * rounds;  // buf[0 .. rest) hold these chunks
#pragma unroll
  for (int i = 0; i < NB - 1; ++i)
    if (i < rest) fold(buf[i]);
}

// Second stage of a split row (one column block per row, cut into `segs`
// segments that a first stage reduced with SPLIT semantics into seg_loss, and
// into SegPairs seg_max / seg_sum, at flat index k * n_rows + row).  One wave
// per row, lane k holding segment k (segs <= 64): the row's lse = M + log S
// from its segments' pairs under the
// golden's rule (a NaN logit, a +inf or an all -inf row give NaN), and the
// loss adds the lse term the first stage left out (pytorch_impl.py:54-70):
// lse where the row holds the label, smoothing * lse elsewhere with smoothing,
// 0 with SPLIT; plus z = lse_square_scale * lse^2 without SPLIT.  The segment
// losses sum to the rest of the golden's loss (-logit_label and the smoothing
// sums are additive over segments).
constexpr int kCombineRowsPerBlock = 4;  // waves of a 256-lane workgroup

__global__ __launch_bounds__(256) void ce_combine(
    const float* __restrict__ seg_loss, const float* __restrict__ seg_sum,
    const float* __restrict__ seg_max, const void* __restrict__ labels, int label_i64,
    float* __restrict__ loss, float* __restrict__ lse_out, float* __restrict__ z_out,
    int64_t n_rows, int n_cols, int segs, CeScalars c) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kCombineRowsPerBlock +
                      static_cast<int>(threadIdx.x >> 6);
  if (row >= n_rows) return;  // a whole wave
  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const Span ssl = VBH_SPAN(seg_loss, segs * n_rows), sss = VBH_SPAN(seg_sum, segs * n_rows);
  const Span ssm = VBH_SPAN(seg_max, segs * n_rows);
  const Span sb = VBH_LABEL_SPAN(labels, label_i64, n_rows);
  const CeOutSpans so{VBH_SPAN(loss, n_rows), VBH_SPAN(lse_out, n_rows), VBH_SPAN(z_out, n_rows)};
  // lane k < segs: segment k's SPLIT loss and SegPair, one load each
  const bool has = lane < segs;
  float sl = 0.f, mk = 0.f, tk = 0.f;
  if (has) {
    const int64_t i = static_cast<int64_t>(lane) * n_rows + row;
    load_f32<float, 1>(seg_loss + i, &sl, ssl);
    load_f32<float, 1>(seg_max + i, &mk, ssm);
    load_f32<float, 1>(seg_sum + i, &tk, sss);
  }
  const float rest = wave_allreduce<Sum>(sl, kWave);
  const RowPairs rp = wave_combine_seg_pairs(has, mk, tk);
  if (lane != 0) return;
  // a +inf max gives inf - inf in the golden: NaN, as an all -inf row does
  const float lse = rp.nan || __builtin_isinf(rp.m) ? __builtin_nanf("") : fast_log(rp.s) + rp.m;
  if (VBH_IN_SPAN(so.lse, lse_out + row, sizeof(float))) lse_out[row] = lse;
  const int64_t label = read_label(labels, label_i64, row, sb);
  float l = 0.f, z = 0.f;
  if (label != c.ignored_index) {
    const int64_t adj = label - c.class_start;
    const bool in_row = adj >= 0 && adj < n_cols;
    if (!c.split) {
      const float base = in_row ? lse : (c.has_smoothing ? c.smoothing * lse : 0.f);
      z = c.lse_square_scale * lse * lse;
      l = base + rest + z;
    } else {
      l = rest;
    }
  }
  if (VBH_IN_SPAN(so.loss, loss + row, sizeof(float))) loss[row] = l;
  if (VBH_IN_SPAN(so.z, z_out + row, sizeof(float))) z_out[row] = z;
}

// Backward: elementwise over the rows.  One 256-lane workgroup per tile of
// 256 vectors of one row (one 16-byte vector per lane, the shape of the copy
// kernel that sets the measured peak); the row's label, dloss and lse are
// read once per workgroup.
constexpr int kBwdLanes = kCeBwdLanes;

// Per-row factors of the backward: p = exp(x * logit_scale - lse) is computed as
// 2^(x * exp_scale - lb) * 2^-res with lb = lse * log2 e rounded and res its
// rounding error (exact, one FMA), so each element costs one FMA ahead of
// v_exp_f32; 2^-res rides on the factor (1 + 2 * lss * lse) that multiplies p.
// Rows whose lse is too large for that form (shift_fma_ok; `form` 0) take
// exp(x * logit_scale - lse) on a multiply and a subtract, with pf = 1 + 2 * lss * lse.
struct CeBwdRow {
  float lse, lb, pf, hit, smooth_neg, scale;
  int form;  // ce_grad's FORM for the row
};

// dlogits of one element: q = p + 2 * lss * lse * p, minus the (smoothed)
// one-hot (`is_label`); times dloss * logit_scale.  FMA: the row's form of p.
// FORM 1: the FMA form (scale 1); 2: the FMA form on the rounded product
// x * logit_scale (any other scale: x * exp_scale would carry exp_scale's own
// rounding, |x * scale| * 2^-24 in the exponent, where the golden rounds the
// product and subtracts lse); 0: the subtract form.
template <int FORM>
__device__ __forceinline__ float ce_grad(float xv, bool is_label, const CeBwdRow& b,
                                         const CeScalars& c) {
  const float p =
      FORM == 1   ? __builtin_amdgcn_exp2f(fmaf(xv, c.exp_scale, -b.lb))
      : FORM == 2 ? __builtin_amdgcn_exp2f(fmaf(mul_rn(xv, c.logit_scale), kLog2e, -b.lb))
                  : fast_exp(mul_rn(xv, c.logit_scale) - b.lse);
  float q = p * b.pf;
  if (is_label) q = q - b.hit;
  if (c.has_smoothing) q = q - b.smooth_neg;
  return b.scale * q;
}

// MIS: rows not a multiple of V long (same offset within a vector for logits
// and dlogits rows): tiles cover the row's aligned body; tile 0 also writes
// the scalar head (before the first 16-byte boundary) and tail elements.
template <typename T, int V, int SP, bool MIS>
__global__ __launch_bounds__(kBwdLanes) void ce_bwd_tiles(
    const float* __restrict__ dloss, const T* __restrict__ logits,
    const float* __restrict__ lse, const void* __restrict__ labels, int label_i64,
    T* __restrict__ dlogits, int n_cols, uint32_t tiles_per_row, int64_t ld_in,
    int64_t ld_out, int64_t dloss_stride, CeScalars c) {
  const uint32_t row32 = blockIdx.x / tiles_per_row;
  const int tix = static_cast<int>(blockIdx.x - row32 * tiles_per_row);
  const int j0 = tix * kBwdLanes;
  const int64_t row = row32;
  const int64_t in0 = row * ld_in;
  int head = 0, nvec = n_cols / V, tail = 0;
  if constexpr (MIS) {
    head = static_cast<int>((V - in0 % V) % V);
    if (head > n_cols) head = n_cols;
    nvec = (n_cols - head) / V;
    tail = n_cols - head - nvec * V;
  }
  const T* lr = logits + in0 + head;     // 16-byte aligned body
  T* dr = dlogits + row * ld_out + head;
  // the grid is the row count times tiles_per_row
  [[maybe_unused]] const int64_t n_rows = gridDim.x / tiles_per_row;
  const Span sx = VBH_SPAN(logits, strided_extent(n_rows, ld_in, n_cols));
  const Span sd = VBH_SPAN(dlogits, strided_extent(n_rows, ld_out, n_cols));
  const Span sdl = VBH_SPAN(dloss, strided_extent(n_rows, dloss_stride, 1));
  const Span sl = VBH_SPAN(lse, n_rows), sb = VBH_LABEL_SPAN(labels, label_i64, n_rows);
  const int j = j0 + static_cast<int>(threadIdx.x);
  // the tile's logits load goes out first; the row's label, dloss and lse
  // (independent loads: dloss is read for ignored rows too) while it is in flight
  typename Raw<T, V>::type r{};
  if (j < nvec) r = load_raw<T, V, SP != kStoreCached>(lr + static_cast<int64_t>(j) * V, sx);
  const int64_t label = read_label(labels, label_i64, row, sb);
  float dlv, lse_r;
  load_f32<float, 1>(dloss + row * dloss_stride, &dlv, sdl);
  load_f32<float, 1>(lse + row, &lse_r, sl);
  const float dl = label != c.ignored_index ? dlv : 0.f;
  const int64_t adj = label - c.class_start;
  CeBwdRow b;
  b.lse = lse_r;
  // the workgroup's tile is one row's: a scalar branch on the row's form
  const bool fma = __builtin_amdgcn_readfirstlane(static_cast<int>(shift_fma_ok(lse_r))) != 0;
  b.form = fma ? (c.logit_scale == 1.f ? 1 : 2) : 0;
  b.lb = lse_r * kLog2e;
  b.pf = (fma ? __builtin_amdgcn_exp2f(-shift_residual(lse_r, b.lb)) : 1.0f) *
         (1.0f + c.two_lse_square_scale * lse_r);
  // (dl * logit_scale) is a Python-double product in the golden
  b.scale = static_cast<float>(static_cast<double>(dl) * c.logit_scale);
  b.smooth_neg = c.has_smoothing ? c.smooth_negative : 0.f;
  b.hit = c.has_smoothing ? c.one_minus_smoothing : 1.0f;
  const int tile = nvec - j0 < kBwdLanes ? nvec - j0 : kBwdLanes;  // <= 0: no body here
  const OutWindow<T, SP> out(dr + static_cast<int64_t>(j0) * V,
                             static_cast<int64_t>(tile > 0 ? tile : 0) * V);
  if (j < nvec) {
    const int64_t rel = adj - head - static_cast<int64_t>(j) * V;  // label's place in r
    float o[V];
    if (b.form == 1) {
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = ce_grad<1>(raw_at<T, V>(r, k), rel == k, b, c);
    } else if (b.form == 2) {
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = ce_grad<2>(raw_at<T, V>(r, k), rel == k, b, c);
    } else {
#pragma unroll
      for (int k = 0; k < V; ++k) o[k] = ce_grad<0>(raw_at<T, V>(r, k), rel == k, b, c);
    }
    out.template store<V>(dr + static_cast<int64_t>(j) * V, static_cast<int>(threadIdx.x) * V, o,
                          sd);
  }
  if (MIS && tix == 0) {
    const int t = static_cast<int>(threadIdx.x);
    auto grad = [&](float v, bool is_label) {
      return b.form == 1   ? ce_grad<1>(v, is_label, b, c)
             : b.form == 2 ? ce_grad<2>(v, is_label, b, c)
                           : ce_grad<0>(v, is_label, b, c);
    };
    if (t < head) {
      float v;
      load_f32<T, 1>(logits + in0 + t, &v, sx);
      const float o = grad(v, adj == t);
      store_from_f32<T, 1>(dr - head + t, &o, sd);
    }
    if (t < tail) {
      const int64_t k = static_cast<int64_t>(nvec) * V + t;
      float v;
      load_f32<T, 1>(lr + k, &v, sx);
      const float o = grad(v, adj == head + k);
      store_from_f32<T, 1>(dr + k, &o, sd);
    }
  }
}

}  // namespace

hipError_t launch_cross_entropy_fwd(const CeArgs& a, const Geometry& g, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  CeScalars c =
      make_scalars(a.smoothing, a.logit_scale, a.lse_square_scale, a.total_classes,
                   a.ignored_index, a.class_start, a.has_smoothing, a.split);
  c.empty_neg_inf = a.empty_neg_inf;
  c.pair_out = a.pair_out;
  const int64_t nseg = a.n_rows * a.ncb;
  dispatch_float_type(a.logits_dt, [&](auto tt) {
    using T = typename decltype(tt)::type;
    constexpr int VN = Vec<T>::n;
    auto go = [&](auto vc) {
      constexpr int V = decltype(vc)::value;
      if (g.stream) {
        launch_kernel((ce_fwd_stream<T, V>), dim3(nseg), dim3(g.block), 0, s,
                           static_cast<const T*>(a.logits), a.labels, a.label_i64, a.loss,
                           a.lse, a.z_loss, a.n_rows, a.n_cols, a.ld, a.block_size, a.ncb,
                           c);
        err = hipGetLastError();
        return;
      }
      dispatch_maxit(g.maxit, [&](auto mc) {
        constexpr int M = decltype(mc)::value;
        if constexpr (M <= lane_cap(V)) {
          auto launch = [&](auto kern) {
            launch_kernel(kern, dim3(grid_for(nseg, g)), dim3(g.block), 0, s,
                               static_cast<const T*>(a.logits), a.labels, a.label_i64, a.loss,
                               a.lse, a.z_loss, a.n_rows, a.n_cols, a.ld, a.block_size, a.ncb,
                               g.tpr, c);
            err = hipGetLastError();
          };
          auto pick = [&](auto sl) {
            constexpr bool SL = decltype(sl)::value;
            if (V > 1 && g.mis) launch(ce_fwd_rows<T, V, M, true, V != 1, SL>);
            else if (g.nt) launch(ce_fwd_rows<T, V, M, true, false, SL>);
            else launch(ce_fwd_rows<T, V, M, false, false, SL>);
          };
          if (c.has_smoothing || c.empty_neg_inf) pick(std::true_type{});
          else pick(std::false_type{});
        }
      });
    };
    if (g.v == 1) go(std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, VN>{});
  });
  return err;
}

bool cross_entropy_fwd_persist_fits(int logits_dtype, int64_t n_cols) {
  return logits_dtype == kF32 && n_cols % 4 == 0 && n_cols / 4 >= kCePersistChunk &&
         n_cols * 4 < (int64_t(1) << 30);
}

int64_t cross_entropy_fwd_persist_chunk_cols() { return int64_t(kCePersistChunk) * 4; }

// Chunks per CU from which the launcher's default takes 256-lane workgroups
// (measured on MI355X; see ce_fwd_persist).
constexpr int64_t kCePersistWideChunksPerCu = 64;

hipError_t launch_cross_entropy_fwd_persist(const CeArgs& a, int64_t max_grid, int lanes,
                                            hipStream_t s) {
  if (!cross_entropy_fwd_persist_fits(a.logits_dt, a.n_cols) || a.ncb != 1 || a.pair_out ||
      a.empty_neg_inf || (lanes != 0 && lanes != 256 && lanes != 512))
    return hipErrorInvalidValue;
  const CeScalars c =
      make_scalars(a.smoothing, a.logit_scale, a.lse_square_scale, a.total_classes,
                   a.ignored_index, a.class_start, a.has_smoothing, a.split);
  if (lanes == 0) {
    const int64_t cpr = (a.n_cols / 4 + kCePersistChunk - 1) / kCePersistChunk;
    const int64_t cus = resident_blocks(
        reinterpret_cast<const void*>(ce_fwd_persist<false, int64_t, true, 256>), 256, 1);
    lanes = a.n_rows * cpr >= kCePersistWideChunksPerCu * cus ? 256 : 512;
  }
  hipError_t err = hipErrorInvalidValue;
  auto launch = [&](auto kern, auto labels, int block) {
    const int64_t cus = resident_blocks(reinterpret_cast<const void*>(kern), block, 1);
    int64_t grid = std::min<int64_t>(a.n_rows, std::max<int64_t>(cus, 1));
    if (max_grid > 0) grid = std::min(grid, max_grid);
    launch_kernel(kern, dim3(grid), dim3(block), 0, s, static_cast<const float*>(a.logits),
                  labels, a.loss, a.lse, a.z_loss, a.n_rows, a.n_cols, a.ld, c);
    err = hipGetLastError();
  };
  auto pick = [&](auto lt, auto lc) {
    using LabelT = typename decltype(lt)::type;
    constexpr int L = decltype(lc)::value;
    const LabelT* labels = static_cast<const LabelT*>(a.labels);
    if (c.logit_scale == 1.f) {
      if (c.has_smoothing) launch(ce_fwd_persist<true, LabelT, true, L>, labels, L);
      else launch(ce_fwd_persist<false, LabelT, true, L>, labels, L);
    } else {
      if (c.has_smoothing) launch(ce_fwd_persist<true, LabelT, false, L>, labels, L);
      else launch(ce_fwd_persist<false, LabelT, false, L>, labels, L);
    }
  };
  auto by_labels = [&](auto lc) {
    if (a.label_i64) pick(TypeTag<int64_t>{}, lc);
    else pick(TypeTag<int32_t>{}, lc);
  };
  if (lanes == 256) by_labels(std::integral_constant<int, 256>{});
  else by_labels(std::integral_constant<int, 512>{});
  return err;
}

hipError_t launch_cross_entropy_combine(const CeArgs& a, const float* seg_loss,
                                        const float* seg_sum, const float* seg_max, int segs,
                                        hipStream_t s) {
  const CeScalars c =
      make_scalars(a.smoothing, a.logit_scale, a.lse_square_scale, a.total_classes,
                   a.ignored_index, a.class_start, a.has_smoothing, a.split);
  launch_kernel(ce_combine,
                dim3((a.n_rows + kCombineRowsPerBlock - 1) / kCombineRowsPerBlock),
                dim3(kCombineRowsPerBlock * kWave), 0, s, seg_loss, seg_sum, seg_max, a.labels,
                a.label_i64, a.loss, a.lse, a.z_loss, a.n_rows, a.n_cols, segs, c);
  return hipGetLastError();
}

hipError_t launch_cross_entropy_bwd(const CeBwdArgs& a, hipStream_t s) {
  hipError_t err = hipErrorInvalidValue;
  const CeScalars c =
      make_scalars(a.smoothing, a.logit_scale, a.lse_square_scale, a.total_classes,
                   a.ignored_index, a.class_start, a.has_smoothing, 0);
  Geometry g;
  g.nt = a.nt != 0;
  g.wt = a.wt != 0;
  dispatch_float_type(a.logits_dt, [&](auto tt) {
    using T = typename decltype(tt)::type;
    constexpr int VN = Vec<T>::n;
    auto go = [&](auto vc) {
      constexpr int V = decltype(vc)::value;
      const int64_t nvec = a.n_cols / V;
      const int64_t tiles = (nvec + kBwdLanes - 1) / kBwdLanes;
      dispatch_store_policy<V>(g, [&](auto sp) {
        constexpr int SP = decltype(sp)::value;
        auto launch = [&](auto kern) {
          launch_kernel(kern, dim3(a.n_rows * tiles), dim3(kBwdLanes), 0, s, a.dloss,
                             static_cast<const T*>(a.logits), a.lse, a.labels, a.label_i64,
                             static_cast<T*>(a.dlogits), a.n_cols, static_cast<uint32_t>(tiles),
                             a.ld_logits, a.ld_dlogits, a.dloss_stride, c);
        };
        if (V > 1 && a.mis) launch(ce_bwd_tiles<T, V, SP, V != 1>);
        else launch(ce_bwd_tiles<T, V, SP, false>);
      });
      err = hipGetLastError();
    };
    if (a.vec == 1) go(std::integral_constant<int, 1>{});
    else go(std::integral_constant<int, VN>{});
  });
  return err;
}

}  // namespace vbh

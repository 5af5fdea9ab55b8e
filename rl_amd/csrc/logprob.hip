// Selected-token log-probabilities over the vocabulary: forward (online
// log-sum-exp with the target gather fused in) and backward (softmax
// recomputed from the saved row statistics, one read + one write).
//
// Semantics follow nemo_rl/distributed/model_utils.py:87-135 and :228-349
// (ChunkedDistributedLogprob with a vocab group of size 1).  Chunking along
// the sequence only changes how the reference schedules work; every row here
// is independent, so the result does not depend on any chunk size.
//
// Layout: one workgroup of W waves owns one row of V logits.  Each lane
// streams 16-byte vectors (8 bf16 / 4 fp32) at stride 64*W vectors, U vectors
// in flight per lane, and keeps a private (offset, sum) pair; lanes and waves
// are merged once at the end of the row.  Nothing of size V is ever written
// in the forward.  The backward walks the gradient as one flat block of 8 KB
// pieces when logits and gradient share a contiguous layout, and row by row
// (zero rows first, then rows with a non-zero upstream gradient) otherwise.

#include "common.h"

// Offsets and rescale factors below rely on exact fp32 rounding of each
// product; contractions are written out explicitly with fmaf where wanted.
#pragma clang fp contract(off)

namespace mirl {
namespace {

// Per-lane log-sum-exp state kept in base-2 "offset" form: the running sum is
// sum_i 2^(x_i*log2e - off) with off = fl(m*log2e), m the running max.
// Four partial sums break the add dependency chain.
struct LseState {
  float m = -INFINITY;
  float off = 0.f;
  float s[4] = {0.f, 0.f, 0.f, 0.f};

  template <int N>
  __device__ __forceinline__ void add(const float (&v)[N]) {
    float bm = v[0];
#pragma unroll
    for (int i = 1; i < N; ++i) bm = fmaxf(bm, v[i]);
    const float mn = fmaxf(m, bm);
    if (mn == -INFINITY) return;  // nothing finite yet on this lane
    if (mn != m) {
      const float noff = mn * kLog2e;
      // m == -inf gives 2^-inf = 0, which is the correct (empty) rescale.
      const float sc = (m == -INFINITY) ? 0.f : fast_exp2(off - noff);
#pragma unroll
      for (int k = 0; k < 4; ++k) s[k] *= sc;
      m = mn;
      off = noff;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) s[i & 3] += fast_exp2(fmaf(v[i], kLog2e, -off));
  }
};

// Streams one row of V logits through per-lane online log-sum-exp states and
// merges lanes and waves.  On thread 0 it returns the row max M and
// logsum = log(sum exp(x - M)); other threads' outputs are unspecified.
// `between` runs once, after the first batch of loads is issued, so that the
// caller's own scalar loads overlap the row's first vector loads.  With
// 0 <= pick < V, *picked (thread 0) is x[pick], taken from the streamed
// values by the lane that holds it (no load of its own that would have to wait
// for the target index), and 0 otherwise.
template <class E, int W, int U, class F>
__device__ __forceinline__ void row_lse(const typename E::raw* x, int64_t V, int tid, F&& between,
                                        float& M_out, float& logsum_out, int64_t pick = -1,
                                        float* picked = nullptr) {
  constexpr int NT = 64 * W;
  constexpr int VEC = E::kVec;
  constexpr int BATCH = U * NT;  // vectors per workgroup per batch
  const RowSpan<E> span(x, V);
  const vu4* xv = reinterpret_cast<const vu4*>(x + span.head);
  const int nvec = (int)span.nvec;
  const int nbatch = (nvec + BATCH - 1) / BATCH;

  // Every batch is U loads per lane issued together; lanes past the end of the
  // row read the row's last vector again and take -inf in its place, which
  // leaves the running max and sum unchanged.  Masking the last batch instead of
  // finishing it one vector at a time keeps the whole row's loads in flight when
  // a lane has only one batch (short rows); issuing every load unconditionally
  // (the mask applied where the values are used) lets the scalar loads that
  // follow go out while the batch is still in flight.
  vu4 q[U];
  uint32_t live = 0;  // bit u: vector u of the batch is inside the row
  auto issue = [&](int base) {
    live = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = base + u * NT;
      q[u] = __builtin_nontemporal_load(xv + min(j, nvec - 1));
      live |= (j < nvec ? 1u : 0u) << u;
    }
  };
  if (nbatch > 0) issue(tid);
  between();
  // scalar head and tail elements (fewer than 2*VEC per row)
  float ht[2];
  ht[0] = (tid < span.head) ? E::load(x + tid) : -INFINITY;
  const int64_t ti = span.tail0 + tid;
  ht[1] = (ti < V) ? E::load(x + ti) : -INFINITY;
  // keep the batch's loads ahead of the arithmetic that consumes them
  __builtin_amdgcn_sched_barrier(0);

  // the picked element's vector and position in it (pvec = -1: in the head or
  // tail, or no pick)
  const bool want = picked != nullptr && pick >= 0 && pick < V;
  const int64_t pb = want ? pick - span.head : -1;
  const int pvec = (pb >= 0 && pb < (int64_t)nvec * VEC) ? (int)(pb / VEC) : -1;
  const int pel = pvec >= 0 ? (int)(pb - (int64_t)pvec * VEC) : 0;
  float pv = 0.f;
  LseState st;
  for (int k = 0; k < nbatch; ++k) {
    float v[U * VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float w[VEC];
      E::unpack(q[u], w);
      const bool in_row = ((live >> u) & 1u) != 0u;
#pragma unroll
      for (int e = 0; e < VEC; ++e) v[u * VEC + e] = in_row ? w[e] : -INFINITY;
      if (tid + k * BATCH + u * NT == pvec) {
#pragma unroll
        for (int e = 0; e < VEC; ++e)
          if (e == pel) pv = w[e];
      }
    }
    st.add(v);
    if (k + 1 < nbatch) issue(tid + (k + 1) * BATCH);
    __builtin_amdgcn_sched_barrier(0);
  }
  st.add(ht);
  if (want && pvec < 0) {
    if (tid == pick) pv = ht[0];
    if (ti == pick) pv = ht[1];
  }

  // merge lanes: the row max and the sum re-based to it
  float M = wave_max(st.m);
  float s = st.s[0] + st.s[1] + st.s[2] + st.s[3];
  const float OFF = M * kLog2e;
  s = (st.m == -INFINITY) ? 0.f : s * fast_exp2(st.off - OFF);
  s = wave_sum(s);
  // one lane holds the picked value, every other lane 0: the sums are exact
  if (want) pv = wave_sum(pv);
  if constexpr (W > 1) {
    __shared__ float sm[W], ss[W], sp[W];
    const int wv = tid / 64, lane = tid % 64;
    if (lane == 0) {
      sm[wv] = M;
      ss[wv] = s;
      sp[wv] = pv;
    }
    __syncthreads();
    if (tid == 0) {
      float Mb = sm[0];
#pragma unroll
      for (int k = 1; k < W; ++k) Mb = fmaxf(Mb, sm[k]);
      const float OFFb = Mb * kLog2e;
      float sb2 = 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k)
        sb2 += (sm[k] == -INFINITY) ? 0.f : ss[k] * fast_exp2(sm[k] * kLog2e - OFFb);
      M = Mb;
      s = sb2;
      if (want) {
        float pt = 0.f;
#pragma unroll
        for (int k = 0; k < W; ++k) pt += sp[k];
        pv = pt;
      }
    }
  }
  if (picked != nullptr) *picked = pv;
  // s = sum 2^(x*log2e - fl(M*log2e)); undo the rounding of the offset so
  // that logsum = log(sum exp(x - M)).
  const float corr = fmaf(M, kLog2e, -(M * kLog2e));
  M_out = M;
  logsum_out = logf(s) - corr * 0.6931471805599453f;
}

template <class E, int W, int U>
__global__ __launch_bounds__(64 * W) void logprob_fwd_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t V, int64_t sb, int64_t sr,
    const int64_t* __restrict__ target, int64_t tsb, int64_t tsr, int64_t vs, int64_t ve,
    float* __restrict__ out, float* __restrict__ stats) {
  const int64_t row = blockIdx.x;
  const int64_t b = row / R;
  const int64_t r = row - b * R;
  const typename E::raw* x = logits + b * sb + r * sr;
  const int tid = threadIdx.x;

  const int64_t t = target[b * tsb + r * tsr];
  // targets outside the vocabulary slice (or past this row) carry no one-hot
  const bool tmask = (t < vs) || (t >= ve) || (t - vs >= V);
  const int64_t tl = tmask ? -1 : (t - vs);
  float xt = 0.f, M, logsum;
  row_lse<E, W, U>(x, V, tid, [] {}, M, logsum, tl, &xt);
  if (tid == 0) {
    const float lp = (xt - M) - logsum;
    out[row] = tmask ? 0.f : lp;
    if (stats != nullptr) {
      stats[2 * row] = M;
      stats[2 * row + 1] = logsum;
    }
  }
}

// Logprobs at K given vocabulary ids per row (ChunkedDistributedGatherLogprob,
// reference model_utils.py:691-748): the row's log-sum-exp as in
// logprob_fwd_kernel, then out[row, k] = (x[id_k] - M) - logsum for ids in
// [vs, ve) and 0 for the others.  Thread k < 64*W loads x[id_k] while the
// row's first loads are in flight (as the single-target kernel does with its
// target); ids beyond the first 64*W are read after the row.
template <class E, int W, int U>
__global__ __launch_bounds__(64 * W) void gather_logprob_fwd_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t V, int64_t sb, int64_t sr,
    const int64_t* __restrict__ idx, int64_t K, int64_t isb, int64_t isr, int64_t isk,
    int64_t vs, int64_t ve, float* __restrict__ out, float* __restrict__ stats) {
  constexpr int NT = 64 * W;
  const int64_t row = blockIdx.x;
  const int64_t b = row / R;
  const int64_t r = row - b * R;
  const typename E::raw* x = logits + b * sb + r * sr;
  const int tid = threadIdx.x;
  const int64_t* ir = idx + b * isb + r * isr;
  const bool mine = tid < K;
  const int64_t t = mine ? ir[tid * isk] : 0;
  const bool in_range = mine && (t >= vs) && (t < ve) && (t - vs < V);
  float xk = 0.f, M, logsum;
  row_lse<E, W, U>(x, V, tid, [&] { if (in_range) xk = E::load(x + (t - vs)); }, M, logsum);
  __shared__ float sh[2];
  if (tid == 0) {
    sh[0] = M;
    sh[1] = logsum;
    if (stats != nullptr) {
      stats[2 * row] = M;
      stats[2 * row + 1] = logsum;
    }
  }
  __syncthreads();
  M = sh[0];
  logsum = sh[1];
  if (mine) out[row * K + tid] = in_range ? (xk - M) - logsum : 0.f;
  for (int64_t k = NT + tid; k < K; k += NT) {
    const int64_t tk = ir[k * isk];
    const bool ok = (tk >= vs) && (tk < ve) && (tk - vs < V);
    out[row * K + k] = ok ? (E::load(x + (tk - vs)) - M) - logsum : 0.f;
  }
}

// The backward runs in two launches over the same grid of rows:
//   kZeroRows    rows whose upstream gradient is exactly 0 (masked prompt and
//                padding positions, rows past R): write zeros, never read;
//   kActiveRows  all other rows: read the logits row, write the gradient.
// Keeping the write-only traffic apart from the read+write traffic lets each
// phase run at its own HBM efficiency instead of a blend of the two
// (measured on MI355X: 1.42 ms vs 1.55 ms for one mixed launch on the
// [8, 2048, 151936] bf16 GRPO workload).
enum BwdPhase { kZeroRows = 0, kActiveRows = 1 };

template <class E, int W, int U, int PHASE>
__global__ __launch_bounds__(64 * W) void logprob_bwd_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t Rt, int64_t V, int64_t sb,
    int64_t sr, const int64_t* __restrict__ target, int64_t tsb, int64_t tsr, int64_t vs,
    int64_t ve, const float* __restrict__ stats, const float* __restrict__ g, int64_t gsb,
    int64_t gsr, typename E::raw* gin, int64_t gisb, int64_t gisr) {
  using raw = typename E::raw;
  constexpr int NT = 64 * W;
  constexpr int VEC = E::kVec;
  const int64_t row = blockIdx.x;
  const int64_t b = row / Rt;
  const int64_t r = row - b * Rt;
  const int tid = threadIdx.x;
  raw* y = gin + b * gisb + r * gisr;
  const float gv = (r < R) ? g[b * gsb + r * gsr] : 0.f;
  const RowSpan<E> ys(y, V);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  const int nvec = (int)ys.nvec;

  if (gv == 0.f) {
    // (onehot - p) * 0 == 0: write the row without reading the logits.
    if constexpr (PHASE != kZeroRows) return;
    const raw z = E::from_float(0.f);
    if (tid < ys.head) y[tid] = z;
    if (ys.tail0 + tid < V) y[ys.tail0 + tid] = z;
    // Nontemporal stores: plain stores leave the memory-side cache full of
    // dirty lines whose write-back slows the next read-heavy kernel (the
    // following forward) by ~30%; streaming stores do not.
    const vu4 zq = vu4{0u, 0u, 0u, 0u};
    int i = tid;
    for (; i + (U - 1) * NT < nvec; i += U * NT) {
#pragma unroll
      for (int u = 0; u < U; ++u) __builtin_nontemporal_store(zq, yv + i + u * NT);
    }
    for (; i < nvec; i += NT) __builtin_nontemporal_store(zq, yv + i);
    return;
  }
  if constexpr (PHASE != kActiveRows) return;

  const raw* x = logits + b * sb + r * sr;
  const int64_t srow = b * R + r;
  const float M = stats[2 * srow];
  const float LS = stats[2 * srow + 1];
  const int64_t t = target[b * tsb + r * tsr];
  // targets outside the vocabulary slice (or past this row) carry no one-hot
  const bool tmask = (t < vs) || (t >= ve) || (t - vs >= V);
  const int64_t tl = tmask ? -1 : (t - vs);

  const RowSpan<E> xs(x, V);
  if (xs.head != ys.head) {
    // Input and output rows are not co-aligned: element-wise path.
    for (int64_t j = tid; j < V; j += NT) {
      const float p = fast_exp2(((E::load(x + j) - M) - LS) * kLog2e);
      const float o = (j == tl) ? (1.f - p) * gv : -p * gv;
      y[j] = E::from_float(o);
    }
    return;
  }
  auto scalar = [&](int64_t j) {
    const float p = fast_exp2(((E::load(x + j) - M) - LS) * kLog2e);
    y[j] = E::from_float((j == tl) ? (1.f - p) * gv : -p * gv);
  };
  if (tid < ys.head) scalar(tid);
  if (ys.tail0 + tid < V) scalar(ys.tail0 + tid);

  const vu4* xv = reinterpret_cast<const vu4*>(x + xs.head);
  // vector index holding the target (or -1)
  const int tv = (tl >= xs.head && tl < xs.tail0) ? (int)((tl - xs.head) / VEC) : -1;
  const int tj = (tv >= 0) ? (int)((tl - xs.head) - (int64_t)tv * VEC) : 0;
  const float ng = -gv;
  auto grad_vec = [&](const vu4& q, int vi) -> vu4 {
    float w[VEC];
    E::unpack(q, w);
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = fast_exp2(((w[k] - M) - LS) * kLog2e) * ng;
    if (vi == tv) {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (k == tj) o[k] = (1.f - fast_exp2(((w[k] - M) - LS) * kLog2e)) * gv;
    }
    return E::pack(o);
  };
  int i = tid;
  for (; i + (U - 1) * NT < nvec; i += U * NT) {
    vu4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = __builtin_nontemporal_load(xv + i + u * NT);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(grad_vec(q[u], i + u * NT), yv + i + u * NT);
  }
  for (; i < nvec; i += NT) __builtin_nontemporal_store(grad_vec(__builtin_nontemporal_load(xv + i), i), yv + i);
}

// `flags` (nflags ints, or null) makes a launch conditional: it does nothing
// unless some flag is set (the early-backward recheck's redo).  Each thread
// loads at most a few flags and the workgroup ORs them in one barrier (a
// serial loop over 64 flags per thread measured 13 us for a launch that then
// did nothing); every thread of the workgroup must call it.
__device__ __forceinline__ bool any_flag(const int* __restrict__ flags, int nflags) {
  if (flags == nullptr) return true;
  int v = 0;
  for (int k = threadIdx.x; k < nflags; k += blockDim.x) v |= flags[k];
  return __syncthreads_or(v) != 0;
}

// Backward over a contiguous [B, Rt, V] gradient whose logits share its layout
// (V a multiple of the vector width, both 16-byte aligned): one 4 KB piece of
// the flat gradient per 128-thread workgroup (two 16-byte vectors per lane,
// 2 KB apart), piece boundaries on 4 KB addresses.  Each lane finds the rows
// of its two vectors and loads their upstream gradient, statistics and target
// together; vectors of rows with a zero upstream gradient are written as zeros
// without reading the logits, the others get (onehot - p) * g.  Short
// workgroups dispatched in order keep the traffic inside a narrow address
// window.  Measured on MI355X (backward of the [8, 2048, 151936] GRPO rows /
// of the [1, 32768, 131072] rows): 128 x 2 vectors with nontemporal loads
// 1.198 / 2.722 ms; 256 x 2 with plain loads 1.231 / 2.849 ms; one vector per
// lane (the per-vector row lookups dominate) 1.34-1.45 / 3.07-3.19 ms; 256 x 4
// and 512 x 2 1.30-1.34 / 2.92 ms.  Arithmetic is that of logprob_bwd_kernel.
constexpr int kFlatThreads = 128;
constexpr int kFlatVecs = 2;

struct FlatBwd {
  const void* logits;
  int64_t R;
  uint32_t Rt, nvr, nvec;
  int shift;
  const int64_t* target;
  int64_t tsb, tsr, vs, ve, V;
  const float* stats;
  const float* g;
  int64_t gsb, gsr;
  void* gin;
  const float* gu;  // redo only: the [B, R] upstream gradient the gradient was formed with
};

// One span of NT * U 16-byte vectors (piece `piece` of that size; 256 vectors
// is a 4 KB piece) by a workgroup of NT threads, U vectors per lane NT
// vectors apart.  SKIP (the redo): vectors of rows whose upstream gradient
// equals A.gu's bit for bit already hold what this would write (same
// arithmetic from the same inputs) and are neither read nor written; rows past
// R hold zeros either way.
template <class E, int NT, int U, bool SKIP = false>
__device__ __forceinline__ void bwd_flat_piece(const FlatBwd& A, int64_t piece) {
  static_assert((NT * U) % (kFlatThreads * kFlatVecs) == 0, "whole 4 KB pieces");
  constexpr int VEC = E::kVec;
  const int64_t R = A.R, vs = A.vs, ve = A.ve, V = A.V;
  const uint32_t Rt = A.Rt, nvr = A.nvr, nvec = A.nvec;
  const float* __restrict__ stats = A.stats;
  const float* __restrict__ g = A.g;
  const int64_t* __restrict__ target = A.target;
  const int64_t gsb = A.gsb, gsr = A.gsr, tsb = A.tsb, tsr = A.tsr;
  vu4* yv = static_cast<vu4*>(A.gin);
  const vu4* xv = static_cast<const vu4*>(A.logits);
  const int64_t base = piece * (NT * U) + threadIdx.x - A.shift;
  bool ok[U];
  uint32_t row[U];
  float gv[U], M[U], LS[U];
  int64_t t[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + u * NT;
    ok[u] = i >= 0 && i < (int64_t)nvec;
    row[u] = (ok[u] ? (uint32_t)i : 0u) / nvr;
    const uint32_t b = row[u] / Rt, r = row[u] - b * Rt;
    gv[u] = 0.f;
    M[u] = LS[u] = 0.f;
    t[u] = -1;
    if (SKIP && (int64_t)r >= R) ok[u] = false;
    if (ok[u] && (int64_t)r < R) {
      const int64_t srow = (int64_t)b * R + r;
      gv[u] = g[(int64_t)b * gsb + (int64_t)r * gsr];
      if (SKIP && __float_as_uint(gv[u]) == __float_as_uint(A.gu[srow])) ok[u] = false;
      M[u] = stats[2 * srow];
      LS[u] = stats[2 * srow + 1];
      t[u] = target[(int64_t)b * tsb + (int64_t)r * tsr];
    }
  }
  // Nontemporal loads and stores: with 4 KB pieces the streaming loads measured
  // 2-4% faster than plain ones, and plain stores slow both this kernel and the
  // next forward by ~15% (they leave the memory-side cache full of dirty lines).
  vu4 q[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (ok[u] && gv[u] != 0.f) q[u] = __builtin_nontemporal_load(xv + base + u * NT);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    const int64_t i = base + u * NT;
    if (gv[u] == 0.f) {
      // (onehot - p) * 0 == 0: written without reading the logits
      __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + i);
      continue;
    }
    const bool tmask = (t[u] < vs) || (t[u] >= ve) || (t[u] - vs >= V);
    const int64_t j0 = (int64_t)((uint32_t)i - row[u] * nvr) * VEC;  // row element of lane 0
    const int tj = tmask ? -1 : (int)(t[u] - vs - j0);               // target lane, if here
    float w[VEC];
    E::unpack(q[u], w);
    const float ng = -gv[u];
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = fast_exp2(((w[k] - M[u]) - LS[u]) * kLog2e) * ng;
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      if (k == tj) o[k] = (1.f - fast_exp2(((w[k] - M[u]) - LS[u]) * kLog2e)) * gv[u];
    __builtin_nontemporal_store(E::pack(o), yv + i);
  }
}

template <class E>
__global__ __launch_bounds__(kFlatThreads) void logprob_bwd_flat_kernel(FlatBwd A) {
  bwd_flat_piece<E, kFlatThreads, kFlatVecs>(A, blockIdx.x);
}

// The early-backward recheck's redo on the flat schedule.  Launches with no
// flag set are the common case, and their cost is the number of (empty)
// workgroups dispatched; the redo itself is fastest with one workgroup per
// piece.  Compromise: single-wave workgroups in a grid-stride loop, kRedoGrid
// of them (two per wave slot, so the later ones fill slots that free up
// early), one 4 KB piece (four vectors per lane) per step.  Measured on the
// backward of the [8, 2048, 151936] bf16 GRPO rows: 1.50 ms and 15 us with no
// flag set; two pieces per step 1.54 ms; one two-wave workgroup per piece
// 1.26 ms but 0.28 ms with no flag set; two-wave workgroups over all 8192
// wave slots 1.62 ms.  The flags are tested per wave (one load per lane and a
// ballot, no barrier).  Same pieces and arithmetic as logprob_bwd_flat_kernel.
// SKIP: rows whose upstream gradient matched (the zero-gradient rows of a
// scaled loss) are left as the early backward wrote them.
constexpr int kRedoPieces = 1;  // 4 KB pieces per grid-stride step
template <class E, bool SKIP>
__global__ __launch_bounds__(64) void logprob_bwd_flat_redo_kernel(
    FlatBwd A, int64_t npieces, const int* __restrict__ flags, int nflags) {
  const int lane = threadIdx.x & 63;
  const int f = lane < nflags ? flags[lane] : 0;
  if (__ballot(f != 0) == 0ull) return;
  const int64_t nsteps = (npieces + kRedoPieces - 1) / kRedoPieces;
  for (int64_t step = blockIdx.x; step < nsteps; step += gridDim.x)
    bwd_flat_piece<E, 64, 4 * kRedoPieces, SKIP>(A, step);
}

// The early-backward recheck's redo over the listed rows only (the rows
// whose upstream gradient differs from the one the early backward used, in
// the check workgroups' lists): a grid-stride loop of waves over 8 KB pieces
// of those rows (64 lanes x 8 vectors), each piece inside one row, so the
// row's gradient, statistics and target are the wave's (scalar loads, the
// next piece's loaded while this one's logits are in flight).  The skipped
// rows cost nothing here, where the loop over every piece of every row spent
// a round trip of loads on each of theirs.  Measured on the scaled-loss redo
// of the [8, 2048, 151936] bf16 GRPO rows (5.30 GB): 0.99 ms with the check,
// 1.22 ms for the loop over every piece; 4 KB pieces 1.01 ms, 2 KB 1.02 ms.
// Same arithmetic as logprob_bwd_flat_kernel.  Launches whose counts are all
// zero return at once.
constexpr int kListRedoVecs = 8;  // 16-byte vectors per lane and piece
constexpr int kListRedoWaves = 4;
template <class E>
__global__ __launch_bounds__(64 * kListRedoWaves) void logprob_bwd_list_redo_kernel(
    FlatBwd A, const int* __restrict__ counts, int nblk, int64_t per,
    const int32_t* __restrict__ list) {
  constexpr int VEC = E::kVec, U = kListRedoVecs, PV = 64 * U;
  const int lane = threadIdx.x & 63;
  const uint32_t c = lane < nblk ? (uint32_t)counts[lane] : 0u;
  uint32_t incl = c;  // inclusive prefix of the counts over the lanes
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = (uint32_t)__shfl_up((int)incl, off, 64);
    if (lane >= off) incl += o;
  }
  const uint32_t total = (uint32_t)__shfl((int)incl, 63, 64);
  if (total == 0u) return;
  const uint32_t nvr = A.nvr;
  const uint32_t ppr = (nvr + PV - 1) / PV;
  const int64_t items = (int64_t)total * ppr;
  const int64_t R = A.R, vs = A.vs, ve = A.ve, V = A.V;
  const vu4* xv = static_cast<const vu4*>(A.logits);
  vu4* yv = static_cast<vu4*>(A.gin);
  // item it: piece pc of the row at list position k (wave-uniform values)
  auto row_of = [&](int64_t it, uint32_t& pc) -> int64_t {
    const uint32_t k = (uint32_t)(it / ppr);
    pc = (uint32_t)(it - (int64_t)k * ppr);
    // the check workgroup whose list holds position k
    const int blk = __popcll(__ballot(lane < nblk && incl <= k));
    const uint32_t excl = (uint32_t)__builtin_amdgcn_readlane((int)(incl - c), blk);
    return (int64_t)list[(int64_t)blk * per + (k - excl)];
  };
  struct RowData {
    float gv, M, LS;
    int64_t t;
  };
  auto data_of = [&](int64_t i) {
    const int64_t b = i / R, r = i - b * R;
    return RowData{A.g[b * A.gsb + r * A.gsr], A.stats[2 * i], A.stats[2 * i + 1],
                   A.target[b * A.tsb + r * A.tsr]};
  };
  const int64_t wstride = (int64_t)gridDim.x * kListRedoWaves;
  int64_t it = (int64_t)blockIdx.x * kListRedoWaves + (threadIdx.x >> 6);
  if (it >= items) return;
  uint32_t pc;
  int64_t i = row_of(it, pc);
  RowData d = data_of(i);
  // the next item's row and row data are loaded while this item's logits are
  // in flight
  for (;;) {
    const int64_t itn = it + wstride;
    const bool more = itn < items;
    uint32_t pcn = 0u;
    const int64_t in_ = more ? row_of(itn, pcn) : 0;
    const int64_t b = i / R, r = i - b * R;
    const int64_t rv = (b * (int64_t)A.Rt + r) * (int64_t)nvr;  // the row's first vector
    const uint32_t o0 = pc * PV + (uint32_t)lane;
    vu4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (d.gv != 0.f && o0 + u * 64 < nvr) q[u] = __builtin_nontemporal_load(xv + rv + o0 + u * 64);
    RowData dn{};
    if (more) dn = data_of(in_);
    const bool tmask = (d.t < vs) || (d.t >= ve) || (d.t - vs >= V);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t o = o0 + u * 64;
      if (o >= nvr) continue;
      if (d.gv == 0.f) {
        __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + rv + o);
        continue;
      }
      const int64_t j0 = (int64_t)o * VEC;  // row element of lane 0
      const int tj = tmask ? -1 : (int)(d.t - vs - j0);
      float w[VEC];
      E::unpack(q[u], w);
      const float ng = -d.gv;
      float out[VEC];
#pragma unroll
      for (int kk = 0; kk < VEC; ++kk) out[kk] = fast_exp2(((w[kk] - d.M) - d.LS) * kLog2e) * ng;
#pragma unroll
      for (int kk = 0; kk < VEC; ++kk)
        if (kk == tj) out[kk] = (1.f - fast_exp2(((w[kk] - d.M) - d.LS) * kLog2e)) * d.gv;
      __builtin_nontemporal_store(E::pack(out), yv + rv + o);
    }
    if (!more) break;
    it = itn;
    pc = pcn;
    i = in_;
    d = dn;
  }
}

// Backward of the K-id gather (reference model_utils.py:750-805):
//   grad = -p * sum_k g_k, plus g_k added at each in-range id_k, in fp32,
// rounded once to the logits dtype.  Three launches: gather_gsum_kernel forms
// sum_k g_k per row, the logprob backward writes the dense -p * gsum part (no
// target), and gather_fixup_kernel rewrites the <= K entries at the ids.  (A
// single launch that stages each 8 KB piece's ids in LDS measured slower on
// the [8, 2048, 151936] bf16 rows with 21 ids, 1.47 vs 1.30 ms: the staging
// round in front of every piece's logits load cuts the bytes in flight.)
//
// `flags` (nflags ints, or null) makes a launch conditional (the early-backward
// recheck's redo); any_flag above tests them.

__global__ __launch_bounds__(256) void gather_gsum_kernel(const float* __restrict__ g, int64_t R,
                                                         int64_t gsb, int64_t gsr, int64_t gsk,
                                                         int64_t K, int64_t rows,
                                                         float* __restrict__ gsum,
                                                         const int* __restrict__ flags, int nflags) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (!any_flag(flags, nflags) || row >= rows) return;
  const int64_t b = row / R, r = row - b * R;
  const float* gr = g + b * gsb + r * gsr;
  float s = 0.f;
  for (int64_t k = 0; k < K; ++k) s += gr[k * gsk];
  gsum[row] = s;
}

// One thread per (row, k).  The first occurrence of each in-range id in a row
// recomputes the dense value -p * gsum exactly as the dense pass formed it,
// adds the upstream gradient of every k' with the same id in k' order (the
// order of scatter_add), and stores the sum rounded to the dtype; repeated
// and out-of-range ids write nothing.
template <class E>
__global__ __launch_bounds__(256) void gather_fixup_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t V, int64_t sb, int64_t sr,
    const int64_t* __restrict__ idx, int64_t K, int64_t isb, int64_t isr, int64_t isk,
    int64_t vs, int64_t ve, const float* __restrict__ stats, const float* __restrict__ g,
    int64_t gsb, int64_t gsr, int64_t gsk, const float* __restrict__ gsum,
    typename E::raw* gin, int64_t gisb, int64_t gisr, int64_t total,
    const int* __restrict__ flags, int nflags) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (!any_flag(flags, nflags) || i >= total) return;
  const int64_t row = i / K, k = i - row * K;
  const int64_t b = row / R, r = row - b * R;
  const int64_t* ir = idx + b * isb + r * isr;
  const int64_t t = ir[k * isk];
  if (t < vs || t >= ve || t - vs >= V) return;
  for (int64_t j = 0; j < k; ++j)
    if (ir[j * isk] == t) return;
  const int64_t tl = t - vs;
  const float M = stats[2 * row], LS = stats[2 * row + 1];
  const float xv = E::load(logits + b * sb + r * sr + tl);
  float o = fast_exp2(((xv - M) - LS) * kLog2e) * (-gsum[row]);
  const float* gr = g + b * gsb + r * gsr;
  for (int64_t j = k; j < K; ++j)
    if (ir[j * isk] == t) o += gr[j * gsk];
  gin[b * gisb + r * gisr + tl] = E::from_float(o);
}

// The same fix-up with one wave per row, for K <= 64: lane k holds id_k and
// g_k, and the duplicate test and the in-order sum over equal ids read the
// other lanes' values through cross-lane shuffles instead of up to K dependent
// loads per thread (the per-(row, k) kernel above measured 25 us on the
// [8, 2048] rows with 21 ids).  Same arithmetic in the same order.
constexpr int kFixupRowsPerBlock = 4;

template <class E>
__global__ __launch_bounds__(64 * kFixupRowsPerBlock) void gather_fixup_wave_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t V, int64_t sb, int64_t sr,
    const int64_t* __restrict__ idx, int64_t K, int64_t isb, int64_t isr, int64_t isk,
    int64_t vs, int64_t ve, const float* __restrict__ stats, const float* __restrict__ g,
    int64_t gsb, int64_t gsr, int64_t gsk, const float* __restrict__ gsum,
    typename E::raw* gin, int64_t gisb, int64_t gisr, int64_t rows,
    const int* __restrict__ flags, int nflags) {
  const int64_t row = (int64_t)blockIdx.x * kFixupRowsPerBlock + threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  // both conditions are uniform over the wave, so every shuffle below sees all 64 lanes
  if (!any_flag(flags, nflags) || row >= rows) return;
  const int64_t b = row / R, r = row - b * R;
  const int64_t* ir = idx + b * isb + r * isr;
  const float* gr = g + b * gsb + r * gsr;
  const bool has = lane < K;
  const int64_t t = has ? ir[lane * isk] : int64_t(-1);
  const float gk = has ? gr[lane * gsk] : 0.f;
  const bool in_range = has && !(t < vs || t >= ve || t - vs >= V);
  float o = 0.f;
  if (in_range) {
    const float M = stats[2 * row], LS = stats[2 * row + 1];
    const float xv = E::load(logits + b * sb + r * sr + (t - vs));
    o = fast_exp2(((xv - M) - LS) * kLog2e) * (-gsum[row]);
  }
  bool first = in_range;
  const int tlo = (int)(uint32_t)(uint64_t)t, thi = (int)(uint32_t)((uint64_t)t >> 32);
  for (int j = 0; j < (int)K; ++j) {
    const int jlo = __shfl(tlo, j, 64), jhi = __shfl(thi, j, 64);
    const float gj = __shfl(gk, j, 64);
    const bool same = (jlo == tlo) && (jhi == thi);
    if (same && j < lane) first = false;  // an earlier k holds the same id
    if (same && j >= lane) o += gj;       // scatter_add order: k, then later equal ids
  }
  if (first) gin[b * gisb + r * gisr + (t - vs)] = E::from_float(o);
}

template <class E>
void launch_gather_fixup(int64_t rows, hipStream_t st, const typename E::raw* logits, int64_t R,
                         int64_t V, int64_t sb, int64_t sr, const int64_t* idx, int64_t K,
                         int64_t isb, int64_t isr, int64_t isk, int64_t vs, int64_t ve,
                         const float* stats, const float* g, int64_t gsb, int64_t gsr,
                         int64_t gsk, const float* gsum, typename E::raw* gin, int64_t gisb,
                         int64_t gisr, const int* flags, int nflags) {
  if (K <= 64) {
    const int64_t grid = (rows + kFixupRowsPerBlock - 1) / kFixupRowsPerBlock;
    hipLaunchKernelGGL((gather_fixup_wave_kernel<E>), dim3((unsigned)grid),
                       dim3(64 * kFixupRowsPerBlock), 0, st, logits, R, V, sb, sr, idx, K, isb,
                       isr, isk, vs, ve, stats, g, gsb, gsr, gsk, gsum, gin, gisb, gisr, rows,
                       flags, nflags);
    return;
  }
  const int64_t total = rows * K;
  hipLaunchKernelGGL((gather_fixup_kernel<E>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     st, logits, R, V, sb, sr, idx, K, isb, isr, isk, vs, ve, stats, g, gsb, gsr,
                     gsk, gsum, gin, gisb, gisr, total, flags, nflags);
}

// Early-backward check.  A caller that knows the upstream gradient in closed
// form launches the logprob backward for it (`g_used`) before autograd asks
// for it; when autograd does, bwd_check_kernel compares the real upstream
// gradient with g_used bit for bit (up to kCheckBlocks workgroups, each writing
// its own flag), and bwd_redo_kernel recomputes the whole gradient from the
// real one only when some flag is set (a scaled loss, a second consumer of the
// logprobs).  Otherwise both launches are a few microseconds of GPU time.
// Each workgroup compares a contiguous share of the [B, R] gradients and
// writes its own flag slot outright (no atomics, nothing to clear first).
constexpr int kCheckBlocks = 64;

// With `list`, a workgroup also lists the rows of its share that differ, in
// order, at list[i0 ...] (i0 = the share's first row), and its flag is their
// count.
__global__ __launch_bounds__(256) void bwd_check_kernel(const float* __restrict__ g, int64_t gsb,
                                                        int64_t gsr, const float* __restrict__ g_used,
                                                        int64_t B, int64_t R, int* __restrict__ flags,
                                                        int32_t* __restrict__ list) {
  __shared__ int s_any[4];
  int any = 0;
  const int64_t n = B * R;
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t i0 = (int64_t)blockIdx.x * per;
  const int64_t i1 = (i0 + per < n) ? i0 + per : n;
  if (list != nullptr) {
    __shared__ uint32_t s_w[4];
    const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t count = 0u;  // rows listed so far (the same in every thread)
    for (int64_t c0 = i0; c0 < i1; c0 += 256) {
      const int64_t i = c0 + threadIdx.x;
      bool d = false;
      if (i < i1) {
        const int64_t b = i / R, r = i - b * R;
        d = __float_as_uint(g[b * gsb + r * gsr]) != __float_as_uint(g_used[i]);
      }
      const uint64_t bal = __ballot(d);
      if (lane == 0) s_w[wv] = (uint32_t)__popcll(bal);
      __syncthreads();
      uint32_t before = count, total = 0u;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        before += v < wv ? s_w[v] : 0u;
        total += s_w[v];
      }
      if (d) list[i0 + before + (uint32_t)__popcll(bal & below)] = (int32_t)i;
      count += total;
      __syncthreads();  // s_w is written again
    }
    if (threadIdx.x == 0) flags[blockIdx.x] = (int)count;
    return;
  }
  for (int64_t i = i0 + threadIdx.x; i < i1; i += 256) {
    const int64_t b = i / R, r = i - b * R;
    any |= (__float_as_uint(g[b * gsb + r * gsr]) != __float_as_uint(g_used[i])) ? 1 : 0;
  }
  const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
  const bool w = __ballot(any != 0) != 0ull;
  if (lane == 0) s_any[wv] = w ? 1 : 0;
  __syncthreads();
  if (threadIdx.x == 0) flags[blockIdx.x] = s_any[0] | s_any[1] | s_any[2] | s_any[3];
}

// Grid-stride recomputation of (onehot - p) * g over rows [0, B * Rt), run only
// when the check flagged a difference (every workgroup returns at once
// otherwise).  Same arithmetic as the other backward kernels.
template <class E>
__global__ __launch_bounds__(256) void bwd_redo_kernel(
    const typename E::raw* __restrict__ logits, int64_t R, int64_t Rt, int64_t V, int64_t sb,
    int64_t sr, const int64_t* __restrict__ target, int64_t tsb, int64_t tsr, int64_t vs,
    int64_t ve, const float* __restrict__ stats, const float* __restrict__ g, int64_t gsb,
    int64_t gsr, typename E::raw* gin, int64_t gisb, int64_t gisr, int64_t rows,
    const int* __restrict__ flags, int nflags) {
  if (!any_flag(flags, nflags)) return;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const int64_t b = row / Rt, r = row - b * Rt;
    typename E::raw* y = gin + b * gisb + r * gisr;
    const float gv = (r < R) ? g[b * gsb + r * gsr] : 0.f;
    if (gv == 0.f) {
      for (int64_t j = threadIdx.x; j < V; j += 256) y[j] = E::from_float(0.f);
      continue;
    }
    const typename E::raw* x = logits + b * sb + r * sr;
    const int64_t srow = b * R + r;
    const float M = stats[2 * srow], LS = stats[2 * srow + 1];
    const int64_t t = target[b * tsb + r * tsr];
    const bool tmask = (t < vs) || (t >= ve) || (t - vs >= V);
    const int64_t tl = tmask ? -1 : (t - vs);
    for (int64_t j = threadIdx.x; j < V; j += 256) {
      const float p = fast_exp2(((E::load(x + j) - M) - LS) * kLog2e);
      y[j] = E::from_float((j == tl) ? (1.f - p) * gv : -p * gv);
    }
  }
}

// Waves per row for the forward: 4 (fewer rows in flight at a time keeps the
// concurrently streamed address window narrower, measured +5% read bandwidth
// over one wave per row), 8 when there are too few rows to give every CU work.
// Not 16: two 512-thread rows fit a CU at these register counts, one
// 1024-thread row does, so 510 rows of 1024 threads ran in two rounds (fp32
// [2, 255, 32000]: 15.6 us at 16 waves, 13.9 us at 8).
int pick_waves(int64_t rows) { return rows * 4 < 8192 ? 8 : 4; }

// The backward always uses 16-wave (1024-thread) rows: measured best for
// both phases on the GRPO workload.
constexpr int kBwdWaves = 16;

template <class E, int W, int U = 8>
void launch_fwd(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t V, int64_t sb,
                int64_t sr, const int64_t* target, int64_t tsb, int64_t tsr, int64_t vs, int64_t ve,
                float* out, float* stats) {
  hipLaunchKernelGGL((logprob_fwd_kernel<E, W, U>), dim3((unsigned)rows), dim3(64 * W), 0, st,
                     static_cast<const typename E::raw*>(logits), R, V, sb, sr, target, tsb, tsr, vs,
                     ve, out, stats);
}

template <class E>
void dispatch_fwd(int w, int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t V,
                  int64_t sb, int64_t sr, const int64_t* target, int64_t tsb, int64_t tsr,
                  int64_t vs, int64_t ve, float* out, float* stats) {
  switch (w) {
    case 4: launch_fwd<E, 4>(rows, st, logits, R, V, sb, sr, target, tsb, tsr, vs, ve, out, stats); break;
    default: launch_fwd<E, 8>(rows, st, logits, R, V, sb, sr, target, tsb, tsr, vs, ve, out, stats); break;
  }
}

template <class E, int W>
void launch_gather_fwd(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t V,
                       int64_t sb, int64_t sr, const int64_t* idx, int64_t K, int64_t isb,
                       int64_t isr, int64_t isk, int64_t vs, int64_t ve, float* out,
                       float* stats) {
  constexpr int U = 8;
  hipLaunchKernelGGL((gather_logprob_fwd_kernel<E, W, U>), dim3((unsigned)rows), dim3(64 * W), 0,
                     st, static_cast<const typename E::raw*>(logits), R, V, sb, sr, idx, K, isb,
                     isr, isk, vs, ve, out, stats);
}

template <class E>
void dispatch_gather_fwd(int w, int64_t rows, hipStream_t st, const void* logits, int64_t R,
                         int64_t V, int64_t sb, int64_t sr, const int64_t* idx, int64_t K,
                         int64_t isb, int64_t isr, int64_t isk, int64_t vs, int64_t ve,
                         float* out, float* stats) {
  switch (w) {
    case 4: launch_gather_fwd<E, 4>(rows, st, logits, R, V, sb, sr, idx, K, isb, isr, isk, vs, ve, out, stats); break;
    case 8: launch_gather_fwd<E, 8>(rows, st, logits, R, V, sb, sr, idx, K, isb, isr, isk, vs, ve, out, stats); break;
    default: launch_gather_fwd<E, 16>(rows, st, logits, R, V, sb, sr, idx, K, isb, isr, isk, vs, ve, out, stats); break;
  }
}

// The flat backward applies when gradient and logits share one contiguous,
// 16-byte aligned [B, Rt, V] layout with whole vectors per row and the vector
// count fits 32-bit indexing; fills the launch arguments and the piece count.
template <class E>
bool flat_bwd_layout(int64_t rows, const void* logits, int64_t R, int64_t Rt, int64_t V,
                     int64_t sb, int64_t sr, const int64_t* target, int64_t tsb, int64_t tsr,
                     int64_t vs, int64_t ve, const float* stats, const float* g, int64_t gsb,
                     int64_t gsr, void* gin, int64_t gisb, int64_t gisr, FlatBwd* A,
                     int64_t* npieces) {
  constexpr int VEC = E::kVec;
  const uintptr_t ya = reinterpret_cast<uintptr_t>(gin), xa = reinterpret_cast<uintptr_t>(logits);
  const bool contiguous = gisr == V && (rows == Rt || gisb == Rt * V);
  const bool shared_layout = R == 0 || (sr == gisr && (rows == Rt || sb == gisb));
  const int64_t nvr = V / VEC;
  const int64_t nvec = rows * nvr;
  if (!(V % VEC == 0 && contiguous && shared_layout && (ya & 15u) == 0 && (xa & 15u) == 0 &&
        nvec + 512 < (int64_t(1) << 32) && rows < (int64_t(1) << 31)))
    return false;
  constexpr int P = kFlatThreads * kFlatVecs;  // vectors per 4 KB piece
  const int to4k = (int)(((4096u - (ya & 4095u)) & 4095u) / 16u);  // vectors before a 4 KB boundary
  const int shift = (P - to4k) & (P - 1);
  *npieces = (nvec + shift + P - 1) / P;
  *A = FlatBwd{logits, R, (uint32_t)Rt, (uint32_t)nvr, (uint32_t)nvec, shift, target, tsb, tsr,
               vs, ve, V, stats, g, gsb, gsr, gin, nullptr};
  return true;
}

// Single-wave workgroups of the flat redo's grid-stride launch: two per wave
// slot of the 256 CUs (32 slots each).
constexpr int64_t kRedoGrid = 256 * 32 * 2;
static_assert(kCheckBlocks <= 64, "the flat redo tests at most 64 flags, one per lane");

// Redo of the backward after a failed early-backward check (every launch
// returns at once when no flag is set): the flat schedule when the layout
// allows it, row by row otherwise.  g_used (contiguous [B, R], or null): the
// upstream gradient the early backward used; the flat redo leaves the rows
// where it equals g alone.
template <class E>
void dispatch_bwd_redo(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t Rt,
                       int64_t V, int64_t sb, int64_t sr, const int64_t* target, int64_t tsb,
                       int64_t tsr, int64_t vs, int64_t ve, const float* stats, const float* g,
                       int64_t gsb, int64_t gsr, void* gin, int64_t gisb, int64_t gisr,
                       const int* flags, int nflags, const float* g_used) {
  using raw = typename E::raw;
  FlatBwd A;
  int64_t npieces = 0;
  if (flat_bwd_layout<E>(rows, logits, R, Rt, V, sb, sr, target, tsb, tsr, vs, ve, stats, g, gsb,
                         gsr, gin, gisb, gisr, &A, &npieces)) {
    const int64_t grid = npieces < kRedoGrid ? npieces : kRedoGrid;
    A.gu = g_used;
    if (g_used)
      hipLaunchKernelGGL((logprob_bwd_flat_redo_kernel<E, true>), dim3((unsigned)grid), dim3(64), 0,
                         st, A, npieces, flags, nflags);
    else
      hipLaunchKernelGGL((logprob_bwd_flat_redo_kernel<E, false>), dim3((unsigned)grid), dim3(64),
                         0, st, A, npieces, flags, nflags);
    return;
  }
  const unsigned grid = (unsigned)(rows < 1024 ? rows : 1024);
  hipLaunchKernelGGL((bwd_redo_kernel<E>), dim3(grid), dim3(256), 0, st,
                     static_cast<const raw*>(logits), R, Rt, V, sb, sr, target, tsb, tsr, vs, ve,
                     stats, g, gsb, gsr, static_cast<raw*>(gin), gisb, gisr, rows, flags, nflags);
}

// The early-backward check, then the redo: over the listed rows when a list
// buffer is given and the layout is the flat one, else dispatch_bwd_redo.
constexpr int64_t kListRedoGrid = 256 * 32 * 2 / kListRedoWaves;
template <class E>
void recheck(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t Rt, int64_t V,
             int64_t sb, int64_t sr, const int64_t* target, int64_t tsb, int64_t tsr, int64_t vs,
             int64_t ve, const float* stats, const float* g, int64_t gsb, int64_t gsr, void* gin,
             int64_t gisb, int64_t gisr, int* flags, int nflags, const float* g_used, int64_t B,
             int32_t* row_list) {
  FlatBwd A;
  int64_t npieces = 0;
  const bool listed = row_list != nullptr &&
                      flat_bwd_layout<E>(rows, logits, R, Rt, V, sb, sr, target, tsb, tsr, vs, ve, stats,
                                         g, gsb, gsr, gin, gisb, gisr, &A, &npieces);
  hipLaunchKernelGGL(bwd_check_kernel, dim3((unsigned)nflags), dim3(256), 0, st, g, gsb, gsr, g_used, B, R,
                     flags, listed ? row_list : nullptr);
  if (!listed) {
    dispatch_bwd_redo<E>(rows, st, logits, R, Rt, V, sb, sr, target, tsb, tsr, vs, ve, stats, g, gsb, gsr,
                         gin, gisb, gisr, flags, nflags, g_used);
    return;
  }
  const int64_t n = B * R;
  const int64_t per = (n + nflags - 1) / nflags;  // the check's share per workgroup
  hipLaunchKernelGGL((logprob_bwd_list_redo_kernel<E>), dim3((unsigned)kListRedoGrid),
                     dim3(64 * kListRedoWaves), 0, st, A, flags, nflags, per, row_list);
}

template <class E>
void dispatch_bwd(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t Rt,
                  int64_t V, int64_t sb, int64_t sr, const int64_t* target, int64_t tsb,
                  int64_t tsr, int64_t vs, int64_t ve, const float* stats, const float* g,
                  int64_t gsb, int64_t gsr, void* gin, int64_t gisb, int64_t gisr) {
  constexpr int W = kBwdWaves, U = 4;
  using raw = typename E::raw;
  FlatBwd A;
  int64_t npieces = 0;
  if (flat_bwd_layout<E>(rows, logits, R, Rt, V, sb, sr, target, tsb, tsr, vs, ve, stats, g, gsb,
                         gsr, gin, gisb, gisr, &A, &npieces)) {
    hipLaunchKernelGGL((logprob_bwd_flat_kernel<E>), dim3((unsigned)npieces), dim3(kFlatThreads), 0,
                       st, A);
    return;
  }
  hipLaunchKernelGGL((logprob_bwd_kernel<E, W, U, kZeroRows>), dim3((unsigned)rows), dim3(64 * W),
                     0, st, static_cast<const raw*>(logits), R, Rt, V, sb, sr, target, tsb, tsr,
                     vs, ve, stats, g, gsb, gsr, static_cast<raw*>(gin), gisb, gisr);
  if (R == 0) return;
  hipLaunchKernelGGL((logprob_bwd_kernel<E, W, U, kActiveRows>), dim3((unsigned)rows),
                     dim3(64 * W), 0, st, static_cast<const raw*>(logits), R, Rt, V, sb, sr,
                     target, tsb, tsr, vs, ve, stats, g, gsb, gsr, static_cast<raw*>(gin), gisb,
                     gisr);
}

template <class E>
void gather_bwd(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t V,
                int64_t sb, int64_t sr, const int64_t* idx, int64_t K, int64_t isb, int64_t isr,
                int64_t isk, int64_t vs, int64_t ve, const float* stats, const float* g,
                int64_t gsb, int64_t gsr, int64_t gsk, float* gsum, void* gin, int64_t gisb,
                int64_t gisr) {
  hipLaunchKernelGGL(gather_gsum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                     g, R, gsb, gsr, gsk, K, rows, gsum, nullptr, 0);
  // dense part: no target (an empty vocabulary slice masks every id), upstream gsum
  dispatch_bwd<E>(rows, st, logits, R, R, V, sb, sr, idx, isb, isr, 0, 0, stats, gsum, R, 1,
                  gin, gisb, gisr);
  const int64_t total = rows * K;
  if (total == 0) return;
  launch_gather_fixup<E>(rows, st, static_cast<const typename E::raw*>(logits), R, V, sb, sr, idx,
                         K, isb, isr, isk, vs, ve, stats, g, gsb, gsr, gsk, gsum,
                         static_cast<typename E::raw*>(gin), gisb, gisr, nullptr, 0);
}

// The K-id gather's early-backward recheck: gather_check_kernel compares the
// real [B, R, K] upstream gradient with the one the early launch used (flags as
// in bwd_check_kernel), then the three backward parts run again, each launch
// returning at once unless a flag is set.  The dense part's redo is
// bwd_redo_kernel with no target, whose arithmetic equals the flat kernel's.
constexpr int kGatherCheckThreads = 1024;

__global__ __launch_bounds__(kGatherCheckThreads) void gather_check_kernel(
    const float* __restrict__ g, int64_t R, int64_t K, int64_t gsb, int64_t gsr, int64_t gsk,
    const float* __restrict__ g_used, int64_t n, int* __restrict__ flags) {
  constexpr int NT = kGatherCheckThreads, U = 4;  // U loads in flight per thread
  int any = 0;
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t i0 = (int64_t)blockIdx.x * per;
  const int64_t i1 = (i0 + per < n) ? i0 + per : n;
  const bool flat = gsk == 1 && gsr == K && gsb == R * K;  // g laid out like g_used
  for (int64_t i = i0 + threadIdx.x; i < i1; i += U * NT) {
    float a[U], c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + u * NT;
      a[u] = c[u] = 0.f;
      if (j < i1) {
        int64_t off = j;
        if (!flat) {
          const int64_t row = j / K, k = j - row * K;
          const int64_t b = row / R, r = row - b * R;
          off = b * gsb + r * gsr + k * gsk;
        }
        a[u] = g[off];
        c[u] = g_used[j];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) any |= (__float_as_uint(a[u]) != __float_as_uint(c[u])) ? 1 : 0;
  }
  any = __syncthreads_or(any);
  if (threadIdx.x == 0) flags[blockIdx.x] = any != 0 ? 1 : 0;
}

template <class E>
void gather_bwd_recheck(int64_t rows, hipStream_t st, const void* logits, int64_t R, int64_t V,
                        int64_t sb, int64_t sr, const int64_t* idx, int64_t K, int64_t isb,
                        int64_t isr, int64_t isk, int64_t vs, int64_t ve, const float* stats,
                        const float* g, int64_t gsb, int64_t gsr, int64_t gsk, const float* g_used,
                        int* flags, float* gsum, void* gin, int64_t gisb, int64_t gisr) {
  using raw = typename E::raw;
  const int64_t total = rows * K;
  const int nflags = (int)(total < kCheckBlocks ? total : kCheckBlocks);
  hipLaunchKernelGGL(gather_check_kernel, dim3((unsigned)nflags), dim3(kGatherCheckThreads), 0, st,
                     g, R, K, gsb, gsr, gsk, g_used, total, flags);
  hipLaunchKernelGGL(gather_gsum_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st,
                     g, R, gsb, gsr, gsk, K, rows, gsum, flags, nflags);
  dispatch_bwd_redo<E>(rows, st, logits, R, R, V, sb, sr, idx, isb, isr, 0, 0, stats, gsum, R, 1,
                       gin, gisb, gisr, flags, nflags, nullptr);
  launch_gather_fixup<E>(rows, st, static_cast<const raw*>(logits), R, V, sb, sr, idx, K, isb, isr,
                         isk, vs, ve, stats, g, gsb, gsr, gsk, gsum, static_cast<raw*>(gin), gisb,
                         gisr, flags, nflags);
}

int check_dtype(int dtype) {
  if (dtype == MIRL_DTYPE_F32 || dtype == MIRL_DTYPE_BF16 || dtype == MIRL_DTYPE_F16) return 0;
  set_error("unsupported logits dtype code %d (expected f32, bf16 or f16)", dtype);
  return MIRL_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                                int64_t stride_b, int64_t stride_r, const int64_t* target,
                                int64_t t_stride_b, int64_t t_stride_r, int64_t vocab_start,
                                int64_t vocab_end, float* out, float* row_stats, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0, "invalid shape B=%lld R=%lld V=%lld", (long long)B,
               (long long)R, (long long)V);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(logits && target && out, "null pointer argument");
  const int w = pick_waves(rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      dispatch_fwd<F32>(w, rows, st, logits, R, V, stride_b, stride_r, target, t_stride_b,
                        t_stride_r, vocab_start, vocab_end, out, row_stats);
      break;
    case MIRL_DTYPE_BF16:
      dispatch_fwd<BF16>(w, rows, st, logits, R, V, stride_b, stride_r, target, t_stride_b,
                         t_stride_r, vocab_start, vocab_end, out, row_stats);
      break;
    default:
      dispatch_fwd<F16>(w, rows, st, logits, R, V, stride_b, stride_r, target, t_stride_b,
                        t_stride_r, vocab_start, vocab_end, out, row_stats);
      break;
  }
  return check_launch("mirl_logprob_fwd");
}

extern "C" int mirl_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                                int64_t R_total, int64_t V, int64_t stride_b, int64_t stride_r,
                                const int64_t* target, int64_t t_stride_b, int64_t t_stride_r,
                                int64_t vocab_start, int64_t vocab_end, const float* row_stats,
                                const float* grad_out, int64_t g_stride_b, int64_t g_stride_r,
                                void* grad_in, int64_t gi_stride_b, int64_t gi_stride_r,
                                void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && R_total >= R && V > 0,
               "invalid shape B=%lld R=%lld R_total=%lld V=%lld", (long long)B, (long long)R,
               (long long)R_total, (long long)V);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  const int64_t rows = B * R_total;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(grad_in != nullptr, "null grad_in");
  MIRL_REQUIRE(R == 0 || (logits && target && row_stats && grad_out), "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      dispatch_bwd<F32>(rows, st, logits, R, R_total, V, stride_b, stride_r, target,
                        t_stride_b, t_stride_r, vocab_start, vocab_end, row_stats, grad_out,
                        g_stride_b, g_stride_r, grad_in, gi_stride_b, gi_stride_r);
      break;
    case MIRL_DTYPE_BF16:
      dispatch_bwd<BF16>(rows, st, logits, R, R_total, V, stride_b, stride_r, target,
                         t_stride_b, t_stride_r, vocab_start, vocab_end, row_stats, grad_out,
                         g_stride_b, g_stride_r, grad_in, gi_stride_b, gi_stride_r);
      break;
    default:
      dispatch_bwd<F16>(rows, st, logits, R, R_total, V, stride_b, stride_r, target,
                        t_stride_b, t_stride_r, vocab_start, vocab_end, row_stats, grad_out,
                        g_stride_b, g_stride_r, grad_in, gi_stride_b, gi_stride_r);
      break;
  }
  return check_launch("mirl_logprob_bwd");
}

extern "C" int mirl_gather_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R,
                                       int64_t V, int64_t stride_b, int64_t stride_r,
                                       const int64_t* indices, int64_t K, int64_t i_stride_b,
                                       int64_t i_stride_r, int64_t i_stride_k,
                                       int64_t vocab_start, int64_t vocab_end, float* out,
                                       float* row_stats, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0 && K >= 0, "invalid shape B=%lld R=%lld V=%lld K=%lld",
               (long long)B, (long long)R, (long long)V, (long long)K);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(logits && (K == 0 || indices) && (K == 0 || out), "null pointer argument");
  const int w = pick_waves(rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      dispatch_gather_fwd<F32>(w, rows, st, logits, R, V, stride_b, stride_r, indices, K,
                               i_stride_b, i_stride_r, i_stride_k, vocab_start, vocab_end, out,
                               row_stats);
      break;
    case MIRL_DTYPE_BF16:
      dispatch_gather_fwd<BF16>(w, rows, st, logits, R, V, stride_b, stride_r, indices, K,
                                i_stride_b, i_stride_r, i_stride_k, vocab_start, vocab_end, out,
                                row_stats);
      break;
    default:
      dispatch_gather_fwd<F16>(w, rows, st, logits, R, V, stride_b, stride_r, indices, K,
                               i_stride_b, i_stride_r, i_stride_k, vocab_start, vocab_end, out,
                               row_stats);
      break;
  }
  return check_launch("mirl_gather_logprob_fwd");
}

extern "C" int64_t mirl_gather_logprob_workspace_elems(int64_t B, int64_t R) { return B * R; }

extern "C" int mirl_gather_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                                       int64_t V, int64_t stride_b, int64_t stride_r,
                                       const int64_t* indices, int64_t K, int64_t i_stride_b,
                                       int64_t i_stride_r, int64_t i_stride_k,
                                       int64_t vocab_start, int64_t vocab_end,
                                       const float* row_stats, const float* grad_out,
                                       int64_t g_stride_b, int64_t g_stride_r,
                                       int64_t g_stride_k, float* workspace, void* grad_in,
                                       int64_t gi_stride_b, int64_t gi_stride_r, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0 && K >= 0, "invalid shape B=%lld R=%lld V=%lld K=%lld",
               (long long)B, (long long)R, (long long)V, (long long)K);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31) && rows * K < (int64_t(1) << 40), "too many rows (%lld)",
               (long long)rows);
  MIRL_REQUIRE(K > 0, "at least one id per row is required (K=%lld)", (long long)K);
  MIRL_REQUIRE(logits && indices && row_stats && grad_in && workspace && grad_out,
               "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      gather_bwd<F32>(rows, st, logits, R, V, stride_b, stride_r, indices, K, i_stride_b,
                      i_stride_r, i_stride_k, vocab_start, vocab_end, row_stats, grad_out,
                      g_stride_b, g_stride_r, g_stride_k, workspace, grad_in, gi_stride_b,
                      gi_stride_r);
      break;
    case MIRL_DTYPE_BF16:
      gather_bwd<BF16>(rows, st, logits, R, V, stride_b, stride_r, indices, K, i_stride_b,
                       i_stride_r, i_stride_k, vocab_start, vocab_end, row_stats, grad_out,
                       g_stride_b, g_stride_r, g_stride_k, workspace, grad_in, gi_stride_b,
                       gi_stride_r);
      break;
    default:
      gather_bwd<F16>(rows, st, logits, R, V, stride_b, stride_r, indices, K, i_stride_b,
                      i_stride_r, i_stride_k, vocab_start, vocab_end, row_stats, grad_out,
                      g_stride_b, g_stride_r, g_stride_k, workspace, grad_in, gi_stride_b,
                      gi_stride_r);
      break;
  }
  return check_launch("mirl_gather_logprob_bwd");
}

extern "C" int mirl_gather_logprob_bwd_recheck(
    const void* logits, int dtype, int64_t B, int64_t R, int64_t V, int64_t stride_b,
    int64_t stride_r, const int64_t* indices, int64_t K, int64_t i_stride_b, int64_t i_stride_r,
    int64_t i_stride_k, int64_t vocab_start, int64_t vocab_end, const float* row_stats,
    const float* grad_out, int64_t g_stride_b, int64_t g_stride_r, int64_t g_stride_k,
    const float* grad_used, int* flags, float* workspace, void* grad_in, int64_t gi_stride_b,
    int64_t gi_stride_r, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0 && K >= 0, "invalid shape B=%lld R=%lld V=%lld K=%lld",
               (long long)B, (long long)R, (long long)V, (long long)K);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31) && rows * K < (int64_t(1) << 40), "too many rows (%lld)",
               (long long)rows);
  MIRL_REQUIRE(K > 0, "at least one id per row is required (K=%lld)", (long long)K);
  MIRL_REQUIRE(logits && indices && row_stats && grad_in && workspace && grad_out && grad_used &&
                   flags,
               "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define MIRL_GATHER_RECHECK(E)                                                                   \
  gather_bwd_recheck<E>(rows, st, logits, R, V, stride_b, stride_r, indices, K, i_stride_b,      \
                        i_stride_r, i_stride_k, vocab_start, vocab_end, row_stats, grad_out,     \
                        g_stride_b, g_stride_r, g_stride_k, grad_used, flags, workspace,         \
                        grad_in, gi_stride_b, gi_stride_r)
  switch (dtype) {
    case MIRL_DTYPE_F32: MIRL_GATHER_RECHECK(F32); break;
    case MIRL_DTYPE_BF16: MIRL_GATHER_RECHECK(BF16); break;
    default: MIRL_GATHER_RECHECK(F16); break;
  }
#undef MIRL_GATHER_RECHECK
  return check_launch("mirl_gather_logprob_bwd_recheck");
}

extern "C" int mirl_logprob_bwd_recheck(const void* logits, int dtype, int64_t B, int64_t R,
                                        int64_t R_total, int64_t V, int64_t stride_b,
                                        int64_t stride_r, const int64_t* target,
                                        int64_t t_stride_b, int64_t t_stride_r,
                                        int64_t vocab_start, int64_t vocab_end,
                                        const float* row_stats, const float* grad_out,
                                        int64_t g_stride_b, int64_t g_stride_r,
                                        const float* grad_used, void* grad_in,
                                        int64_t gi_stride_b, int64_t gi_stride_r, int* flag,
                                        int32_t* row_list, void* stream) {
  clear_error();
  if (int e = check_dtype(dtype)) return e;
  MIRL_REQUIRE(B >= 0 && R >= 0 && R_total >= R && V > 0,
               "invalid shape B=%lld R=%lld R_total=%lld V=%lld", (long long)B, (long long)R,
               (long long)R_total, (long long)V);
  const int64_t rows = B * R_total;
  if (rows == 0 || R == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(logits && target && row_stats && grad_out && grad_used && grad_in && flag,
               "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = B * R;
  const int nflags = (int)(n < kCheckBlocks ? n : kCheckBlocks);
#define MIRL_REDO(E)                                                                          \
  recheck<E>(rows, st, logits, R, R_total, V, stride_b, stride_r, target, t_stride_b,          \
             t_stride_r, vocab_start, vocab_end, row_stats, grad_out, g_stride_b, g_stride_r,  \
             grad_in, gi_stride_b, gi_stride_r, flag, nflags, grad_used, B, row_list)
  switch (dtype) {
    case MIRL_DTYPE_F32: MIRL_REDO(F32); break;
    case MIRL_DTYPE_BF16: MIRL_REDO(BF16); break;
    default: MIRL_REDO(F16); break;
  }
#undef MIRL_REDO
  return check_launch("mirl_logprob_bwd_recheck");
}

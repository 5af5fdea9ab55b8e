// Per-token divergences between the student distribution p = softmax(x) and a
// fixed teacher distribution q = softmax(y) over the vocabulary, and their
// gradients with respect to the student logits.
//
// Semantics follow nemo_rl/distributed/model_utils.py:2199-2538 with a vocab
// group of size 1:
//   entropy        L = sum_v p_v log p_v              (ChunkedDistributedEntropy)
//   cross entropy  L = -sum_v p_v log q_v             (ChunkedDistributedCrossEntropyToFixedLogits)
//   reverse KL     L = sum_v p_v (log p_v - log q_v)  (ChunkedDistributedReverseKLToFixedLogits)
//   backward       dL/dx_v = (p_v (w_v - L)) g,  w = log p | -log q | log p - log q,
//                  formed in fp32 and rounded once to the logits dtype.
//
// Forward: one pass over the row(s).  Each lane keeps, in base-2 offset form
// (y = x*log2e - off, off = fl(m*log2e) for its running max m):
//   s = sum 2^y,   t = sum 2^y * y,   u = sum 2^y * (x_teacher - c),
// plus the teacher's own (max, sum).  A rise of the running max by d = off -
// off' rescales them as s' = 2^d s, t' = 2^d (t + d s), u' = 2^d u.  At the end
//   sum p log p = ln2 * t/s - ln s,   sum p x_teacher = c + u/s,
//   -sum p log q = (M_t + logZ_t - c) - u/s,
// where c is the teacher's first logit of the row (0 if not finite), which keeps
// u free of cancellation when the teacher logits share a large offset.  Lanes
// past the end of a row read -2^100 (-2^15 for fp16) instead of -inf: a power of
// two, so x*log2e is exact and a lane that sees nothing else gets y = 0 and
// finite sums, which the merge then scales by 2^(-huge) = 0; next to real
// logits the padding gives 2^y = 0 with y finite.  Either way no padding term
// turns into 0 * inf.
//
// Backward: the gradient is walked as one flat array of 16-byte vectors when the
// student, teacher and gradient share one contiguous layout (the autograd
// case), one workgroup per row otherwise.  Rows whose upstream gradient is 0
// are written as zeros without reading the logits.

#include "common.h"

#pragma clang fp contract(off)

namespace mirl {
namespace {

constexpr float kLn2 = 0.6931471805599453f;

template <int KIND>
struct DivTraits {
  static constexpr bool kT = KIND != MIRL_DIV_CROSS_ENTROPY;  // needs sum 2^y * y
  static constexpr bool kTeacher = KIND != MIRL_DIV_ENTROPY;  // reads teacher logits
};

template <int KIND>
struct DivState {
  static constexpr bool kT = DivTraits<KIND>::kT;
  static constexpr bool kTeacher = DivTraits<KIND>::kTeacher;
  float m = -INFINITY, off = 0.f;
  float s[2] = {0.f, 0.f}, t[2] = {0.f, 0.f}, u[2] = {0.f, 0.f};
  float mt = -INFINITY, offt = 0.f;
  float st[2] = {0.f, 0.f};
  float c = 0.f;  // teacher shift

  template <int N>
  __device__ __forceinline__ void add(const float (&xs)[N], const float (&ys)[N]) {
    float bm = xs[0];
#pragma unroll
    for (int i = 1; i < N; ++i) bm = fmaxf(bm, xs[i]);
    const float mn = fmaxf(m, bm);
    if (mn != -INFINITY) {
      if (mn != m) {
        const float noff = mn * kLog2e;
        const float d = off - noff;
        const float sc = (m == -INFINITY) ? 0.f : fast_exp2(d);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          if constexpr (kT) t[k] = sc * fmaf(d, s[k], t[k]);
          if constexpr (kTeacher) u[k] *= sc;
          s[k] *= sc;
        }
        m = mn;
        off = noff;
      }
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const float y = fmaf(xs[i], kLog2e, -off);
        const float e = fast_exp2(y);
        s[i & 1] += e;
        if constexpr (kT) t[i & 1] = fmaf(e, y, t[i & 1]);
        if constexpr (kTeacher) u[i & 1] = fmaf(e, ys[i] - c, u[i & 1]);
      }
    }
    if constexpr (kTeacher) {
      float bt = ys[0];
#pragma unroll
      for (int i = 1; i < N; ++i) bt = fmaxf(bt, ys[i]);
      const float mtn = fmaxf(mt, bt);
      if (mtn == -INFINITY) return;
      if (mtn != mt) {
        const float noff = mtn * kLog2e;
        const float sc = (mt == -INFINITY) ? 0.f : fast_exp2(offt - noff);
        st[0] *= sc;
        st[1] *= sc;
        mt = mtn;
        offt = noff;
      }
#pragma unroll
      for (int i = 0; i < N; ++i) st[i & 1] += fast_exp2(fmaf(ys[i], kLog2e, -offt));
    }
  }
};

template <class E, int W, int U, int KIND>
__global__ __launch_bounds__(64 * W) void divergence_fwd_kernel(
    const typename E::raw* __restrict__ xs, const typename E::raw* __restrict__ xt, int64_t R,
    int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, float* __restrict__ out,
    float* __restrict__ stats) {
  using raw = typename E::raw;
  constexpr bool kT = DivTraits<KIND>::kT;
  constexpr bool kTeacher = DivTraits<KIND>::kTeacher;
  constexpr int NT = 64 * W;
  constexpr int VEC = E::kVec;
  constexpr int BATCH = U * NT;
  const int64_t row = blockIdx.x;
  const int64_t b = row / R;
  const int64_t r = row - b * R;
  const int tid = threadIdx.x;
  const raw* x = xs + b * ssb + r * ssr;
  const raw* y = kTeacher ? xt + b * tsb + r * tsr : x;

  DivState<KIND> st;
  if constexpr (kTeacher) {
    const float c0 = E::load(y);
    st.c = isfinite(c0) ? c0 : 0.f;
  }
  const RowSpan<E> sx(x, V);
  const RowSpan<E> sy(y, V);
  if (sx.head != sy.head) {
    // student and teacher rows not co-aligned: element-wise path
    for (int64_t j = tid; j < V; j += NT) {
      const float a[1] = {E::load(x + j)};
      const float bt[1] = {E::load(y + j)};
      st.add(a, bt);
    }
  } else {
    const vu4* xv = reinterpret_cast<const vu4*>(x + sx.head);
    const vu4* yv = reinterpret_cast<const vu4*>(y + sx.head);
    const int nvec = (int)sx.nvec;
    const int nbatch = (nvec + BATCH - 1) / BATCH;
    const vu4 pad = vu4{E::kLowPad2, E::kLowPad2, E::kLowPad2, E::kLowPad2};
    vu4 q[U], qt[U];
    auto issue = [&](int base) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * NT;
        q[u] = (j < nvec) ? __builtin_nontemporal_load(xv + j) : pad;
        if constexpr (kTeacher) qt[u] = (j < nvec) ? __builtin_nontemporal_load(yv + j) : pad;
      }
    };
    if (nbatch > 0) issue(tid);
    const float lowpad = -0x1p100f;
    float hx[2], hy[2];
    hx[0] = (tid < sx.head) ? E::load(x + tid) : lowpad;
    hy[0] = (kTeacher && tid < sx.head) ? E::load(y + tid) : lowpad;
    const int64_t ti = sx.tail0 + tid;
    hx[1] = (ti < V) ? E::load(x + ti) : lowpad;
    hy[1] = (kTeacher && ti < V) ? E::load(y + ti) : lowpad;
    __builtin_amdgcn_sched_barrier(0);
    for (int k = 0; k < nbatch; ++k) {
      float v[U * VEC], vt[U * VEC];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float w[VEC];
        E::unpack(q[u], w);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[u * VEC + e] = w[e];
        if constexpr (kTeacher) {
          E::unpack(qt[u], w);
#pragma unroll
          for (int e = 0; e < VEC; ++e) vt[u * VEC + e] = w[e];
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) vt[u * VEC + e] = 0.f;
        }
      }
      st.add(v, vt);
      if (k + 1 < nbatch) issue(tid + (k + 1) * BATCH);
      __builtin_amdgcn_sched_barrier(0);
    }
    st.add(hx, hy);
  }

  // merge lanes
  float M = wave_max(st.m);
  const float OFF = M * kLog2e;
  float S, T = 0.f, Uu = 0.f;
  {
    const float d = st.off - OFF;
    const float sc = (st.m == -INFINITY) ? 0.f : fast_exp2(d);
    const float s0 = st.s[0] + st.s[1];
    S = sc * s0;
    if constexpr (kT) T = sc * fmaf(d, s0, st.t[0] + st.t[1]);
    if constexpr (kTeacher) Uu = sc * (st.u[0] + st.u[1]);
  }
  S = wave_sum(S);
  if constexpr (kT) T = wave_sum(T);
  if constexpr (kTeacher) Uu = wave_sum(Uu);
  float Mt = 0.f, St = 0.f;
  if constexpr (kTeacher) {
    Mt = wave_max(st.mt);
    St = (st.mt == -INFINITY) ? 0.f : (st.st[0] + st.st[1]) * fast_exp2(st.offt - Mt * kLog2e);
    St = wave_sum(St);
  }
  if constexpr (W > 1) {
    __shared__ float sm[W], ss[W], stt[W], su[W], smt[W], sst[W];
    const int wv = tid / 64, lane = tid % 64;
    if (lane == 0) {
      sm[wv] = M;
      ss[wv] = S;
      stt[wv] = T;
      su[wv] = Uu;
      smt[wv] = Mt;
      sst[wv] = St;
    }
    __syncthreads();
    if (tid == 0) {
      float Mb = sm[0];
#pragma unroll
      for (int k = 1; k < W; ++k) Mb = fmaxf(Mb, sm[k]);
      const float OFFb = Mb * kLog2e;
      float Sb = 0.f, Tb = 0.f, Ub = 0.f;
#pragma unroll
      for (int k = 0; k < W; ++k) {
        if (sm[k] == -INFINITY) continue;
        const float d = sm[k] * kLog2e - OFFb;
        const float sc = fast_exp2(d);
        Sb += sc * ss[k];
        if constexpr (kT) Tb += sc * fmaf(d, ss[k], stt[k]);
        if constexpr (kTeacher) Ub += sc * su[k];
      }
      M = Mb;
      S = Sb;
      T = Tb;
      Uu = Ub;
      if constexpr (kTeacher) {
        float Mtb = smt[0];
#pragma unroll
        for (int k = 1; k < W; ++k) Mtb = fmaxf(Mtb, smt[k]);
        const float OFFt = Mtb * kLog2e;
        float Stb = 0.f;
#pragma unroll
        for (int k = 0; k < W; ++k)
          Stb += (smt[k] == -INFINITY) ? 0.f : sst[k] * fast_exp2(smt[k] * kLog2e - OFFt);
        Mt = Mtb;
        St = Stb;
      }
    }
  }
  if (tid == 0) {
    const float OFFf = M * kLog2e;
    const float corr = fmaf(M, kLog2e, -OFFf);
    const float lnS = logf(S);
    const float logZ = lnS - corr * kLn2;
    float L = 0.f, logZt = 0.f;
    if constexpr (kT) L = kLn2 * (T / S) - lnS;
    if constexpr (kTeacher) {
      const float corrt = fmaf(Mt, kLog2e, -(Mt * kLog2e));
      logZt = logf(St) - corrt * kLn2;
      const float ce = ((Mt - st.c) + logZt) - Uu / S;
      L = (KIND == MIRL_DIV_CROSS_ENTROPY) ? ce : L + ce;
    }
    out[row] = L;
    if (stats != nullptr) {
      float* o = stats + 4 * row;
      o[0] = M;
      o[1] = logZ;
      o[2] = Mt;
      o[3] = logZt;
    }
  }
}

// Gradient of one element: (p (w - L)) g with p = exp((x - M) - logZ).
template <int KIND>
__device__ __forceinline__ float div_grad(float xs, float xt, float M, float logZ, float Mt,
                                          float logZt, float L, float g) {
  const float lps = (xs - M) - logZ;
  const float p = fast_exp2(lps * kLog2e);
  float w;
  if constexpr (KIND == MIRL_DIV_ENTROPY) {
    w = lps;
  } else {
    const float lpt = (xt - Mt) - logZt;
    w = (KIND == MIRL_DIV_CROSS_ENTROPY) ? -lpt : lps - lpt;
  }
  return (p * (w - L)) * g;
}

// Flat backward over contiguous [rows, V] student / teacher / gradient arrays
// with whole 16-byte vectors per row: one 4 KB piece of the gradient per
// 128-thread workgroup (two vectors per lane, 2 KB apart), piece boundaries on
// 4 KB gradient addresses, nontemporal loads and stores (reverse KL on bf16
// [8, 2048, 151936]: 1.59 ms, against 1.67 ms for 8 KB pieces of 256 threads
// with plain loads).
constexpr int kDivFlatThreads = 128;

template <class E, int KIND>
__global__ __launch_bounds__(kDivFlatThreads) void divergence_bwd_flat_kernel(
    const typename E::raw* __restrict__ xs, const typename E::raw* __restrict__ xt, uint32_t nvr,
    uint32_t nvec, int shift, const float* __restrict__ Lrow, const float* __restrict__ stats,
    const float* __restrict__ g, int64_t R, int64_t gsb, int64_t gsr, typename E::raw* gin) {
  constexpr bool kTeacher = DivTraits<KIND>::kTeacher;
  constexpr int VEC = E::kVec;
  constexpr int NT = kDivFlatThreads, U = 2;
  vu4* yv = reinterpret_cast<vu4*>(gin);
  const vu4* xv = reinterpret_cast<const vu4*>(xs);
  const vu4* tv = reinterpret_cast<const vu4*>(xt);
  const int64_t base = (int64_t)blockIdx.x * (NT * U) + threadIdx.x - shift;
  bool ok[U];
  float gv[U], M[U], LZ[U], Mt[U], LZt[U], L[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + u * NT;
    ok[u] = i >= 0 && i < (int64_t)nvec;
    const uint32_t row = (ok[u] ? (uint32_t)i : 0u) / nvr;
    gv[u] = M[u] = LZ[u] = Mt[u] = LZt[u] = L[u] = 0.f;
    if (ok[u]) {
      const int64_t b = row / R, r = row - b * R;
      gv[u] = g[b * gsb + r * gsr];
      const float* o = stats + 4 * (int64_t)row;
      M[u] = o[0];
      LZ[u] = o[1];
      Mt[u] = o[2];
      LZt[u] = o[3];
      L[u] = Lrow[row];
    }
  }
  vu4 q[U], qt[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (ok[u] && gv[u] != 0.f) {
      q[u] = __builtin_nontemporal_load(xv + base + u * NT);
      if constexpr (kTeacher) qt[u] = __builtin_nontemporal_load(tv + base + u * NT);
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    const int64_t i = base + u * NT;
    if (gv[u] == 0.f) {
      __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + i);
      continue;
    }
    float w[VEC], wt[VEC], o[VEC];
    E::unpack(q[u], w);
    if constexpr (kTeacher) E::unpack(qt[u], wt);
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      o[k] = div_grad<KIND>(w[k], kTeacher ? wt[k] : 0.f, M[u], LZ[u], Mt[u], LZt[u], L[u], gv[u]);
    __builtin_nontemporal_store(E::pack(o), yv + i);
  }
}

// Row-per-workgroup backward for any strides (vector body when the student,
// teacher and gradient rows are co-aligned, element-wise otherwise).
template <class E, int KIND>
__global__ __launch_bounds__(256) void divergence_bwd_row_kernel(
    const typename E::raw* __restrict__ xs, const typename E::raw* __restrict__ xt, int64_t R,
    int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr,
    const float* __restrict__ Lrow, const float* __restrict__ stats,
    const float* __restrict__ g, int64_t gsb, int64_t gsr, typename E::raw* gin, int64_t gisb,
    int64_t gisr) {
  using raw = typename E::raw;
  constexpr bool kTeacher = DivTraits<KIND>::kTeacher;
  constexpr int VEC = E::kVec;
  constexpr int NT = 256;
  const int64_t row = blockIdx.x;
  const int64_t b = row / R, r = row - b * R;
  const int tid = threadIdx.x;
  raw* y = gin + b * gisb + r * gisr;
  const float gv = g[b * gsb + r * gsr];
  const RowSpan<E> ys(y, V);
  if (gv == 0.f) {
    const raw z = E::from_float(0.f);
    vu4* yvec = reinterpret_cast<vu4*>(y + ys.head);
    if (tid < ys.head) y[tid] = z;
    if (ys.tail0 + tid < V) y[ys.tail0 + tid] = z;
    for (int64_t i = tid; i < ys.nvec; i += NT)
      __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yvec + i);
    return;
  }
  const raw* x = xs + b * ssb + r * ssr;
  const raw* t = kTeacher ? xt + b * tsb + r * tsr : x;
  const float* o = stats + 4 * row;
  const float M = o[0], LZ = o[1], Mt = o[2], LZt = o[3], L = Lrow[row];
  const RowSpan<E> xsp(x, V), tsp(t, V);
  if (xsp.head != ys.head || tsp.head != ys.head) {
    for (int64_t j = tid; j < V; j += NT)
      y[j] = E::from_float(div_grad<KIND>(E::load(x + j), kTeacher ? E::load(t + j) : 0.f, M, LZ,
                                          Mt, LZt, L, gv));
    return;
  }
  auto scalar = [&](int64_t j) {
    y[j] = E::from_float(
        div_grad<KIND>(E::load(x + j), kTeacher ? E::load(t + j) : 0.f, M, LZ, Mt, LZt, L, gv));
  };
  if (tid < ys.head) scalar(tid);
  if (ys.tail0 + tid < V) scalar(ys.tail0 + tid);
  const vu4* xv = reinterpret_cast<const vu4*>(x + ys.head);
  const vu4* tv = reinterpret_cast<const vu4*>(t + ys.head);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  for (int64_t i = tid; i < ys.nvec; i += NT) {
    float w[VEC], wt[VEC], out[VEC];
    E::unpack(xv[i], w);
    if constexpr (kTeacher) E::unpack(tv[i], wt);
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      out[k] = div_grad<KIND>(w[k], kTeacher ? wt[k] : 0.f, M, LZ, Mt, LZt, L, gv);
    __builtin_nontemporal_store(E::pack(out), yv + i);
  }
}

int pick_waves(int64_t rows) {
  int w = 4;
  while (w < 16 && rows * w < 8192) w <<= 1;
  return w;
}

template <class E, int KIND, int W>
void launch_fwd(int64_t rows, hipStream_t st, const void* xs, const void* xt, int64_t R,
                int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, float* out,
                float* stats) {
  // two inputs in flight per batch for the teacher kinds
  constexpr int U = DivTraits<KIND>::kTeacher ? 4 : 8;
  using raw = typename E::raw;
  hipLaunchKernelGGL((divergence_fwd_kernel<E, W, U, KIND>), dim3((unsigned)rows), dim3(64 * W),
                     0, st, static_cast<const raw*>(xs), static_cast<const raw*>(xt), R, V, ssb,
                     ssr, tsb, tsr, out, stats);
}

template <class E, int KIND>
void dispatch_fwd(int64_t rows, hipStream_t st, const void* xs, const void* xt, int64_t R,
                  int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, float* out,
                  float* stats) {
  switch (pick_waves(rows)) {
    case 4: launch_fwd<E, KIND, 4>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats); break;
    case 8: launch_fwd<E, KIND, 8>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats); break;
    default: launch_fwd<E, KIND, 16>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats); break;
  }
}

template <class E, int KIND>
void dispatch_bwd(int64_t rows, hipStream_t st, const void* xs, const void* xt, int64_t R,
                  int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, const float* L,
                  const float* stats, const float* g, int64_t gsb, int64_t gsr, void* gin,
                  int64_t gisb, int64_t gisr) {
  using raw = typename E::raw;
  constexpr int VEC = E::kVec;
  constexpr bool kTeacher = DivTraits<KIND>::kTeacher;
  const uintptr_t ya = reinterpret_cast<uintptr_t>(gin), xa = reinterpret_cast<uintptr_t>(xs),
                  ta = reinterpret_cast<uintptr_t>(xt);
  // every [B, R, V] array contiguous with the same layout
  const bool contig = gisr == V && gisb == R * V && ssr == V && ssb == R * V &&
                      (!kTeacher || (tsr == V && tsb == R * V));
  const int64_t nvr = V / VEC;
  const int64_t nvec = rows * nvr;
  if (V % VEC == 0 && contig && (ya & 15u) == 0 && (xa & 15u) == 0 &&
      (!kTeacher || (ta & 15u) == 0) && nvec + 512 < (int64_t(1) << 32)) {
    const int to4k = (int)(((4096u - (ya & 4095u)) & 4095u) / 16u);
    constexpr int P = kDivFlatThreads * 2;  // vectors per 4 KB piece
    const int shift = (P - to4k) & (P - 1);
    const int64_t grid = (nvec + shift + P - 1) / P;
    hipLaunchKernelGGL((divergence_bwd_flat_kernel<E, KIND>), dim3((unsigned)grid),
                       dim3(kDivFlatThreads), 0, st, static_cast<const raw*>(xs),
                       static_cast<const raw*>(xt), (uint32_t)nvr, (uint32_t)nvec, shift, L, stats,
                       g, R, gsb, gsr, static_cast<raw*>(gin));
    return;
  }
  hipLaunchKernelGGL((divergence_bwd_row_kernel<E, KIND>), dim3((unsigned)rows), dim3(256), 0, st,
                     static_cast<const raw*>(xs), static_cast<const raw*>(xt), R, V, ssb, ssr, tsb,
                     tsr, L, stats, g, gsb, gsr, static_cast<raw*>(gin), gisb, gisr);
}

template <class E>
void fwd_kind(int kind, int64_t rows, hipStream_t st, const void* xs, const void* xt, int64_t R,
              int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, float* out,
              float* stats) {
  switch (kind) {
    case MIRL_DIV_ENTROPY:
      dispatch_fwd<E, MIRL_DIV_ENTROPY>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats);
      break;
    case MIRL_DIV_CROSS_ENTROPY:
      dispatch_fwd<E, MIRL_DIV_CROSS_ENTROPY>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats);
      break;
    default:
      dispatch_fwd<E, MIRL_DIV_REVERSE_KL>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, out, stats);
      break;
  }
}

template <class E>
void bwd_kind(int kind, int64_t rows, hipStream_t st, const void* xs, const void* xt, int64_t R,
              int64_t V, int64_t ssb, int64_t ssr, int64_t tsb, int64_t tsr, const float* L,
              const float* stats, const float* g, int64_t gsb, int64_t gsr, void* gin,
              int64_t gisb, int64_t gisr) {
  switch (kind) {
    case MIRL_DIV_ENTROPY:
      dispatch_bwd<E, MIRL_DIV_ENTROPY>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, L, stats, g,
                                        gsb, gsr, gin, gisb, gisr);
      break;
    case MIRL_DIV_CROSS_ENTROPY:
      dispatch_bwd<E, MIRL_DIV_CROSS_ENTROPY>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, L, stats,
                                              g, gsb, gsr, gin, gisb, gisr);
      break;
    default:
      dispatch_bwd<E, MIRL_DIV_REVERSE_KL>(rows, st, xs, xt, R, V, ssb, ssr, tsb, tsr, L, stats, g,
                                           gsb, gsr, gin, gisb, gisr);
      break;
  }
}

int check_args(int kind, int dtype, int64_t B, int64_t R, int64_t V, const void* xs,
               const void* xt) {
  MIRL_REQUIRE(kind == MIRL_DIV_ENTROPY || kind == MIRL_DIV_CROSS_ENTROPY ||
                   kind == MIRL_DIV_REVERSE_KL,
               "invalid divergence kind %d", kind);
  if (!(dtype == MIRL_DTYPE_F32 || dtype == MIRL_DTYPE_BF16 || dtype == MIRL_DTYPE_F16)) {
    set_error("unsupported logits dtype code %d (expected f32, bf16 or f16)", dtype);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0, "invalid shape B=%lld R=%lld V=%lld", (long long)B,
               (long long)R, (long long)V);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  MIRL_REQUIRE(B * R < (int64_t(1) << 31), "too many rows (%lld)", (long long)(B * R));
  MIRL_REQUIRE(xs != nullptr, "null student logits");
  MIRL_REQUIRE(kind == MIRL_DIV_ENTROPY || xt != nullptr, "teacher logits required");
  return MIRL_OK;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_divergence_fwd(int kind, const void* student, const void* teacher, int dtype,
                                   int64_t B, int64_t R, int64_t V, int64_t s_stride_b,
                                   int64_t s_stride_r, int64_t t_stride_b, int64_t t_stride_r,
                                   float* out, float* row_stats, void* stream) {
  clear_error();
  if (int e = check_args(kind, dtype, B, R, V, student, teacher)) return e;
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(out != nullptr, "null output");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      fwd_kind<F32>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                    t_stride_r, out, row_stats);
      break;
    case MIRL_DTYPE_BF16:
      fwd_kind<BF16>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                     t_stride_r, out, row_stats);
      break;
    default:
      fwd_kind<F16>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                    t_stride_r, out, row_stats);
      break;
  }
  return check_launch("mirl_divergence_fwd");
}

extern "C" int mirl_divergence_bwd(int kind, const void* student, const void* teacher, int dtype,
                                   int64_t B, int64_t R, int64_t V, int64_t s_stride_b,
                                   int64_t s_stride_r, int64_t t_stride_b, int64_t t_stride_r,
                                   const float* out, const float* row_stats,
                                   const float* grad_out, int64_t g_stride_b, int64_t g_stride_r,
                                   void* grad_in, int64_t gi_stride_b, int64_t gi_stride_r,
                                   void* stream) {
  clear_error();
  if (int e = check_args(kind, dtype, B, R, V, student, teacher)) return e;
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(out && row_stats && grad_out && grad_in, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case MIRL_DTYPE_F32:
      bwd_kind<F32>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                    t_stride_r, out, row_stats, grad_out, g_stride_b, g_stride_r, grad_in,
                    gi_stride_b, gi_stride_r);
      break;
    case MIRL_DTYPE_BF16:
      bwd_kind<BF16>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                     t_stride_r, out, row_stats, grad_out, g_stride_b, g_stride_r, grad_in,
                     gi_stride_b, gi_stride_r);
      break;
    default:
      bwd_kind<F16>(kind, rows, st, student, teacher, R, V, s_stride_b, s_stride_r, t_stride_b,
                    t_stride_r, out, row_stats, grad_out, g_stride_b, g_stride_r, grad_in,
                    gi_stride_b, gi_stride_r);
      break;
  }
  return check_launch("mirl_divergence_bwd");
}

// Top-k / top-p / temperature-filtered token logprobs.
//
// Semantics (reference nemo_rl/algorithms/logits_sampling_utils.py:69-212 and
// nemo_rl/distributed/model_utils.py:352-479, in the production chain of
// model_utils.py:1660-1718): y = dtype(fl32(float(x) * fl32(1.0 / T))) — the
// in-place division of automodel/train.py:248-262 as torch runs it on the GPU
// (a product with the rounded reciprocal), skipped when T == 1 — read as fp32;
//   top-k: keep y >= the k-th largest y (every tie at the k-th value kept);
//   top-p: over the kept-k values in ascending order with ties ordered by
//          vocabulary index (a stable sort), p = softmax, cum = cumulative sum
//          accumulated in double and rounded to fp32, keep cum > fp32(1 - top_p),
//          always keep the maximum;
//   logprob(t) = (y_t - m) - log(sum_kept exp(y - m)), -inf when t is not kept.
// The kept set is always a suffix of that ascending order, so it is described
// by one lexicographic cut (v_cut, i_cut): j kept <=> y_j > v_cut or
// (y_j == v_cut and j >= i_cut).
//
// Forward, fast path (1 <= k <= 1024): one workgroup per row streams the row
// once, keeping per-lane maxima and per-(lane, group-of-vectors) maxima.  The
// k-th largest lane maximum is a lower bound tau on the k-th largest value
// (k distinct elements are >= it), so only groups whose maximum reaches tau
// can hold a kept element; those few groups are listed in LDS and re-read by
// the whole workgroup as independent loads (a few KB per row), and their
// elements >= tau collected in LDS.  Sorting the candidates by (value, index)
// gives the exact top-k value (the k-th largest), the stable-order top-p cut
// and the kept-set log-sum-exp.  Rows whose candidates overflow LDS are
// flagged and redone by the general path.
//
// Forward, general path (top-p without top-k, k > 1024, flagged rows): 16-bit
// rows go to the histogram kernels (topk_hist.hip), fp32 rows to the two-pass
// kernel (topk_f32.hip); what those cannot finish (values outside their
// tables, candidate overflow) to an exact multi-pass radix selection over the
// row (count histograms for the top-k value, probability-mass histograms for
// the top-p cut), re-reading the row for each 8-bit digit.
//
// Backward: grad = (onehot(t) - p) * g on the kept set, 0 elsewhere, rounded
// to the logits dtype, then multiplied by fl32(1.0 / T) and rounded to that
// dtype again (the reference's autograd chain through .to(float32) and div_,
// as torch runs it on the GPU).  A write-only pass zeroes the
// rows; a second, small pass stores the kept entries from the kept list saved
// by the forward (<= kKeepCap entries), without reading the logits.  Rows with
// larger kept sets are re-read and rewritten whole by the second pass.

#include <cstdlib>

#include "filter.h"

namespace mirl {
namespace {

constexpr int kCandCap = 1024;  // candidates held in LDS by the fast path
constexpr int kMaxGroups = 20;  // vector groups per lane in the fast path
constexpr int kGeneralThreads = 1024;

// Upper 16 bits of okey(v), rounded up: from_okey(hi << 16) >= v.  Exact for
// 16-bit inputs, whose keys have zero low halves.
__device__ __forceinline__ uint16_t okey_hi_up(float v) {
  const uint32_t k = okey(v);
  const uint32_t hi = k >> 16;
  return (uint16_t)(((k & 0xffffu) != 0u && hi < 0xffffu) ? hi + 1u : hi);
}
// k-th largest of the NT order keys okey(vals[i]) (vals in LDS), computed by
// one wave: the largest c with #{key >= c} >= k, one bit per round from bit 31
// down to LOW_BIT, counted by ballot.  Bits below LOW_BIT are left zero, so the
// result is a lower bound when the keys have nonzero low bits (exact for values
// of a 16-bit type with LOW_BIT = 16).  Only wave 0 may call it.
template <int NT, int LOW_BIT>
__device__ uint32_t wave_kth_largest(const float* vals, int k) {
  constexpr int PER = NT / 64;
  const int lane = threadIdx.x % 64;
  uint32_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) key[i] = okey(vals[lane + 64 * i]);
  uint32_t prefix = 0;
  for (int bit = 31; bit >= LOW_BIT; --bit) {
    const uint32_t cand = prefix | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) cnt += __popcll(__ballot(key[i] >= cand));
    if (cnt >= k) prefix = cand;
  }
  return prefix;
}

// Ascending sort of n <= kCandCap distinct 64-bit keys in LDS by the whole
// workgroup: each key's rank is the number of smaller keys.  Must be entered
// after a barrier that publishes the keys; ends with a barrier.
template <int NT>
__device__ void block_rank_sort(uint64_t* keys, int n) {
  constexpr int PER = (kCandCap + NT - 1) / NT;
  const int tid = threadIdx.x;
  uint64_t mine[PER];
  int rank[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int i = tid + p * NT;
    mine[p] = i < n ? keys[i] : ~0ull;
    rank[p] = 0;
  }
  for (int j = 0; j < n; ++j) {
    const uint64_t kj = keys[j];
#pragma unroll
    for (int p = 0; p < PER; ++p) rank[p] += (kj < mine[p]) ? 1 : 0;
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < PER; ++p)
    if (tid + p * NT < n) keys[rank[p]] = mine[p];
  __syncthreads();
}

// Writes the row's results; run by wave 0 alone (the other waves may have
// left).  `skeys` holds the kept-k candidates sorted ascending as
// (okey(y) << 32 | index); `thr` is the top-k value; `yt` is the target's
// scaled logit (lane 0 only; NaN when there is no target in range).
template <class E, bool DEC16>
__device__ void finish_row(const FilterParams& P, int64_t row, const uint64_t* skeys, int n_k,
                           float thr, float yt, int64_t t) {
  const int lane = threadIdx.x;
  auto y_at = [&](int i) { return from_okey((uint32_t)(skeys[i] >> 32)); };
  const float m = y_at(n_k - 1);
  int first = 0;
  if (P.has_p) {
    // the softmax normaliser, summed in double and rounded once to fp32
    double zpart = 0.0;
    for (int i = lane; i < n_k; i += 64) zpart += (double)expf(y_at(i) - m);
    const float Z = (float)wave_sum(zpart);
    first = n_k - 1;  // the maximum is always kept
    if constexpr (DEC16) {
      // probabilities rounded to the logits dtype; the cumulative sum is
      // accumulated one element at a time in fp32, in ascending order (every
      // lane holds the same running sum and adds each element read from its
      // lane), and each partial sum is rounded to the dtype before the compare
      float S = 0.f;
      for (int base = 0; base < n_k; base += 64) {
        const int i = base + lane;
        const float p = (i < n_k) ? round_trip<E>(expf(y_at(i) - m) / Z) : 0.f;
        float mine = 0.f;
        const int n_here = n_k - base < 64 ? n_k - base : 64;
        for (int l = 0; l < n_here; ++l) {
          S += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), l));
          mine = (lane == l) ? S : mine;
        }
        const uint64_t bal = __ballot((i < n_k) && (round_trip<E>(mine) > P.thr16));
        if (bal != 0ull) {
          first = base + __ffsll((long long)bal) - 1;
          break;
        }
      }
    } else {
      // cumulative probability in ascending order, accumulated in double
      const float inv = 1.0f / Z;
      double run = 0.0;
      for (int base = 0; base < n_k; base += 64) {
        const int i = base + lane;
        double inc = (i < n_k) ? (double)(expf(y_at(i) - m) * inv) : 0.0;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const double o = __shfl_up(inc, off, 64);
          if (lane >= off) inc += o;
        }
        const bool hit = (i < n_k) && ((float)(run + inc) > P.cut);
        const uint64_t bal = __ballot(hit);
        if (bal != 0ull) {
          first = base + __ffsll((long long)bal) - 1;
          break;
        }
        run += __shfl(inc, 63, 64);
      }
    }
  }
  const uint64_t ck = skeys[first];
  const float v_cut = P.has_p ? from_okey((uint32_t)(ck >> 32)) : thr;
  const int32_t i_cut = P.has_p ? (int32_t)(ck & 0xffffffffu) : 0;
  const int n_kept = n_k - first;
  float spart = 0.f;
  for (int i = first + lane; i < n_k; i += 64) spart += expf(y_at(i) - m);
  const float logsum = logf(wave_sum(spart));
  if (n_kept <= kKeepCap) {
    int32_t* ki = P.kept_idx + row * kKeepCap;
    float* kp = P.kept_p + row * kKeepCap;
    for (int i = first + lane; i < n_k; i += 64) {
      ki[i - first] = (int32_t)(skeys[i] & 0xffffffffu);
      kp[i - first] = expf((y_at(i) - m) - logsum);
    }
  }
  if (lane == 0) {
    RowInfo ri;
    ri.m = m;
    ri.logsum = logsum;
    ri.v_cut = v_cut;
    ri.i_cut = i_cut;
    ri.n_kept = n_kept;
    ri.flags = 0;
    P.info[row] = ri;
    if (P.out != nullptr) {
      float lp = -INFINITY;
      if (t >= 0 && t < P.V && kept_lex(yt, t, v_cut, i_cut)) lp = (yt - m) - logsum;
      P.out[row] = lp;
    }
  }
}

// Top-k export epilogue: `top` holds the k largest (okey(y) << 32 | ~index)
// keys in ascending order; entry i of the output is the (i+1)-th largest, its
// value re-read from the logits (exact, including the sign of zero).
template <class E>
__device__ void export_topk(const FilterParams& P, int64_t row, const typename E::raw* x,
                            const uint64_t* top) {
  const int k = P.top_k;
  for (int i = threadIdx.x; i < k; i += blockDim.x) {
    const int64_t j = (int64_t)(~(uint32_t)(top[k - 1 - i] & 0xffffffffu));
    P.tk_vals[row * k + i] = E::load(x + j);
    P.tk_idx[row * k + i] = P.tk_base + j;
  }
  if (threadIdx.x == 0) P.info[row].flags = 0;
}

// Order key of the export: every NaN (either sign) above +inf, as torch.topk ranks it.
__device__ __forceinline__ uint32_t okey_export(float y) {
  return (y != y) ? 0xffffffffu : okey(y);
}

// k-th largest order key of the row by radix selection (8 bits per pass), and
// how many elements equal to it belong to the top k ("remaining").
template <int NT, class Y>
__device__ uint32_t radix_kth_key(Y&& yat, int64_t V, int k, int* hist_i, uint32_t* s_sel,
                                  int* remaining_out, bool nan_high) {
  const int tid = threadIdx.x;
  uint32_t prefix = 0, mask = 0;
  int remaining = k;
  for (int d = 3; d >= 0; --d) {
    const int shift = 8 * d;
    for (int i = tid; i < 256; i += NT) hist_i[i] = 0;
    __syncthreads();
    for (int64_t j = tid; j < V; j += NT) {
      const float y = yat(j);
      const uint32_t kk = nan_high ? okey_export(y) : okey(y);
      if ((kk & mask) == prefix) atomicAdd(&hist_i[(kk >> shift) & 255u], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0, bsel = 0;
      for (int bin = 255; bin >= 0; --bin) {
        if (acc + hist_i[bin] >= remaining) {
          bsel = bin;
          break;
        }
        acc += hist_i[bin];
      }
      s_sel[0] = (uint32_t)bsel;
      s_sel[1] = (uint32_t)(remaining - acc);
    }
    __syncthreads();
    prefix |= s_sel[0] << shift;
    mask |= 255u << shift;
    remaining = (int)s_sel[1];
    __syncthreads();
  }
  *remaining_out = remaining;
  return prefix;
}

// The export's exact cut for k: the k-th largest order key thr (radix
// selection over the value bits) and i_last, the index of the last element
// equal to thr that belongs to the top k (the `remaining`-th smallest index
// among them, by radix selection over the index bits).  The top k are then the
// elements with key > thr, or key == thr and index <= i_last.
template <int NT, class Y>
__device__ void export_cut(Y&& yat, int64_t V, int k, int* hist_i, uint32_t* s_sel, uint32_t* thr_out,
                           uint32_t* i_last_out) {
  const int tid = threadIdx.x;
  int remaining = 0;
  const uint32_t thr = radix_kth_key<NT>(yat, V, k, hist_i, s_sel, &remaining, true);

  // the remaining-th smallest index among the elements whose key equals thr
  int top_bit = 0;
  while ((int64_t(1) << (top_bit + 1)) < V) ++top_bit;
  uint32_t iprefix = 0, imask = 0;
  int need = remaining;
  for (int hi = top_bit; hi >= 0; hi -= 8) {
    const int lo = hi >= 7 ? hi - 7 : 0;
    const int nb = hi - lo + 1;
    const uint32_t dmask = (1u << nb) - 1u;
    for (int i = tid; i < 256; i += NT) hist_i[i] = 0;
    __syncthreads();
    for (int64_t j = tid; j < V; j += NT) {
      if (okey_export(yat(j)) != thr) continue;
      const uint32_t jj = (uint32_t)j;
      if ((jj & imask) != iprefix) continue;
      atomicAdd(&hist_i[(jj >> lo) & dmask], 1);
    }
    __syncthreads();
    if (tid == 0) {
      int acc = 0, bsel = 0;
      for (int bin = 0; bin <= (int)dmask; ++bin) {
        if (acc + hist_i[bin] >= need) {
          bsel = bin;
          break;
        }
        acc += hist_i[bin];
      }
      s_sel[0] = (uint32_t)bsel;
      s_sel[1] = (uint32_t)(need - acc);
    }
    __syncthreads();
    iprefix |= s_sel[0] << lo;
    imask |= dmask << lo;
    need = (int)s_sel[1];
    __syncthreads();
  }
  *thr_out = thr;
  *i_last_out = iprefix;
}

// General top-k export for the rows the fast path flagged (candidate
// overflow, i.e. many equal values): the exact cut, then exactly k entries
// collected and rank-sorted.
template <class E>
__global__ __launch_bounds__(kGeneralThreads) void topk_export_general_kernel(FilterParams P) {
  using raw = typename E::raw;
  constexpr int NT = kGeneralThreads;
  __shared__ int hist_i[256];
  __shared__ uint32_t s_sel[2];
  __shared__ int s_cnt;
  __shared__ uint64_t s_cand[kCandCap];
  const int64_t row = blockIdx.x;
  if ((P.info[row].flags & 1) == 0) return;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;
  auto yat = [&](int64_t j) { return E::load(x + j); };
  uint32_t thr, i_last;
  export_cut<NT>(yat, V, P.top_k, hist_i, s_sel, &thr, &i_last);

  if (tid == 0) s_cnt = 0;
  __syncthreads();
  for (int64_t j = tid; j < V; j += NT) {
    const uint32_t kk = okey_export(yat(j));
    if (kk > thr || (kk == thr && (uint32_t)j <= i_last)) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < kCandCap) s_cand[slot] = ((uint64_t)kk << 32) | (uint64_t)(~(uint32_t)j);
    }
  }
  __syncthreads();
  block_rank_sort<NT>(s_cand, P.top_k);
  export_topk<E>(P, row, x, s_cand);
}

// Descending sort of n 64-bit keys at `a` (LDS or global memory) by the whole
// workgroup: a bitonic network in which every merge compares in the same
// direction (the first step of each merge pairs i with its mirror in the
// block), so positions >= n act as keys below every real one and are never
// touched, for any n.  Every thread must enter it.
template <int NT>
__device__ void bitonic_sort_desc(uint64_t* a, int64_t n) {
  int64_t N = 1;
  while (N < n) N <<= 1;
  for (int64_t blk = 2; blk <= N; blk <<= 1) {
    // mirror step: i in the lower half of its block against blk - 1 - (i mod blk)
    for (int64_t t = threadIdx.x; t < N / 2; t += NT) {
      const int64_t base = (t / (blk / 2)) * blk, off = t % (blk / 2);
      const int64_t i = base + off, l = base + blk - 1 - off;
      if (l < n) {
        const uint64_t u = a[i], v = a[l];
        if (u < v) {
          a[i] = v;
          a[l] = u;
        }
      }
    }
    __syncthreads();
    for (int64_t j = blk / 4; j >= 1; j >>= 1) {
      for (int64_t t = threadIdx.x; t < N / 2; t += NT) {
        const int64_t i = (t / j) * 2 * j + (t % j), l = i + j;
        if (l < n) {
          const uint64_t u = a[i], v = a[l];
          if (u < v) {
            a[i] = v;
            a[l] = u;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Rows held in LDS by the large-k export's sort (16384 keys, 128 KB); larger
// k sort in place in the row's own index output.
constexpr int kExportLdsKeys = 16384;

// Top-k export for k > kCandCap: the exact cut, the k entries collected as
// sort keys (order key << 32 | ~index: larger = higher value, then lower id)
// and sorted descending, then written out with their values re-read.
template <class E>
__global__ __launch_bounds__(kGeneralThreads) void topk_export_large_kernel(FilterParams P) {
  using raw = typename E::raw;
  constexpr int NT = kGeneralThreads;
  __shared__ int hist_i[256];
  __shared__ uint32_t s_sel[2];
  __shared__ int s_cnt;
  __shared__ uint64_t s_keys[kExportLdsKeys];
  const int64_t row = blockIdx.x;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;
  const int k = P.top_k;
  auto yat = [&](int64_t j) { return E::load(x + j); };
  uint32_t thr, i_last;
  export_cut<NT>(yat, V, k, hist_i, s_sel, &thr, &i_last);
  uint64_t* keys = k <= kExportLdsKeys ? s_keys
                                       : reinterpret_cast<uint64_t*>(P.tk_idx + row * (int64_t)k);
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  for (int64_t j = tid; j < V; j += NT) {
    const uint32_t kk = okey_export(yat(j));
    if (kk > thr || (kk == thr && (uint32_t)j <= i_last)) {
      const int slot = atomicAdd(&s_cnt, 1);
      if (slot < k) keys[slot] = ((uint64_t)kk << 32) | (uint64_t)(~(uint32_t)j);
    }
  }
  __syncthreads();
  bitonic_sort_desc<NT>(keys, k);
  // each thread reads its keys before any output is written over them
  for (int64_t i0 = 0; i0 < k; i0 += NT) {
    const int64_t i = i0 + tid;
    uint64_t key = 0;
    if (i < k) key = keys[i];
    __syncthreads();
    if (i < k) {
      const int64_t j = (int64_t)(~(uint32_t)(key & 0xffffffffu));
      P.tk_vals[row * k + i] = E::load(x + j);
      P.tk_idx[row * k + i] = P.tk_base + j;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// fast path
// ---------------------------------------------------------------------------
template <class E, int W, int U, bool EXPORT = false, bool DEC16 = false>
__global__ __launch_bounds__(64 * W) void filter_fast_kernel(FilterParams P) {
  using raw = typename E::raw;
  constexpr int NT = 64 * W;
  constexpr int VEC = E::kVec;
  __shared__ uint16_t s_gkey[kMaxGroups * NT];  // per-group maxima, okey_hi_up
  __shared__ float s_lmax[NT];
  __shared__ uint64_t s_cand[kCandCap];
  __shared__ uint16_t s_pairs[kCandCap];  // (lane, group) pairs to re-read
  __shared__ int s_count, s_npairs;
  __shared__ float s_tau;

  const int64_t row = blockIdx.x;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const RowSpan<E> sp(x, P.V);
  const vu4* xv = reinterpret_cast<const vu4*>(x + sp.head);
  const int nvec = (int)sp.nvec;
  // vectors of lane tid: tid + j*NT, j < Jmax, in groups of GS consecutive j
  // (at most kMaxGroups groups).  Small groups keep the re-read short: each
  // re-read vector costs a whole memory line.  GS is a power of two below U
  // (whole groups inside one batch of U loads) or a multiple of U.
  const int Jmax = (nvec + NT - 1) / NT;
  int GS = (Jmax + kMaxGroups - 1) / kMaxGroups;
  if (GS < U) {
    int p2 = 1;
    while (p2 < GS) p2 <<= 1;
    GS = p2;
  } else {
    GS = U * ((GS + U - 1) / U);
  }
  const int G = (Jmax + GS - 1) / GS;
  if (tid == 0) {
    s_count = 0;
    s_npairs = 0;
  }
  // the target's logit, loaded now so that its latency overlaps the stream
  int64_t t = -1;
  float yt = NAN;
  if (tid == 0 && P.out != nullptr) {
    t = P.target[b * P.tsb + r * P.tsr];
    if (t >= 0 && t < P.V) yt = scaled<E>(E::load(x + t), P);
  }

  // ---- pass 1: stream the row, per-group maxima of the raw values ----------
  float lmax = -INFINITY, cur = -INFINITY;
  bool saw_nan = false;  // the export ranks NaN above every number; fmaxf drops it
  int curg = 0;
  int j = 0;
  for (; tid + (j + U - 1) * NT < nvec; j += U) {
    vu4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = __builtin_nontemporal_load(xv + tid + (j + u) * NT);
    float mm[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float w[VEC];
      E::unpack(q[u], w);
      mm[u] = w[0];
#pragma unroll
      for (int k = 1; k < VEC; ++k) mm[u] = fmaxf(mm[u], w[k]);
      if constexpr (EXPORT) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) saw_nan |= (w[k] != w[k]);
      }
    }
    if (GS >= U) {
      const int g = j / GS;
      if (g != curg) {
        s_gkey[curg * NT + tid] = okey_hi_up(cur);
        lmax = fmaxf(lmax, cur);
        curg = g;
        cur = -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) cur = fmaxf(cur, mm[u]);
    } else {
      // U / GS whole groups: reduce pairwise, mm[u] holds group u / GS at u % GS == 0
#pragma unroll
      for (int h = 1; h < U; h <<= 1)
        if (h < GS) {
#pragma unroll
          for (int u = 0; u + h < U; u += 2 * h) mm[u] = fmaxf(mm[u], mm[u + h]);
        }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u % GS == 0) {
          s_gkey[((j + u) / GS) * NT + tid] = okey_hi_up(mm[u]);
          lmax = fmaxf(lmax, mm[u]);
        }
    }
  }
  if (GS < U) curg = j / GS;  // every group so far is complete and stored
  for (; tid + j * NT < nvec; ++j) {
    const int g = j / GS;
    if (g != curg) {
      s_gkey[curg * NT + tid] = okey_hi_up(cur);
      lmax = fmaxf(lmax, cur);
      curg = g;
      cur = -INFINITY;
    }
    float w[VEC];
    E::unpack(xv[tid + j * NT], w);
#pragma unroll
    for (int k = 0; k < VEC; ++k) cur = fmaxf(cur, w[k]);
    if constexpr (EXPORT) {
#pragma unroll
      for (int k = 0; k < VEC; ++k) saw_nan |= (w[k] != w[k]);
    }
  }
  if (curg < G) {
    s_gkey[curg * NT + tid] = okey_hi_up(cur);
    lmax = fmaxf(lmax, cur);
  }
  for (int g = curg + 1; g < G; ++g) s_gkey[g * NT + tid] = okey_hi_up(-INFINITY);
  const float hv = (tid < sp.head) ? E::load(x + tid) : -INFINITY;
  const float tv = (sp.tail0 + tid < P.V) ? E::load(x + sp.tail0 + tid) : -INFINITY;
  lmax = fmaxf(lmax, fmaxf(hv, tv));
  s_lmax[tid] = lmax;
  if constexpr (EXPORT) {
    saw_nan |= (hv != hv) || (tv != tv);
    if (__syncthreads_or(saw_nan)) {
      // a NaN is the largest element: the exact general path handles the row
      if (tid == 0) P.info[row].flags = 1;
      return;
    }
  }
  __syncthreads();

  // ---- lower bound tau: the k-th largest lane maximum ------------------------
  if (tid < 64) {
    const uint32_t kk = wave_kth_largest<NT, sizeof(raw) == 2 ? 16 : 0>(s_lmax, P.top_k);
    if (tid == 0) s_tau = scaled<E>(from_okey(kk), P);
  }
  __syncthreads();
  const float tau = s_tau;

  // ---- pass 2: re-read groups that can hold candidates ------------------------
  // (value key, index) for the filter; (value key, ~index) for the export, so
  // that among equal values the lower index sorts higher
  auto push = [&](float y, int64_t idx) {
    const int slot = atomicAdd(&s_count, 1);
    const uint32_t lo = EXPORT ? ~(uint32_t)idx : (uint32_t)idx;
    if (slot < kCandCap) s_cand[slot] = ((uint64_t)okey(y) << 32) | (uint64_t)lo;
  };
  // flagged groups are listed first, then their vectors are spread over the
  // whole workgroup so that the re-reads are independent loads
  for (int g = 0; g < G; ++g) {
    if (scaled<E>(from_okey((uint32_t)s_gkey[g * NT + tid] << 16), P) >= tau) {
      const int slot = atomicAdd(&s_npairs, 1);
      if (slot < kCandCap) s_pairs[slot] = (uint16_t)(tid * kMaxGroups + g);
    }
  }
  __syncthreads();
  const int npairs = s_npairs;
  if (npairs > kCandCap) {
    // more flagged groups than candidate slots: every flagged group holds at
    // least one element >= tau, so the candidates overflow as well
    if (tid == 0) s_count = kCandCap + 1;
  } else {
    constexpr int UR = 4;
    const int nload = npairs * GS;
    for (int i0 = 0; i0 < nload; i0 += NT * UR) {
      vu4 q[UR];
      int vi[UR];
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        const int i = i0 + u * NT + tid;
        vi[u] = -1;
        if (i < nload) {
          const int pr = s_pairs[i / GS];
          const int v = pr / kMaxGroups + ((pr % kMaxGroups) * GS + i % GS) * NT;
          if (v < nvec) vi[u] = v;
        }
        if (vi[u] >= 0) q[u] = xv[vi[u]];
      }
#pragma unroll
      for (int u = 0; u < UR; ++u) {
        if (vi[u] < 0) continue;
        float w[VEC];
        E::unpack(q[u], w);
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          const float y = scaled<E>(w[k], P);
          if (y >= tau) push(y, sp.head + (int64_t)vi[u] * VEC + k);
        }
      }
    }
  }
  if (tid < sp.head) {
    const float y = scaled<E>(hv, P);
    if (y >= tau) push(y, tid);
  }
  if (sp.tail0 + tid < P.V) {
    const float y = scaled<E>(tv, P);
    if (y >= tau) push(y, sp.tail0 + tid);
  }
  __syncthreads();
  const int C = s_count;
  if (C > kCandCap || C < P.top_k) {
    if (tid == 0) {
      RowInfo ri{};
      ri.flags = 1;
      P.info[row] = ri;
    }
    return;
  }

  // ---- sort the candidates; the k-th largest is the exact top-k value ----------
  block_rank_sort<NT>(s_cand, C);
  if constexpr (EXPORT) {
    export_topk<E>(P, row, x, s_cand + (C - P.top_k));
    return;
  }
  const uint32_t thr_key = (uint32_t)(s_cand[C - P.top_k] >> 32);
  // kept-k = the sorted suffix with key >= thr_key
  int cnt = 0;
  for (int i = tid; i < C; i += NT) cnt += ((uint32_t)(s_cand[i] >> 32) >= thr_key) ? 1 : 0;
  __shared__ int redi[NT / 64];
  const int n_k = block_sum_i<NT>(cnt, redi);
  if (tid < 64) finish_row<E, DEC16>(P, row, s_cand + (C - n_k), n_k, from_okey(thr_key), yt, t);
}

// ---------------------------------------------------------------------------
// general path: exact multi-pass radix selection over the row
// ---------------------------------------------------------------------------
template <class E>
__global__ __launch_bounds__(kGeneralThreads) void filter_general_kernel(FilterParams P,
                                                                         int all_rows) {
  using raw = typename E::raw;
  constexpr int NT = kGeneralThreads;
  __shared__ int hist_i[256];
  __shared__ double hist_d[256];
  __shared__ float redf[NT / 64];
  __shared__ int redi[NT / 64];
  __shared__ uint32_t s_sel[2];
  __shared__ double s_below;
  __shared__ int s_cnt;
  __shared__ int s_grp;  // elements under the last selected digit
  __shared__ uint64_t s_cand[kKeepCap];

  const int64_t row = blockIdx.x;
  if (!all_rows && (P.info[row].flags & 1) == 0) return;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;
  auto yat = [&](int64_t j) { return scaled<E>(E::load(x + j), P); };

  // row maximum
  float mx = -INFINITY;
  for (int64_t j = tid; j < V; j += NT) mx = fmaxf(mx, yat(j));
  const float m = block_max_f<NT>(mx, redf);

  // top-k value: radix select on the 32-bit order key, 8 bits per pass
  uint32_t thr_key = 0;
  if (P.top_k > 0) {
    int remaining = 0;
    thr_key = radix_kth_key<NT>(yat, V, P.top_k, hist_i, s_sel, &remaining, false);
  }

  // top-p cut: the smallest (key, index) whose cumulative probability > cut
  float v_cut = from_okey(thr_key);
  int32_t i_cut = 0;
  if (P.has_p) {
    // the normaliser summed in double and rounded once; p = fl32(e * fl32(1 / Z))
    double zp = 0.0;
    for (int64_t j = tid; j < V; j += NT) {
      const float y = yat(j);
      if (okey(y) >= thr_key) zp += (double)expf(y - m);
    }
    const float Z = (float)block_sum_d<NT>(zp, hist_d);
    const float inv = 1.0f / Z;
    if (tid == 0) s_below = 0.0;
    uint32_t prefix = 0, mask = 0;
    bool done = false;
    // value digits, then index digits among the elements tied at the value
    for (int phase = 0; phase < 2 && !done; ++phase) {
      int top_bit = 31;
      if (phase == 1) {
        top_bit = 0;
        while ((int64_t(1) << (top_bit + 1)) < V) ++top_bit;
      }
      uint32_t iprefix = 0, imask = 0;
      for (int hi = top_bit; hi >= 0; hi -= 8) {
        const int lo = hi >= 7 ? hi - 7 : 0;
        const int shift = lo;
        const int nb = hi - lo + 1;
        const uint32_t dmask = (nb >= 32) ? 0xffffffffu : ((1u << nb) - 1u);
        for (int i = tid; i < 256; i += NT) {
          hist_d[i] = 0.0;
          hist_i[i] = 0;
        }
        __syncthreads();
        for (int64_t j = tid; j < V; j += NT) {
          const float y = yat(j);
          const uint32_t k = okey(y);
          if (k < thr_key) continue;
          uint32_t digit;
          if (phase == 0) {
            if ((k & mask) != prefix) continue;
            digit = (k >> shift) & dmask;
          } else {
            if (k != prefix) continue;
            const uint32_t jj = (uint32_t)j;
            if ((jj & imask) != iprefix) continue;
            digit = (jj >> shift) & dmask;
          }
          atomicAdd(&hist_d[digit], (double)(expf(y - m) * inv));
          atomicAdd(&hist_i[digit], 1);
        }
        __syncthreads();
        if (tid == 0) {
          double below = s_below;
          int bsel = -1, last_nonempty = -1;
          for (int bin = 0; bin <= (int)dmask; ++bin) {
            if (hist_d[bin] == 0.0) continue;
            last_nonempty = bin;
            if ((float)(below + hist_d[bin]) > P.cut) {
              bsel = bin;
              break;
            }
            below += hist_d[bin];
          }
          if (bsel < 0) {
            // no cumulative value exceeds the cut: only the maximum is kept
            bsel = last_nonempty;
            below -= hist_d[bsel];
          }
          s_below = below;
          s_sel[0] = (uint32_t)bsel;
          s_grp = hist_i[bsel];
        }
        __syncthreads();
        if (phase == 0) {
          prefix |= s_sel[0] << shift;
          mask |= dmask << shift;
        } else {
          iprefix |= s_sel[0] << shift;
          imask |= dmask << shift;
        }
        __syncthreads();
      }
      if (phase == 1) i_cut = (int32_t)iprefix;
      // a value held by one element needs no index digits (i_cut 0 keeps it)
      if (phase == 0 && s_grp == 1) done = true;
    }
    v_cut = from_okey(prefix);
  }

  // kept-set log-sum-exp, count and (small) kept list
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  float sp = 0.f;
  int cnt = 0;
  for (int64_t j = tid; j < V; j += NT) {
    const float y = yat(j);
    if (!kept_lex(y, j, v_cut, i_cut)) continue;
    sp += expf(y - m);
    ++cnt;
    const int slot = atomicAdd(&s_cnt, 1);
    if (slot < kKeepCap) s_cand[slot] = ((uint64_t)okey(y) << 32) | (uint64_t)(uint32_t)j;
  }
  const float s = block_sum_f<NT>(sp, redf);
  const int n_kept = block_sum_i<NT>(cnt, redi);
  const float logsum = logf(s);
  if (n_kept <= kKeepCap) {
    int32_t* ki = P.kept_idx + row * kKeepCap;
    float* kp = P.kept_p + row * kKeepCap;
    for (int i = tid; i < n_kept; i += NT) {
      const float y = from_okey((uint32_t)(s_cand[i] >> 32));
      ki[i] = (int32_t)(s_cand[i] & 0xffffffffu);
      kp[i] = expf((y - m) - logsum);
    }
  }
  if (tid == 0) {
    RowInfo ri;
    ri.m = m;
    ri.logsum = logsum;
    ri.v_cut = v_cut;
    ri.i_cut = i_cut;
    ri.n_kept = n_kept;
    ri.flags = 0;
    P.info[row] = ri;
    if (P.out != nullptr) {
      const int64_t t = P.target[b * P.tsb + r * P.tsr];
      float lp = -INFINITY;
      if (t >= 0 && t < V) {
        const float yt = yat(t);
        if (kept_lex(yt, t, v_cut, i_cut)) lp = (yt - m) - logsum;
      }
      P.out[row] = lp;
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
struct FilterBwdParams {
  const void* logits;
  int64_t R, Rt, V, sb, sr;
  const int64_t* target;
  int64_t tsb, tsr;
  float rT;   // temperature_recip of the fused temperature
  int has_t;
  float rGT;  // temperature_recip of an earlier in-place division, applied to the gradient last
  int has_gt;
  int zero_rows;  // phase 2 zeroes the rows it does not rewrite (no phase 1)
  const RowInfo* info;
  const int32_t* kept_idx;
  const float* kept_p;
  const float* g;
  int64_t gsb, gsr;
  void* gin;
  int64_t gisb, gisr;
};

template <class E>
__device__ __forceinline__ typename E::raw grad_to_dtype(float g32, const FilterBwdParams& P) {
  if (!P.has_t && !P.has_gt) return E::from_float(g32);
  // dtype(g), then the backward of the fused temperature (fl32 product with
  // rT, rounded to the dtype), then that of an in-place division applied to
  // the logits before this call (the same with rGT): autograd's chain of the
  // fp32 upcast and the two divisions as torch runs them on the GPU
  float r = round_trip<E>(g32);
  if (P.has_t) r = round_trip<E>(mul_rn(r, P.rT));
  if (P.has_gt) r = round_trip<E>(mul_rn(r, P.rGT));
  return E::from_float(r);
}

// Phase 1 over a contiguous gradient: zeros over the whole [rows, V] block,
// one 4 KB piece per workgroup with piece boundaries on 4 KB addresses.  Many
// short workgroups dispatched in order keep the stores inside a narrow
// address window, which is what lets a pure write stream reach the HBM write
// rate; row-shaped workgroups over rows that are not 4 KB multiples fall
// short of it.
template <class E>
__global__ __launch_bounds__(256) void filter_bwd_zero_flat_kernel(void* gin, int64_t n, int shift) {
  using raw = typename E::raw;
  raw* y = static_cast<raw*>(gin);
  const RowSpan<E> ys(y, n);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x - shift;
  if (i >= 0 && i < ys.nvec) __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + i);
  if (blockIdx.x == 0) {
    const raw zr = E::from_float(0.f);
    if (threadIdx.x < ys.head) y[threadIdx.x] = zr;
    if (ys.tail0 + threadIdx.x < n) y[ys.tail0 + threadIdx.x] = zr;
  }
}

// Phase 1 over strided rows: zeros row by row.
template <class E, int W>
__global__ __launch_bounds__(64 * W) void filter_bwd_zero_rows_kernel(FilterBwdParams P) {
  using raw = typename E::raw;
  constexpr int NT = 64 * W;
  const int64_t row = blockIdx.x;
  const int64_t b = row / P.Rt, r = row - b * P.Rt;
  raw* y = static_cast<raw*>(P.gin) + b * P.gisb + r * P.gisr;
  const RowSpan<E> ys(y, P.V);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  for (int64_t i = threadIdx.x; i < ys.nvec; i += NT)
    __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + i);
  const raw zr = E::from_float(0.f);
  if (threadIdx.x < ys.head) y[threadIdx.x] = zr;
  if (ys.tail0 + threadIdx.x < P.V) y[ys.tail0 + threadIdx.x] = zr;
}

// How the whole-row walk narrows an fp32 gradient to the dtype.
enum GradConv {
  kConvPlain = 0,  // no temperature: round to the dtype
  kConvGT = 1,     // an earlier in-place temperature only: round, product with rGT, round
  kConvT = 2,      // the fused temperature only: values scaled; round, product with rT, round
  kConvTwo = 3,    // both: values scaled; grad_to_dtype
};
template <int CONV>
constexpr bool conv_scales_values() {
  return CONV == kConvT || CONV == kConvTwo;
}
template <int CONV>
constexpr bool conv_one_product() {
  return CONV == kConvGT || CONV == kConvT;
}
// The GradConv for a launch's temperatures.
__host__ __device__ inline int grad_conv(bool has_t, bool has_gt) {
  return has_t ? (has_gt ? kConvTwo : kConvT) : (has_gt ? kConvGT : kConvPlain);
}

// Per-row arithmetic of the whole-row walks below: the kept test of elements
// equal to v_cut, the probability of a kept element and the gradient narrowed
// to the dtype.
// The least float above v (for non-NaN y: y > v <=> y >= next_float_up(v)):
// -0.0 taken as +0.0, NaN above +inf and NaN (nothing compares >= it).
__device__ __forceinline__ float next_float_up(float v) {
  v = v + 0.0f;
  const uint32_t u = __float_as_uint(v);
  if (v != v || u == 0x7f800000u) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((int32_t)u >= 0 ? u + 1u : u - 1u);
}

template <class E, int CONV>
struct WalkMath {
  using raw = typename E::raw;
  const FilterBwdParams& P;
  const RowInfo& ri;
  float gv, ngv, c, rone, vc;
  int64_t t;
  bool rank_form;
  uint32_t rcut;
  int32_t icut;
  __device__ WalkMath(const FilterBwdParams& P_, const RowInfo& ri_, float gv_, int64_t t_)
      : P(P_), ri(ri_), gv(gv_), t(t_) {
    vc = ri.v_cut;
    rank_form = ri.i_cut < 0;
    rcut = rank_form ? (uint32_t)(-1 - ri.i_cut) : 0u;
    icut = ri.i_cut;
    // p = exp(y - m - logsum); for the 16-bit dtypes as exp2(y log2e - c) in
    // one fma (its absolute error in the exponent, a few 1e-6, is far below the
    // dtype's resolution), for fp32 gradients from the differences
    c = (ri.m + ri.logsum) * kLog2e;
    ngv = -gv;
    rone = CONV == kConvT ? P.rT : P.rGT;
  }
  __device__ float yval(float xf) const {
    if constexpr (conv_scales_values<CONV>())
      return round_trip<E>(mul_rn(xf, P.rT));
    else
      return xf;
  }
  __device__ float prob(float yy) const {
    if constexpr (std::is_same<E, F32>::value)
      return fast_exp2(((yy - ri.m) - ri.logsum) * kLog2e);
    else
      return fast_exp2(__builtin_fmaf(yy, kLog2e, -c));
  }
  // gradient of a non-target element, narrowed to the dtype
  __device__ raw narrow(float g32) const {
    if constexpr (CONV == kConvPlain) {
      return E::from_float(g32);
    } else if constexpr (conv_one_product<CONV>()) {
      return E::from_float(mul_rn(round_trip<E>(g32), rone));
    } else {
      return grad_to_dtype<E>(g32, P);
    }
  }
  // the non-target gradients -p g of one vector (0 outside the kept set)
  template <class Kept>
  __device__ void narrow_vec(const float (&w)[E::kVec], raw (&vals)[E::kVec], Kept kept) const {
    float g[E::kVec];
#pragma unroll
    for (int k = 0; k < E::kVec; ++k) g[k] = kept(k) ? prob(w[k]) * ngv : 0.f;
    if constexpr (conv_one_product<CONV>()) {
      // round to the dtype two at a time, multiply, round again
#pragma unroll
      for (int k = 0; k < E::kVec; k += 2) {
        float a = g[k], b = g[k + 1];
        round_trip2<E>(a, b);
        a = mul_rn(a, rone);
        b = mul_rn(b, rone);
        vals[k] = E::from_float(a);
        vals[k + 1] = E::from_float(b);
      }
    } else {
#pragma unroll
      for (int k = 0; k < E::kVec; ++k) vals[k] = narrow(g[k]);
    }
  }
  // a vector of fp32 gradients narrowed to the dtype as narrow() does, packed
  __device__ vu4 pack_vec(float (&g)[E::kVec]) const {
    if constexpr (CONV == kConvPlain) {
      return E::pack(g);
    } else if constexpr (conv_one_product<CONV>()) {
#pragma unroll
      for (int k = 0; k < E::kVec; k += 2) {
        round_trip2<E>(g[k], g[k + 1]);
        g[k] = mul_rn(g[k], rone);
        g[k + 1] = mul_rn(g[k + 1], rone);
      }
      return E::pack(g);
    } else {
      raw vals[E::kVec];
#pragma unroll
      for (int k = 0; k < E::kVec; ++k) vals[k] = grad_to_dtype<E>(g[k], P);
      vu4 out;
      __builtin_memcpy(&out, vals, sizeof(out));
      return out;
    }
  }
  __device__ raw grad_at(float yy, int64_t j, bool kept) const {
    float g32 = 0.f;
    if (kept) {
      const float p = prob(yy);
      g32 = ((j == t) ? 1.f - p : -p) * gv;
    }
    return grad_to_dtype<E>(g32, P);
  }
  __device__ bool tied_kept(uint32_t rank, int64_t j) const { return rank_form ? rank >= rcut : j >= icut; }
};

// The whole-row walk of the filtered backward: re-read the logits x of one
// row and write the gradient y of the whole row, in index order (the head, the
// 16-byte vectors, the tail).  The elements equal to v_cut are counted as they
// come (the same count in every lane), so that a cut in rank form is applied
// too; their ranks are only worked out for vectors where a tie occurs.
// Elements outside the kept set get the gradient 0.  One wave per row.
template <class E, int CONV>
__device__ __forceinline__ void walk_row(const FilterBwdParams& P, const RowInfo& ri,
                                         const typename E::raw* x, typename E::raw* y, float gv,
                                         int64_t t, int lane) {
  using raw = typename E::raw;
  constexpr int VEC = E::kVec;
  constexpr int U = 4;
  const WalkMath<E, CONV> W(P, ri, gv, t);
  const float vc = W.vc;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t seen = 0;
  // one element per lane, consecutive indices across the lanes; every lane calls it
  auto lane_step = [&](int64_t j, bool valid) {
    const float yy = valid ? W.yval(E::load(x + j)) : 0.f;
    const bool tie = valid && yy == vc;
    const uint64_t bal = __ballot(tie);
    bool kept = valid && yy > vc;
    if (tie) kept = W.tied_kept(seen + (uint32_t)__popcll(bal & below), j);
    seen += (uint32_t)__popcll(bal);
    if (valid) y[j] = W.grad_at(yy, j, kept);
  };
  const RowSpan<E> xs(x, P.V);
  const RowSpan<E> ys(y, P.V);
  if (xs.head != ys.head) {
    for (int64_t j0r = 0; j0r < P.V; j0r += 64) lane_step(j0r + lane, j0r + lane < P.V);
    return;
  }
  lane_step(lane, lane < ys.head);
  const vu4* xv = reinterpret_cast<const vu4*>(x + xs.head);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  const int64_t nvec = ys.nvec;
  for (int64_t base = 0; base < nvec; base += 64 * U) {
    vu4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * 64 + lane;
      q[u] = i < nvec ? __builtin_nontemporal_load(xv + i) : vu4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * 64 + lane;
      const bool valid = i < nvec;
      const int64_t jb = ys.head + i * VEC;
      float w[VEC];
      E::unpack(q[u], w);
#pragma unroll
      for (int k = 0; k < VEC; ++k) w[k] = W.yval(w[k]);
      bool tie = false;
#pragma unroll
      for (int k = 0; k < VEC; ++k) tie = tie || w[k] == vc;
      tie = tie && valid;
      raw vals[VEC];
      // keep bits of a vector with ties; all ones: no tie in the wave's vectors
      uint32_t keep8 = ~0u;
      if (__ballot(tie) != 0ull) {
        // ranks of the tied elements: the wave's exclusive prefix of the counts
        uint32_t tie8 = 0;
        keep8 = 0;
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          tie8 |= (valid && w[k] == vc ? 1u : 0u) << k;
          keep8 |= (w[k] > vc ? 1u : 0u) << k;
        }
        const uint32_t cnt = (uint32_t)__popc(tie8);
        uint32_t inc = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const uint32_t o = (uint32_t)__shfl_up((int)inc, off, 64);
          if (lane >= off) inc += o;
        }
        const uint32_t ex = inc - cnt;
        const uint32_t total = (uint32_t)__shfl((int)inc, 63, 64);
        for (uint32_t m = tie8; m != 0u; m &= m - 1u) {
          const int k = __ffs(m) - 1;
          if (W.tied_kept(seen + ex + (uint32_t)__popc(tie8 & ((1u << k) - 1u)), jb + k)) keep8 |= 1u << k;
        }
        seen += total;
        W.narrow_vec(w, vals, [&](int k) { return ((keep8 >> k) & 1u) != 0u; });
      } else {
        W.narrow_vec(w, vals, [&](int k) { return w[k] > vc; });
      }
      // the target element (1 - p) g, narrowed exactly
      const int64_t dt = t - jb;
      if (dt >= 0 && dt < VEC) {
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k == dt) vals[k] = W.grad_at(w[k], jb + k, keep8 == ~0u ? w[k] > vc : ((keep8 >> k) & 1u) != 0u);
      }
      if (valid) {
        vu4 out;
        __builtin_memcpy(&out, vals, sizeof(out));
        __builtin_nontemporal_store(out, yv + i);
      }
    }
  }
  lane_step(ys.tail0 + lane, ys.tail0 + lane < P.V);
}

// The whole-row walk by a workgroup of kRowWaves waves per row: each round
// covers kRowThreads * kRowVecs consecutive 16-byte vectors (vector
// base + u * kRowThreads + thread), so far fewer rows are streamed at once
// than with one wave per row and the traffic stays in a narrower address
// window.  A cut in rank form needs each tied element's rank among the row's
// ties in index order: every wave counts its ties per u, the counts meet in
// LDS (one barrier per round, the count array alternating between two halves
// so that a round's writes never meet the previous round's reads), and each
// wave takes the exclusive prefix over the (u, wave) order.  The head and the
// tail are counted by every wave alike (the same running count everywhere)
// and written by wave 0.  Measured on the top-p-alone backward of bf16
// [4, 4096, 151936] rows (9.48 GB): one wave per row 1.99 ms; 16-wave rows,
// two per CU, 1.87 ms; 12-wave rows, two per CU (6 waves per SIMD, so more
// scalar registers per wave), 1.84 ms.  The walk is issue-bound rather than
// HBM-bound: about 25 VALU instructions per element (the probability, its
// rounding, the division of an earlier in-place temperature, the kept test),
// 93% of the VALU issue slots over the kernel (SQ_INSTS_VALU against
// GRBM_GUI_ACTIVE).
// Sum of a 32-bit count over the 64 lanes of a wave (every lane gets the sum).
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, 64);
  return v;
}

constexpr int kRowWaves = 12;
constexpr int kRowThreads = 64 * kRowWaves;
constexpr int kRowVecs = 2;

template <class E, int CONV>
__device__ __forceinline__ void walk_row_block(const FilterBwdParams& P, const RowInfo& ri,
                                               const typename E::raw* x, typename E::raw* y,
                                               float gv, int64_t t, uint32_t* s_cnt) {
  using raw = typename E::raw;
  constexpr int VEC = E::kVec;
  constexpr int U = kRowVecs;
  constexpr int NT = kRowThreads;
  constexpr int NC = U * kRowWaves;  // counts per round
  static_assert(NC <= 64, "one count per lane");
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const WalkMath<E, CONV> W(P, ri, gv, t);
  const float vc = W.vc;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t seen = 0;  // ties before the current position, the same in every wave
  auto lane_step = [&](int64_t j, bool valid, bool write) {
    const float yy = valid ? W.yval(E::load(x + j)) : 0.f;
    const bool tie = valid && yy == vc;
    const uint64_t bal = __ballot(tie);
    bool kept = valid && yy > vc;
    if (tie) kept = W.tied_kept(seen + (uint32_t)__popcll(bal & below), j);
    seen += (uint32_t)__popcll(bal);
    if (valid && write) y[j] = W.grad_at(yy, j, kept);
  };
  auto incl_scan = [&](uint32_t v) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)v, off, 64);
      if (lane >= off) v += o;
    }
    return v;
  };
  const RowSpan<E> xs(x, P.V);
  const RowSpan<E> ys(y, P.V);
  if (xs.head != ys.head) {
    // logits and gradient not co-aligned: one wave walks the row element by element
    if (wave == 0)
      for (int64_t j0r = 0; j0r < P.V; j0r += 64) lane_step(j0r + lane, j0r + lane < P.V, true);
    return;
  }
  lane_step(lane, lane < ys.head, wave == 0);
  const vu4* xv = reinterpret_cast<const vu4*>(x + xs.head);
  vu4* yv = reinterpret_cast<vu4*>(y + ys.head);
  // 32-bit indices in the vector loop (rows hold fewer than 2^31 elements)
  const int nvec = (int)ys.nvec;
  const int head = (int)ys.head;
  const int tt = (t >= 0 && t < P.V) ? (int)t : -1;
  int par = 0;
  float t_y = 0.f;
  bool t_kept = false, t_mine = false;
  // the next round's loads are issued before this round is worked on (two
  // rounds in flight); indices past the row are clamped to its last vector
  // (loaded, never used), so that no load is conditional
  const int last = nvec > 0 ? nvec - 1 : 0;
  vu4 q[U], qn[U];
  if (nvec > 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = u * NT + tid;
      q[u] = __builtin_nontemporal_load(xv + (i < last ? i : last));
    }
  }
  for (int base = 0; base < nvec; base += NT * U) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + NT * U + u * NT + tid;
      qn[u] = __builtin_nontemporal_load(xv + (i < last ? i : last));
    }
    // Ties (elements equal to v_cut) are rare and a row's kept ties are the
    // tail of its ties in index order (rank >= rcut, or index >= i_cut).  So
    // each (wave, u) span of the round is one of: all its ties dropped, all
    // kept, or the one span of the row holding the cut, where each tie's rank
    // (or index) is worked out.  Ranks need the wave counts of the round's
    // earlier spans: they meet in LDS, one barrier per round, and only while
    // the running count has not yet reached rcut (the mode is the same for
    // the whole workgroup).
    // the round's values (after the fused temperature, when there is one)
    float w[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      E::unpack(q[u], w[u]);
#pragma unroll
      for (int k = 0; k < VEC; ++k) w[u][k] = W.yval(w[u][k]);
    }
    // this lane's ties (elements equal to v_cut) in span u, one bit per element
    auto tie_bits = [&](int u) {
      uint32_t m = 0u;
      if (base + u * NT + tid < nvec) {
#pragma unroll
        for (int k = 0; k < VEC; ++k) m |= (w[u][k] == vc ? 1u : 0u) << k;
      }
      return m;
    };
    // per span (wave-uniform): 0 = drop its ties, 1 = keep them, 2 = exact (keepT bits)
    int mode[U];
    uint32_t keepT[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mode[u] = 0;
      keepT[u] = 0u;
    }
    if (W.rank_form) {
      if (seen >= W.rcut) {
#pragma unroll
        for (int u = 0; u < U; ++u) mode[u] = 1;
      } else {
        // the tie counts of the round's (wave, u) spans: a count per lane, summed
        // over the wave (two instructions per element, only while the cut lies ahead)
        uint32_t wcnt[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          uint32_t cl = 0u;
          if (base + u * NT + tid < nvec) {
#pragma unroll
            for (int k = 0; k < VEC; ++k) cl += (w[u][k] == vc) ? 1u : 0u;
          }
          wcnt[u] = wave_sum_u32(cl);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (lane == 0) s_cnt[par * NC + u * kRowWaves + wave] = wcnt[u];
        __syncthreads();
        const uint32_t c = lane < NC ? s_cnt[par * NC + lane] : 0u;
        const uint32_t inc = incl_scan(c);
        const uint32_t total = (uint32_t)__shfl((int)inc, NC - 1, 64);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t start = seen + (uint32_t)__shfl((int)(inc - c), u * kRowWaves + wave, 64);
          if (start >= W.rcut) {
            mode[u] = 1;
          } else if (start + wcnt[u] > W.rcut) {
            // the span holding the cut: this lane's ties ranked after the
            // ties of the wave's earlier lanes
            mode[u] = 2;
            const uint32_t tb = tie_bits(u);
            const uint32_t cnt = (uint32_t)__popc(tb);
            const uint32_t r0 = start + incl_scan(cnt) - cnt;
            for (uint32_t m = tb; m != 0u; m &= m - 1u) {
              const int k = __ffs(m) - 1;
              if (r0 + (uint32_t)__popc(tb & ((1u << k) - 1u)) >= W.rcut) keepT[u] |= 1u << k;
            }
          }
        }
        seen += total;
        par ^= 1;
      }
    } else {
      // index form: a tie is kept from index i_cut on
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int span0 = head + (base + u * NT + wave * 64) * VEC;
        if (span0 >= W.icut) {
          mode[u] = 1;
        } else if (span0 + 64 * VEC > W.icut) {
          mode[u] = 2;
          const int jb = head + (base + u * NT + tid) * VEC;
          for (uint32_t m = tie_bits(u); m != 0u; m &= m - 1u) {
            const int k = __ffs(m) - 1;
            if (jb + k >= W.icut) keepT[u] |= 1u << k;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = base + u * NT + tid;
      const int jb = head + i * VEC;
      raw vals[VEC];
      const uint32_t kt = keepT[u];
      // the mode is the same in every lane of the wave: a scalar branch
      const int md = __builtin_amdgcn_readfirstlane(mode[u]);
      if (md == 2)
        W.narrow_vec(w[u], vals, [&](int k) { return w[u][k] > vc || ((kt >> k) & 1u) != 0u; });
      else if (md == 1)
        W.narrow_vec(w[u], vals, [&](int k) { return w[u][k] >= vc; });
      else
        W.narrow_vec(w[u], vals, [&](int k) { return w[u][k] > vc; });
      // the target element: its value and kept test are kept for the store
      // of (1 - p) g after the walk, by this thread
      const int dt = tt - jb;
      if (dt >= 0 && dt < VEC && i < nvec) {
#pragma unroll
        for (int k = 0; k < VEC; ++k)
          if (k == dt) {
            const bool tk = md == 2 ? ((kt >> k) & 1u) != 0u : md == 1;
            t_y = w[u][k];
            t_kept = w[u][k] > vc || (w[u][k] == vc && tk);
            t_mine = true;
          }
      }
      if (i < nvec) {
        vu4 out;
        __builtin_memcpy(&out, vals, sizeof(out));
        __builtin_nontemporal_store(out, yv + i);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = qn[u];
  }
  // the target's (1 - p) g, narrowed exactly, over the -p g stored above (a
  // later store of the same thread)
  if (t_mine) y[t] = W.grad_at(t_y, t, t_kept);
  lane_step(ys.tail0 + lane, ys.tail0 + lane < P.V, wave == 0);
}

// The backward when no row has a kept list (top-p without top-k, k above the
// kept-list cap): one kRowThreads workgroup per row writes the whole row, as
// zeros (rows past R and rows with a zero upstream gradient) or by the walk.
// (two workgroups per CU: 6 waves per SIMD).  KIND
// is the GradConv of the launch (the temperatures it applies to the gradient),
// so that each kernel holds the walk it uses and no more.
template <class E, int KIND>
__global__ __launch_bounds__(kRowThreads, 6) void filter_bwd_row_kernel(FilterBwdParams P) {
  using raw = typename E::raw;
  __shared__ uint32_t s_cnt[2 * kRowVecs * kRowWaves];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const int64_t b = row / P.Rt, r = row - b * P.Rt;
  raw* y = static_cast<raw*>(P.gin) + b * P.gisb + r * P.gisr;
  float gv = 0.f;
  int64_t srow = 0;
  if (r < P.R) {
    srow = b * P.R + r;
    gv = P.g[b * P.gsb + r * P.gsr];
  }
  if (gv == 0.f) {
    const RowSpan<E> zs(y, P.V);
    vu4* zv = reinterpret_cast<vu4*>(y + zs.head);
    for (int64_t i = tid; i < zs.nvec; i += kRowThreads) __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, zv + i);
    const raw zr = E::from_float(0.f);
    if (tid < zs.head) y[tid] = zr;
    if (zs.tail0 + tid < P.V) y[zs.tail0 + tid] = zr;
    return;
  }
  const RowInfo ri = P.info[srow];
  const int64_t t = P.target[b * P.tsb + r * P.tsr];
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  walk_row_block<E, KIND>(P, ri, x, y, gv, t, s_cnt);
}

// The backward of rows without kept lists on 8 KB pieces: a workgroup of 256
// threads writes one piece of one row, two 16-byte vectors per thread (the
// first piece of a row also the elements before the row's first 16-byte
// boundary, the last one those after its last), pieces numbered in address
// order within the row and rows one after another.  Consecutive workgroups
// then cover consecutive addresses, so the chip's reads and writes stay in a
// narrow address window: a plain copy of [16380, 151936] bf16 rows moves at
// 6.4 TB/s on such pieces and at 5.2 TB/s with a workgroup streaming each
// row (the DRAM pages of hundreds of rows open at once).  The row's upstream
// gradient, cut and target are the workgroup's (scalar loads, issued
// together).  Measured on the top-k 2000 backward of bf16 [4, 4096, 151936]
// rows (9.48 GB): 1.49 ms on 8 KB pieces, 1.83 ms on 4 KB pieces (a piece's
// dependent loads amortized over half the bytes), 1.65 ms on 16 KB pieces;
// 2.10 ms for the row walk.
//
// A cut in index form (j kept among the elements equal to v_cut from i_cut
// on) is applied per element.  In rank form (kept among those ties from rank
// rcut on, in index order) a piece cannot know its ties' ranks: it writes
// every tie as kept, stores its tie count, and lists its ties' offsets in
// index order (up to kPieceTieCap; a workgroup scan ranks them); a per-row
// fix-up then ranks the pieces by their counts and writes zeros over the ties
// of rank < rcut, reading a piece again only where its list overflowed.
constexpr int kPcThreads = 256;
constexpr int kPcVecs = 2;                          // 16-byte vectors per thread
constexpr int kPcVectors = kPcThreads * kPcVecs;    // per piece
constexpr int kPieceTieCap = MIRL_FILTER_PIECE_TIE_CAP;
static_assert(kPieceTieCap % 2 == 0, "a piece's list is read as 32-bit words");

struct PieceGeom {
  int ppr;            // pieces per row
  int nvec;           // 16-byte vectors per row (the same in every row)
  int head;           // elements before the first vector
  uint32_t* tie_cnt;  // [B * R * ppr]: the piece's tie count (rank-form rows with rcut > 0)
  uint16_t* tie_pos;  // [B * R * ppr][kPieceTieCap]: tie offsets from the piece's first element
};

// first element of piece pc (piece 0 starts at the row's element 0)
__device__ __forceinline__ int piece_j0(const PieceGeom& Gm, int pc, int vec) {
  return pc == 0 ? 0 : Gm.head + pc * kPcVectors * vec;
}

template <class E, int CONV>
__global__ __launch_bounds__(kPcThreads) void filter_bwd_piece_kernel(FilterBwdParams P, PieceGeom Gm) {
  using raw = typename E::raw;
  constexpr int VEC = E::kVec, NT = kPcThreads, U = kPcVecs, NW = NT / 64;
  __shared__ uint32_t s_cnt[U * NW + 2];  // body ties per (u, wave), then the head's and the tail's
  // 32-bit index arithmetic: rows < 2^31, V < 2^31
  const uint32_t blk = blockIdx.x;
  const uint32_t row = blk / (uint32_t)Gm.ppr;
  const int pc = (int)(blk - row * (uint32_t)Gm.ppr);
  const uint32_t b = row / (uint32_t)P.Rt, r = row - b * (uint32_t)P.Rt;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // the row's upstream gradient, cut and target, loaded together
  const bool live = r < (uint32_t)P.R;
  const uint32_t srow = b * (uint32_t)P.R + r;
  float gv = 0.f;
  RowInfo ri{};
  int64_t t = -1;
  if (live) {
    gv = P.g[(int64_t)b * P.gsb + (int64_t)r * P.gsr];
    ri = P.info[srow];
    t = P.target[(int64_t)b * P.tsb + (int64_t)r * P.tsr];
  }
  raw* y = static_cast<raw*>(P.gin) + (int64_t)b * P.gisb + (int64_t)r * P.gisr;
  vu4* yv = reinterpret_cast<vu4*>(y + Gm.head);
  const int i0 = pc * kPcVectors + tid;  // this thread's first vector
  const int tail0 = Gm.head + Gm.nvec * VEC;
  const bool hv = pc == 0 && tid < Gm.head;                         // a head element
  const bool tv = pc == Gm.ppr - 1 && tail0 + tid < (int)P.V;       // a tail element
  const raw zr = E::from_float(0.f);
  if (gv == 0.f) {
    // rows past R and rows with a zero upstream gradient: zeros, the logits unread
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i0 + u * NT < Gm.nvec) __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, yv + i0 + u * NT);
    if (hv) y[tid] = zr;
    if (tv) y[tail0 + tid] = zr;
    return;
  }
  const raw* x = static_cast<const raw*>(P.logits) + (int64_t)b * P.sb + (int64_t)r * P.sr;
  const vu4* xv = reinterpret_cast<const vu4*>(x + Gm.head);
  vu4 q[U];
#pragma unroll
  for (int u = 0; u < U; ++u)
    q[u] = i0 + u * NT < Gm.nvec ? __builtin_nontemporal_load(xv + i0 + u * NT) : vu4{0u, 0u, 0u, 0u};
  const float xh = hv ? E::load(x + tid) : 0.f;
  const float xt = tv ? E::load(x + tail0 + tid) : 0.f;
  const WalkMath<E, CONV> W(P, ri, gv, t);
  const float vc = W.vc;
  const float yh = W.yval(xh), ytl = W.yval(xt);
  float w[U][VEC];
  bool anyt[U];  // the vector holds an element equal to v_cut
#pragma unroll
  for (int u = 0; u < U; ++u) {
    E::unpack(q[u], w[u]);
    bool a = false;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      w[u][k] = W.yval(w[u][k]);
      a = a || w[u][k] == vc;
    }
    anyt[u] = a && i0 + u * NT < Gm.nvec;
  }
  auto tie_bits = [&](int u) {
    uint32_t m = 0u;
#pragma unroll
    for (int k = 0; k < VEC; ++k) m |= (w[u][k] == vc ? 1u : 0u) << k;
    return anyt[u] ? m : 0u;
  };
  const bool th = hv && yh == vc, tt = tv && ytl == vc;
  // per vector: kept <=> y >= thr (v_cut: its ties kept; the next float up:
  // dropped), then the ties in `drop` zeroed, which only the vector holding an
  // index-form cut has.  Rank form: every tie kept here (settled by the
  // fix-up where rcut > 0).
  const float vnext = next_float_up(vc);
  float thr[U];
  uint32_t drop[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    thr[u] = vc;
    drop[u] = 0u;
  }
  bool keepH = th, keepTl = tt;
  if (!W.rank_form) {
    const int icut = W.icut;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int jb = Gm.head + (i0 + u * NT) * VEC;
      if (jb + VEC <= icut) thr[u] = vnext;
      const bool cutvec = jb < icut && jb + VEC > icut && anyt[u];
      if (__ballot(cutvec) != 0ull && cutvec) drop[u] = tie_bits(u) & ((1u << (icut - jb)) - 1u);
    }
    keepH = th && tid >= icut;
    keepTl = tt && tail0 + tid >= icut;
  } else if (W.rcut > 0u) {
    // the piece's ties in index order: the head's, the body's by (u, thread), the tail's
    uint32_t tb[U], cnt[U], inc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      tb[u] = 0u;
      inc[u] = 0u;
      if (__ballot(anyt[u]) != 0ull) {
        tb[u] = tie_bits(u);
        inc[u] = wave_scan_dpp((uint32_t)__popc(tb[u]));
      }
      cnt[u] = (uint32_t)__popc(tb[u]);
      if (lane == 63) s_cnt[u * NW + wave] = inc[u];
    }
    const uint64_t bh = __ballot(th), bt = __ballot(tt);
    if (tid == 0) {
      s_cnt[U * NW] = (uint32_t)__popcll(bh);
      s_cnt[U * NW + 1] = (uint32_t)__popcll(bt);
    }
    __syncthreads();
    const uint32_t nh = s_cnt[U * NW];
    uint32_t before[U];  // ties of the piece before this thread's span u
    uint32_t base = nh;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t span = 0u;
      before[u] = base;
#pragma unroll
      for (int v = 0; v < NW; ++v) {
        before[u] += v < wave ? s_cnt[u * NW + v] : 0u;
        span += s_cnt[u * NW + v];
      }
      before[u] += inc[u] - cnt[u];
      base += span;
    }
    // the count and the list (offsets in index order, up to kPieceTieCap)
    const uint64_t below = (1ull << lane) - 1ull;
    const int j0 = piece_j0(Gm, pc, VEC);
    const int64_t slot = (int64_t)srow * Gm.ppr + pc;
    uint16_t* lst = Gm.tie_pos + slot * kPieceTieCap;
    if (th) {
      const uint32_t a = (uint32_t)__popcll(bh & below);
      if (a < (uint32_t)kPieceTieCap) lst[a] = (uint16_t)(tid - j0);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int jb = Gm.head + (i0 + u * NT) * VEC;
      uint32_t a = before[u];
      for (uint32_t m = tb[u]; m != 0u; m &= m - 1u, ++a) {
        const int k = __ffs(m) - 1;
        if (a < (uint32_t)kPieceTieCap) lst[a] = (uint16_t)(jb + k - j0);
      }
    }
    if (tt) {
      const uint32_t at = base + (uint32_t)__popcll(bt & below);
      if (at < (uint32_t)kPieceTieCap) lst[at] = (uint16_t)(tail0 + tid - j0);
    }
    if (tid == 0) Gm.tie_cnt[slot] = base + s_cnt[U * NW + 1];
  }
  const float ngv = -gv;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = i0 + u * NT;
    const int jb = Gm.head + i * VEC;
    float o[VEC];
#pragma unroll
    for (int k = 0; k < VEC; ++k) o[k] = w[u][k] >= thr[u] ? W.prob(w[u][k]) * ngv : 0.f;
    if (__ballot(drop[u] != 0u) != 0ull) {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if ((drop[u] >> k) & 1u) o[k] = 0.f;
    }
    // the target element: (1 - p) g where kept
    const int64_t dt = t - jb;
    if (dt >= 0 && dt < VEC) {
#pragma unroll
      for (int k = 0; k < VEC; ++k)
        if (k == dt) {
          const bool kept = w[u][k] >= thr[u] && ((drop[u] >> k) & 1u) == 0u;
          o[k] = kept ? (1.f - W.prob(w[u][k])) * gv : 0.f;
        }
    }
    const vu4 out = W.pack_vec(o);
    if (i < Gm.nvec) __builtin_nontemporal_store(out, yv + i);
  }
  if (hv) y[tid] = W.grad_at(yh, tid, yh > vc || keepH);
  if (tv) y[tail0 + tid] = W.grad_at(ytl, tail0 + tid, ytl > vc || keepTl);
}

// Per row with a rank-form cut and rcut > 0 (one wave each): the pieces'
// tie counts scanned in order, and the listed ties of rank < rcut written as
// zeros (a piece whose list overflowed is read again, its ties ranked by
// ballot).  Measured on the top-p backward of bf16 [4, 4096, 151936] rows
// (about 75 zeros per row): 0.17 ms, the cost of that many scattered 2-byte
// writes into lines already written back.  A decoupled look-back in the piece
// kernel (each piece adding up the counts its row's earlier pieces publish,
// so that every tie is written once) measured 2.9 ms for the piece kernel
// alone: pieces waiting on pieces of other XCDs hold their slots.
template <class E, int CONV>
__global__ __launch_bounds__(256) void filter_bwd_piece_fixup_kernel(FilterBwdParams P, PieceGeom Gm,
                                                                     int64_t nrows) {
  using raw = typename E::raw;
  constexpr int VEC = E::kVec;
  const int lane = threadIdx.x & 63;
  const int64_t srow = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (srow >= nrows) return;
  const int64_t b = srow / P.R, r = srow - b * P.R;
  const float gv = P.g[b * P.gsb + r * P.gsr];
  if (gv == 0.f) return;
  const RowInfo ri = P.info[srow];
  if (ri.i_cut >= -1) return;  // index form, or every tie kept
  const uint32_t rcut = (uint32_t)(-1 - ri.i_cut);
  raw* y = static_cast<raw*>(P.gin) + b * P.gisb + r * P.gisr;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const raw zr = E::from_float(0.f);
  const WalkMath<E, CONV> W(P, ri, gv, -1);
  const uint32_t* cnt = Gm.tie_cnt + srow * Gm.ppr;
  const uint16_t* pos = Gm.tie_pos + srow * Gm.ppr * kPieceTieCap;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t seen = 0u;
  for (int c0 = 0; c0 < Gm.ppr && seen < rcut; c0 += 64) {
    const int pc = c0 + lane;
    const uint32_t n = pc < Gm.ppr ? cnt[pc] : 0u;
    const uint32_t inc = wave_scan_dpp(n);
    const uint32_t start = seen + inc - n;
    const bool need = n > 0u && start < rcut;
    if (need && n <= (uint32_t)kPieceTieCap) {
      // the piece's list read whole (independent loads), then the zeros stored
      const int j0 = piece_j0(Gm, pc, VEC);
      const uint32_t m = min(n, rcut - start);
      const uint32_t* pw = reinterpret_cast<const uint32_t*>(pos + pc * kPieceTieCap);
      uint32_t wv[kPieceTieCap / 2];
#pragma unroll
      for (int a = 0; a < kPieceTieCap / 2; ++a) wv[a] = 2u * a < m ? pw[a] : 0u;
#pragma unroll
      for (int a = 0; a < kPieceTieCap; ++a)
        if ((uint32_t)a < m) y[j0 + ((wv[a >> 1] >> (16 * (a & 1))) & 0xffffu)] = zr;
    }
    for (uint64_t ov = __ballot(need && n > (uint32_t)kPieceTieCap); ov != 0ull; ov &= ov - 1ull) {
      const int l = __ffsll((unsigned long long)ov) - 1;
      const int pv = c0 + l;
      uint32_t rk = (uint32_t)__shfl((int)start, l, 64);
      const int64_t j0 = piece_j0(Gm, pv, VEC);
      const int64_t j1 = pv == Gm.ppr - 1 ? P.V : (int64_t)Gm.head + (int64_t)(pv + 1) * kPcVectors * VEC;
      for (int64_t jj = j0; jj < j1 && rk < rcut; jj += 64) {
        const int64_t j = jj + lane;
        const bool tie = j < j1 && W.yval(E::load(x + j)) == W.vc;
        const uint64_t bal = __ballot(tie);
        if (tie && rk + (uint32_t)__popcll(bal & below) < rcut) y[j] = zr;
        rk += (uint32_t)__popcll(bal);
      }
    }
    seen += (uint32_t)__shfl((int)inc, 63, 64);
  }
}

// Phase 2, one wave per row with a non-zero upstream gradient: with the saved
// kept list each kept entry is stored on its own (phase 1 zeroed the rest);
// otherwise the row is re-read and rewritten whole.
template <class E>
__global__ __launch_bounds__(256) void filter_bwd_scatter_kernel(FilterBwdParams P, int64_t rows) {
  using raw = typename E::raw;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int64_t b = row / P.Rt, r = row - b * P.Rt;
  raw* y = static_cast<raw*>(P.gin) + b * P.gisb + r * P.gisr;
  // zeros over the row (zero_rows mode: rows not rewritten below)
  auto zero_row = [&]() {
    const RowSpan<E> zs(y, P.V);
    vu4* zv = reinterpret_cast<vu4*>(y + zs.head);
    for (int64_t i = lane; i < zs.nvec; i += 64) __builtin_nontemporal_store(vu4{0u, 0u, 0u, 0u}, zv + i);
    const raw zr = E::from_float(0.f);
    if (lane < zs.head) y[lane] = zr;
    if (zs.tail0 + lane < P.V) y[zs.tail0 + lane] = zr;
  };
  if (r >= P.R) {
    if (P.zero_rows) zero_row();
    return;
  }
  const int64_t srow = b * P.R + r;
  // independent loads, issued together
  const float gv = P.g[b * P.gsb + r * P.gsr];
  const RowInfo ri = P.info[srow];
  const int64_t t = P.target[b * P.tsb + r * P.tsr];
  const int32_t j0 = P.kept_idx[srow * kKeepCap + lane];
  const float p0 = P.kept_p[srow * kKeepCap + lane];
  if (gv == 0.f) {
    if (P.zero_rows) zero_row();
    return;
  }

  if (!P.zero_rows && ri.n_kept <= kKeepCap && (ri.flags & kFlagNoKeptList) == 0) {
    for (int i = lane; i < ri.n_kept; i += 64) {
      const int64_t j = (i == lane) ? j0 : P.kept_idx[srow * kKeepCap + i];
      const float p = (i == lane) ? p0 : P.kept_p[srow * kKeepCap + i];
      y[j] = grad_to_dtype<E>(((j == t) ? 1.f - p : -p) * gv, P);
    }
    return;
  }

  // Whole row: re-read the logits and re-apply the cut.
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  switch (grad_conv(P.has_t, P.has_gt)) {
    case kConvPlain: walk_row<E, kConvPlain>(P, ri, x, y, gv, t, lane); break;
    case kConvGT: walk_row<E, kConvGT>(P, ri, x, y, gv, t, lane); break;
    case kConvT: walk_row<E, kConvT>(P, ri, x, y, gv, t, lane); break;
    default: walk_row<E, kConvTwo>(P, ri, x, y, gv, t, lane); break;
  }
}

// filtered logits (-inf outside the kept set) and the keep mask
template <class E, int W>
__global__ __launch_bounds__(64 * W) void filter_mask_kernel(FilterParams P, void* filtered,
                                                             uint8_t* keep, int64_t fsr,
                                                             int64_t ksr) {
  using raw = typename E::raw;
  constexpr int NT = 64 * W;
  const int64_t row = blockIdx.x;
  const raw* x = static_cast<const raw*>(P.logits) + row * P.sr;
  raw* f = static_cast<raw*>(filtered) + row * fsr;
  uint8_t* kk = keep + row * ksr;
  const RowInfo ri = P.info[row];
  const raw ninf = E::from_float(-INFINITY);
  for (int64_t j = threadIdx.x; j < P.V; j += NT) {
    const raw xr = x[j];
    const bool k = kept_lex(E::load_raw(xr), j, ri.v_cut, ri.i_cut);
    f[j] = k ? xr : ninf;
    kk[j] = k ? 1 : 0;
  }
}

// Waves per row of the fast path (at least k lanes); 8 waves stream 4 vectors
// per lane per batch.  Measured on bf16 [4, 4096, 151936] rows (k = 50) / on
// the [8, 2048, 151936] top-k export (k = 64): 8 waves x 4 vectors 0.795 /
// 0.818 ms; x 8 vectors 0.825 / 0.912; x 2 vectors 0.801 / 0.810; x 16 vectors
// 0.815 / 1.53; 4 waves x 8 vectors 0.838 / 0.846; 16 waves x 2 vectors
// 0.857 / 0.823.
int fast_waves(int top_k) {
  int w = 8;
  while (w < 16 && 64 * w < top_k) w <<= 1;
  return w;
}

template <class E>
int launch_fwd(const FilterParams& P, int64_t rows, hipStream_t st) {
  const bool fast = P.top_k >= 1 && P.top_k <= 1024 && P.top_k <= P.V;
  if (fast) {
    switch (fast_waves(P.top_k)) {
      case 8:
        if (P.dec16)
          hipLaunchKernelGGL((filter_fast_kernel<E, 8, 4, false, true>), dim3((unsigned)rows), dim3(512),
                             0, st, P);
        else
          hipLaunchKernelGGL((filter_fast_kernel<E, 8, 4>), dim3((unsigned)rows), dim3(512), 0, st, P);
        break;
      default:
        if (P.dec16)
          hipLaunchKernelGGL((filter_fast_kernel<E, 16, 4, false, true>), dim3((unsigned)rows),
                             dim3(1024), 0, st, P);
        else
          hipLaunchKernelGGL((filter_fast_kernel<E, 16, 4>), dim3((unsigned)rows), dim3(1024), 0, st,
                             P);
        break;
    }
    if (int e = check_launch("filter_fast_kernel")) return e;
  }
  // the rows left to a general path: all of them, or those the fast kernel flagged
  if (sizeof(typename E::raw) == 2 && P.V <= kHistMaxV)
    return launch_hist_rows(P, dtype_code<E>(), rows, fast ? 0 : 1, st);
  bool all = !fast;
  if (std::is_same<E, F32>::value && !fast) {
    // fp32 rows in two passes; the rows it flags go to the radix kernel
    if (int e = launch_f32_rows(P, rows, st)) return e;
    all = false;
  }
  hipLaunchKernelGGL((filter_general_kernel<E>), dim3((unsigned)rows), dim3(kGeneralThreads), 0, st,
                     P, all ? 1 : 0);
  return check_launch("filter_general_kernel");
}

template <class E>
int launch_topk_export(const FilterParams& P, int64_t rows, hipStream_t st) {
  if (P.top_k > kCandCap) {
    hipLaunchKernelGGL((topk_export_large_kernel<E>), dim3((unsigned)rows), dim3(kGeneralThreads), 0,
                       st, P);
    return check_launch("topk_export_large_kernel");
  }
  switch (fast_waves(P.top_k)) {
    case 8:
      hipLaunchKernelGGL((filter_fast_kernel<E, 8, 4, true>), dim3((unsigned)rows), dim3(512), 0, st, P);
      break;
    default:
      hipLaunchKernelGGL((filter_fast_kernel<E, 16, 4, true>), dim3((unsigned)rows), dim3(1024), 0,
                         st, P);
      break;
  }
  if (int e = check_launch("filter_fast_kernel(export)")) return e;
  hipLaunchKernelGGL((topk_export_general_kernel<E>), dim3((unsigned)rows), dim3(kGeneralThreads), 0,
                     st, P);
  return check_launch("topk_export_general_kernel");
}

// Pieces per row bound (16-byte vectors of V elements, 4 KB pieces), for the workspace size.
int64_t piece_ppr_bound(int64_t V, int64_t esz) {
  const int64_t nv = V * esz / 16;
  return nv > 0 ? (nv + kPcVectors - 1) / kPcVectors : 1;
}

// The piece schedule's geometry when the layout allows it (logits and gradient
// co-aligned, every row at the same 16-byte offset, rows whole in 32-bit
// indexing), else ppr = 0.
template <class E>
PieceGeom piece_geom(const FilterBwdParams& P, int64_t B, int64_t rows, void* ws) {
  PieceGeom Gm{};
  constexpr int64_t esz = sizeof(typename E::raw);
  const uintptr_t ax = reinterpret_cast<uintptr_t>(P.logits), ay = reinterpret_cast<uintptr_t>(P.gin);
  auto row_step_ok = [&](int64_t stride, int64_t extent) { return extent <= 1 || (stride * esz) % 16 == 0; };
  if (ws == nullptr || ax % esz != 0 || ay % esz != 0 || ax % 16 != ay % 16) return Gm;
  if (!row_step_ok(P.sb, B) || !row_step_ok(P.sr, P.R) || !row_step_ok(P.gisb, B) || !row_step_ok(P.gisr, P.Rt))
    return Gm;
  int64_t head = (int64_t)(((16u - (ay & 15u)) & 15u) / esz);
  if (head > P.V) head = P.V;
  const int64_t nvec = (P.V - head) / E::kVec;
  const int64_t ppr = nvec > 0 ? (nvec + kPcVectors - 1) / kPcVectors : 1;
  if (rows * ppr * kPcThreads >= (int64_t(1) << 32)) return Gm;
  // workspace: the tie counts, then the tie lists
  const int64_t slots = B * P.R * piece_ppr_bound(P.V, esz);
  Gm.ppr = (int)ppr;
  Gm.nvec = (int)nvec;
  Gm.head = (int)head;
  Gm.tie_cnt = static_cast<uint32_t*>(ws);
  Gm.tie_pos = reinterpret_cast<uint16_t*>(Gm.tie_cnt + slots);
  return Gm;
}

template <class E>
int launch_bwd(const FilterBwdParams& P, int64_t B, int64_t rows, void* ws, hipStream_t st) {
  if (P.zero_rows) {
    // rows without kept lists: each row written once
    if (rows == 0) return MIRL_OK;
    const PieceGeom Gm = piece_geom<E>(P, B, rows, ws);
    if (Gm.ppr > 0) {
      // 4 KB pieces in address order, then the per-row fix-up of rank-form ties
      const int64_t srows = B * P.R;
      auto launch = [&](auto conv) {
        constexpr int CONV = decltype(conv)::value;
        hipLaunchKernelGGL((filter_bwd_piece_kernel<E, CONV>), dim3((unsigned)(rows * Gm.ppr)),
                           dim3(kPcThreads), 0, st, P, Gm);
        if (srows > 0)
          hipLaunchKernelGGL((filter_bwd_piece_fixup_kernel<E, CONV>), dim3((unsigned)((srows + 3) / 4)),
                             dim3(256), 0, st, P, Gm, srows);
      };
      switch (grad_conv(P.has_t, P.has_gt)) {
        case kConvPlain: launch(std::integral_constant<int, kConvPlain>{}); break;
        case kConvGT: launch(std::integral_constant<int, kConvGT>{}); break;
        case kConvT: launch(std::integral_constant<int, kConvT>{}); break;
        default: launch(std::integral_constant<int, kConvTwo>{}); break;
      }
      return check_launch("filter_bwd_piece_kernel");
    }
    // other layouts: a workgroup walks each row
    auto launch = [&](auto conv) {
      constexpr int CONV = decltype(conv)::value;
      hipLaunchKernelGGL((filter_bwd_row_kernel<E, CONV>), dim3((unsigned)rows), dim3(kRowThreads), 0,
                         st, P);
    };
    switch (grad_conv(P.has_t, P.has_gt)) {
      case kConvPlain: launch(std::integral_constant<int, kConvPlain>{}); break;
      case kConvGT: launch(std::integral_constant<int, kConvGT>{}); break;
      case kConvT: launch(std::integral_constant<int, kConvT>{}); break;
      default: launch(std::integral_constant<int, kConvTwo>{}); break;
    }
    return check_launch("filter_bwd_row_kernel");
  }
  const bool contiguous = P.gisr == P.V && (B == 1 || P.gisb == P.Rt * P.V);
  if (contiguous) {
    const int64_t n = rows * P.V;
    const uintptr_t a = reinterpret_cast<uintptr_t>(P.gin);
    const uintptr_t a16 = (a + 15u) & ~uintptr_t(15);
    const int to4k = (int)(((4096u - (a16 & 4095u)) & 4095u) / 16u);  // vectors before a 4 KB boundary
    const int shift = (256 - to4k) & 255;
    const int64_t nvec = (n * (int64_t)sizeof(typename E::raw)) / 16 + 1;
    const int64_t grid = (nvec + shift + 255) / 256;
    MIRL_REQUIRE(grid < (int64_t(1) << 31), "gradient too large (%lld elements)", (long long)n);
    hipLaunchKernelGGL((filter_bwd_zero_flat_kernel<E>), dim3((unsigned)grid), dim3(256), 0, st,
                       P.gin, n, shift);
  } else {
    hipLaunchKernelGGL((filter_bwd_zero_rows_kernel<E, 16>), dim3((unsigned)rows), dim3(1024), 0,
                       st, P);
  }
  if (int e = check_launch("filter_bwd_zero_kernel")) return e;
  if (P.R == 0) return MIRL_OK;
  hipLaunchKernelGGL((filter_bwd_scatter_kernel<E>), dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     st, P, rows);
  return check_launch("filter_bwd_scatter_kernel");
}

int check_filter_args(int dtype, int64_t B, int64_t R, int64_t V, int top_k, double top_p,
                      double temperature, int p_dtype) {
  if (dtype != MIRL_DTYPE_F32 && dtype != MIRL_DTYPE_BF16 && dtype != MIRL_DTYPE_F16) {
    set_error("unsupported logits dtype code %d", dtype);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(p_dtype == MIRL_DTYPE_F32 || p_dtype == dtype,
               "top-p decision dtype %d must be fp32 (%d) or the logits dtype (%d)", p_dtype,
               MIRL_DTYPE_F32, dtype);
  if (p_dtype != MIRL_DTYPE_F32 && top_p < 1.0 && V > kHistMaxV) {
    set_error("top-p decided in a 16-bit dtype supports vocabularies up to %lld (got %lld)",
              (long long)kHistMaxV, (long long)V);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0, "invalid shape B=%lld R=%lld V=%lld", (long long)B,
               (long long)R, (long long)V);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  MIRL_REQUIRE(top_k <= V, "selected index k out of range (top_k=%d, vocabulary %lld)", top_k,
               (long long)V);
  MIRL_REQUIRE(top_k > 0 || (top_p > 0.0 && top_p < 1.0),
               "no filtering requested (top_k=%d, top_p=%g)", top_k, top_p);
  MIRL_REQUIRE(top_p > 0.0 && top_p <= 1.0, "top_p must be in (0, 1], got %g", top_p);
  MIRL_REQUIRE(temperature > 0.0, "temperature must be positive, got %g", temperature);
  return MIRL_OK;
}

// fp32 -> bf16 -> fp32, round to nearest even (finite inputs)
float round_bf16_host(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float r;
  __builtin_memcpy(&r, &u, 4);
  return r;
}

FilterParams make_params(const void* logits, int64_t R, int64_t V, int64_t sb, int64_t sr,
                         const int64_t* target, int64_t tsb, int64_t tsr, double temperature,
                         int top_k, double top_p, int p_dtype, float* out, void* info,
                         int32_t* kept_idx, float* kept_p) {
  FilterParams P;
  P.logits = logits;
  P.R = R;
  P.V = V;
  P.sb = sb;
  P.sr = sr;
  P.target = target;
  P.tsb = tsb;
  P.tsr = tsr;
  P.rT = temperature_recip(temperature);
  P.has_t = temperature != 1.0;
  P.top_k = top_k > 0 ? top_k : 0;
  P.has_p = top_p < 1.0;
  P.cut = (float)(1.0 - top_p);
  P.dec16 = p_dtype != MIRL_DTYPE_F32 && P.has_p;
  // the Python float 1 - top_p meets a 16-bit tensor as that dtype: double ->
  // float -> dtype, each rounding to nearest even
  P.thr16 = p_dtype == MIRL_DTYPE_BF16 ? round_bf16_host(P.cut)
            : p_dtype == MIRL_DTYPE_F16 ? (float)(_Float16)P.cut : P.cut;
  P.out = out;
  P.info = static_cast<RowInfo*>(info);
  P.kept_idx = kept_idx;
  P.kept_p = kept_p;
  P.tk_vals = nullptr;
  P.tk_idx = nullptr;
  P.tk_base = 0;
  const char* ex = std::getenv("MIRL_F32_FILTER_EXACT_BELOW");
  P.f32_exact_below = (ex != nullptr && ex[0] == '1') ? 1 : 0;
  return P;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_filtered_logprob_fwd(const void* logits, int dtype, int64_t B, int64_t R,
                                         int64_t V, int64_t stride_b, int64_t stride_r,
                                         const int64_t* target, int64_t t_stride_b,
                                         int64_t t_stride_r, double temperature, int top_k,
                                         double top_p, int p_dtype, float* out, void* row_info,
                                         int32_t* kept_idx, float* kept_p, void* stream) {
  clear_error();
  if (int e = check_filter_args(dtype, B, R, V, top_k, top_p, temperature, p_dtype)) return e;
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(logits && row_info && kept_idx && kept_p, "null pointer argument");
  MIRL_REQUIRE(out == nullptr || target != nullptr, "out given without target");
  const FilterParams P = make_params(logits, R, V, stride_b, stride_r, target, t_stride_b,
                                     t_stride_r, temperature, top_k, top_p, p_dtype, out,
                                     row_info, kept_idx, kept_p);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32) return launch_fwd<F32>(P, rows, st);
  if (dtype == MIRL_DTYPE_BF16) return launch_fwd<BF16>(P, rows, st);
  return launch_fwd<F16>(P, rows, st);
}

extern "C" int mirl_filtered_logprob_bwd(const void* logits, int dtype, int64_t B, int64_t R,
                                         int64_t R_total, int64_t V, int64_t stride_b,
                                         int64_t stride_r, const int64_t* target,
                                         int64_t t_stride_b, int64_t t_stride_r,
                                         double temperature, double grad_temperature, int top_k,
                                         const void* row_info, const int32_t* kept_idx,
                                         const float* kept_p, const float* grad_out,
                                         int64_t g_stride_b, int64_t g_stride_r, void* grad_in,
                                         int64_t gi_stride_b, int64_t gi_stride_r, void* workspace,
                                         void* stream) {
  clear_error();
  if (dtype != MIRL_DTYPE_F32 && dtype != MIRL_DTYPE_BF16 && dtype != MIRL_DTYPE_F16) {
    set_error("unsupported logits dtype code %d", dtype);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(B >= 0 && R >= 0 && R_total >= R && V > 0, "invalid shape");
  MIRL_REQUIRE(temperature > 0.0 && grad_temperature > 0.0, "temperature must be positive");
  const int64_t rows = B * R_total;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(grad_in != nullptr, "null grad_in");
  MIRL_REQUIRE(R == 0 || (logits && target && row_info && kept_idx && kept_p && grad_out),
               "null pointer argument");
  FilterBwdParams P;
  P.logits = logits;
  P.R = R;
  P.Rt = R_total;
  P.V = V;
  P.sb = stride_b;
  P.sr = stride_r;
  P.target = target;
  P.tsb = t_stride_b;
  P.tsr = t_stride_r;
  P.rT = temperature_recip(temperature);
  P.has_t = temperature != 1.0;
  P.rGT = temperature_recip(grad_temperature);
  P.has_gt = grad_temperature != 1.0;
  P.info = static_cast<const RowInfo*>(row_info);
  P.kept_idx = kept_idx;
  P.kept_p = kept_p;
  P.g = grad_out;
  P.gsb = g_stride_b;
  P.gsr = g_stride_r;
  P.gin = grad_in;
  P.gisb = gi_stride_b;
  P.gisr = gi_stride_r;
  // the forward keeps kept lists for the rows of 1 <= top_k <= 1024 (fast path):
  // zero the gradient in one flat pass, then scatter; otherwise rows are
  // rewritten whole and each row is written once
  P.zero_rows = !(top_k >= 1 && top_k <= kCandCap);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32) return launch_bwd<F32>(P, B, rows, workspace, st);
  if (dtype == MIRL_DTYPE_BF16) return launch_bwd<BF16>(P, B, rows, workspace, st);
  return launch_bwd<F16>(P, B, rows, workspace, st);
}

extern "C" int64_t mirl_filtered_logprob_bwd_workspace_bytes(int dtype, int64_t B, int64_t R, int64_t V) {
  clear_error();
  const int64_t esz = dtype == MIRL_DTYPE_F32 ? 4 : (dtype == MIRL_DTYPE_BF16 || dtype == MIRL_DTYPE_F16) ? 2 : 0;
  if (esz == 0) {
    set_error("unsupported logits dtype code %d", dtype);
    return -1;
  }
  if (B < 0 || R < 0 || V <= 0) {
    set_error("invalid shape B=%lld R=%lld V=%lld", (long long)B, (long long)R, (long long)V);
    return -1;
  }
  return B * R * piece_ppr_bound(V, esz) * (int64_t)(4 + 2 * kPieceTieCap);
}

extern "C" int mirl_top_k_top_p_mask(const void* logits, int dtype, int64_t N, int64_t V,
                                     int64_t row_stride, int top_k, double top_p, int p_dtype,
                                     void* row_info, int32_t* kept_idx, float* kept_p,
                                     void* filtered, int64_t filtered_row_stride,
                                     uint8_t* keep_mask, int64_t keep_row_stride, void* stream) {
  clear_error();
  if (int e = check_filter_args(dtype, N, 1, V, top_k, top_p, 1.0, p_dtype)) return e;
  if (N == 0) return MIRL_OK;
  MIRL_REQUIRE(N < (int64_t(1) << 31), "too many rows (%lld)", (long long)N);
  MIRL_REQUIRE(logits && row_info && kept_idx && kept_p && filtered && keep_mask,
               "null pointer argument");
  // rows are [N, V] with row stride `row_stride`: R = 1 so that row = b
  const FilterParams P = make_params(logits, 1, V, row_stride, 0, nullptr, 0, 0, 1.0, top_k,
                                     top_p, p_dtype, nullptr, row_info, kept_idx, kept_p);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int e;
  if (dtype == MIRL_DTYPE_F32) e = launch_fwd<F32>(P, N, st);
  else if (dtype == MIRL_DTYPE_BF16) e = launch_fwd<BF16>(P, N, st);
  else e = launch_fwd<F16>(P, N, st);
  if (e) return e;
  if (int e2 = launch_resolve_rows(P, dtype, N, st)) return e2;  // index form for the mask kernel
  FilterParams Q = P;
  Q.sr = row_stride;  // filter_mask_kernel indexes rows by row * sr
  if (dtype == MIRL_DTYPE_F32)
    hipLaunchKernelGGL((filter_mask_kernel<F32, 4>), dim3((unsigned)N), dim3(256), 0, st, Q,
                       filtered, keep_mask, filtered_row_stride, keep_row_stride);
  else if (dtype == MIRL_DTYPE_BF16)
    hipLaunchKernelGGL((filter_mask_kernel<BF16, 4>), dim3((unsigned)N), dim3(256), 0, st, Q,
                       filtered, keep_mask, filtered_row_stride, keep_row_stride);
  else
    hipLaunchKernelGGL((filter_mask_kernel<F16, 4>), dim3((unsigned)N), dim3(256), 0, st, Q,
                       filtered, keep_mask, filtered_row_stride, keep_row_stride);
  return check_launch("mirl_top_k_top_p_mask");
}

extern "C" int64_t mirl_vocab_topk_workspace_bytes(int64_t rows) {
  return rows * (int64_t)sizeof(RowInfo);
}

extern "C" int mirl_vocab_topk(const void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                               int64_t stride_b, int64_t stride_r, int k, int64_t vocab_start,
                               float* values, int64_t* indices, void* workspace, void* stream) {
  clear_error();
  if (dtype != MIRL_DTYPE_F32 && dtype != MIRL_DTYPE_BF16 && dtype != MIRL_DTYPE_F16) {
    set_error("unsupported logits dtype code %d", dtype);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(B >= 0 && R >= 0 && V > 0, "invalid shape B=%lld R=%lld V=%lld", (long long)B,
               (long long)R, (long long)V);
  MIRL_REQUIRE(V < (int64_t(1) << 31), "vocabulary size %lld exceeds 2^31-1", (long long)V);
  MIRL_REQUIRE(k >= 1 && k <= V, "k=%d must be in [1, V=%lld]", k, (long long)V);
  const int64_t rows = B * R;
  if (rows == 0) return MIRL_OK;
  MIRL_REQUIRE(rows < (int64_t(1) << 31), "too many rows (%lld)", (long long)rows);
  MIRL_REQUIRE(logits && values && indices && workspace, "null pointer argument");
  FilterParams P = make_params(logits, R, V, stride_b, stride_r, nullptr, 0, 0, 1.0, k, 1.0,
                               MIRL_DTYPE_F32, nullptr, workspace, nullptr, nullptr);
  P.tk_vals = values;
  P.tk_idx = indices;
  P.tk_base = vocab_start;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32) return launch_topk_export<F32>(P, rows, st);
  if (dtype == MIRL_DTYPE_BF16) return launch_topk_export<BF16>(P, rows, st);
  return launch_topk_export<F16>(P, rows, st);
}

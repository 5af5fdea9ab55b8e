// Top-k / top-p filtered forward for fp32 rows whose filter keeps large sets
// (top-p without top-k, or k > 1024): two passes over each row.
//
// Semantics (those of topk_filter.hip with fp32 decisions; reference
// nemo_rl/algorithms/logits_sampling_utils.py:111-212 on the fp32 tensor of
// nemo_rl/distributed/model_utils.py:1660-1718): y = fl32(x * fl32(1 / T)),
// thr = the k-th largest y (every tie kept); over the kept-k values in
// ascending (value, index) order p = fl32(expf(y - m) * fl32(1 / Z)) with
// Z = fl32(the double sum of expf(y - m)), cum = the double sum of the p up to
// and including an element, rounded to fp32; the cut is the first element
// with cum > fl32(1 - top_p) (the maximum when there is none); kept = the cut
// and everything after it.
//
// The normaliser needs the row maximum before any exponential is summed, and
// an fp32 row of the vocabulary (600 KB) is larger than a CU's LDS, so the
// row is read twice:
//  - pass 1 streams the row once: its maximum, and the number of values under
//    each 16-bit prefix of the fp32 bits (the bf16 truncation) in a 70 KB
//    table over the magnitudes below 512 (word m counts +x in its low half
//    and -x in its high half).  The values under one prefix lie within one
//    part in 128 of each other, so each bin's exp(y - m) has known bounds.
//    From the counts follow the bin of the k-th largest value, and rigorous
//    lower and upper bounds of the ascending cumulative mass at every bin
//    boundary; these give two bins B1 <= B2 that bracket the cut;
//  - pass 2 streams the row again: the exact normaliser (double sum over the
//    kept-k values), the exact sum of expf(y - m) of the kept-k values below
//    B1, the kept count and sum above B2, and every element of bins B1..B2
//    (a few hundred to a few thousand) collected into LDS as
//    (order key << 32 | index).
// The k-th largest value and the cut are then found among the collected
// elements by radix rounds with exact double masses in LDS.  The mass below
// B1 enters as inv * sum(e), which is within 2^-24 (relative) of the sum of
// the rounded p; a row whose cut that interval leaves undecided is summed
// exactly by a third pass.  Rows outside the table (|y| >= 512, inf, NaN),
// with 65536 or more values under one prefix, or with more bracketed
// elements than LDS holds are flagged for filter_general_kernel.

#include "filter.h"

namespace mirl {

namespace {

constexpr int kFT = 512;  // threads per row: two rows per CU
constexpr int kUB = 4;    // 16-byte vectors per lane and batch (two batches in flight)
constexpr int kFW = kFT / kWave;
constexpr uint32_t kMagWords = 0x4400;  // 16-bit magnitude prefixes below 512.0
constexpr int kFWPT = (int)kMagWords / kFT;
constexpr int kFTable = (int)kMagWords + 1;  // + the word counting values outside it
constexpr int kFCand = (kFTable * 4) / 8;    // collected elements over the same bytes
constexpr int kWaveCap = kFCand / kFW;        // collected elements per wave (its own segment)
static_assert(kFWPT * kFT == (int)kMagWords, "table words split evenly over the threads");

struct F32Shared {
  union {
    uint32_t hist[kFTable];
    uint32_t list[kFTable];  // occupied bins: count << 16 | 16-bit order key
    uint64_t cand[kFCand];   // okey(y) << 32 | index
  } u;
  double hd[256];
  uint32_t hc[256];
  float red_f[kFW];
  // one slot per workgroup reduction (each written once, so no barrier before it)
  uint32_t ru_a[4 * kFW], ru_b[kFW], ru_c[kFW], ru_d[kFW];
  double rd_a[2 * kFW], rd_b[2 * kFW], rd_c[kFW], rd_d[kFW], rd_e[kFW], rd_f[2 * kFW];
  uint32_t wcnt[kFW];  // elements each wave collected into its segment
  uint32_t ncand;      // collected elements, contiguous after the compaction
  uint32_t bk16, kprime, b1, b2;
  uint32_t cbk;
  uint32_t sel[4];
  double dsel[1];
  unsigned long long best;
  int status;
};

// -0.0 becomes +0.0 (the order key treats them as one value, and so must the table)
__device__ __forceinline__ float canon(float y) { return y + 0.0f; }

// The filtered value y = fl32(x * fl32(1 / T)); -0.0 is left as it is (the
// float comparisons and the order key treat it as +0.0).
template <bool HAS_T>
__device__ __forceinline__ float y_of(float x, float rT) {
  if constexpr (HAS_T) return mul_rn(x, rT);
  else return x;
}
// Calls f(std::integral_constant<bool, has_t>): the streaming loops are
// compiled once with the temperature's product and once without.
template <class F>
__device__ __forceinline__ void with_t(bool has_t, F&& f) {
  if (has_t) f(std::true_type{});
  else f(std::false_type{});
}

// Exclusive scans (thread order) and totals of N values with one barrier.
// `red` (N * kFW entries) belongs to this reduction alone, so no barrier is
// needed before it is written.
template <class T, int N>
__device__ __forceinline__ void block_scan1(const T (&v)[N], T (&ex)[N], T (&tot)[N], T* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  T inc[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    inc[i] = wave_scan_dpp(v[i]);
    if (lane == 63) red[i * kFW + wv] = inc[i];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    T base = T(0), t = T(0);
#pragma unroll
    for (int w = 0; w < kFW; ++w) {
      const T r = red[i * kFW + w];
      base += (w < wv) ? r : T(0);
      t += r;
    }
    ex[i] = base + (inc[i] - v[i]);
    tot[i] = t;
  }
}
template <class T, int N>
__device__ __forceinline__ void block_sum1(T (&v)[N], T* red) {
  T ex[N];
  block_scan1(v, ex, v, red);
}
template <class T>
__device__ __forceinline__ T block_total1(T v, T* red) {
  T a[1] = {v};
  block_sum1(a, red);
  return a[0];
}

// Bounds of exp(y - m) over the values under a 16-bit order key (a bin): the
// bin's smallest value and the next bin's smallest value, their distance to
// m and its product with log2(e) in fp32 (|y - m| < 1024: within 2^-13.5
// relative after the exponential), the hardware exp2 (about one ulp), and a
// slack of 2^-11 that covers those, exp_le0's error and the fp32 roundings of
// the probabilities.
__device__ __forceinline__ void bin_bounds(uint32_t k16, float M, double& elo, double& ehi) {
  constexpr float kSlack = 1.0f / 2048.0f;
  const float vlo = from_okey(k16 << 16), vhi = from_okey((k16 + 1u) << 16);
  elo = (double)(__builtin_amdgcn_exp2f((vlo - M) * kLog2e) * (1.0f - kSlack));
  ehi = (double)(fminf(__builtin_amdgcn_exp2f((vhi - M) * kLog2e), 1.0f) * (1.0f + kSlack));
}

// Streams the row's fp32 values through f(y, index, valid): an unaligned head
// and tail element by element (visited by every lane of wave 0, valid only
// where an element is, so that a wave's ballots and the counts kept from them
// stay the same in all its lanes), the body as 16-byte vectors in batches of
// UB per lane with the next batch in flight while the current one is visited.
template <int UB, bool HAS_T, class F>
__device__ __forceinline__ void stream_row(const float* x, int64_t V, float rT, F&& f) {
  const int tid = threadIdx.x;
  const RowSpan<F32> sp(x, V);
  if (tid < kWave) {  // the whole of wave 0
    const bool hv = tid < sp.head;
    f(hv ? y_of<HAS_T>(x[tid], rT) : 0.f, (uint32_t)tid, hv);
    const bool tv = sp.tail0 + tid < V;
    f(tv ? y_of<HAS_T>(x[sp.tail0 + tid], rT) : 0.f, (uint32_t)(sp.tail0 + tid), tv);
  }
  const vu4* xv = reinterpret_cast<const vu4*>(x + sp.head);
  const int nv = (int)sp.nvec;  // < 2^29: V < 2^31
  constexpr int kStep = UB * kFT;
  const int nfull = nv / kStep;
  const uint32_t head = (uint32_t)sp.head;
  vu4 qa[UB], qb[UB];
  auto issue = [&](vu4(&q)[UB], int bi) {
#pragma unroll
    for (int u = 0; u < UB; ++u) q[u] = __builtin_nontemporal_load(xv + (bi * kStep + tid + u * kFT));
  };
  auto visit = [&](const vu4(&q)[UB], int bi) {
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const uint32_t j0 = head + 4u * (uint32_t)(bi * kStep + tid + u * kFT);
      f(y_of<HAS_T>(__uint_as_float(q[u].x), rT), j0, true);
      f(y_of<HAS_T>(__uint_as_float(q[u].y), rT), j0 + 1u, true);
      f(y_of<HAS_T>(__uint_as_float(q[u].z), rT), j0 + 2u, true);
      f(y_of<HAS_T>(__uint_as_float(q[u].w), rT), j0 + 3u, true);
      __builtin_amdgcn_sched_barrier(0);  // one vector at a time (register budget)
    }
  };
  if (nfull > 0) issue(qa, 0);
  int bi = 0;
  for (; bi + 1 < nfull; bi += 2) {
    issue(qb, bi + 1);
    visit(qa, bi);
    if (bi + 2 < nfull) issue(qa, bi + 2);
    visit(qb, bi + 1);
  }
  if (bi < nfull) visit(qa, bi);
#pragma unroll
  for (int u = 0; u < UB; ++u) {
    const int v = nfull * kStep + tid + u * kFT;
    // the remaining vectors: every lane of a wave visits them, valid where one is
    const bool vv = v < nv;
    const vu4 q = vv ? __builtin_nontemporal_load(xv + v) : vu4{0u, 0u, 0u, 0u};
    const uint32_t j0 = head + 4u * (uint32_t)v;
    f(y_of<HAS_T>(__uint_as_float(q.x), rT), j0, vv);
    f(y_of<HAS_T>(__uint_as_float(q.y), rT), j0 + 1u, vv);
    f(y_of<HAS_T>(__uint_as_float(q.z), rT), j0 + 2u, vv);
    f(y_of<HAS_T>(__uint_as_float(q.w), rT), j0 + 3u, vv);
  }
}

// exp(x) for x <= 0, as expf evaluates it: x * log2(e) as a rounded product
// plus its rounding error (an fma with the constant's high part, then its low
// part), the nearest integer taken out, exp2 of the remainder on the hardware
// instruction, scaled back by the integer.  expf's own range checks are left
// out (no overflow for x <= 0; below -103.97, where expf returns 0, this may
// return a subnormal).
__device__ __forceinline__ float exp_le0(float x) {
#pragma clang fp contract(off)
  constexpr float kHi = 0x1.715476p+0f, kLo = 0x1.4ae0bep-26f;
  const float ph = x * kHi;
  float pl = __builtin_fmaf(x, kHi, -ph);
  pl = __builtin_fmaf(x, kLo, pl);
  const float e = __builtin_rintf(ph);
  const float a = (ph - e) + pl;
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(a), (int)e);
}

// Probability of a collected value: fl32(exp(y - m) * inv), widened.
__device__ __forceinline__ double prob_of(uint32_t k32, float M, float inv) {
  return (double)(exp_le0(from_okey(k32) - M) * inv);
}

// Calls f(entry) for every collected element.
template <class F>
__device__ __forceinline__ void for_cands(const F32Shared& sh, F&& f) {
  const int n = (int)sh.ncand;
  for (int i = threadIdx.x; i < n; i += kFT) f(sh.u.cand[i]);
}

// The cut among the collected elements of bins B1..B2 (kept-k: key >= thr):
// the first element, in (value, index) order, whose cumulative mass (the
// mass below B1 plus the collected masses up to it) rounds to more than
// `cut`.  The mass below B1 is known to lie in [dlo, dhi].  Returns 0 with
// the key and index in `key`, `idx` when both ends of the interval give the
// same element, 1 when they differ, 2 when no element's cumulative mass
// exceeds the cut, 3 when the mass below the bracket alone exceeds it.
struct Cut {
  int status;
  uint32_t key, idx;
};
__device__ Cut find_cut(F32Shared& sh, uint32_t thr32, uint32_t B1, uint32_t B2, float M,
                        float inv, double dlo, double dhi, float cut, int64_t V) {
  const int tid = threadIdx.x, lane = tid & 63;
  const uint64_t base_key = (uint64_t)B1 << 16;
  const uint32_t span = B2 - B1 + 1u;  // bins in the bracket
  int wb = 16;
  while ((1u << (wb - 16)) < span) ++wb;  // offset bits of the bracket (<= 32)
  uint64_t cur = 0;  // offset prefix: bits below wb are open
  double blo = dlo, bhi = dhi;
  uint32_t ties = 0;
  auto in_bracket = [&](uint32_t k32) {
    const uint32_t k16 = k32 >> 16;
    return k32 >= thr32 && k16 >= B1 && k16 <= B2;
  };
  bool first_round = true;
  while (wb > 0) {
    const int shift = wb > 8 ? wb - 8 : 0;
    const uint32_t nd = 1u << (wb - shift);
    for (int i = tid; i < 256; i += kFT) {
      sh.hd[i] = 0.0;
      sh.hc[i] = 0u;
    }
    __syncthreads();
    for_cands(sh, [&](uint64_t c) {
      const uint32_t k32 = (uint32_t)(c >> 32);
      if (!in_bracket(k32)) return;
      const uint64_t off = (uint64_t)k32 - base_key;
      if ((off >> wb) != (cur >> wb)) return;
      const uint32_t d = (uint32_t)(off >> shift) & (nd - 1u);
      atomicAdd(&sh.hd[d], prob_of(k32, M, inv));
      atomicAdd(&sh.hc[d], 1u);
    });
    __syncthreads();
    if (tid < kWave) {
      // lane l holds digits 4l .. 4l+3: the first occupied digit whose
      // cumulative mass crosses the cut, from each end of the interval
      constexpr int kNone = 1 << 30;
      double s[4], cb[4], lt = 0.0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[j] = sh.hd[4 * lane + j];
        lt += s[j];
      }
      const double inc = wave_scan_dpp(lt);
      double c = __shfl_up(inc, 1, kWave);
      if (lane == 0) c = 0.0;
      int dl = kNone, dh = kNone, last = -1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        cb[j] = c;
        const double c2 = c + s[j];
        if (sh.hc[4 * lane + j] != 0u) {
          last = 4 * lane + j;
          if (dl == kNone && (float)(blo + c2) > cut) dl = 4 * lane + j;
          if (dh == kNone && (float)(bhi + c2) > cut) dh = 4 * lane + j;
        }
        c = c2;
      }
      // digits are ordered by lane: the first lane with a crossing holds the
      // first crossing digit, the last lane with an occupied digit the last one
      const uint64_t bl = __ballot(dl != kNone), bh = __ballot(dh != kNone), bo = __ballot(last >= 0);
      const int gl = bl ? __builtin_amdgcn_readlane(dl, __ffsll((long long)bl) - 1) : kNone;
      const int gh = bh ? __builtin_amdgcn_readlane(dh, __ffsll((long long)bh) - 1) : kNone;
      const int gi = bo ? __builtin_amdgcn_readlane(last, 63 - __clzll((long long)bo)) : -1;
      int d = -1, st = 0;
      if (first_round && (float)bhi > cut) {
        st = 3;  // the mass below the bracket alone crosses: the bracket is wrong
      } else if (gl != gh) {
        st = 1;
      } else if (gl == kNone) {
        // no crossing: in a first round there is none at all; in a later one
        // the previous digit crossed as a whole, so its last occupied digit
        // (a difference in the summation order) is the one
        if (first_round || gi < 0) st = 2;
        else d = gi;
      } else {
        d = gl;
      }
      if (lane == 0) sh.status = st;
      if (d >= 0 && (d >> 2) == lane) {
        sh.sel[0] = (uint32_t)d;
        const int q = d & 3;  // selects without a dynamically indexed array (no scratch)
        sh.dsel[0] = q == 0 ? cb[0] : q == 1 ? cb[1] : q == 2 ? cb[2] : cb[3];
      }
    }
    __syncthreads();
    if (sh.status != 0) return Cut{sh.status, 0u, 0u};
    const uint32_t d = sh.sel[0];
    blo += sh.dsel[0];
    bhi += sh.dsel[0];
    ties = sh.hc[d];
    cur |= (uint64_t)d << shift;
    wb = shift;
    first_round = false;
    __syncthreads();
  }
  const uint32_t key = (uint32_t)(base_key + cur);
  // the cut's value is `key`; `ties` collected elements hold it, each with mass p
  if (ties <= 1u) {
    if (tid == 0) sh.sel[1] = 0xffffffffu;
    __syncthreads();
    for_cands(sh, [&](uint64_t c) {
      if ((uint32_t)(c >> 32) == key) sh.sel[1] = (uint32_t)c;
    });
    __syncthreads();
    return Cut{0, key, sh.sel[1]};
  }
  // ties: the j-th in index order, the smallest j whose cumulative mass crosses
  const double p = prob_of(key, M, inv);
  auto first_j = [&](double base) {
    // the smallest j in [1, ties] with fl32(base + j p) > cut (ties when none)
    uint32_t lo = 1u, hi = ties;
    while (lo < hi) {
      const uint32_t mid = lo + (hi - lo) / 2u;
      if ((float)(base + (double)mid * p) > cut) hi = mid;
      else lo = mid + 1u;
    }
    return lo;
  };
  const uint32_t jl = first_j(blo), jh = first_j(bhi);
  if (jl != jh) return Cut{1, 0u, 0u};
  uint32_t need = jl;
  int nbits = 1;
  while ((int64_t(1) << nbits) < V) ++nbits;
  uint32_t pre = 0;
  int w2 = nbits;
  while (w2 > 0) {
    const int shift = w2 > 8 ? w2 - 8 : 0;
    const uint32_t nd = 1u << (w2 - shift);
    for (int i = tid; i < 256; i += kFT) sh.hc[i] = 0u;
    __syncthreads();
    for_cands(sh, [&](uint64_t c) {
      if ((uint32_t)(c >> 32) != key) return;
      const uint32_t j = (uint32_t)c;
      if ((j >> w2) != (pre >> w2)) return;
      atomicAdd(&sh.hc[(j >> shift) & (nd - 1u)], 1u);
    });
    __syncthreads();
    if (tid < kWave) {
      uint32_t s[4], lt = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s[j] = sh.hc[4 * lane + j];
        lt += s[j];
      }
      uint32_t c = wave_scan_dpp(lt) - lt;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (c < need && c + s[j] >= need) {
          sh.sel[2] = (uint32_t)(4 * lane + j);
          sh.sel[3] = need - c;
        }
        c += s[j];
      }
    }
    __syncthreads();
    pre |= sh.sel[2] << shift;
    need = sh.sel[3];
    w2 = shift;
    __syncthreads();
  }
  return Cut{0, key, pre};
}

// Flags the row for filter_general_kernel (uniform: every thread returns after it).
__device__ __forceinline__ void flag_row(const FilterParams& P, int64_t row) {
  if (threadIdx.x == 0) {
    RowInfo ri{};
    ri.flags = kFlagRedo;
    P.info[row] = ri;
  }
}

// Pass 2 over the row: the double sums of expf(y - m) over the kept-k values
// (`zall`: every value >= vinc, which leaves out the partly kept bin of the
// k-th largest value) and over those below the bracket (`db`: vinc <= y <
// vb1), and the collection of the bracket [vb1, vb2e) and of the k-th largest
// value's bin [vlo, vloe) into LDS.  TOPK: some values fall below the k-th
// largest value's bin (otherwise every value is kept-k and the tests drop).
template <bool TOPK, bool HAS_T>
__device__ __forceinline__ void pass2(const float* x, int64_t V, const FilterParams& P,
                                      F32Shared& sh, float M, float vinc, float vb1, float vb2e,
                                      float vlo, float vloe, double& zall, double& db) {
  // each wave appends to its own segment at a wave-uniform count: no atomics
  uint64_t* seg = sh.u.cand + (threadIdx.x >> 6) * kWaveCap;
  uint32_t wc = 0u;
  stream_row<kUB, HAS_T>(x, V, P.rT, [&](float y, uint32_t j, bool valid) {
    const double de = valid ? (double)exp_le0(y - M) : 0.0;
    const bool below = y < vb1;
    bool coll = valid && !below && y < vb2e;
    if constexpr (TOPK) {
      const bool incl = y >= vinc;
      zall += incl ? de : 0.0;
      db += (incl && below) ? de : 0.0;
      coll = coll || (valid && y >= vlo && y < vloe);
    } else {
      zall += de;
      db += below ? de : 0.0;
    }
    const uint64_t bal = __ballot(coll);
    if (bal != 0ull) {
      if (coll) {
        const uint32_t at = wc + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (at < (uint32_t)kWaveCap) seg[at] = ((uint64_t)okey(y) << 32) | j;
      }
      wc += (uint32_t)__popcll(bal);
    }
  });
  if ((threadIdx.x & 63) == 0) sh.wcnt[threadIdx.x >> 6] = wc;
}

__global__ __launch_bounds__(kFT, 4) void filter_f32_kernel(FilterParams P) {
  __shared__ F32Shared sh;
  const int64_t row = blockIdx.x;
  const int64_t b = row / P.R, r = row - b * P.R;
  const float* x = static_cast<const float*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;

  {
    vu4* h4 = reinterpret_cast<vu4*>(sh.u.hist);
    for (int i = tid; i < kFTable / 4; i += kFT) h4[i] = vu4{0u, 0u, 0u, 0u};
    for (int i = (kFTable / 4) * 4 + tid; i < kFTable; i += kFT) sh.u.hist[i] = 0u;
  }
  if (tid == 0) {
    sh.status = 0;
    sh.bk16 = 0xffffffffu;  // set below by the thread whose bins hold the k-th largest
    sh.b1 = 0u;
    sh.b2 = 0xffffffffu;
  }
  __syncthreads();
  int64_t t = -1;
  float yt = 0.f;
  if (tid == 0 && P.out != nullptr) {
    t = P.target[b * P.tsb + r * P.tsr];
    if (t >= 0 && t < V) yt = canon(P.has_t ? mul_rn(x[t], P.rT) : x[t]);
  }

  // ---- pass 1: the maximum and the 16-bit prefix counts ----
  float mloc = -INFINITY;
  {
    char* hb = reinterpret_cast<char*>(sh.u.hist);
    with_t(P.has_t, [&](auto ht) {
      stream_row<kUB, decltype(ht)::value>(x, V, P.rT, [&](float y, uint32_t, bool valid) {
        if (!valid) return;
        y = canon(y);  // -0.0 counted with +0.0, as the order key has it
        mloc = fmaxf(mloc, y);
        const uint32_t u = __float_as_uint(y);
        const uint32_t m = min((u >> 16) & 0x7fffu, kMagWords);
        atomicAdd(reinterpret_cast<uint32_t*>(hb + (m << 2)), 1u + (u >> 31) * 0xffffu);
      });
    });
  }
  // The serial phases between the passes run at a raised wave priority: the
  // other row on the CU is streaming and tolerates the delay, these phases do not.
  __builtin_amdgcn_s_setprio(2);
  const float M = block_max_f<kFT>(mloc, sh.red_f);  // ends after a barrier

  // ---- the occupied bins as a list in ascending order ----
  // Thread t owns table words kFWPT*t .. kFWPT*t + kFWPT-1 (magnitudes); the
  // ascending order is the negative values by descending magnitude (threads
  // and words in reverse), then the positive ones by ascending magnitude.
  // Entries (count << 16 | 16-bit order key) are written over the table.
  const uint32_t L0 = (uint32_t)tid * (uint32_t)kFWPT;
  uint32_t wd[kFWPT];
  uint32_t cn = 0, cp = 0, zn = 0, zp = 0;
#pragma unroll
  for (int w = 0; w < kFWPT; ++w) {
    wd[w] = sh.u.hist[L0 + w];
    cp += wd[w] & 0xffffu;
    cn += wd[w] >> 16;
    zp += (wd[w] & 0xffffu) != 0u ? 1u : 0u;
    zn += (wd[w] >> 16) != 0u ? 1u : 0u;
  }
  const uint32_t ovf = sh.u.hist[kMagWords];
  const uint32_t va[4] = {cn, cp, zn, zp};
  uint32_t ea[4], ta[4];
  block_scan1(va, ea, ta, sh.ru_a);
  const uint32_t ntot = ta[0], ptot = ta[1], nzn = ta[2], nzp = ta[3], ezn = ea[2], ezp = ea[3];
  const uint32_t N = nzn + nzp;
  // a 16-bit count that wrapped loses a multiple of 65536 from the total
  if (ntot + ptot != (uint32_t)V || ovf != 0u || N > (uint32_t)kFTable) {
    flag_row(P, row);
    return;
  }
  {
    uint32_t at = nzn - ezn - zn;  // negative entries of later threads come first
#pragma unroll
    for (int w = kFWPT - 1; w >= 0; --w) {
      const uint32_t c = wd[w] >> 16;
      if (c != 0u) sh.u.list[at++] = (c << 16) | (0x7fffu - (L0 + (uint32_t)w));
    }
    at = nzn + ezp;
#pragma unroll
    for (int w = 0; w < kFWPT; ++w) {
      const uint32_t c = wd[w] & 0xffffu;
      if (c != 0u) sh.u.list[at++] = (c << 16) | (0x8000u | (L0 + (uint32_t)w));
    }
  }
  __syncthreads();
  // each thread takes a contiguous share of the list
  const uint32_t per = (N + kFT - 1) / kFT;
  const uint32_t i0 = min(N, (uint32_t)tid * per), i1 = min(N, i0 + per);

  // ---- the k-th largest value's bin ----
  const uint32_t k_eff = P.top_k > 0 ? (uint32_t)P.top_k : (uint32_t)V;
  const uint32_t pos0 = (uint32_t)V - k_eff;  // its ascending position
  {
    uint32_t cs = 0;
    for (uint32_t i = i0; i < i1; ++i) cs += sh.u.list[i] >> 16;
    const uint32_t vb[1] = {cs};
    uint32_t eb[1], tb[1];
    block_scan1(vb, eb, tb, sh.ru_b);
    uint32_t at = eb[0];
    for (uint32_t i = i0; i < i1; ++i) {
      const uint32_t e = sh.u.list[i], c = e >> 16;
      if (pos0 >= at && pos0 < at + c) {
        sh.bk16 = e & 0xffffu;
        sh.kprime = at + c - pos0;
        sh.cbk = c;
      }
      at += c;
    }
  }
  __syncthreads();
  const uint32_t lo16 = sh.bk16, kprime = sh.kprime, cbk = sh.cbk;
  if (lo16 == 0xffffffffu) {
    flag_row(P, row);
    return;
  }
  const bool partial = kprime < cbk;  // some values of the bin fall below the k-th largest
  const uint32_t top16 = okey(M) >> 16;
  const float cut = P.cut;

  // ---- the bracket of the top-p cut ----
  uint32_t B1 = lo16, B2 = lo16 - 1u;  // no top-p: nothing bracketed
  if (P.has_p) {
    double sl = 0.0, sh_ = 0.0;
    for (uint32_t i = i0; i < i1; ++i) {
      const uint32_t e = sh.u.list[i], k16 = e & 0xffffu, c = e >> 16;
      if (k16 < lo16) continue;
      double elo, ehi;
      bin_bounds(k16, M, elo, ehi);
      sl += (double)(k16 == lo16 ? kprime : c) * elo;
      sh_ += (double)c * ehi;
    }
    const double vs[2] = {sl, sh_};
    double es[2], ts[2];
    block_scan1(vs, es, ts, sh.rd_a);
    const double Zlo = ts[0], Zhi = ts[1];
    double al = es[0], ah = es[1];
    // B1 = the last bin whose boundary's upper bound U = ah / (ah + Zlo - al)
    // is <= cut; B2 = the first bin after which the lower bound
    // L = al / (al + Zhi - ah) exceeds the cut by more than the fp32 rounding
    const double cutd = (double)cut, cutp = (double)cut * (1.0 + 1.0 / 4194304.0);
    uint32_t my1 = 0u, my2 = 0xffffffffu;
    for (uint32_t i = i0; i < i1; ++i) {
      const uint32_t e = sh.u.list[i], k16 = e & 0xffffu, c = e >> 16;
      if (k16 < lo16) continue;
      if (ah <= cutd * (ah + fmax(Zlo - al, 0.0))) my1 = k16;
      double elo, ehi;
      bin_bounds(k16, M, elo, ehi);
      al += (double)(k16 == lo16 ? kprime : c) * elo;
      ah += (double)c * ehi;
      if (my2 == 0xffffffffu && al > cutp * (al + fmax(Zhi - ah, 0.0))) my2 = k16;
    }
    // one LDS atomic per wave (same-address LDS atomics are serialised)
    my1 = wave_max_u32(my1);
    my2 = wave_min_u32(my2);
    if ((tid & 63) == 0) {
      if (my1 != 0u) atomicMax(&sh.b1, my1);
      if (my2 != 0xffffffffu) atomicMin(&sh.b2, my2);
    }
    __syncthreads();
    B1 = sh.b1;
    B2 = sh.b2 == 0xffffffffu ? top16 : sh.b2;
    if (B1 < lo16 || B2 < B1) {
      flag_row(P, row);
      return;
    }
  }
  // values counted as kept above the bracket (the k-th largest value's bin
  // excepted when it is collected)
  uint32_t na = 0;
  for (uint32_t i = i0; i < i1; ++i) {
    const uint32_t e = sh.u.list[i], k16 = e & 0xffffu;
    if (k16 + 1u > B2 + 1u && !(partial && k16 == lo16)) na += e >> 16;
  }
  const uint32_t nabove = block_total1(na, sh.ru_c);
  __syncthreads();  // the list is read for the last time above

  // ---- pass 2 ----
  auto vstart = [](uint32_t k16) { return from_okey(k16 << 16); };  // a bin's smallest value
  const bool topk = k_eff < (uint32_t)V;
  const float vinc = vstart(partial ? lo16 + 1u : lo16);
  const float vb1 = P.has_p ? vstart(B1) : -INFINITY;
  const float vb2e = P.has_p ? vstart(B2 + 1u) : -INFINITY;
  const float vlo = partial ? vstart(lo16) : INFINITY;
  const float vloe = partial ? vstart(lo16 + 1u) : INFINITY;
  double zall = 0.0, db = 0.0;
  __builtin_amdgcn_s_setprio(0);
  with_t(P.has_t, [&](auto ht) {
    constexpr bool HT = decltype(ht)::value;
    if (topk) pass2<true, HT>(x, V, P, sh, M, vinc, vb1, vb2e, vlo, vloe, zall, db);
    else pass2<false, HT>(x, V, P, sh, M, vinc, vb1, vb2e, vlo, vloe, zall, db);
  });
  __builtin_amdgcn_s_setprio(2);
  double zd[2] = {zall, db};
  block_sum1(zd, sh.rd_b);
  const double zt = zd[0], dbt = zd[1];
  {
    // the waves' segments moved to the front as one array: every thread reads
    // its entries (at most kCompact) into registers, then writes them back
    uint32_t off[kFW + 1];
    off[0] = 0u;
    bool over = false;
#pragma unroll
    for (int w = 0; w < kFW; ++w) {
      over = over || sh.wcnt[w] > (uint32_t)kWaveCap;
      off[w + 1] = off[w] + min(sh.wcnt[w], (uint32_t)kWaveCap);
    }
    if (over) {
      flag_row(P, row);
      return;
    }
    const uint32_t n = off[kFW];
    constexpr int kCompact = (kFCand + kFT - 1) / kFT;
    uint64_t tmp[kCompact];
#pragma unroll
    for (int k = 0; k < kCompact; ++k) {
      const uint32_t v = (uint32_t)tid + (uint32_t)(k * kFT);
      tmp[k] = 0ull;
      if (v < n) {
        uint32_t w = 0u, base = 0u;
#pragma unroll
        for (int q = 1; q < kFW; ++q) {
          const bool past = v >= off[q];
          w = past ? (uint32_t)q : w;
          base = past ? off[q] : base;
        }
        tmp[k] = sh.u.cand[w * (uint32_t)kWaveCap + (v - base)];
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kCompact; ++k) {
      const uint32_t v = (uint32_t)tid + (uint32_t)(k * kFT);
      if (v < n) sh.u.cand[v] = tmp[k];
    }
    if (tid == 0) sh.ncand = n;
    __syncthreads();
  }

  // ---- the k-th largest value among the collected values of its bin ----
  uint32_t thr32 = lo16 << 16;
  if (partial) {
    const int lane = tid & 63;
    uint32_t need = kprime, pre = lo16 << 16;
    for (int shift = 8; shift >= 0; shift -= 8) {
      for (int i = tid; i < 256; i += kFT) sh.hc[i] = 0u;
      __syncthreads();
      for_cands(sh, [&](uint64_t c) {
        const uint32_t k32 = (uint32_t)(c >> 32);
        if ((k32 >> (shift + 8)) == (pre >> (shift + 8))) atomicAdd(&sh.hc[(k32 >> shift) & 255u], 1u);
      });
      __syncthreads();
      if (tid < kWave) {
        // counts from the top digit down: the digit holding the need-th largest
        const int lr = 63 - lane;  // lane lane visits digits 4*lr+3 .. 4*lr
        uint32_t sc[4], lt = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sc[j] = sh.hc[4 * lr + 3 - j];
          lt += sc[j];
        }
        uint32_t c = wave_scan_dpp(lt) - lt;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (c < need && c + sc[j] >= need) {
            sh.sel[2] = (uint32_t)(4 * lr + 3 - j);
            sh.sel[3] = need - c;
          }
          c += sc[j];
        }
      }
      __syncthreads();
      pre |= sh.sel[2] << shift;
      need = sh.sel[3];
      __syncthreads();
    }
    thr32 = pre;
  }
  auto in_kbin = [&](uint32_t k32) { return partial && (k32 >> 16) == lo16; };
  auto in_bracket = [&](uint32_t k32) {
    const uint32_t k16 = k32 >> 16;
    return k16 >= B1 && k16 <= B2;
  };

  // ---- the cut ----
  uint32_t ckey = thr32, cidx = 0u;  // top-k alone: every value >= thr kept
  float inv = 0.f;
  if (P.has_p) {
    // the normaliser: the kept-k values of the partly kept bin join zall
    double zk = 0.0;
    for_cands(sh, [&](uint64_t c) {
      const uint32_t k32 = (uint32_t)(c >> 32);
      if (in_kbin(k32) && k32 >= thr32) zk += (double)exp_le0(from_okey(k32) - M);
    });
    const double Z = zt + block_total1(zk, sh.rd_c);
    inv = 1.0f / (float)Z;
    // the mass below the bracket: the collected kept-k values of that bin
    // below B1 exactly, the others as inv * dbt within 2^-24 relative
    double dk = 0.0;
    for_cands(sh, [&](uint64_t c) {
      const uint32_t k32 = (uint32_t)(c >> 32);
      if (in_kbin(k32) && k32 >= thr32 && (k32 >> 16) < B1) dk += prob_of(k32, M, inv);
    });
    const double dkt = block_total1(dk, sh.rd_d);
    const double below = dbt * (double)inv;
    constexpr double kRel = 1.0 / 8388608.0;  // 2^-23 > the 2^-24 of each rounded p
    Cut cres{1, 0u, 0u};
    if (!P.f32_exact_below)
      cres = find_cut(sh, thr32, B1, B2, M, inv, dkt + below * (1.0 - kRel),
                      dkt + below * (1.0 + kRel), cut, V);
    if (cres.status == 1) {
      // ---- pass 3 (rare): the mass below the bracket summed exactly ----
      double dx = 0.0;
      __builtin_amdgcn_s_setprio(0);
      with_t(P.has_t, [&](auto ht) {
        stream_row<kUB, decltype(ht)::value>(x, V, P.rT, [&](float y, uint32_t, bool valid) {
          const bool below_b1 = valid && y >= vinc && y < vb1;
          dx += below_b1 ? (double)(exp_le0(y - M) * inv) : 0.0;
        });
      });
      __builtin_amdgcn_s_setprio(2);
      const double d = dkt + block_total1(dx, sh.rd_e);
      cres = find_cut(sh, thr32, B1, B2, M, inv, d, d, cut, V);
    }
    int st = cres.status;
    ckey = cres.key;
    cidx = cres.idx;
    if (st == 2) {
      // no cumulative mass exceeds the cut: only the last element is kept, the
      // maximum with the largest index (it is collected when B2 is the top bin)
      if (B2 != top16) {
        st = 3;
      } else {
        uint64_t best = 0ull;
        for_cands(sh, [&](uint64_t c) {
          if ((uint32_t)(c >> 32) >= thr32 && c > best) best = c;
        });
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
          const uint64_t o = __shfl_xor(best, off, kWave);
          best = o > best ? o : best;
        }
        if (tid == 0) sh.best = 0ull;
        __syncthreads();
        if ((tid & 63) == 0) atomicMax(&sh.best, (unsigned long long)best);
        __syncthreads();
        ckey = (uint32_t)(sh.best >> 32);
        cidx = (uint32_t)sh.best;
        st = 0;
      }
    }
    if (st != 0) {
      flag_row(P, row);
      return;
    }
  }

  // ---- the kept set's count and sum ----
  // kept: every value above the bracket (zt - dbt - the bracket's kept-k
  // values), and the collected values from the cut on
  const uint64_t ck = ((uint64_t)ckey << 32) | cidx;
  double sbr = 0.0, sk = 0.0;
  uint32_t nk = 0u;
  for_cands(sh, [&](uint64_t c) {
    const uint32_t k32 = (uint32_t)(c >> 32);
    const double e = (double)exp_le0(from_okey(k32) - M);
    if (in_bracket(k32) && !in_kbin(k32)) sbr += e;
    if (k32 >= thr32 && c >= ck) {
      sk += e;
      ++nk;
    }
  });
  double sf[2] = {sbr, sk};
  block_sum1(sf, sh.rd_f);
  const double S = (zt - dbt - sf[0]) + sf[1];
  const uint32_t n_kept = nabove + block_total1(nk, sh.ru_d);
  if (tid == 0) {
    const float logsum = logf((float)S);
    const float v_cut = from_okey(ckey);
    const int32_t i_cut = (int32_t)cidx;
    RowInfo ri;
    ri.m = M;
    ri.logsum = logsum;
    ri.v_cut = v_cut;
    ri.i_cut = i_cut;
    ri.n_kept = (int32_t)n_kept;
    ri.flags = kFlagNoKeptList;
    P.info[row] = ri;
    if (P.out != nullptr) {
      float lp = -INFINITY;
      if (t >= 0 && t < V && kept_lex(yt, t, v_cut, i_cut)) lp = (yt - M) - logsum;
      P.out[row] = lp;
    }
  }
}

}  // namespace

int launch_f32_rows(const FilterParams& P, int64_t rows, hipStream_t st) {
  hipLaunchKernelGGL(filter_f32_kernel, dim3((unsigned)rows), dim3(kFT), 0, st, P);
  return check_launch("filter_f32_kernel");
}

}  // namespace mirl

// Filtered-logprob forward for 16-bit logits (bf16 / fp16) from an exact
// count table of the row's values: the general path of the filter for top-p
// without top-k, k > 1024, and rows the fast path flagged.
//
// Semantics: those of topk_filter.hip (reference
// nemo_rl/algorithms/logits_sampling_utils.py:111-212 and
// nemo_rl/distributed/model_utils.py:382-432).  The kept set is a suffix of the
// ascending (value, index) order, described by the cut (v_cut, i_cut).
//
// One 1024-thread workgroup per row reads the row with 16-byte nontemporal
// loads.  Every raw value is counted into a table of 65536 16-bit counts in
// LDS (128 KB), indexed by an order-preserving key of the raw bits; the values
// that occur are the table's non-empty entries, and the value y = dtype(x * rT)
// of an entry is computed from its key.  So the top-k value, the normaliser,
// the cumulative probability in ascending order and the kept set's
// log-sum-exp all follow from the table:
//   top-k:  suffix counts over the keys give the k-th largest value;
//   Z:      sum over kept-k keys of count * exp(y - m);
//   top-p:  masses count * p(y) summed in key order give the cumulative
//           probability at the end of every entry; the cut is the first
//           element at which it passes the threshold.  With fp32 decisions the
//           sum is exact in double and rounded to fp32, as the reference's
//           double-accumulated cumsum is.  With 16-bit decisions the
//           reference accumulates the dtype-rounded probabilities one at a
//           time in fp32: the exact sum plus a rigorous bound on that
//           sequence's rounding (zero inside a binade when the addend is a
//           multiple of the accumulator's ulp, half an ulp per binade crossing
//           or per addition otherwise) decides the cut for almost every row;
//           a row where the bound leaves the cut undecided is walked exactly
//           by one wave (additions of equal values inside one binade are
//           applied in closed form).
//
// filter_compact_kernel (first) lists the occupied keys once, with their y and
// exp(y - m), and works over contiguous shares of that list; it leaves the
// index cut inside the tied values in rank form and writes no kept list.
// filter_hist_kernel (for the rows the compact kernel flags) works over the
// table itself, each thread owning 64 consecutive keys; a second sweep over
// the row finds the index cut (the r-th smallest index among the tied
// values), a third writes the kept list of rows with at most
// MIRL_FILTER_KEEP_CAP kept entries, and counts of 65536 or more (which wrap
// the 16-bit entries, so the total differs from V) are repaired by two more
// sweeps that count the affected 256-key blocks exactly.

#include "filter.h"

namespace mirl {
namespace {

constexpr int kHT = 1024;          // threads per row
constexpr int kHW = kHT / 64;      // waves per row
constexpr int kHistWords = 32768;  // 65536 16-bit counts
constexpr int kOvfSlots = 8;       // 256-key blocks with exact 32-bit counts

struct HistShared {
  uint32_t hist[kHistWords];
  uint32_t ovf_cnt[kOvfSlots * 256];
  uint32_t coarse[256];
  uint32_t tcnt[kHT];  // elements per thread's key range
  double red_d[kHW * 4];
  uint32_t red_u[kHW * 4];
  uint32_t ovf_block[kOvfSlots];
  int novf;
  int first_lo, first_hi;
  uint32_t key_lo, pos_lo, key_hi, pos_hi;
  uint32_t kth_key;
  int walk_hit;
  int32_t elem_index;
  int nk;
};

template <class E>
__device__ __forceinline__ uint32_t bits16(typename E::raw v) {
  return (uint32_t)__builtin_bit_cast(uint16_t, v);
}
template <class E>
__device__ __forceinline__ float value16(uint32_t r) {
  if constexpr (std::is_same<E, BF16>::value)
    return __uint_as_float(r << 16);
  else
    return (float)__builtin_bit_cast(_Float16, (uint16_t)r);
}
template <class E>
__device__ __forceinline__ uint32_t raw_of_value16(float f) {
  return bits16<E>(E::from_float(f));
}
// Order-preserving key of raw 16-bit float bits; -0 is counted as +0.
__device__ __forceinline__ uint32_t okey16(uint32_t r) {
  r &= 0xffffu;
  if (r == 0x8000u) r = 0u;
  return (r & 0x8000u) ? (~r & 0xffffu) : (r | 0x8000u);
}
__device__ __forceinline__ uint32_t raw_of_okey16(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
}

// Physical table word of logical word L (= key >> 1).  Thread t owns logical
// words 32t .. 32t + 31 (keys 64t .. 64t + 63); their order inside the block is
// rotated by t / 2 so that the 64 lanes of a wave reading their own word w hit
// 64 different banks.
__device__ __forceinline__ uint32_t hword(uint32_t L) {
  const uint32_t t = L >> 5;
  return (t << 5) | (((L & 31u) + (t >> 1)) & 31u);
}

template <class T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const T o = __shfl_up(v, off, 64);
    if (lane >= off) v += o;
  }
  return v;
}

// Exclusive prefix over the workgroup (NW waves) in thread order; *total = the sum.
template <class T, int NW = kHW>
__device__ T block_excl_scan(T v, T* red, T* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const T inc = wave_incl_scan(v);
  T ex = __shfl_up(inc, 1, 64);
  if (lane == 0) ex = T(0);
  __syncthreads();
  if (lane == 63) red[wv] = inc;
  __syncthreads();
  T base = T(0), tot = T(0);
  for (int w = 0; w < NW; ++w) {
    const T s = red[w];
    if (w < wv) base += s;
    tot += s;
  }
  *total = tot;
  return base + ex;
}

template <class T, int N, int NW = kHW>
__device__ void block_sum_n(T (&v)[N], T* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v[i] += __shfl_xor(v[i], off, 64);
  __syncthreads();
  if (lane == 0)
#pragma unroll
    for (int i = 0; i < N; ++i) red[i * NW + wv] = v[i];
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    T s = T(0);
    for (int w = 0; w < NW; ++w) s += red[i * NW + w];
    v[i] = s;
  }
}

template <int NW = kHW>
__device__ uint32_t block_max_u(uint32_t v, uint32_t* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int w = 1; w < NW; ++w) r = max(r, red[w]);
  return r;
}

// Workgroup-wide exclusive scan (thread order) and total with one barrier.
// `red` (NW entries) must be used by no other reduction of the same kernel
// invocation, so no barrier is needed before it is written.
template <class T, int NW>
__device__ __forceinline__ T block_excl_scan1(T v, T* red, T* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const T inc = wave_scan_dpp(v);
  if (lane == 63) red[wv] = inc;
  __syncthreads();
  T base = T(0), tot = T(0);
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const T s = red[w];
    base += (w < wv) ? s : T(0);
    tot += s;
  }
  *total = tot;
  return base + inc - v;
}
// Workgroup-wide sums of N values with one barrier (`red`: N * NW entries,
// used by no other reduction of the same kernel invocation).
template <class T, int N, int NW>
__device__ __forceinline__ void block_sum1(T (&v)[N], T* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const T inc = wave_scan_dpp(v[i]);
    if (lane == 63) red[i * NW + wv] = inc;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    T s = T(0);
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[i * NW + w];
    v[i] = s;
  }
}

// Relative distance within which the fp32 running sum S is kept from the
// exact sum X: the bound below assumes |S - X| <= kSlack * X, which the
// certification checks as it goes.
constexpr double kSlack = 1.0 / 4096.0;

// Bound on the rounding of n fp32 additions S <- fl(S + p) that take the
// exact running sum from X0 to X1 (> 0), with S within kSlack * X of X.  S
// stays in [X0 (1 - kSlack), X1 (1 + kSlack)], below 2^(e + 1) for
// e = ilogb(X1 (1 + kSlack)), where the ulp is u.  An addend that is a
// multiple of u adds exactly inside each binade and can round only where S
// enters a new binade: once per power of two in that interval, by at most
// half that binade's ulp (<= u / 2).  Any other addend may round on every
// addition, by at most u / 2.
__device__ double run_error_bound(uint32_t n, double p, double X0, double X1) {
  if (p == 0.0 || n == 0u) return 0.0;
  const double hi = X1 * (1.0 + kSlack);
  const int e = ilogb(hi);
  const int eu = (e < -126 ? -126 : e) - 23;
  const double u = ldexp(1.0, eu);
  const double q = ldexp(p, -eu);
  if (q == floor(q)) {
    // the first addition to an empty sum is exact (S = p); binades are entered above it
    const double lo = X0 > 0.0 ? X0 * (1.0 - kSlack) : p;
    const int crossings = e - ilogb(lo);
    return (double)crossings * 0.5 * u;
  }
  return (double)n * 0.5 * u;
}

// Whether the non-negative integer-valued double v is even (every double of
// 2^53 or more is).
__device__ __forceinline__ bool even_int(double v) {
  return v >= 9007199254740992.0 || (((uint64_t)v) & 1u) == 0u;
}

// n additions S <- fl32(S + p) of one value p >= 0.  Returns true when a
// partial sum reaches B (S >= B); *at is then the 1-based addition that did.
// Inside the binade [2^e, 2^(e+1)) of S every addition adds p rounded to the
// binade's ulp u (to nearest, a tie going to the even multiple of u), so runs
// of additions that stay inside the binade are applied at once.
__device__ bool seq_add_run(float& S, float p, uint32_t n, float B, uint32_t* at) {
  uint32_t done = 0;
  while (done < n) {
    if (S == 0.f || n - done <= 2u) {
      S = S + p;
      ++done;
      if (S >= B) {
        *at = done;
        return true;
      }
      continue;
    }
    int eS = ilogbf(S);
    if (eS < -126) eS = -126;
    const int eu = eS - 23;
    const double Su = ldexp((double)S, -eu);  // integer < 2^24
    const double Tu = 16777216.0;             // 2^(eS + 1) in units of u
    const double q = ldexp((double)p, -eu);
    const double fq = floor(q);
    double d;
    if (q == fq) {
      d = q;
    } else if (q - fq != 0.5) {
      d = (q - fq < 0.5) ? fq : fq + 1.0;
    } else if (even_int(Su)) {
      // a tie from an even multiple: rounding to even keeps S even
      d = even_int(fq) ? fq : fq + 1.0;
    } else {
      S = S + p;  // a tie from an odd multiple rounds up to an even one
      ++done;
      if (S >= B) {
        *at = done;
        return true;
      }
      continue;
    }
    if (d == 0.0) return false;  // the remaining additions leave S unchanged
    const double smax = floor((Tu - 1.0 - Su) / d);  // additions that stay in the binade
    const double rem = (double)(n - done);
    const double s = smax < rem ? smax : rem;
    const double Bu = ldexp((double)B, -eu);  // B > S >= 2^eS: an integer in units of u
    if (s > 0.0 && Su + s * d >= Bu) {
      const double need = ceil((Bu - Su) / d);
      S = (float)ldexp(Su + need * d, eu);
      done += (uint32_t)need;
      *at = done;
      return true;
    }
    S = (float)ldexp(Su + s * d, eu);
    done += (uint32_t)s;
    if (done < n && s == smax) {  // the next addition leaves the binade
      S = S + p;
      ++done;
      if (S >= B) {
        *at = done;
        return true;
      }
    }
  }
  return false;
}

// One row of filter_hist_kernel.  WALK = false: a row whose 16-bit cut the
// bound leaves undecided is flagged again (info.flags bit 0) and left to the
// WALK = true launch, which decides it by the exact sequence.
template <class E, int NV, bool WALK>
__device__ __forceinline__ void hist_row(const FilterParams& P, const int64_t row) {
  using raw = typename E::raw;
  __shared__ HistShared sh;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  // (the thread index passes an empty asm once per row, so that nothing
  // derived from it is kept across the rows of filter_hist_kernel's loop)
  int tid_ = threadIdx.x;
  asm volatile("" : "+v"(tid_));
  const int tid = tid_, lane = tid & 63;
  const int64_t V = P.V;
  const RowSpan<E> sp(x, V);
  const vu4* xv = reinterpret_cast<const vu4*>(x + sp.head);
  const int64_t nvec = sp.nvec;

  // ---- pass 1: the row into registers, then every value into the table ----
  vu4 q[NV > 0 ? NV : 1];
  if constexpr (NV > 0) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int64_t v = tid + (int64_t)j * kHT;
      if (v < nvec) q[j] = __builtin_nontemporal_load(xv + v);
    }
  }
  const bool has_h = tid < sp.head;
  const bool has_tl = sp.tail0 + tid < V;
  const uint32_t hraw = has_h ? bits16<E>(x[tid]) : 0u;
  const uint32_t traw = has_tl ? bits16<E>(x[sp.tail0 + tid]) : 0u;
  {
    vu4* h4 = reinterpret_cast<vu4*>(sh.hist);
    for (int i = tid; i < kHistWords / 4; i += kHT) h4[i] = vu4{0u, 0u, 0u, 0u};
  }
  if (tid == 0) {
    sh.novf = 0;
    sh.first_lo = kHT;
    sh.first_hi = kHT;
    sh.nk = 0;
    sh.walk_hit = 0;
    sh.elem_index = 0;
    sh.kth_key = 0;
    sh.key_lo = sh.pos_lo = sh.key_hi = sh.pos_hi = 0;
  }
  __syncthreads();

  // calls f(index, raw bits) for every element of this thread, in index order
  // within each of its segments: head element, register/vector slots, tail
  auto sweep = [&](auto&& f) {
    if (has_h) f((int64_t)tid, hraw);
    if constexpr (NV > 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int64_t v = tid + (int64_t)j * kHT;
        if (v < nvec) {
          const uint32_t w[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
          const int64_t base = sp.head + v * 8;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f(base + 2 * e, w[e] & 0xffffu);
            f(base + 2 * e + 1, w[e] >> 16);
          }
        }
      }
    } else {
      // batches of 8 independent loads per lane
      constexpr int UB = 8;
      for (int64_t v0 = tid; v0 < nvec; v0 += (int64_t)UB * kHT) {
        vu4 t[UB];
#pragma unroll
        for (int u = 0; u < UB; ++u) {
          const int64_t v = v0 + (int64_t)u * kHT;
          if (v < nvec) t[u] = __builtin_nontemporal_load(xv + v);
        }
#pragma unroll
        for (int u = 0; u < UB; ++u) {
          const int64_t v = v0 + (int64_t)u * kHT;
          if (v >= nvec) break;
          const uint32_t w[4] = {t[u].x, t[u].y, t[u].z, t[u].w};
          const int64_t base = sp.head + v * 8;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            f(base + 2 * e, w[e] & 0xffffu);
            f(base + 2 * e + 1, w[e] >> 16);
          }
        }
      }
    }
    if (has_tl) f(sp.tail0 + tid, traw);
  };

  uint32_t kmax = 0;
  sweep([&](int64_t, uint32_t rw) {
    const uint32_t k = okey16(rw);
    atomicAdd(&sh.hist[hword(k >> 1)], (k & 1u) ? 0x10000u : 1u);
    kmax = max(kmax, k);
  });
  const uint32_t kmx = block_max_u(kmax, sh.red_u);  // its barriers complete the table

  // ---- the table: counts, repaired where 16-bit entries wrapped ----------
  const uint32_t k0 = (uint32_t)tid * 64u;
  uint32_t ct = 0;
#pragma unroll 4
  for (int w = 0; w < 32; ++w) {
    const uint32_t word = sh.hist[hword(tid * 32 + w)];
    ct += (word & 0xffffu) + (word >> 16);
  }
  {
    uint32_t tot[1] = {ct};
    block_sum_n<uint32_t, 1>(tot, sh.red_u);
    if (tot[0] != (uint32_t)V) {
      // some value occurs 65536 times or more: find its 256-key blocks by exact
      // block counts, then count those blocks exactly
      for (int i = tid; i < 256; i += kHT) sh.coarse[i] = 0u;
      __syncthreads();
      sweep([&](int64_t, uint32_t rw) { atomicAdd(&sh.coarse[okey16(rw) >> 8], 1u); });
      __syncthreads();
      if (tid < 256) {
        uint32_t fine = 0;
        for (int i = 0; i < 128; ++i) {
          const uint32_t word = sh.hist[hword(tid * 128 + i)];
          fine += (word & 0xffffu) + (word >> 16);
        }
        if (fine != sh.coarse[tid]) {
          const int s = atomicAdd(&sh.novf, 1);
          if (s < kOvfSlots) sh.ovf_block[s] = (uint32_t)tid;
        }
      }
      __syncthreads();
      const int nb = sh.novf;
      if (nb > kOvfSlots) {  // not reachable for V <= kHistMaxV
        if (tid == 0) {
          RowInfo ri{};
          ri.flags = 2;
          P.info[row] = ri;
        }
        return;
      }
      for (int i = tid; i < nb * 256; i += kHT) sh.ovf_cnt[i] = 0u;
      __syncthreads();
      sweep([&](int64_t, uint32_t rw) {
        const uint32_t k = okey16(rw);
        for (int s = 0; s < nb; ++s)
          if (sh.ovf_block[s] == (k >> 8)) atomicAdd(&sh.ovf_cnt[s * 256 + (k & 255u)], 1u);
      });
      __syncthreads();
    }
  }
  const int novf = sh.novf;
  auto kcount = [&](uint32_t k) -> uint32_t {
    if (novf > 0) {
      for (int s = 0; s < novf; ++s)
        if (sh.ovf_block[s] == (k >> 8)) return sh.ovf_cnt[s * 256 + (k & 255u)];
    }
    return (sh.hist[hword(k >> 1)] >> ((k & 1u) << 4)) & 0xffffu;
  };
  // f(key, count) over this thread's 64 keys with a non-zero count, ascending
  auto for_range = [&](auto&& f) {
#pragma unroll 1
    for (int w = 0; w < 32; ++w) {
      const uint32_t word = sh.hist[hword(tid * 32 + w)];
      if (word == 0u && novf == 0) continue;
      const uint32_t ka = k0 + 2u * (uint32_t)w;
      const uint32_t na = novf ? kcount(ka) : (word & 0xffffu);
      const uint32_t nb = novf ? kcount(ka + 1u) : (word >> 16);
      if (na) f(ka, na);
      if (nb) f(ka + 1u, nb);
    }
  };
  if (novf > 0) {
    ct = 0;
    for_range([&](uint32_t, uint32_t n) { ct += n; });
  }
  sh.tcnt[tid] = ct;

  auto yk = [&](uint32_t k) { return scaled<E>(value16<E>(raw_of_okey16(k)), P); };
  // smallest key in [lo, hi] whose value is >= y (hi + 1 if none)
  auto lowest_ge = [&](uint32_t lo, uint32_t hi, float y) {
    uint32_t a = lo, c = hi + 1u;
    while (a < c) {
      const uint32_t mid = (a + c) >> 1;
      if (yk(mid) >= y) c = mid; else a = mid + 1u;
    }
    return a;
  };
  // largest key in [lo, hi] whose value is <= y (lo - 1 if none)
  auto highest_le = [&](uint32_t lo, uint32_t hi, float y) {
    uint32_t a = lo, c = hi + 1u;
    while (a < c) {
      const uint32_t mid = (a + c) >> 1;
      if (yk(mid) <= y) a = mid + 1u; else c = mid;
    }
    return a - 1u;
  };
  const float m = yk(kmx);

  // ---- top-k: the k-th largest value from suffix counts ---------------------
  uint32_t thr_key = 0;
  float y_thr = -INFINITY;
  if (P.top_k > 0) {
    __syncthreads();
    const int rr = kHT - 1 - tid;  // thread tid scans key range rr (descending order)
    const uint32_t crev = sh.tcnt[rr];
    uint32_t tot;
    const uint32_t above = block_excl_scan<uint32_t>(crev, sh.red_u, &tot);
    const uint32_t kk = (uint32_t)P.top_k;
    if (above < kk && kk <= above + crev) {
      uint32_t acc = above;
#pragma unroll 1
      for (int i = 63; i >= 0; --i) {
        const uint32_t key = (uint32_t)rr * 64u + (uint32_t)i;
        acc += kcount(key);
        if (acc >= kk) {
          sh.kth_key = key;
          break;
        }
      }
    }
    __syncthreads();
    y_thr = yk(sh.kth_key);
    thr_key = lowest_ge(0u, sh.kth_key, y_thr);
  }

  // ---- normaliser over the kept-k values ------------------------------------
  double zsum[1] = {0.0};
  for_range([&](uint32_t key, uint32_t n) {
    if (key >= thr_key) zsum[0] += (double)n * (double)expf(yk(key) - m);
  });
  block_sum_n<double, 1>(zsum, sh.red_d);
  const float Z = (float)zsum[0];

  // ---- top-p cut -----------------------------------------------------------
  // (cut_key, cut_pos): the cut is the cut_pos-th element (1-based) of key
  // cut_key in the ascending order; no cut keeps the maximum only
  bool have_cut = false, walked = false;
  uint32_t cut_key = 0, cut_pos = 0;
  if (P.has_p) {
    const float inv = 1.0f / Z;
    auto pmass = [&](uint32_t key) -> double {
      const float e = expf(yk(key) - m);
      return P.dec16 ? (double)round_trip<E>(e / Z) : (double)(e * inv);
    };
    double mt = 0.0;
    for_range([&](uint32_t key, uint32_t n) {
      if (key >= thr_key) mt += (double)n * pmass(key);
    });
    double mtot;
    const double X0 = block_excl_scan<double>(mt, sh.red_d, &mtot);
    // first addition t in [1, n] of a run X + t p for which hit() holds (hit(X + n p) is true)
    auto first_in_run = [&](double X, double p, uint32_t n, auto&& hit) {
      uint32_t a = 1u, c = n;
      while (a < c) {
        const uint32_t mid = a + ((c - a) >> 1);
        if (hit(X + (double)mid * p)) c = mid; else a = mid + 1u;
      }
      return a;
    };
    if (!P.dec16) {
      const float cut = P.cut;
      auto hit = [&](double X) { return (float)X > cut; };
      double X = X0;
      bool found = false;
      uint32_t fk = 0, fp = 0;
      for_range([&](uint32_t key, uint32_t n) {
        if (found || key < thr_key) return;
        const double p = pmass(key);
        if (hit(X + (double)n * p)) {
          found = true;
          fk = key;
          fp = hit(X) ? 1u : first_in_run(X, p, n, hit);
        }
        X += (double)n * p;
      });
      block_first_flagged(found, &sh.first_lo);
      __syncthreads();
      if (sh.first_lo == tid) {
        sh.key_lo = fk;
        sh.pos_lo = fp;
      }
      __syncthreads();
      have_cut = sh.first_lo < kHT;
      cut_key = sh.key_lo;
      cut_pos = sh.pos_lo;
    } else {
      // smallest fp32 S whose rounding to the dtype exceeds thr16
      const float thr = P.thr16;
      const float nxt = value16<E>(raw_of_value16<E>(thr) + 1u);
      const float mid = 0.5f * (thr + nxt);
      const float Bthr = round_trip<E>(mid) > thr ? mid : nextafterf(mid, INFINITY);
      const double Bd = (double)Bthr;
      // rounding bounds of the sequential sum, then the cut for S = X - D and X + D
      double bt = 0.0;
      {
        double X = X0;
        for_range([&](uint32_t key, uint32_t n) {
          if (key < thr_key) return;
          const double p = pmass(key);
          const double X1 = X + (double)n * p;
          bt += run_error_bound(n, p, X, X1);
          X = X1;
        });
      }
      double btot;
      const double D0 = block_excl_scan<double>(bt, sh.red_d, &btot);
      {
        double X = X0, D = D0;
        bool flo = false, fhi = false, slack_ok = true;
        uint32_t klo = 0, plo = 0, khi = 0, phi = 0;
        for_range([&](uint32_t key, uint32_t n) {
          if ((flo && fhi) || key < thr_key) return;
          const double p = pmass(key);
          const double X1 = X + (double)n * p;
          const double Db = D + run_error_bound(n, p, X, X1);
          if (Db > 0.5 * kSlack * X1) slack_ok = false;  // the bound's premise fails: walk the row
          auto hlo = [&](double v) { return v + Db >= Bd; };
          auto hhi = [&](double v) { return v - Db >= Bd; };
          if (!flo && hlo(X1)) {
            flo = true;
            klo = key;
            plo = hlo(X) ? 1u : first_in_run(X, p, n, hlo);
          }
          if (!fhi && hhi(X1)) {
            fhi = true;
            khi = key;
            phi = hhi(X) ? 1u : first_in_run(X, p, n, hhi);
          }
          X = X1;
          D = Db;
        });
        block_first_flagged(flo, &sh.first_lo);
        block_first_flagged(fhi, &sh.first_hi);
        if (!slack_ok) sh.walk_hit = -1;
        __syncthreads();
        if (sh.first_lo == tid) {
          sh.key_lo = klo;
          sh.pos_lo = plo;
        }
        if (sh.first_hi == tid) {
          sh.key_hi = khi;
          sh.pos_hi = phi;
        }
        __syncthreads();
      }
      const bool none_lo = sh.first_lo >= kHT, none_hi = sh.first_hi >= kHT;
      const bool certain = sh.walk_hit == 0 &&
                           ((none_lo && none_hi) ||
                            (!none_lo && !none_hi && sh.key_lo == sh.key_hi &&
                             sh.pos_lo == sh.pos_hi));
      if (certain) {
        have_cut = !none_hi;
        cut_key = sh.key_hi;
        cut_pos = sh.pos_hi;
      } else if constexpr (!WALK) {
        if (tid == 0) {
          RowInfo ri{};
          ri.flags = 1;
          P.info[row] = ri;
        }
        return;
      } else {
        // the exact sequence, one wave: ranges whose additions are all exact
        // and stay inside S's binade below the threshold are added at once
        walked = true;
        __syncthreads();
        if (tid < 64) {
          float S = 0.f;
          bool hit = false;
          uint32_t hk = 0, hp = 0;
          for (int t = 0; t < kHT && !hit; ++t) {
            if (sh.tcnt[t] == 0u) continue;
            const uint32_t key = (uint32_t)t * 64u + (uint32_t)lane;
            const uint32_t n = key >= thr_key ? kcount(key) : 0u;
            const float p = n ? (float)pmass(key) : 0.f;
            bool batched = false;
            if (S > 0.f) {
              int eS = ilogbf(S);
              if (eS < -126) eS = -126;
              const double qp = ldexp((double)p, 23 - eS);
              const bool exact = n == 0u || qp == floor(qp);
              double sum = (double)n * (double)p;
#pragma unroll
              for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
              const double top = ldexp(1.0, eS + 1);
              if (__ballot(!exact) == 0ull && (double)S + sum < top && (double)S + sum < Bd) {
                S = (float)((double)S + sum);
                batched = true;
              }
            }
            if (!batched) {
              uint64_t nz = __ballot(n > 0u);
              while (nz != 0ull) {
                const int l = __ffsll((long long)nz) - 1;
                nz &= nz - 1ull;
                const uint32_t nl = (uint32_t)__builtin_amdgcn_readlane((int)n, l);
                const float pl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), l));
                uint32_t at = 0;
                if (seq_add_run(S, pl, nl, Bthr, &at)) {
                  hit = true;
                  hk = (uint32_t)t * 64u + (uint32_t)l;
                  hp = at;
                  break;
                }
              }
            }
          }
          if (lane == 0) {
            sh.walk_hit = hit ? 1 : 0;
            sh.key_lo = hk;
            sh.pos_lo = hp;
          }
        }
        __syncthreads();
        have_cut = sh.walk_hit != 0;
        cut_key = sh.key_lo;
        cut_pos = sh.pos_lo;
      }
    }
  }

  // ---- the cut's value group, kept count and log-sum-exp --------------------
  uint32_t g_lo, g_hi;
  float v_cut;
  if (!P.has_p) {
    v_cut = y_thr;
    g_lo = thr_key;
    g_hi = highest_le(thr_key, 65535u, y_thr);
  } else {
    const uint32_t ck = have_cut ? cut_key : kmx;
    v_cut = yk(ck);
    g_lo = lowest_ge(thr_key, ck, v_cut);
    g_hi = highest_le(ck, 65535u, v_cut);
  }
  double sums[2] = {0.0, 0.0};      // kept mass above the group, group size (as exact doubles)
  uint32_t cnts[2] = {0u, 0u};      // elements above the group, group elements before the cut
  for_range([&](uint32_t key, uint32_t n) {
    if (key > g_hi) {
      cnts[0] += n;
      sums[0] += (double)n * (double)expf(yk(key) - m);
    } else if (key >= g_lo) {
      sums[1] += (double)n;
      if (have_cut && key < cut_key) cnts[1] += n;
    }
  });
  block_sum_n<double, 2>(sums, sh.red_d);
  block_sum_n<uint32_t, 2>(cnts, sh.red_u);
  const uint32_t n_group = (uint32_t)sums[1];
  uint32_t rcut = 0;  // group elements (in index order) before the cut
  if (P.has_p) rcut = have_cut ? cnts[1] + cut_pos - 1u : n_group - 1u;
  const uint32_t n_kept = cnts[0] + (n_group - rcut);
  const double ksum = sums[0] + (double)(n_group - rcut) * (double)expf(v_cut - m);
  const float logsum = logf((float)ksum);

  // ---- index cut inside the group: its rcut-th smallest index ---------------
  int32_t i_cut = 0;
  if (rcut > 0u) {
    auto member = [&](uint32_t rw) {
      const uint32_t k = okey16(rw);
      return k >= g_lo && k <= g_hi;
    };
    uint32_t run = 0;
    bool done = false;
    // one segment of consecutive indices per thread: base index and a bit
    // mask of its members (bit e = element base + e)
    auto segment = [&](int64_t base, uint32_t mask) {
      const uint32_t c = (uint32_t)__popc(mask);
      uint32_t tot;
      const uint32_t ex = block_excl_scan<uint32_t>(c, sh.red_u, &tot);
      if (run + tot > rcut) {
        const uint32_t want = rcut - run;
        if (ex <= want && want < ex + c) {
          uint32_t mm = mask;
          for (uint32_t i = 0; i < want - ex; ++i) mm &= mm - 1u;
          sh.elem_index = (int32_t)(base + (__ffs(mm) - 1));
        }
        done = true;
      }
      run += tot;
    };
    segment((int64_t)tid, (has_h && member(hraw)) ? 1u : 0u);
    if constexpr (NV > 0) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (done) break;
        const int64_t v = tid + (int64_t)j * kHT;
        if ((int64_t)j * kHT >= nvec) break;
        uint32_t mask = 0;
        if (v < nvec) {
          const uint32_t w[4] = {q[j].x, q[j].y, q[j].z, q[j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            mask |= member(w[e] & 0xffffu) ? (1u << (2 * e)) : 0u;
            mask |= member(w[e] >> 16) ? (2u << (2 * e)) : 0u;
          }
        }
        segment(sp.head + v * 8, mask);
      }
    } else {
      for (int64_t v0 = 0; v0 < nvec && !done; v0 += kHT) {
        const int64_t v = v0 + tid;
        uint32_t mask = 0;
        if (v < nvec) {
          const vu4 t = xv[v];
          const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            mask |= member(w[e] & 0xffffu) ? (1u << (2 * e)) : 0u;
            mask |= member(w[e] >> 16) ? (2u << (2 * e)) : 0u;
          }
        }
        segment(sp.head + v * 8, mask);
      }
    }
    if (!done) segment(sp.tail0 + tid, (has_tl && member(traw)) ? 1u : 0u);
    __syncthreads();
    i_cut = sh.elem_index;
  }

  // ---- kept list for the backward -------------------------------------------
  if (n_kept <= (uint32_t)kKeepCap) {
    int32_t* ki = P.kept_idx + row * kKeepCap;
    float* kp = P.kept_p + row * kKeepCap;
    sweep([&](int64_t j, uint32_t rw) {
      const uint32_t k = okey16(rw);
      if (k > g_hi || (k >= g_lo && j >= (int64_t)i_cut)) {
        const int s = atomicAdd(&sh.nk, 1);
        if (s < kKeepCap) {
          ki[s] = (int32_t)j;
          kp[s] = expf((yk(k) - m) - logsum);
        }
      }
    });
  }

  if (tid == 0) {
    RowInfo ri;
    ri.m = m;
    ri.logsum = logsum;
    ri.v_cut = v_cut;
    ri.i_cut = i_cut;
    ri.n_kept = (int32_t)n_kept;
    ri.flags = walked ? kFlagWalked : 0;
    P.info[row] = ri;
    if (P.out != nullptr) {
      const int64_t t = P.target[b * P.tsb + r * P.tsr];
      float lp = -INFINITY;
      if (t >= 0 && t < V) {
        const float yt = scaled<E>(E::load(x + t), P);
        if (kept_lex(yt, t, v_cut, i_cut)) lp = (yt - m) - logsum;
      }
      P.out[row] = lp;
    }
  }
}

// The rows flagged (info.flags bit 0) among this workgroup's share, rows
// blockIdx.x + k gridDim.x for k < per (<= kHT): their flags are read at once,
// the flagged rows listed in LDS and decided one after another, so that a
// launch over rows of which few or none are flagged costs a few microseconds.
template <class E, int NV, bool WALK>
__global__ __launch_bounds__(kHT) void filter_hist_kernel(FilterParams P, int64_t rows, int per) {
  __shared__ int s_n;
  __shared__ int64_t s_rows[kHT];
  const int tid = threadIdx.x;
  if (tid == 0) s_n = 0;
  __syncthreads();
  if (tid < per) {
    const int64_t row = (int64_t)blockIdx.x + (int64_t)tid * gridDim.x;
    if (row < rows && (P.info[row].flags & 1) != 0) s_rows[atomicAdd(&s_n, 1)] = row;
  }
  __syncthreads();
  // (the count and the rows are uniform: in scalar registers, as blockIdx.x
  // would be, so that the loop is not taken for a divergent one)
  const int n = __builtin_amdgcn_readfirstlane(s_n);
  for (int i = 0; i < n; ++i) {
    const uint64_t rw = (uint64_t)s_rows[i];
    const int64_t row = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(rw >> 32)) << 32) |
                                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)rw));
    hist_row<E, NV, WALK>(P, row);
    __syncthreads();  // the row's last reads of the table before the next row clears it
  }
}

// ---------------------------------------------------------------------------
// Compact form: the occupied keys as an entry list
// ---------------------------------------------------------------------------
// The table phases above evaluate y = dtype(x * rT) and exp(y - m) per occupied
// key, several times, and a thread owns 64 consecutive keys, so the occupied
// keys (a few thousand of the 65536) crowd into a few waves.  This kernel
// counts the row the same way, then lists the occupied keys in ascending
// order as entries {key | count << 16, y, exp(y - m)} over the table's
// memory, each computed once and spread over all lanes; top-k, the normaliser,
// the cut and the value group then run over contiguous shares of the list.
// The index cut inside the value group is left in rank form (the group's
// rcut-th element in index order, RowInfo.i_cut = -1 - rcut) for the
// consumers that walk the row in index order, so the row is read once; the
// target's rank is counted only when its value is the cut value.  No kept
// list is written (flags bit 2): the backward rewrites such rows whole.
// A 16-bit cut that the rounding bound leaves undecided is walked exactly over
// the list by one wave.  Rows it cannot finish (a count of 65536 or more, more
// than kEntCap occupied keys) are flagged (flags bit 0) for filter_hist_kernel.
//
// Two table geometries:
//  - CompactFull: 1024 threads, every one of the 65536 keys (fp16 logits, and
//    bf16 rows outside the window below);
//  - CompactWindow: 512 threads, the bf16 values of |x| < 512: word m (the
//    magnitude bits, m < 0x4400) counts +x in its low half and -x in its high
//    half (70 KB of counts), so two rows share a CU and one row's list phases
//    run while the other row is being counted.  Per value: an and and a clamp
//    (two values at a time), an address and an increment.  A value outside
//    the window (|x| >= 512, +-inf, NaN) lands in word 0x4400 and flags the
//    row for filter_hist_kernel.
struct CompactFull {
  static constexpr int NT = 1024;
  static constexpr uint32_t kBase = 0;      // first key of the table
  static constexpr int kWords = 32768;      // logical words (2 keys each)
  static constexpr bool kWindow = false;
  static constexpr bool kPad = true;        // one pad word per 32 (strided reads of 32 words)
  // Lean entries: the key and count only (y and exp(y - m) are formed again
  // from the key where an entry other than the thread's own is read), so that
  // an fp16 row's distinct values fit (about 14000-16000 on N(0, 1) rows of
  // 151936): at most 18 per thread.
  static constexpr bool kLean = true;
  static constexpr int kLeanCap = 18 * NT;
};
struct CompactWindow {
  static constexpr int NT = 512;
  static constexpr uint32_t kBase = 0u;     // (unused: words are indexed by magnitude)
  static constexpr int kWords = 0x4400;     // magnitudes below bf16 512.0
  static constexpr bool kWindow = true;
  static constexpr bool kPad = false;       // strided reads of 34 words: 2-way bank conflicts
  static constexpr bool kLean = false;      // 12-byte entries: key and count, y, exp(y - m)
  static constexpr int kLeanCap = 0;
};

template <class G>
struct CompactShared {
  static constexpr int kWPT = G::kWords / G::NT;          // logical words per thread
  // the table's physical words, then one word counting the values outside it
  static constexpr int kPadWords = G::kWords + (G::kPad ? G::kWords / 32 : 0) + 1;
  // entries over the same bytes: 12 bytes each, or 4 (lean)
  static constexpr int kEntCap = G::kLean ? G::kLeanCap : kPadWords / 3;
  static constexpr int kYE = G::kLean ? 1 : kEntCap;  // (unused in the lean layout)
  static constexpr int NW = G::NT / 64;
  static_assert(kWPT * G::NT == G::kWords, "table words split evenly over the threads");
  static_assert(!G::kLean || kEntCap <= kPadWords, "lean entries over the table's bytes");
  union {
    uint32_t hist[kPadWords];  // logical word L at L (+ L / 32 with padding)
    struct {
      uint32_t kc[kEntCap];
      float y[kYE];
      float e[kYE];
    } ent;
  } u;
  // one slot of NW entries per reduction of a row (each written once)
  double red_d[NW * 4];
  uint32_t red_u[NW * 9];
  uint32_t sel[4];
  int first_lo, first_hi;
  uint32_t ent_lo, pos_lo, ent_hi, pos_hi;
  int fail;
  int walk_hit;
  uint32_t walk_ent, walk_pos;
};

__device__ __forceinline__ uint32_t padded(uint32_t L) { return L + (L >> 5); }

// Order keys of the two 16-bit values of a word, in the word's halves: a
// negative value's bits inverted, a positive value's sign bit set.
__device__ __forceinline__ uint32_t okey16x2(uint32_t w) {
  const uint32_t neg = (w >> 15) & 0x00010001u;
  return w ^ ((neg * 0xffffu) | 0x80008000u);
}

// The second launch bound is the minimum number of waves per SIMD: four 128-register
// waves (two 512-thread rows per CU for the window table; one 1024-thread row for
// the full one).
template <class E, class G, bool DEC16>
__global__ __launch_bounds__(G::NT, 2048 / G::NT) void filter_compact_kernel(FilterParams P) {
  using raw = typename E::raw;
  using SH = CompactShared<G>;
  constexpr int NT = G::NT, NW = SH::NW, kWPT = SH::kWPT, kEntCap = SH::kEntCap;
  __shared__ SH sh;
  const int64_t row = blockIdx.x;
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;
  const RowSpan<E> sp(x, V);
  const vu4* xv = reinterpret_cast<const vu4*>(x + sp.head);
  const int64_t nvec = sp.nvec;

  {
    vu4* h4 = reinterpret_cast<vu4*>(sh.u.hist);
    for (int i = tid; i < SH::kPadWords / 4; i += NT) h4[i] = vu4{0u, 0u, 0u, 0u};
    for (int i = (SH::kPadWords / 4) * 4 + tid; i < SH::kPadWords; i += NT) sh.u.hist[i] = 0u;
  }
  if (tid == 0) {
    sh.first_lo = NT;
    sh.first_hi = NT;
    sh.fail = 0;
    sh.sel[0] = sh.sel[1] = sh.sel[2] = sh.sel[3] = 0u;
    sh.ent_lo = sh.pos_lo = sh.ent_hi = sh.pos_hi = 0u;
  }
  __syncthreads();
  // the target and its value, loaded while the row is counted
  int64_t t = -1;
  uint32_t xt_bits = 0u;
  if (P.out != nullptr) {
    t = P.target[b * P.tsb + r * P.tsr];
    if (t >= 0 && t < V) xt_bits = bits16<E>(x[t]);
  }

  // ---- one pass over the row: every value counted under its order key ----
  // A key outside the table (window geometry) is clamped to kLimit, whose
  // logical word kWords is the word after the table: it counts those values
  // (kLimit is even, so in its low half).  Branch-free per element.
  constexpr uint32_t kLimit = 2u * (uint32_t)G::kWords;
  auto phys = [](uint32_t L) { return G::kPad ? padded(L) : L; };
  auto count_key = [&](uint32_t k) {
    const uint32_t rel = min(k - G::kBase, kLimit);
    atomicAdd(&sh.u.hist[phys(rel >> 1)], 1u + (rel & 1u) * 0xffffu);
  };
  // two values per 32-bit word; the window layout clamps both magnitudes in
  // one packed 16-bit operation and takes byte addresses straight from them
  typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
  auto count_word = [&](uint32_t w) {
    if constexpr (G::kPad) {
      const uint32_t k2 = okey16x2(w);
      count_key(k2 & 0xffffu);
      count_key(k2 >> 16);
    } else {
      // word min(|x| bits, kWords), the sign choosing the half.  Eight VALU
      // instructions for the two values (the compiler's form took eleven):
      // each half's byte address by one shift that reads the half directly
      // (SDWA operand select), each increment 1 + sign * 0xffff by a bit
      // extract and one 24-bit multiply-add.
      const u16x2 mag = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
      const uint32_t c =
          __builtin_bit_cast(uint32_t, __builtin_elementwise_min(mag, (u16x2)(uint16_t)G::kWords));
      uint32_t alo, ahi, ilo, ihi;
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_0"
          : "=v"(alo) : "v"(c));
      asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:WORD_1"
          : "=v"(ahi) : "v"(c));
      asm("v_bfe_u32 %0, %1, 15, 1\n\tv_mad_u32_u24 %0, %0, %2, 1" : "=&v"(ilo) : "v"(w), "s"(0xffffu));
      asm("v_lshrrev_b32 %0, 31, %1\n\tv_mad_u32_u24 %0, %0, %2, 1" : "=&v"(ihi) : "v"(w), "s"(0xffffu));
      char* base = reinterpret_cast<char*>(sh.u.hist);
      atomicAdd(reinterpret_cast<uint32_t*>(base + alo), ilo);
      atomicAdd(reinterpret_cast<uint32_t*>(base + ahi), ihi);
    }
  };
  // one value (a row's unaligned head and tail), in the table's layout
  auto count_one = [&](uint32_t r) {
    if constexpr (G::kWindow) {
      const uint32_t c = min(r & 0x7fffu, (uint32_t)G::kWords);
      atomicAdd(&sh.u.hist[c], 1u + ((r >> 15) & 1u) * 0xffffu);
    } else {
      count_key(okey16x2(r) & 0xffffu);
    }
  };
  if (tid < sp.head) count_one(bits16<E>(x[tid]));
  if (sp.tail0 + tid < V) count_one(bits16<E>(x[sp.tail0 + tid]));
  {
    // Full batches (UB vectors per lane, every lane in bounds) are addressed
    // from a uniform batch base plus per-lane offsets that do not change, and
    // two are in flight: the next one is issued before the current one is
    // counted.  A prefetch past the last full batch reads the row's first
    // vector in every lane (one line, not counted), so that every issue is
    // unconditional and the waits exact.  The remaining vectors follow as one
    // guarded batch.
    constexpr int UB = 8;
    constexpr int kStep = UB * NT;
    const int nv = (int)nvec;  // < 2^28: V < 2^31
    const int nfull = nv / kStep;
    const char* xb = reinterpret_cast<const char*>(xv);
    vu4 qa[UB], qb[UB];
    auto issue = [&](vu4(&q)[UB], int bi) {
      // all ones for a batch of the row, zero past the last one (masks, not
      // selects: the compiler keeps masks branch-free)
      const uint32_t real = 0u - (uint32_t)(bi < nfull);
      const char* bp = xb + (size_t)((uint32_t)bi & real) * (size_t)kStep * 16u;
#pragma unroll
      for (int u = 0; u < UB; ++u)
        q[u] = __builtin_nontemporal_load(
            reinterpret_cast<const vu4*>(bp + (((uint32_t)(tid + u * NT) * 16u) & real)));
      __builtin_amdgcn_sched_barrier(0);  // every load issued before the counting that follows
    };
    auto count_vec = [&](const vu4& q) {
      count_word(q.x);
      count_word(q.y);
      count_word(q.z);
      count_word(q.w);
    };
    // one vector at a time: the scheduler is kept from hoisting the key
    // arithmetic of later vectors (registers for two workgroups per CU)
    auto count_batch = [&](const vu4(&q)[UB]) {
#pragma unroll
      for (int u = 0; u < UB; ++u) {
        count_vec(q[u]);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // pairs of batches with unconditional uses (so that no load is moved
    // past the counting it should overlap); an odd last batch is in qa
    if (nfull > 0) issue(qa, 0);
    const int npairs = nfull / 2;
    for (int pi = 0; pi < npairs; ++pi) {
      issue(qb, 2 * pi + 1);
      count_batch(qa);
      issue(qa, 2 * pi + 2);
      count_batch(qb);
    }
    if (nfull & 1) count_batch(qa);
#pragma unroll
    for (int u = 0; u < UB; ++u) {
      const int v = nfull * kStep + tid + u * NT;
      if (v < nv) count_vec(__builtin_nontemporal_load(xv + v));
    }
  }
  __syncthreads();

  // ---- the occupied keys: counted, checked, listed in ascending order ------
  // Thread t owns logical words kWPT*t .. kWPT*t + kWPT - 1.  Key layout: word
  // L holds keys kBase + 2L (low half) and kBase + 2L + 1.  Window layout: word
  // m holds +m (low half, key 0x8000 | m) and -m (high half, key 0x7fff - m),
  // so the list is the negative entries by descending m (threads in reverse
  // order), then the positive ones by ascending m.
  const uint32_t L0 = (uint32_t)tid * (uint32_t)kWPT;
  const uint32_t key0 = G::kBase + 2u * L0;
  // The thread's words are read once, into registers, for the counts here and
  // the entries below; the entries may then overwrite the table after the one
  // barrier of the offsets.
  uint32_t wd[kWPT];
#pragma unroll
  for (int w = 0; w < kWPT; ++w) wd[w] = sh.u.hist[phys(L0 + (uint32_t)w)];
  const uint32_t outside = sh.u.hist[phys((uint32_t)G::kWords)];
  uint32_t ct = 0, nzp = 0, nzn = 0, kloc = 0;
  if constexpr (G::kWindow) {
    // per word: the count of both halves by one sum of absolute differences,
    // the occupied halves as (lo != 0) | (hi != 0) << 16 by one packed minimum,
    // the last occupied positive and the first occupied negative word as
    // maxima of (w + 1) and (kWPT - w) over the occupied words
    typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
    uint32_t occ = 0, wpos = 0, wneg = 0;
#pragma unroll
    for (int w = 0; w < kWPT; ++w) {
      ct = __builtin_amdgcn_sad_u16(wd[w], 0u, ct);
      const uint32_t o = __builtin_bit_cast(
          uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, wd[w]), (u16x2)(uint16_t)1));
      occ += o;
      wpos = max(wpos, (o & 1u) * (uint32_t)(w + 1));
      wneg = max(wneg, (o >> 16) * (uint32_t)(kWPT - w));
    }
    nzp = occ & 0xffffu;
    nzn = occ >> 16;
    const uint32_t kpos = wpos != 0u ? 0x8000u | (L0 + wpos - 1u) : 0u;
    const uint32_t kneg = wneg != 0u ? 0x7fffu - (L0 + (uint32_t)kWPT - wneg) : 0u;
    kloc = kpos != 0u ? kpos : kneg;  // key 0 (the largest NaN) orders below every other
  } else {
    uint32_t kpos = 0;
#pragma unroll 8
    for (int w = 0; w < kWPT; ++w) {
      const uint32_t lo = wd[w] & 0xffffu, hi = wd[w] >> 16;
      ct += lo + hi;
      nzp += (lo != 0u ? 1u : 0u) + (hi != 0u ? 1u : 0u);
      if (lo != 0u) kpos = key0 + 2u * (uint32_t)w;
      if (hi != 0u) kpos = key0 + 2u * (uint32_t)w + 1u;
    }
    kloc = kpos;
  }
  // one barrier for the entry offsets, the numbers of entries, the total
  // count and the largest occupied key
  uint32_t N, Nn, tot, kmx;
  uint32_t off_p, off_n;
  {
    const int lane = tid & 63, wv = tid >> 6;
    const uint32_t ip = wave_scan_dpp(nzp);
    const uint32_t in_ = wave_scan_dpp(nzn);
    const uint32_t ict = wave_scan_dpp(ct);
    const uint32_t ikm = wave_scan_dpp(kloc, OpMaxU());
    if (lane == 63) {
      sh.red_u[wv] = ip;
      sh.red_u[NW + wv] = in_;
      sh.red_u[2 * NW + wv] = ict;
      sh.red_u[3 * NW + wv] = ikm;
    }
    __syncthreads();
    uint32_t bp = 0u, bn = 0u, Np = 0u;
    Nn = 0u;
    tot = 0u;
    kmx = 0u;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const uint32_t a = sh.red_u[w], an = sh.red_u[NW + w];
      bp += (w < wv) ? a : 0u;
      bn += (w < wv) ? an : 0u;
      Np += a;
      Nn += an;
      tot += sh.red_u[2 * NW + w];
      kmx = max(kmx, sh.red_u[3 * NW + w]);
    }
    N = Np + Nn;
    off_p = Nn + bp + ip - nzp;  // the positive (or key-layout) entries, ascending
    off_n = Nn - (bn + in_);     // the negative entries of later threads come first
  }
  // a 16-bit count that wrapped loses a multiple of 65536 from the total
  if (tot != (uint32_t)V || outside != 0u || N > (uint32_t)kEntCap) {
    if (tid == 0) {
      RowInfo ri{};
      ri.flags = 1;
      P.info[row] = ri;
    }
    return;
  }
  // (every table word was read before the offsets' barrier)
  if constexpr (G::kWindow) {
    // Branch-free: a half with no values writes to this thread's own slot past
    // the entry list (kc[kEntCap + tid], inside the y array, which is written
    // after the next barrier and read only below N), so that no lane waits on
    // the others' branches.
    static_assert(kEntCap + NT <= 3 * kEntCap, "the spare slots lie inside the entry arrays");
    const uint32_t spare = (uint32_t)kEntCap + (uint32_t)tid;
    // (a wave whose words are all empty, most of the table, skips both loops)
    if (nzn != 0u) {
      uint32_t j = off_n;
#pragma unroll
      for (int w = kWPT - 1; w >= 0; --w) {
        const uint32_t hi = wd[w] >> 16;
        sh.u.ent.kc[hi != 0u ? j : spare] = (0x7fffu - (L0 + (uint32_t)w)) | (hi << 16);
        j += hi != 0u ? 1u : 0u;
      }
    }
    if (nzp != 0u) {
      uint32_t j = off_p;
#pragma unroll
      for (int w = 0; w < kWPT; ++w) {
        const uint32_t lo = wd[w] & 0xffffu;
        sh.u.ent.kc[lo != 0u ? j : spare] = (0x8000u | (L0 + (uint32_t)w)) | (lo << 16);
        j += lo != 0u ? 1u : 0u;
      }
    }
  } else {
    uint32_t j = off_p;
#pragma unroll
    for (int w = 0; w < kWPT; ++w) {
      const uint32_t lo = wd[w] & 0xffffu, hi = wd[w] >> 16;
      const uint32_t k0 = key0 + 2u * (uint32_t)w;
      if (lo != 0u) sh.u.ent.kc[j++] = k0 | (lo << 16);
      if (hi != 0u) sh.u.ent.kc[j++] = (k0 + 1u) | (hi << 16);
    }
  }
  __syncthreads();
  auto yk = [&](uint32_t k) { return scaled<E>(value16<E>(raw_of_okey16(k)), P); };
  const float m = yk(kmx);
  // Each thread's share of the list (entries j0 .. j1 - 1, at most CMAX) is
  // evaluated once and kept in registers for the phases below; y and
  // exp(y - m) also go to LDS for the searches and the exact walk.
  constexpr int CMAX = (kEntCap + NT - 1) / NT;
  const uint32_t C = (N + NT - 1) / NT;  // the same for every thread
  const uint32_t j0 = min(N, (uint32_t)tid * C), j1 = min(N, j0 + C);
  uint32_t rn[CMAX];  // counts, 0 past the share
  float re[CMAX];     // exp(y - m)
#pragma unroll
  for (int i = 0; i < CMAX; ++i) {
    rn[i] = 0u;
    re[i] = 0.f;
    if ((uint32_t)i < C && j0 + (uint32_t)i < j1) {
      const uint32_t j = j0 + (uint32_t)i;
      const uint32_t kcj = sh.u.ent.kc[j];
      const float y = yk(kcj & 0xffffu);
      const float e = expf(y - m);
      if constexpr (!G::kLean) {
        sh.u.ent.y[j] = y;
        sh.u.ent.e[j] = e;
      }
      rn[i] = kcj >> 16;
      re[i] = e;
    }
  }
  __syncthreads();
  const uint32_t* kc = sh.u.ent.kc;
  // entry j's y and exp(y - m): from LDS, or formed again from its key (lean)
  auto yat = [&](uint32_t j) -> float {
    if constexpr (G::kLean) return yk(kc[j] & 0xffffu);
    else return sh.u.ent.y[j];
  };
  auto eat = [&](uint32_t j) -> float {
    if constexpr (G::kLean) return expf(yat(j) - m);
    else return sh.u.ent.e[j];
  };
  auto cnt = [&](uint32_t j) { return kc[j] >> 16; };
  // first entry in [lo, hi] whose y >= v (hi + 1 if none); last entry whose y <= v (lo - 1 if none)
  auto first_ge = [&](uint32_t lo, uint32_t hi, float v) {
    uint32_t a = lo, c = hi + 1u;
    while (a < c) {
      const uint32_t mid = (a + c) >> 1;
      if (yat(mid) >= v) c = mid; else a = mid + 1u;
    }
    return a;
  };
  auto last_le = [&](uint32_t lo, uint32_t hi, float v) {
    uint32_t a = lo, c = hi + 1u;
    while (a < c) {
      const uint32_t mid = (a + c) >> 1;
      if (yat(mid) <= v) a = mid + 1u; else c = mid;
    }
    return a - 1u;
  };

  // ---- top-k: the k-th largest value by suffix counts over the list --------
  uint32_t thr = 0;  // first entry of the kept-k values
  float y_thr = -INFINITY;
  if (P.top_k > 0) {
    uint32_t cr = 0;
#pragma unroll
    for (int i = 0; i < CMAX; ++i) cr += rn[i];
    uint32_t tk;
    const uint32_t below = block_excl_scan1<uint32_t, NW>(cr, sh.red_u + 4 * NW, &tk);
    const uint32_t above = tk - below - cr;  // elements of the later (larger) entries
    const uint32_t kk = (uint32_t)P.top_k;
    if (above < kk && kk <= above + cr) {
      uint32_t acc = above;
      bool done = false;
#pragma unroll
      for (int i = CMAX - 1; i >= 0; --i) {
        acc += rn[i];
        if (!done && rn[i] != 0u && acc >= kk) {
          sh.sel[0] = j0 + (uint32_t)i;
          done = true;
        }
      }
    }
    __syncthreads();
    const uint32_t jk = sh.sel[0];
    y_thr = yat(jk);
    thr = (jk == 0u || yat(jk - 1u) < y_thr) ? jk : first_ge(0u, jk, y_thr);
  }
  // entry i of the share is inside the kept-k values
  auto in_k = [&](int i) { return rn[i] != 0u && j0 + (uint32_t)i >= thr; };

  // ---- normaliser over the kept-k values ------------------------------------
  double zs[1] = {0.0};
#pragma unroll
  for (int i = 0; i < CMAX; ++i)
    if (in_k(i)) zs[0] += (double)rn[i] * (double)re[i];
  block_sum1<double, 1, NW>(zs, sh.red_d);
  const float Z = (float)zs[0];

  // ---- top-p cut: (entry, 1-based position inside it) -----------------------
  bool have_cut = false, walked = false;
  uint32_t cut_ent = 0, cut_pos = 0;
  if (P.has_p) {
    const float inv = 1.0f / Z;
    auto pmass = [&](uint32_t j) -> double {
      return DEC16 ? (double)round_trip<E>(eat(j) / Z) : (double)(eat(j) * inv);
    };
    // the share's probabilities (in place of the exponentials, which the
    // group phase reads from LDS)
    float* rp = re;
#pragma unroll
    for (int i = 0; i < CMAX; ++i) rp[i] = DEC16 ? round_trip<E>(re[i] / Z) : re[i] * inv;
    double mt = 0.0;
#pragma unroll
    for (int i = 0; i < CMAX; ++i)
      if (in_k(i)) mt += (double)rn[i] * (double)rp[i];
    double mtot;
    const double X0 = block_excl_scan1<double, NW>(mt, sh.red_d + NW, &mtot);
    // first addition t in [1, n] of a run X + t p for which hit() holds
    // (hit(X + n p) holds, and hit is monotone in t), where v is about the
    // least value hit() accepts: t = ceil((v - X) / p) is checked with its
    // neighbour, and a binary search finishes only when that misses
    auto first_in_run = [&](double X, double p, uint32_t n, double v, auto&& hit) {
      uint32_t a = 1u, c = n;  // the answer lies in [a, c]
      const double te = ceil((v - X) / p);
      if (te > 1.0 && te < (double)n) {  // (false for NaN)
        const uint32_t t = (uint32_t)te;
        if (hit(X + (double)t * p)) {
          c = t;
          if (hit(X + (double)(t - 1u) * p)) c = t - 1u; else a = t;
        } else {
          a = t + 1u;
          if (hit(X + (double)(t + 1u) * p)) c = t + 1u; else a = t + 2u;
        }
      }
      while (a < c) {
        const uint32_t mid = a + ((c - a) >> 1);
        if (hit(X + (double)mid * p)) c = mid; else a = mid + 1u;
      }
      return a;
    };
    if constexpr (!DEC16) {
      const float cut = P.cut;
      auto hit = [&](double X) { return (float)X > cut; };
      // the midpoint above cut, about where the fp32 rounding passes it
      const double vcut = 0.5 * ((double)cut + (double)nextafterf(cut, INFINITY));
      double X = X0;
      bool found = false;
      uint32_t fk = 0, fp = 0;
#pragma unroll
      for (int i = 0; i < CMAX; ++i) {
        if (!found && in_k(i)) {
          const double p = (double)rp[i];
          const uint32_t n = rn[i];
          if (hit(X + (double)n * p)) {
            found = true;
            fk = j0 + (uint32_t)i;
            fp = hit(X) ? 1u : first_in_run(X, p, n, vcut, hit);
          }
          X += (double)n * p;
        }
      }
      block_first_flagged(found, &sh.first_lo);
      __syncthreads();
      if (sh.first_lo == tid) {
        sh.ent_lo = fk;
        sh.pos_lo = fp;
      }
      __syncthreads();
      have_cut = sh.first_lo < NT;
      cut_ent = sh.ent_lo;
      cut_pos = sh.pos_lo;
    } else {
      // smallest fp32 S whose rounding to the dtype exceeds thr16
      const float t16 = P.thr16;
      const float nxt = value16<E>(raw_of_value16<E>(t16) + 1u);
      const float mid = 0.5f * (t16 + nxt);
      const float Bthr = round_trip<E>(mid) > t16 ? mid : nextafterf(mid, INFINITY);
      const double Bd = (double)Bthr;
      // the share's bound bt, its end Xe, and for the tests below without
      // the other threads' bound D0: smin = min over entries of
      // (kSlack / 2) X1 - (bound so far), hmax = max of X1 - (bound so far)
      double bt = 0.0, Xe = X0, smin = INFINITY, hmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < CMAX; ++i) {
        if (in_k(i)) {
          const double p = (double)rp[i];
          const uint32_t n = rn[i];
          const double X1 = Xe + (double)n * p;
          bt += run_error_bound(n, p, Xe, X1);
          smin = fmin(smin, 0.5 * kSlack * X1 - bt);
          hmax = fmax(hmax, X1 - bt);
          Xe = X1;
        }
      }
      double btot;
      const double D0 = block_excl_scan1<double, NW>(bt, sh.red_d + 2 * NW, &btot);
      bool flo = false, fhi = false, slack_ok = true;
      uint32_t klo = 0, plo = 0, khi = 0, phi = 0;
      // The search below runs in the shares that may hold the lower or upper
      // crossing (a margin of 2^-40 over the differently associated sums);
      // every other share checks each entry's slack, D0 + bound <= (kSlack /
      // 2) X1, at once.
      const double Bm = Bd * (1.0 - 0x1p-40);
      const bool search = Xe + D0 + bt >= Bm || hmax - D0 >= Bm;
      if (!search) slack_ok = D0 <= smin;
      if (search) {
        double X = X0, D = D0;
#pragma unroll
        for (int i = 0; i < CMAX; ++i) {
          if (!(flo && fhi) && in_k(i)) {
            const double p = (double)rp[i];
            const uint32_t n = rn[i];
            const uint32_t j = j0 + (uint32_t)i;
            const double X1 = X + (double)n * p;
            const double Db = D + run_error_bound(n, p, X, X1);
            if (Db > 0.5 * kSlack * X1) slack_ok = false;
            auto hlo = [&](double v) { return v + Db >= Bd; };
            auto hhi = [&](double v) { return v - Db >= Bd; };
            if (!flo && hlo(X1)) {
              flo = true;
              klo = j;
              plo = hlo(X) ? 1u : first_in_run(X, p, n, Bd - Db, hlo);
            }
            if (!fhi && hhi(X1)) {
              fhi = true;
              khi = j;
              phi = hhi(X) ? 1u : first_in_run(X, p, n, Bd + Db, hhi);
            }
            X = X1;
            D = Db;
          }
        }
      }
      block_first_flagged(flo, &sh.first_lo);
      block_first_flagged(fhi, &sh.first_hi);
      if (!slack_ok) sh.fail = 1;
      __syncthreads();
      if (sh.first_lo == tid) {
        sh.ent_lo = klo;
        sh.pos_lo = plo;
      }
      if (sh.first_hi == tid) {
        sh.ent_hi = khi;
        sh.pos_hi = phi;
      }
      __syncthreads();
      const bool none_lo = sh.first_lo >= NT, none_hi = sh.first_hi >= NT;
      const bool certain = sh.fail == 0 &&
                           ((none_lo && none_hi) ||
                            (!none_lo && !none_hi && sh.ent_lo == sh.ent_hi && sh.pos_lo == sh.pos_hi));
      if (certain) {
        have_cut = !none_hi;
        cut_ent = sh.ent_hi;
        cut_pos = sh.pos_hi;
      } else {
        walked = true;
        // the exact sequence, one wave, 64 entries at a time: the lanes whose
        // additions stay inside S's binade below the threshold are added at
        // once, the others entry by entry (a run of one value in closed form)
        __syncthreads();  // every thread has read the certification's results
        if (tid < 64) {
          const int lane = tid;
          float S = 0.f;
          bool hit = false;
          uint32_t hk = 0, hp = 0;
          for (uint32_t g0 = thr; g0 < N && !hit; g0 += 64u) {
            const uint32_t j = g0 + (uint32_t)lane;
            const uint32_t n = j < N ? cnt(j) : 0u;
            const float p = n ? (float)pmass(j) : 0.f;
            int l0 = 0;  // first lane of the group not added yet
            while (l0 < 64 && !hit) {
              if (S > 0.f) {
                // Inside S's binade (ulp u), with S = s u, an addition of p
                // = P u rounds s + P to an integer: s + round(P), except that
                // a P ending in exactly one half goes to the even neighbour,
                // so the step depends on s's parity.  Every run of n equal
                // additions is then a map s -> s + d[s & 1] (its pair d,
                // closed form below), the maps compose (f then g: d[b] =
                // f.d[b] + g.d[(b + f.d[b]) & 1]), and a scan over the lanes
                // gives s after each lane's run.  Lanes l0.. up to the first
                // that would leave the binade or reach the threshold are added
                // at once.  A step of 2^25 or more leaves the binade (s < 2^24)
                // and is held at 2^25, so that 64 of them fit 32 bits.
                int eS = ilogbf(S);
                if (eS < -126) eS = -126;
                const int eu = eS - 23;
                const uint32_t s0 = (uint32_t)ldexp((double)S, -eu);  // < 2^24
                const double q = ldexp((double)p, -eu);
                const bool mine = lane >= l0;
                constexpr double kBig = 33554432.0;  // 2^25
                uint32_t d0 = 0u, d1 = 0u;  // identity for the lanes before l0 and past N
                if (mine && n != 0u) {
                  const double fq = floor(q), nd = (double)n;
                  if (q - fq == 0.5) {
                    // from an even s every step ends even; from an odd s the
                    // first step does
                    const bool odd_a = fq < kBig && (((uint32_t)fq) & 1u) != 0u;
                    const double e0 = nd * (odd_a ? fq + 1.0 : fq);
                    const double e1 = odd_a ? e0 - 1.0 : e0 + 1.0;
                    d0 = e0 >= kBig ? (uint32_t)kBig : (uint32_t)e0;
                    d1 = e1 >= kBig ? (uint32_t)kBig : (uint32_t)e1;
                  } else {
                    const double e = nd * (q - fq < 0.5 ? fq : fq + 1.0);
                    d0 = d1 = e >= kBig ? (uint32_t)kBig : (uint32_t)e;
                  }
                }
                auto past = [&](uint32_t sv) {
                  return sv >= 16777216u || ldexp((double)sv, eu) >= Bd;
                };
                // lane l0 alone already leaves the binade or reaches the
                // threshold: no scan
                const uint32_t own0 =
                    (uint32_t)__builtin_amdgcn_readlane((int)((s0 & 1u) ? d1 : d0), l0);
                if (!past(s0 + own0)) {
                  // the scan by DPP moves (the lanes with no source read the
                  // identity map 0): the earlier lanes' map, then this one's
                  auto after = [&](uint32_t f0, uint32_t f1) {
                    const uint32_t g0 = f0 + ((f0 & 1u) ? d1 : d0);
                    const uint32_t g1 = f1 + ((f1 & 1u) ? d0 : d1);
                    d0 = g0;
                    d1 = g1;
                  };
                  after(dpp_u32<0x111>(d0), dpp_u32<0x111>(d1));
                  after(dpp_u32<0x112>(d0), dpp_u32<0x112>(d1));
                  after(dpp_u32<0x114>(d0), dpp_u32<0x114>(d1));
                  after(dpp_u32<0x118>(d0), dpp_u32<0x118>(d1));
                  after(dpp_u32<0x142, 0xa>(d0), dpp_u32<0x142, 0xa>(d1));
                  after(dpp_u32<0x143, 0xc>(d0), dpp_u32<0x143, 0xc>(d1));
                  const uint32_t sl = s0 + ((s0 & 1u) ? d1 : d0);
                  const uint64_t badm = __ballot(mine && past(sl));
                  const int lb = badm ? __ffsll((long long)badm) - 1 : 64;
                  // (lb > l0: lane l0 itself stays inside)
                  S = (float)ldexp((double)(uint32_t)__builtin_amdgcn_readlane((int)sl, lb - 1), eu);
                  l0 = lb;
                  continue;
                }
              }
              // lane l0 alone: a binade crossing, the threshold, or S == 0
              const uint32_t nl = (uint32_t)__builtin_amdgcn_readlane((int)n, l0);
              const float pl = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), l0));
              uint32_t at = 0;
              if (nl != 0u && seq_add_run(S, pl, nl, Bthr, &at)) {
                hit = true;
                hk = g0 + (uint32_t)l0;
                hp = at;
              }
              ++l0;
            }
          }
          if (lane == 0) {
            sh.walk_hit = hit ? 1 : 0;
            sh.walk_ent = hk;
            sh.walk_pos = hp;
          }
        }
        __syncthreads();
        have_cut = sh.walk_hit != 0;
        cut_ent = sh.walk_ent;
        cut_pos = sh.walk_pos;
      }
    }
  }

  // ---- the cut's value group, kept count and log-sum-exp --------------------
  uint32_t g_lo, g_hi;
  float v_cut;
  // (entries hold distinct keys: equal values only where the temperature
  // merges keys, so the group is usually the one entry, seen from its
  // neighbours without a search)
  if (!P.has_p && P.top_k <= 0) {
    v_cut = y_thr;
    g_lo = thr;
    g_hi = last_le(thr, N - 1u, y_thr);
  } else {
    const uint32_t ck = !P.has_p ? thr : have_cut ? cut_ent : N - 1u;
    v_cut = yat(ck);  // (y_thr when there is no top-p)
    g_lo = (ck == thr || yat(ck - 1u) < v_cut) ? ck : first_ge(thr, ck, v_cut);
    g_hi = (ck == N - 1u || yat(ck + 1u) > v_cut) ? ck : last_le(ck, N - 1u, v_cut);
  }
  double ksum_above = 0.0;  // kept mass above the group
  uint32_t cnts[3] = {0u, 0u, 0u};  // elements above the group, in it, in it before the cut entry
#pragma unroll
  for (int i = 0; i < CMAX; ++i) {
    const uint32_t j = j0 + (uint32_t)i;
    const uint32_t n = rn[i];
    if (n == 0u) continue;
    if (j > g_hi) {
      cnts[0] += n;
      ksum_above += (double)n * (double)eat(j);
    } else if (j >= g_lo) {
      cnts[1] += n;
      if (have_cut && j < cut_ent) cnts[2] += n;
    }
  }
  {  // the four sums with one barrier
    const int lane = tid & 63, wv = tid >> 6;
    const double isum = wave_scan_dpp(ksum_above);
    uint32_t ic[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) ic[q] = wave_scan_dpp(cnts[q]);
    if (lane == 63) {
      sh.red_d[3 * NW + wv] = isum;
#pragma unroll
      for (int q = 0; q < 3; ++q) sh.red_u[(5 + q) * NW + wv] = ic[q];
    }
    __syncthreads();
    ksum_above = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) ksum_above += sh.red_d[3 * NW + w];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      uint32_t sq = 0u;
#pragma unroll
      for (int w = 0; w < NW; ++w) sq += sh.red_u[(5 + q) * NW + w];
      cnts[q] = sq;
    }
  }
  double sums[1] = {ksum_above};
  const uint32_t n_group = cnts[1];
  uint32_t rcut = 0;  // group elements (in index order) before the cut
  if (P.has_p) rcut = have_cut ? cnts[2] + cut_pos - 1u : n_group - 1u;
  const uint32_t n_kept = cnts[0] + (n_group - rcut);
  const double ksum = sums[0] + (double)(n_group - rcut) * (double)eat(g_lo);
  const float logsum = logf((float)ksum);
  const uint32_t gk_lo = kc[g_lo] & 0xffffu, gk_hi = kc[g_hi] & 0xffffu;

  // ---- the target --------------------------------------------------------
  float lp = -INFINITY;
  if (t >= 0 && t < V) {
    const uint32_t kt = okey16x2(xt_bits) & 0xffffu;
    const float yt = yk(kt);
    bool kept = yt > v_cut;
    if (yt == v_cut) {
      kept = true;
      if (rcut > 0u) {
        // the target's rank among the group's elements in index order
        uint32_t before = 0;
        for (int64_t j = tid; j < t; j += NT) {
          const uint32_t kj = okey16x2(bits16<E>(x[j])) & 0xffffu;
          before += (kj >= gk_lo && kj <= gk_hi) ? 1u : 0u;
        }
        uint32_t bs[1] = {before};
        block_sum1<uint32_t, 1, NW>(bs, sh.red_u + 8 * NW);
        kept = bs[0] >= rcut;
      }
    }
    if (kept) lp = (yt - m) - logsum;
  }

  if (tid == 0) {
    RowInfo ri;
    ri.m = m;
    ri.logsum = logsum;
    ri.v_cut = v_cut;
    ri.i_cut = rcut > 0u ? -1 - (int32_t)rcut : 0;
    ri.n_kept = (int32_t)n_kept;
    ri.flags = kFlagNoKeptList | (walked ? kFlagWalked : 0);
    P.info[row] = ri;
    if (P.out != nullptr) P.out[row] = lp;
  }
}

// The index cut of a row left in rank form (i_cut = -1 - rcut): the index of
// the group's element of rank rcut in index order, the group being the
// elements whose scaled value equals v_cut.  One workgroup per row; rows in
// index form return at once.  Each thread counts the group's elements in its
// own contiguous share of the row, a workgroup scan places the shares, and
// the thread holding rank rcut reads its share again.
template <class E>
__global__ __launch_bounds__(kHT) void filter_resolve_kernel(FilterParams P) {
  using raw = typename E::raw;
  __shared__ uint32_t red[kHW * 4];
  __shared__ int32_t s_idx;
  const int64_t row = blockIdx.x;
  const RowInfo ri = P.info[row];
  if (ri.i_cut >= 0) return;
  const uint32_t rcut = (uint32_t)(-1 - ri.i_cut);
  const int64_t b = row / P.R, r = row - b * P.R;
  const raw* x = static_cast<const raw*>(P.logits) + b * P.sb + r * P.sr;
  const int tid = threadIdx.x;
  const int64_t V = P.V;
  auto yk = [&](uint32_t k) { return scaled<E>(value16<E>(raw_of_okey16(k)), P); };
  // the group's key range, searched between the keys of -inf and +inf (NaN keys lie outside)
  const uint32_t klo = okey16x2(raw_of_value16<E>(-INFINITY)) & 0xffffu;
  const uint32_t khi = okey16x2(raw_of_value16<E>(INFINITY)) & 0xffffu;
  const float v = ri.v_cut;
  uint32_t a = klo, c = khi + 1u;
  while (a < c) {
    const uint32_t mid = (a + c) >> 1;
    if (yk(mid) >= v) c = mid; else a = mid + 1u;
  }
  const uint32_t g_lo = a;
  a = klo;
  c = khi + 1u;
  while (a < c) {
    const uint32_t mid = (a + c) >> 1;
    if (yk(mid) <= v) a = mid + 1u; else c = mid;
  }
  const uint32_t g_hi = a - 1u;
  auto member = [&](int64_t j) {
    const uint32_t k = okey16x2(bits16<E>(x[j])) & 0xffffu;
    return k >= g_lo && k <= g_hi;
  };
  const int64_t C = (V + kHT - 1) / kHT;
  const int64_t j0 = min(V, (int64_t)tid * C), j1 = min(V, j0 + C);
  uint32_t n = 0;
  for (int64_t j = j0; j < j1; ++j) n += member(j) ? 1u : 0u;
  uint32_t tot;
  const uint32_t before = block_excl_scan<uint32_t>(n, red, &tot);
  if (tid == 0) s_idx = 0;
  __syncthreads();
  if (before <= rcut && rcut < before + n) {
    uint32_t seen = before;
    for (int64_t j = j0; j < j1; ++j) {
      if (!member(j)) continue;
      if (seen == rcut) {
        s_idx = (int32_t)j;
        break;
      }
      ++seen;
    }
  }
  __syncthreads();
  if (tid == 0) P.info[row].i_cut = s_idx;
}

template <class E>
int launch_hist(const FilterParams& P, int64_t rows, int all_rows, hipStream_t st) {
  // the compact kernel first; the rows it flags go to filter_hist_kernel
  using G = typename std::conditional<std::is_same<E, BF16>::value, CompactWindow,
                                      CompactFull>::type;
  // (after the fast kernel, all_rows == 0, the few rows it flagged, if any, go
  // straight to filter_hist_kernel: a compact launch over every row to find
  // them would cost more than it saves)
  if (all_rows) {
    if (P.dec16)
      hipLaunchKernelGGL((filter_compact_kernel<E, G, true>), dim3((unsigned)rows), dim3(G::NT), 0,
                         st, P);
    else
      hipLaunchKernelGGL((filter_compact_kernel<E, G, false>), dim3((unsigned)rows), dim3(G::NT), 0,
                         st, P);
    if (int e = check_launch("filter_compact_kernel")) return e;
  }
  // the flagged rows, each workgroup over a share of at most kHT rows
  const int64_t grid = std::min<int64_t>(rows, std::max<int64_t>(256, (rows + kHT - 1) / kHT));
  const int per = (int)((rows + grid - 1) / grid);
  hipLaunchKernelGGL((filter_hist_kernel<E, 0, false>), dim3((unsigned)grid), dim3(kHT), 0, st, P,
                     rows, per);
  if (int e = check_launch("filter_hist_kernel")) return e;
  if (!P.dec16) return MIRL_OK;
  // rows the rounding bound left undecided
  hipLaunchKernelGGL((filter_hist_kernel<E, 0, true>), dim3((unsigned)grid), dim3(kHT), 0, st, P,
                     rows, per);
  return check_launch("filter_hist_kernel(walk)");
}

}  // namespace

int launch_resolve_rows(const FilterParams& P, int dtype, int64_t rows, hipStream_t st) {
  if (dtype == MIRL_DTYPE_BF16)
    hipLaunchKernelGGL((filter_resolve_kernel<BF16>), dim3((unsigned)rows), dim3(kHT), 0, st, P);
  else if (dtype == MIRL_DTYPE_F16)
    hipLaunchKernelGGL((filter_resolve_kernel<F16>), dim3((unsigned)rows), dim3(kHT), 0, st, P);
  else
    return MIRL_OK;  // fp32 rows never leave the cut in rank form
  return check_launch("filter_resolve_kernel");
}

int launch_hist_rows(const FilterParams& P, int dtype, int64_t rows, int all_rows,
                     hipStream_t st) {
  MIRL_REQUIRE(P.V <= kHistMaxV, "vocabulary %lld exceeds the histogram path's %lld",
               (long long)P.V, (long long)kHistMaxV);
  if (dtype == MIRL_DTYPE_BF16) return launch_hist<BF16>(P, rows, all_rows, st);
  MIRL_REQUIRE(dtype == MIRL_DTYPE_F16, "histogram path: 16-bit logits only (dtype %d)", dtype);
  return launch_hist<F16>(P, rows, all_rows, st);
}

}  // namespace mirl

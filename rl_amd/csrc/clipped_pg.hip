// Fused ClippedPG loss: forward value, every metric of the reference's metric
// dictionary, and the closed-form gradient with respect to the token
// log-probabilities, in two launches over [B, L] tokens:
//
//   pg_rows_kernel   one workgroup per sequence b: row masks, sequence-level
//                    ratios / IS weights, per-token loss terms and gradients,
//                    and the row's partial sums for the loss and metrics;
//   pg_final_kernel  one workgroup: reduces the row partials in row order
//                    (deterministic), writes the loss and metrics, and adds
//                    the one cross-row gradient term (VAPO NLL, whose
//                    normaliser is the batch's correct-token count).
//
// Semantics: nemo_rl/algorithms/loss/loss_functions.py:698-1183 (__call__),
// nemo_rl/algorithms/loss/clipped_pg.py:38-194 (objective, diagnostics),
// nemo_rl/algorithms/utils.py:56-115 (calculate_kl), :294-306 (masked_mean).
// Gradient rules are PyTorch's autograd rules for the same op sequence:
// maximum/minimum split the gradient 50/50 on exact ties, clamp passes it on
// the closed interval, where() passes it to the selected branch, nan_to_num
// passes it where the input was finite.

#include <mutex>

#include "common.h"
#include "pg_token.h"

namespace mirl {
namespace {

using namespace pg;

// Threads per sequence row: 1024 for fp32 rows (measured 25 vs 29 us at 256 on
// 8 rows of 2047 tokens, where one workgroup per row leaves most CUs idle),
// 512 for fp64, whose kernel would spill registers at 1024.
template <class T>
constexpr int row_threads() { return sizeof(T) == 4 ? 1024 : 512; }
constexpr int kFinalThreads = 1024;

// row partial-sum slots
enum Slot {
  P_ACTOR = 0,
  P_KL,
  P_TMPE,
  P_RATIO,
  P_RATIO_C,
  P_RATIO_MIN,
  P_RATIO_MAX,
  P_RATIO_C_MIN,
  P_RATIO_C_MAX,
  P_GEN_KL,
  P_POL_KL,
  P_JS,
  P_ENT,
  P_SIR,
  P_NVS,
  P_CVT,
  P_NLL,
  P_OOB,
  P_EXCL,
  P_SC,  // score-centering correction
  P_HM,  // score-centering head mass
  NUM_SLOTS
};

// Block-wide reductions over row_threads<T>() / kFinalThreads threads.
template <class T, int NT>
__device__ T block_sum(T v, T* scratch) {
  v = wave_sum(v);
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();
  if (lane == 0) scratch[wv] = v;
  __syncthreads();
  T r = T(0);
#pragma unroll
  for (int k = 0; k < NT / 64; ++k) r += scratch[k];
  return r;
}

// Reductions of N values at once.  Value k is reduced with kind(k): a sum, or a
// min / max that propagates NaN (torch's amin / amax).  Each value takes the
// same xor butterfly inside a wave and the same wave order as a separate
// block_sum would (the N shuffle chains interleave instead of running one after
// the other behind two barriers each), so the results are bitwise the same.
enum RedKind { R_SUM = 0, R_MIN = 1, R_MAX = 2 };

template <class T>
__device__ __forceinline__ T red_combine(int kind, T a, T b) {
  if (kind == R_MIN) return (b < a || isnan(b)) ? b : a;
  if (kind == R_MAX) return (b > a || isnan(b)) ? b : a;
  return a + b;
}

// Leaves wave w's result for value k in scratch[k * (NT / 64) + w]; scratch
// holds N * (NT / 64) values.
template <class T, int NT, int N, class Kind>
__device__ __forceinline__ void block_exchange_n(T (&v)[N], Kind kind, T* scratch) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    T o[N];
#pragma unroll
    for (int k = 0; k < N; ++k) o[k] = __shfl_xor(v[k], off, 64);
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = red_combine(kind(k), v[k], o[k]);
  }
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();  // an earlier reduction's readers are done with scratch
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < N; ++k) scratch[k * (NT / 64) + wv] = v[k];
  }
  __syncthreads();
}

// Workgroup total of value k over the wave partials left by block_exchange_n.
template <class T, int NT>
__device__ __forceinline__ T block_total(int kind, int k, const T* scratch) {
  const T* p = scratch + k * (NT / 64);
  T r = (kind == R_SUM) ? T(0) : p[0];
  for (int w = (kind == R_SUM) ? 0 : 1; w < NT / 64; ++w) r = red_combine(kind, r, p[w]);
  return r;
}

// N sums at once, every thread receiving every total.
template <class T, int NT, int N>
__device__ __forceinline__ void block_sum_n(T (&v)[N], T* scratch) {
  block_exchange_n<T, NT, N>(v, [](int) { return int(R_SUM); }, scratch);
#pragma unroll
  for (int k = 0; k < N; ++k) v[k] = block_total<T, NT>(R_SUM, k, scratch);
}

__device__ __forceinline__ int slot_kind(int k) {
  if (k == P_RATIO_MIN || k == P_RATIO_C_MIN) return R_MIN;
  if (k == P_RATIO_MAX || k == P_RATIO_C_MAX) return R_MAX;
  return R_SUM;
}

// torch.maximum / torch.minimum: NaN in either operand propagates.
template <class T>
__device__ __forceinline__ T tmaximum(T a, T b) {
  return (isnan(a) || isnan(b)) ? a + b : (a > b ? a : b);
}
template <class T>
__device__ __forceinline__ T tminimum(T a, T b) {
  return (isnan(a) || isnan(b)) ? a + b : (a < b ? a : b);
}

// adaptive_ppo_clip_kept_mask (clipped_pg.py:38-50)
template <class T>
__device__ __forceinline__ bool adaptive_kept(T w, T A, T lo, T hi, T outer) {
  return (w <= outer) && ((A >= T(0)) || (w >= lo)) && ((A <= T(0)) || (w <= hi));
}

// Score centering of one active token (score_centering.py:76-129): returns
// term = sum_k coef_k plog_k and the head mass sum_k q_k, and writes
// coef_k * scale to out[k] (contiguous).  A is the token's advantage (read by
// adaptive-ppo-clip only).
template <class T>
__device__ void score_centering_token(const mirl_score_centering_args& sc, int64_t b, int64_t l,
                                      T A, T scale, T* __restrict__ out, T* term_out,
                                      T* head_out) {
  const T* pl = static_cast<const T*>(sc.plog) + b * sc.p_sb + l * sc.p_sl;
  const T* ql = static_cast<const T*>(sc.qlog) + b * sc.q_sb + l * sc.q_sl;
  const int64_t K = sc.K;
  // The ids are read kChunk at a time, all loads of a chunk issued before any
  // is used (one dependent load per id measured 15 us for 16 K tokens x 20 ids);
  // sums still run in k order.
  constexpr int kChunk = 8;
  T head = T(0), psum = T(0);
  for (int64_t k0 = 0; k0 < K; k0 += kChunk) {
    T qv[kChunk], pv[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int64_t k = k0 + u < K ? k0 + u : K - 1;
      qv[u] = ql[k * sc.q_sk];
      pv[u] = pl[k * sc.p_sk];
    }
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      if (k0 + u < K) {
        head += dexp(qv[u]);
        psum += dexp(pv[u]);
      }
    }
  }
  // rho = clamp(1 - head, min=0) / clamp(1 - sum p, min=1e-6)
  T num = T(1) - head;
  num = isnan(num) ? num : (num < T(0) ? T(0) : num);
  T den = T(1) - psum;
  den = isnan(den) ? den : (den < T(1e-6) ? T(1e-6) : den);
  const T rho = num / den;
  const T lo = T(sc.lo), hi = T(sc.hi), outer = T(sc.outer);
  T alpha;
  switch (sc.mode) {
    case MIRL_SC_OFF: alpha = rho; break;
    case MIRL_SC_IS: alpha = T(1); break;
    case MIRL_SC_TIS: alpha = tminimum(tmaximum(T(1), lo * rho), hi * rho); break;
    case MIRL_SC_ICEPOP: {
      const T tr = T(1) / rho;
      alpha = (tr >= lo && tr <= hi) ? T(1) : T(0);
      break;
    }
    default: alpha = adaptive_kept(T(1) / rho, A, lo, hi, outer) ? T(1) : T(0); break;
  }
  T term = T(0);
  for (int64_t k0 = 0; k0 < K; k0 += kChunk) {
    T pv[kChunk], qv[kChunk];
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int64_t k = k0 + u < K ? k0 + u : K - 1;
      pv[u] = pl[k * sc.p_sk];
      qv[u] = ql[k * sc.q_sk];
    }
#pragma unroll
    for (int u = 0; u < kChunk; ++u) {
      const int64_t k = k0 + u;
      if (k >= K) break;
      const T plk = pv[u], qlk = qv[u];
      const T p = dexp(plk), q = dexp(qlk);
      T mass;
      switch (sc.mode) {
        case MIRL_SC_OFF: mass = q; break;
        case MIRL_SC_IS: mass = p; break;
        case MIRL_SC_TIS: mass = tminimum(tmaximum(p, lo * q), hi * q); break;
        case MIRL_SC_ICEPOP: {
          const T r = dexp(plk - qlk);
          mass = (r >= lo && r <= hi) ? p : T(0);
          break;
        }
        default: mass = adaptive_kept(dexp(plk - qlk), A, lo, hi, outer) ? p : T(0); break;
      }
      const T coef = mass - alpha * p;
      term += coef * plk;
      out[k] = coef * scale;
    }
  }
  *term_out = term;
  *head_out = head;
}

// Score-centering scratch: per-token term and head mass (written by
// sc_term_kernel) and the gradient scale alpha * A (written by pg_rows_kernel,
// read by sc_scale_kernel); each [B, L].
template <class T>
struct ScWork {
  T* term;
  T* head;
  T* scale;
};

template <class T>
struct Inputs {
  View<T> curr, unf, tm, adv, prev, gen, ref;
  MaskView psm;
  const T* sample_mask;
  const T* rewards;
  const T* gvs;
  const T* gvt;
};

template <class T, int NT>
__global__ __launch_bounds__(NT) void pg_rows_kernel(mirl_pg_config cfg, int64_t L,
                                                              Inputs<T> in, T* __restrict__ gcurr,
                                                              T* __restrict__ gunf,
                                                              T* __restrict__ part,
                                                              ScWork<T> sc_ws, int has_sc) {
  __shared__ T scratch[NUM_SLOTS * (NT / 64)];
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const T eps = T(1e-8);
  const T gvt = *in.gvt + eps;
  const T gvs = *in.gvs + eps;
  const bool has_kl = cfg.kl_penalty != 0.0;

  // ---- pass A: row masks --------------------------------------------------
  // support'(l) = psm & ~isneginf(prev) & ~isneginf(gen)
  auto support = [&](int64_t l) -> bool {
    if (!cfg.has_support_mask) return true;
    const T pv = cfg.force_on_policy ? in.curr(b, l) : in.prev(b, l);
    return in.psm(b, l) && !(isinf(pv) && pv < 0) && !(isinf(in.gen(b, l)) && in.gen(b, l) < 0);
  };
  T any_tm = 0, any_tm2 = 0, sum_tm = 0, sum_tm2 = 0;
  for (int64_t l = tid; l < L; l += NT) {
    const T tmv = in.tm(b, l);
    const T tm2 = tmv * (support(l) ? T(1) : T(0));
    any_tm += (tmv != T(0)) ? T(1) : T(0);
    any_tm2 += (tm2 != T(0)) ? T(1) : T(0);
    sum_tm += tmv;
    sum_tm2 += tm2;
  }
  {
    T r[4] = {any_tm, any_tm2, sum_tm, sum_tm2};
    block_sum_n<T, NT>(r, scratch);
    any_tm = r[0];
    any_tm2 = r[1];
    sum_tm = r[2];
    sum_tm2 = r[3];
  }
  const T sm = in.sample_mask[b] * (any_tm > T(0) ? T(1) : T(0));
  const T sm2 = cfg.has_support_mask ? sm * (any_tm2 > T(0) ? T(1) : T(0)) : sm;
  // tokens of this row after the support adjustment (token_mask in the objective)
  auto tm2_at = [&](int64_t l) -> T {
    const T tmv = in.tm(b, l);
    return cfg.has_support_mask ? tmv * (support(l) ? T(1) : T(0)) : tmv;
  };
  // sanitised operands: where(mask2 != 0, x, 0)
  auto prev_of = [&](int64_t l) -> T { return cfg.force_on_policy ? in.curr(b, l) : in.prev(b, l); };

  // ---- pass B: sequence-level quantities ----------------------------------
  T seq_lr = 0, seq_is = 0, seq_lir = 0;
  {
    for (int64_t l = tid; l < L; l += NT) {
      const T tm2 = tm2_at(l);
      const T mask2 = tm2 * sm2;
      const bool on = mask2 != T(0);
      const T c = on ? in.curr(b, l) : T(0);
      const T pv = on ? prev_of(l) : T(0);
      const T gv = on ? in.gen(b, l) : T(0);
      seq_lr += (c - pv) * tm2;
      seq_is += (pv - gv) * mask2;
      seq_lir += nan_to_zero_all(pv - gv) * tm2;
    }
    T r[3] = {seq_lr, seq_is, seq_lir};
    block_sum_n<T, NT>(r, scratch);
    seq_lr = r[0];
    seq_is = r[1];
    seq_lir = r[2];
  }
  const bool seq_ratio = cfg.sequence_level_is && !cfg.disable_ppo_ratio && !cfg.force_on_policy;
  const T r_seq = seq_ratio ? dexp(seq_lr / (sum_tm2 + eps)) : T(0);
  const T w_seq = nan_to_zero_all(dexp(seq_is));
  T seq_kept = T(1);
  if (cfg.tis_type == MIRL_TIS_SEQ_MASK) {
    const T g = dexp(seq_lir / (sum_tm2 + eps));
    seq_kept = (g >= T(cfg.tis_ratio_min) && g <= T(cfg.tis_ratio)) ? T(1) : T(0);
  }

  // ---- pass C: per-token terms -------------------------------------------
  T acc[NUM_SLOTS];
#pragma unroll
  for (int k = 0; k < NUM_SLOTS; ++k) acc[k] = T(0);
  acc[P_RATIO_MIN] = T(INFINITY);
  acc[P_RATIO_C_MIN] = T(INFINITY);
  acc[P_RATIO_MAX] = T(-INFINITY);
  acc[P_RATIO_C_MAX] = T(-INFINITY);
  T gspo_sum = 0;  // sum_t alpha_t * w_t * dcl_t/dr_seq  (sequence-level ratio)
  const T actor_row_norm = sum_tm2 + eps;
  const T kl_row_norm = sum_tm + eps;
  const bool correct = cfg.has_rewards && cfg.nll_weight > 0.0 && in.rewards[b] > T(0);

  for (int64_t l = tid; l < L; l += NT) {
    const T tmv = in.tm(b, l);
    const T tm2 = tm2_at(l);
    const T mask2 = tm2 * sm2;
    const T kl_mask = tmv * sm;
    const bool on = mask2 != T(0);
    const T craw = in.curr(b, l);
    const T c = on ? craw : T(0);
    const T pv = on ? prev_of(l) : T(0);
    const T gv = on ? in.gen(b, l) : T(0);
    // score centering zeroes the advantages outside the final mask
    // (loss_functions.py:841-842)
    const T A = (has_sc && !on) ? T(0) : in.adv(b, l);
    TokenIn<T> ti;
    ti.tmv = tmv;
    ti.tm2 = tm2;
    ti.sm = sm;
    ti.sm2 = sm2;
    ti.craw = craw;
    ti.c = c;
    ti.pv = pv;
    ti.gv = gv;
    ti.A = A;
    const bool kon = kl_mask != T(0);
    ti.cu = (has_kl && kon) ? (cfg.has_unfiltered ? in.unf(b, l) : craw) : T(0);
    ti.rf = (has_kl && kon) ? in.ref(b, l) : T(0);
    ti.kgen = (has_kl && kon) ? in.gen(b, l) : T(0);
    ti.gvt = gvt;
    ti.gvs = gvs;
    ti.actor_row_norm = actor_row_norm;
    ti.kl_row_norm = kl_row_norm;
    ti.r_seq = r_seq;
    ti.w_seq = w_seq;
    ti.seq_kept = seq_kept;
    ti.seq_ratio = seq_ratio;
    const TokenOut<T> to = token_terms<T>(cfg, ti);
    T gc = to.gc;  // dloss/dcurr (this token)
    const T gu = to.gu;  // dloss/dunfiltered
    if (has_kl) acc[P_KL] += to.klt * (cfg.token_level_loss ? kl_mask : tmv);
    const T w = to.w;
    if (cfg.need_is) acc[P_OOB] += (to.oob ? T(1) : T(0)) * mask2;
    const T r = to.r, rc = to.rc;
    const T alpha = to.alpha;
    acc[P_ACTOR] += to.v * (cfg.token_level_loss ? mask2 : tm2);
    if (has_sc) {
      // correction A * term, normalised like the actor loss (loss_functions.py:1070-1097);
      // term / head come from sc_term_kernel, the gradient scale goes to sc_scale_kernel
      const int64_t i = b * L + l;
      if (on) {
        acc[P_SC] += (A * sc_ws.term[i]) * (cfg.token_level_loss ? mask2 : tm2);
        acc[P_HM] += sc_ws.head[i] * mask2;
      }
      sc_ws.scale[i] = on ? alpha * A : T(0);
    }
    if (seq_ratio) gspo_sum += to.gspo;

    // NLL bookkeeping (gradient added by the final kernel)
    if (correct) {
      acc[P_CVT] += mask2;
      acc[P_NLL] += (-c) * mask2;
    }

    // metrics ---------------------------------------------------------------
    acc[P_TMPE] += dexp(dabs(gv - pv) * mask2) * mask2;
    if (cfg.full_metrics) {
      acc[P_RATIO] += r * mask2;
      acc[P_RATIO_C] += rc * mask2;
      if (on) {
        acc[P_RATIO_MIN] = (r < acc[P_RATIO_MIN] || isnan(r)) ? r : acc[P_RATIO_MIN];
        acc[P_RATIO_MAX] = (r > acc[P_RATIO_MAX] || isnan(r)) ? r : acc[P_RATIO_MAX];
        acc[P_RATIO_C_MIN] = (rc < acc[P_RATIO_C_MIN] || isnan(rc)) ? rc : acc[P_RATIO_C_MIN];
        acc[P_RATIO_C_MAX] = (rc > acc[P_RATIO_C_MAX] || isnan(rc)) ? rc : acc[P_RATIO_C_MAX];
      }
      acc[P_GEN_KL] += kl_value<T>(cfg.kl_type, pv - gv) * mask2;
      acc[P_POL_KL] += kl_value<T>(cfg.kl_type, gv - pv) * mask2;
      const T lm = dlog(T(0.5) * dexp(pv) + T(0.5) * dexp(gv));
      const T a = pv - lm, bb = gv - lm;
      const T js = T(0.5) * ((dexp(a) - a) - T(1)) + T(0.5) * ((dexp(bb) - bb) - T(1));
      acc[P_JS] += js * mask2;
      acc[P_ENT] += (dexp(c - gv) * c) * mask2;
    }
    if (cfg.need_is && !cfg.sequence_level_is) acc[P_SIR] += w * mask2;
    acc[P_EXCL] += kl_mask - mask2;

    gcurr[b * L + l] = gc;
    if (cfg.has_unfiltered) gunf[b * L + l] = gu;
  }

  // sequence-level ratio gradient: every token of the row shares r_seq
  if (seq_ratio) {
    gspo_sum = block_sum<T, NT>(gspo_sum, scratch);
    const T coef = gspo_sum * r_seq / (sum_tm2 + eps);
    for (int64_t l = tid; l < L; l += NT) {
      const T tm2 = tm2_at(l);
      if (tm2 * sm2 != T(0)) gcurr[b * L + l] += coef * tm2;
    }
  }

  // ---- row partials ------------------------------------------------------
  T* out = part + b * NUM_SLOTS;
  block_exchange_n<T, NT, NUM_SLOTS>(acc, [](int k) { return slot_kind(k); }, scratch);
  if (tid < NUM_SLOTS) {
    const int k = tid;  // thread k finishes slot k
    T v = block_total<T, NT>(slot_kind(k), k, scratch);
    if ((k == P_ACTOR || k == P_SC) && !cfg.token_level_loss) v = sm2 * (v / actor_row_norm);
    if (k == P_KL && !cfg.token_level_loss) v = sm * (v / kl_row_norm);
    if (k == P_SIR && cfg.sequence_level_is) {
      bool oob = false;
      v = truncate_is(cfg, w_seq, T(0), seq_kept, &oob) * sm2;
    }
    if (k == P_NVS) v = sm2;
    if (k == P_OOB && cfg.tis_type == MIRL_TIS_SEQ_MASK) v = (T(1) - seq_kept) * sm2;
    out[k] = v;
  }
}

template <class T>
__global__ __launch_bounds__(kFinalThreads) void pg_final_kernel(mirl_pg_config cfg, int64_t B,
                                                                 int64_t L, Inputs<T> in,
                                                                 const T* __restrict__ part,
                                                                 T* __restrict__ metrics,
                                                                 T* __restrict__ loss_out,
                                                                 T* __restrict__ gcurr,
                                                                 int has_sc) {
  __shared__ T tot[NUM_SLOTS];
  const int tid = threadIdx.x;
  if (tid < NUM_SLOTS) {
    const int k = tid;
    T v;
    if (k == P_RATIO_MIN || k == P_RATIO_C_MIN) {
      v = T(INFINITY);
      for (int64_t b = 0; b < B; ++b) {
        const T x = part[b * NUM_SLOTS + k];
        v = (x < v || isnan(x)) ? x : v;
      }
    } else if (k == P_RATIO_MAX || k == P_RATIO_C_MAX) {
      v = T(-INFINITY);
      for (int64_t b = 0; b < B; ++b) {
        const T x = part[b * NUM_SLOTS + k];
        v = (x > v || isnan(x)) ? x : v;
      }
    } else {
      v = T(0);
      for (int64_t b = 0; b < B; ++b) v += part[b * NUM_SLOTS + k];
    }
    tot[k] = v;
  }
  __syncthreads();
  const T eps = T(1e-8);
  const T gvt = *in.gvt + eps;
  const T gvs = *in.gvs + eps;
  const T cvt = tot[P_CVT];
  const bool nll_on = cfg.has_rewards && cfg.nll_weight > 0.0;
  if (tid == 0) {
    T actor = tot[P_ACTOR] / (cfg.token_level_loss ? gvt : gvs);
    if (has_sc) actor = actor + tot[P_SC] / (cfg.token_level_loss ? gvt : gvs);
    const T kl = cfg.kl_penalty != 0.0 ? tot[P_KL] / (cfg.token_level_loss ? gvt : gvs) : T(0);
    const T nll = (nll_on && cvt > T(0)) ? tot[P_NLL] / (cvt + eps) : T(0);
    const T loss = (actor + kl) + T(cfg.nll_weight) * nll;
    T* m = metrics;
    m[MIRL_M_LOSS] = loss;
    if (loss_out != nullptr) *loss_out = loss;  // the loss on its own, for callers that want it apart
    m[MIRL_M_TOKEN_MULT_PROB_ERROR] = tot[P_TMPE] / gvt;
    m[MIRL_M_PROBS_RATIO] = tot[P_RATIO] / gvt;
    m[MIRL_M_PROBS_RATIO_CLAMPED] = tot[P_RATIO_C] / gvt;
    m[MIRL_M_PROBS_RATIO_MIN] = tot[P_RATIO_MIN];
    m[MIRL_M_PROBS_RATIO_MAX] = tot[P_RATIO_MAX];
    m[MIRL_M_PROBS_RATIO_CLAMPED_MIN] = tot[P_RATIO_C_MIN];
    m[MIRL_M_PROBS_RATIO_CLAMPED_MAX] = tot[P_RATIO_C_MAX];
    m[MIRL_M_GEN_KL_ERROR] = tot[P_GEN_KL] / gvt;
    m[MIRL_M_POLICY_KL_ERROR] = tot[P_POL_KL] / gvt;
    m[MIRL_M_JS_DIVERGENCE_ERROR] = tot[P_JS] / gvt;
    m[MIRL_M_APPROX_ENTROPY] = -(tot[P_ENT] / gvt);
    m[MIRL_M_SAMPLING_IMPORTANCE_RATIO] = tot[P_SIR] / (cfg.sequence_level_is ? gvs : gvt);
    m[MIRL_M_KL_PENALTY] = cfg.kl_penalty != 0.0 ? kl / T(cfg.kl_penalty) : T(0);
    m[MIRL_M_NUM_VALID_SAMPLES] = tot[P_NVS];
    m[MIRL_M_POSITIVE_NLL_LOSS] = nll;
    m[MIRL_M_IS_OOB_RATIO] = tot[P_OOB] / (cfg.tis_type == MIRL_TIS_SEQ_MASK ? gvs : gvt);
    m[MIRL_M_POLICY_SUPPORT_EXCLUDED_TOKENS] = tot[P_EXCL];
    m[MIRL_M_SCORE_CENTERING_HEAD_MASS] = has_sc ? tot[P_HM] / gvt : T(0);
  }
  if (nll_on && cvt > T(0)) {
    // d(mu * nll)/dcurr = -mu * correct_mask / (cvt + 1e-8)
    const T coef = -T(cfg.nll_weight) / (cvt + eps);
    for (int64_t i = tid; i < B * L; i += kFinalThreads) {
      const int64_t b = i / L, l = i - b * L;
      if (!(in.rewards[b] > T(0))) continue;
      const T tmv = in.tm(b, l);
      T tm2 = tmv;
      if (cfg.has_support_mask) {
        const T pv = cfg.force_on_policy ? in.curr(b, l) : in.prev(b, l);
        const bool sup = in.psm(b, l) && !(isinf(pv) && pv < 0) && !(isinf(in.gen(b, l)) && in.gen(b, l) < 0);
        tm2 = sup ? tmv : T(0);
      }
      // sm2 for row b: recover from the row partial (num valid samples slot)
      const T sm2 = part[b * NUM_SLOTS + P_NVS];
      const T mask2 = tm2 * sm2;
      if (mask2 != T(0)) gcurr[i] += coef * mask2;
    }
  }
}

// compute_score_centering_term over [B, L] tokens, one thread per token.
// Tokens with token_mask == 0 (or, when `sample_mask` is given, in a sample
// whose mask is 0) get zero term, head mass and coefficients.
// 64 threads per workgroup: one token per thread, spread over as many CUs as
// there are 64-token groups.
constexpr int kScTermThreads = 64;

template <class T>
__global__ __launch_bounds__(kScTermThreads) void sc_term_kernel(mirl_score_centering_args sc, int64_t B,
                                                      int64_t L, View<T> tm,
                                                      const T* __restrict__ sample_mask,
                                                      View<T> adv, int has_adv,
                                                      T* __restrict__ term,
                                                      T* __restrict__ head) {
  const int64_t i = (int64_t)blockIdx.x * kScTermThreads + threadIdx.x;
  if (i >= B * L) return;
  const int64_t b = i / L, l = i - b * L;
  T* coef = static_cast<T*>(sc.grad) + i * sc.K;
  if (tm(b, l) == T(0) || (sample_mask != nullptr && sample_mask[b] == T(0))) {
    term[i] = T(0);
    head[i] = T(0);
    for (int64_t k = 0; k < sc.K; ++k) coef[k] = T(0);
    return;
  }
  const T A = has_adv ? adv(b, l) : T(0);
  T t, h;
  score_centering_token<T>(sc, b, l, A, T(1), coef, &t, &h);
  term[i] = t;
  head[i] = h;
}

// dloss/dplog[b, l, k] = coef[b, l, k] * scale[b, l]; exactly 0 where the
// scale is 0 (tokens outside the final loss mask).  One thread per element.
template <class T>
__global__ __launch_bounds__(256) void sc_scale_kernel(T* __restrict__ grad,
                                                       const T* __restrict__ scale, int64_t K,
                                                       int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const T sc = scale[i / K];
  grad[i] = (sc == T(0)) ? T(0) : grad[i] * sc;
}

template <class T>
int run(const mirl_pg_config* cfg, int64_t B, int64_t L, const mirl_view2d* v,
        const void* sample_mask, const void* rewards, const void* gvs, const void* gvt,
        void* metrics, void* loss_out, void* gcurr, void* gunf,
        const mirl_score_centering_args* sc, void* ws, hipStream_t st) {
  Inputs<T> in;
  auto mk = [](const mirl_view2d& x) { return View<T>{static_cast<const T*>(x.ptr), x.sb, x.sl}; };
  in.curr = mk(v[0]);
  in.unf = mk(v[1]);
  in.tm = mk(v[2]);
  in.adv = mk(v[3]);
  in.prev = mk(v[4]);
  in.gen = mk(v[5]);
  in.ref = mk(v[6]);
  in.psm = MaskView{static_cast<const uint8_t*>(v[7].ptr), v[7].sb, v[7].sl};
  in.sample_mask = static_cast<const T*>(sample_mask);
  in.rewards = static_cast<const T*>(rewards);
  in.gvs = static_cast<const T*>(gvs);
  in.gvt = static_cast<const T*>(gvt);
  T* part = static_cast<T*>(ws);
  const int has_sc = sc != nullptr ? 1 : 0;
  ScWork<T> scw{nullptr, nullptr, nullptr};
  const int64_t n = B * L;
  if (has_sc) {
    // workspace layout: row partials, then term, head mass and scale ([B, L] each)
    scw.term = part + B * NUM_SLOTS;
    scw.head = scw.term + n;
    scw.scale = scw.head + n;
    if (n > 0)
      hipLaunchKernelGGL((sc_term_kernel<T>), dim3((unsigned)((n + kScTermThreads - 1) / kScTermThreads)),
                         dim3(kScTermThreads), 0, st,
                         *sc, B, L, in.tm, in.sample_mask, in.adv, 1, scw.term, scw.head);
  }
  hipLaunchKernelGGL((pg_rows_kernel<T, row_threads<T>()>), dim3((unsigned)B), dim3(row_threads<T>()), 0, st, *cfg, L, in,
                     static_cast<T*>(gcurr), static_cast<T*>(gunf), part, scw, has_sc);
  if (int e = check_launch("mirl_clipped_pg(rows)")) return e;
  hipLaunchKernelGGL((pg_final_kernel<T>), dim3(1), dim3(kFinalThreads), 0, st, *cfg, B, L, in,
                     static_cast<const T*>(part), static_cast<T*>(metrics),
                     static_cast<T*>(loss_out), static_cast<T*>(gcurr), has_sc);
  if (has_sc && n * sc->K > 0) {
    const int64_t ne = n * sc->K;
    hipLaunchKernelGGL((sc_scale_kernel<T>), dim3((unsigned)((ne + 255) / 256)), dim3(256), 0, st,
                       static_cast<T*>(sc->grad), static_cast<const T*>(scw.scale), sc->K, ne);
  }
  return check_launch("mirl_clipped_pg(final)");
}

template <class T>
int run_sc_term(int64_t B, int64_t L, const mirl_score_centering_args* sc, mirl_view2d tm,
                mirl_view2d adv, void* term, void* head, hipStream_t st) {
  const int64_t n = B * L;
  View<T> tmv{static_cast<const T*>(tm.ptr), tm.sb, tm.sl};
  View<T> av{static_cast<const T*>(adv.ptr), adv.sb, adv.sl};
  hipLaunchKernelGGL((sc_term_kernel<T>), dim3((unsigned)((n + kScTermThreads - 1) / kScTermThreads)),
                         dim3(kScTermThreads), 0, st, *sc,
                     B, L, tmv, static_cast<const T*>(nullptr), av, adv.ptr != nullptr ? 1 : 0,
                     static_cast<T*>(term), static_cast<T*>(head));
  return check_launch("mirl_score_centering_term");
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int64_t mirl_clipped_pg_workspace_elems(int64_t B, int64_t L, int score_centering) {
  return B * NUM_SLOTS + (score_centering ? 3 * B * L : 0);
}

// ---------------------------------------------------------------------------
// Scratch of mirl_clipped_pg_noalloc: a fixed array in the library's own
// device data, one copy on every GPU the library runs on, held until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the device symbol): the device address of
// each GPU's copy is looked up once per device with hipGetSymbolAddress and
// that address is what the kernels receive.
// ---------------------------------------------------------------------------
namespace mirl {
namespace {

constexpr int64_t kNoAllocScratchBytes = int64_t(4) << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch copy (looked up on the first
// call per device, then cached).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return MIRL_ERR_HIP;
  }
  MIRL_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                hipGetErrorString(e));
      return MIRL_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MIRL_OK;
}

}  // namespace
}  // namespace mirl

extern "C" int64_t mirl_clipped_pg_noalloc_max_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int mirl_clipped_pg_noalloc(const mirl_pg_config* cfg, int dtype, int64_t B, int64_t L,
                                       mirl_view2d curr, mirl_view2d unfiltered,
                                       mirl_view2d token_mask, mirl_view2d advantages,
                                       mirl_view2d prev, mirl_view2d generation,
                                       mirl_view2d reference, mirl_view2d support_mask,
                                       const void* sample_mask, const void* rewards,
                                       const void* global_valid_seqs,
                                       const void* global_valid_toks, void* metrics, void* loss,
                                       void* grad_curr, void* grad_unfiltered,
                                       const mirl_score_centering_args* score_centering,
                                       void* stream) {
  clear_error();
  MIRL_REQUIRE(dtype == MIRL_DTYPE_F32 || dtype == MIRL_DTYPE_F64,
               "mirl_clipped_pg_noalloc: dtype must be f32 or f64 (got %d)", dtype);
  MIRL_REQUIRE(B > 0 && L >= 0 && B < (int64_t(1) << 31) && L < (int64_t(1) << 40),
               "invalid shape B=%lld L=%lld", (long long)B, (long long)L);
  const int64_t elem = dtype == MIRL_DTYPE_F64 ? 8 : 4;
  const int64_t need =
      mirl_clipped_pg_workspace_elems(B, L, score_centering != nullptr ? 1 : 0) * elem;
  MIRL_REQUIRE(need <= kNoAllocScratchBytes,
               "mirl_clipped_pg_noalloc: B=%lld L=%lld needs %lld bytes of scratch; the "
               "no-allocation entry point holds at most %lld bytes (use mirl_clipped_pg with a "
               "caller workspace)",
               (long long)B, (long long)L, (long long)need, (long long)kNoAllocScratchBytes);
  void* ws = nullptr;
  if (int e = scratch_address(&ws)) return e;
  // Every scratch element the kernels read is written earlier in the same
  // call (row partials by pg_rows_kernel, score-centering terms by
  // sc_term_kernel), so nothing needs clearing between calls.
  return mirl_clipped_pg(cfg, dtype, B, L, curr, unfiltered, token_mask, advantages, prev,
                         generation, reference, support_mask, sample_mask, rewards,
                         global_valid_seqs, global_valid_toks, metrics, loss, grad_curr,
                         grad_unfiltered, score_centering, ws, stream);
}

extern "C" int mirl_clipped_pg(const mirl_pg_config* cfg, int dtype, int64_t B, int64_t L,
                               mirl_view2d curr, mirl_view2d unfiltered, mirl_view2d token_mask,
                               mirl_view2d advantages, mirl_view2d prev, mirl_view2d generation,
                               mirl_view2d reference, mirl_view2d support_mask,
                               const void* sample_mask, const void* rewards,
                               const void* global_valid_seqs, const void* global_valid_toks,
                               void* metrics, void* loss, void* grad_curr, void* grad_unfiltered,
                               const mirl_score_centering_args* score_centering, void* workspace,
                               void* stream) {
  clear_error();
  MIRL_REQUIRE(cfg != nullptr, "null config");
  MIRL_REQUIRE(B > 0 && L >= 0, "invalid shape B=%lld L=%lld", (long long)B, (long long)L);
  MIRL_REQUIRE(B < (int64_t(1) << 31), "batch too large");
  MIRL_REQUIRE(curr.ptr && token_mask.ptr && advantages.ptr && generation.ptr && sample_mask &&
                   global_valid_seqs && global_valid_toks && metrics && grad_curr && workspace,
               "null pointer argument");
  MIRL_REQUIRE(cfg->force_on_policy || prev.ptr, "prev_logprobs required");
  MIRL_REQUIRE(cfg->kl_penalty == 0.0 || reference.ptr, "reference_policy_logprobs required");
  MIRL_REQUIRE(!cfg->has_unfiltered || (unfiltered.ptr && grad_unfiltered),
               "curr_logprobs_unfiltered and its gradient buffer required");
  MIRL_REQUIRE(!cfg->has_support_mask || support_mask.ptr, "policy_support_mask required");
  MIRL_REQUIRE(!cfg->has_rewards || rewards, "rewards required");
  MIRL_REQUIRE(cfg->kl_type >= MIRL_KL_K1 && cfg->kl_type <= MIRL_KL_K3, "invalid KL type %d",
               cfg->kl_type);
  MIRL_REQUIRE(cfg->tis_type >= MIRL_TIS_NONE && cfg->tis_type <= MIRL_TIS_SEQ_MASK,
               "invalid truncated IS type %d", cfg->tis_type);
  if (score_centering != nullptr) {
    const mirl_score_centering_args& sc = *score_centering;
    MIRL_REQUIRE(sc.mode >= MIRL_SC_OFF && sc.mode <= MIRL_SC_ADAPTIVE,
                 "invalid score-centering mode %d", sc.mode);
    MIRL_REQUIRE(sc.K >= 0, "invalid score-centering K=%lld", (long long)sc.K);
    MIRL_REQUIRE(sc.K == 0 || (sc.plog && sc.qlog && sc.grad),
                 "score centering needs plog, qlog and a gradient buffer");
  }
  const mirl_view2d views[8] = {curr, unfiltered, token_mask, advantages,
                                prev, generation, reference, support_mask};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32)
    return run<float>(cfg, B, L, views, sample_mask, rewards, global_valid_seqs, global_valid_toks,
                      metrics, loss, grad_curr, grad_unfiltered, score_centering, workspace, st);
  if (dtype == MIRL_DTYPE_F64)
    return run<double>(cfg, B, L, views, sample_mask, rewards, global_valid_seqs,
                       global_valid_toks, metrics, loss, grad_curr, grad_unfiltered, score_centering,
                       workspace, st);
  set_error("mirl_clipped_pg: dtype must be f32 or f64 (got %d)", dtype);
  return MIRL_ERR_UNSUPPORTED;
}

extern "C" int mirl_score_centering_term(int dtype, int64_t B, int64_t L,
                                         const mirl_score_centering_args* args,
                                         mirl_view2d token_mask, mirl_view2d advantages,
                                         void* term, void* head_mass, void* stream) {
  clear_error();
  MIRL_REQUIRE(args != nullptr, "null score-centering arguments");
  MIRL_REQUIRE(B >= 0 && L >= 0 && args->K >= 0, "invalid shape B=%lld L=%lld K=%lld",
               (long long)B, (long long)L, (long long)args->K);
  MIRL_REQUIRE(args->mode >= MIRL_SC_OFF && args->mode <= MIRL_SC_ADAPTIVE,
               "invalid score-centering mode %d", args->mode);
  MIRL_REQUIRE(args->mode != MIRL_SC_ADAPTIVE || advantages.ptr != nullptr,
               "adaptive-ppo-clip score centering needs the advantages");
  if (B * L == 0) return MIRL_OK;
  MIRL_REQUIRE(B * L < (int64_t(1) << 40), "too many tokens");
  MIRL_REQUIRE(token_mask.ptr && term && head_mass && (args->K == 0 || (args->plog && args->qlog && args->grad)),
               "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32)
    return run_sc_term<float>(B, L, args, token_mask, advantages, term, head_mass, st);
  if (dtype == MIRL_DTYPE_F64)
    return run_sc_term<double>(B, L, args, token_mask, advantages, term, head_mass, st);
  set_error("mirl_score_centering_term: dtype must be f32 or f64 (got %d)", dtype);
  return MIRL_ERR_UNSUPPORTED;
}

// Per-token arithmetic of the ClippedPG objective (the terms pg_rows_kernel
// accumulates and the closed-form gradient of one token), as one function with
// floating-point contraction off: any kernel that evaluates a token's loss
// gradient with it gets the loss kernel's bits, which a device-side comparison
// with the loss kernel's gradient (an early-started backward's check) needs.
//
// Semantics: nemo_rl/algorithms/loss/loss_functions.py:840-1130 (the per-token
// terms of __call__), nemo_rl/algorithms/loss/clipped_pg.py:131-194
// (clipped_pg_actor_objective), nemo_rl/algorithms/utils.py:56-115
// (calculate_kl).  Gradient rules are PyTorch's autograd rules for the same op
// sequence: maximum/minimum split the gradient 50/50 on exact ties, clamp
// passes it on the closed interval, nan_to_num passes it where the input was
// finite.

#pragma once

#include "common.h"

namespace mirl {
namespace pg {

template <class T>
struct View {
  const T* p;
  int64_t sb, sl;
  __device__ __forceinline__ T operator()(int64_t b, int64_t l) const { return p[b * sb + l * sl]; }
};

struct MaskView {
  const uint8_t* p;
  int64_t sb, sl;
  __device__ __forceinline__ bool operator()(int64_t b, int64_t l) const {
    return p[b * sb + l * sl] != 0;
  }
};

template <class T>
__device__ __forceinline__ T dexp(T x) {
  if constexpr (sizeof(T) == 8) return exp(x); else return expf(x);
}
template <class T>
__device__ __forceinline__ T dlog(T x) {
  if constexpr (sizeof(T) == 8) return log(x); else return logf(x);
}
template <class T>
__device__ __forceinline__ T dabs(T x) {
  if constexpr (sizeof(T) == 8) return fabs(x); else return fabsf(x);
}
template <class T>
__device__ __forceinline__ T nan_to_zero_all(T x) {
  // nan_to_num(x, nan=0, posinf=0, neginf=0)
  return isfinite(x) ? x : T(0);
}
template <class T>
__device__ __forceinline__ T dclamp(T x, T lo, T hi) {
  // torch.clamp: min then max, NaN propagates
  if (isnan(x)) return x;
  return x < lo ? lo : (x > hi ? hi : x);
}

// maximum(a, b) gradient share of a (PyTorch: ties split evenly)
template <class T>
__device__ __forceinline__ T max_share_a(T a, T b) {
  return a > b ? T(1) : (a < b ? T(0) : T(0.5));
}

// Per-token KL estimate k(logr) and its derivative dk/dlogr.
template <class T>
__device__ __forceinline__ T kl_value(int type, T lr) {
  if (type == MIRL_KL_K1) return -lr;
  if (type == MIRL_KL_K2) return (lr * lr) / T(2);
  return (dexp(lr) - T(1)) - lr;
}
template <class T>
__device__ __forceinline__ T kl_deriv(int type, T lr) {
  if (type == MIRL_KL_K1) return T(-1);
  if (type == MIRL_KL_K2) return lr;
  return dexp(lr) - T(1);
}

// Truncated importance sampling applied to one weight (loss_functions.py:921-1013).
// `oob` reports whether the weight fell outside the truncation bounds.
template <class T>
__device__ __forceinline__ T truncate_is(const mirl_pg_config& cfg, T w, T A, T seq_kept, bool* oob) {
  if (cfg.tis_type == MIRL_TIS_TIS) {
    const T tmin = T(cfg.tis_ratio_min), tmax = T(cfg.tis_ratio);
    *oob = (w > tmax) || (w < tmin);
    return dclamp(w, tmin, tmax);
  }
  if (cfg.tis_type == MIRL_TIS_ICEPOP) {
    const bool kept = (w >= T(cfg.tis_ratio_min)) && (w <= T(cfg.tis_ratio));
    *oob = !kept;
    return kept ? w : T(0);
  }
  if (cfg.tis_type == MIRL_TIS_ADAPTIVE) {
    const bool kept = (w <= T(cfg.adaptive_outer)) && ((A >= T(0)) || (w >= T(cfg.tis_ratio_min))) &&
                      ((A <= T(0)) || (w <= T(cfg.adaptive_hi)));
    *oob = !kept;
    return kept ? w : T(0);
  }
  if (cfg.tis_type == MIRL_TIS_SEQ_MASK) {
    *oob = false;
    return w * seq_kept;
  }
  *oob = false;
  return w;
}

// One token's operands.  pv, gv are the sanitised prev / generation logprobs
// (0 outside the final mask); cu, rf, kgen the KL operands (0 outside the KL
// mask).  The row quantities (masks, normalisers, sequence-level ratio and IS
// weight) come from the caller.
template <class T>
struct TokenIn {
  T tmv, tm2, sm, sm2;   // token mask, after the support adjustment; row masks
  T craw, c, pv, gv, A;  // current logprob (raw and masked), prev, generation, advantage
  T cu, rf, kgen;        // KL operands
  T gvt, gvs;            // global normalisers (+1e-8)
  T actor_row_norm, kl_row_norm;
  T r_seq, w_seq, seq_kept;
  bool seq_ratio;
};

// What the loss kernels accumulate from one token, and its gradient.
template <class T>
struct TokenOut {
  T gc;     // d(loss)/d(curr) of this token (grad_loss = 1), without the NLL term
  T gu;     // d(loss)/d(unfiltered curr)
  T klt;    // beta * clamped KL estimate (0 without KL)
  T w;      // importance weight after truncation (1 when not needed)
  bool oob; // the weight fell outside the truncation bounds
  T r, rc;  // ratio and clamped ratio
  T v;      // weighted clipped objective
  T alpha;  // the token's weight in the actor loss
  T gspo;   // alpha * w * dcl/dr (sequence-level ratio gradient share)
};

template <class T>
__device__ __forceinline__ TokenOut<T> token_terms(const mirl_pg_config& cfg, const TokenIn<T>& t) {
#pragma clang fp contract(off)
  TokenOut<T> o;
  const T mask2 = t.tm2 * t.sm2;
  const T kl_mask = t.tmv * t.sm;
  const bool on = mask2 != T(0);
  const T beta = T(cfg.kl_penalty);
  const T A = t.A;
  const T c = t.c, pv = t.pv, gv = t.gv;
  o.gc = T(0);
  o.gu = T(0);
  o.klt = T(0);

  // KL term (utils.py:56-115) ----------------------------------------------
  if (cfg.kl_penalty != 0.0) {
    const bool kon = kl_mask != T(0);
    const T cu = t.cu, rf = t.rf, kgen = t.kgen;
    // importance weight exp(cu - X), X detached
    const T e = cfg.use_on_policy_kl ? dexp(cu - kgen) : dexp(cu - cu);
    const T w = nan_to_zero_all(e);
    const T dw = isfinite(e) ? e : T(0);
    T lr = rf - cu;
    T dlr_pass = T(1);  // d(clamped logr)/d(logr)
    bool w_grad = true;
    if (cfg.has_kl_input_clamp) {
      const T ic = T(cfg.kl_input_clamp);
      const T lc = dclamp(lr, -ic, ic);
      w_grad = (lr == lc);
      dlr_pass = (lr >= -ic && lr <= ic) ? T(1) : T(0);
      lr = lc;
    }
    const T k = kl_value<T>(cfg.kl_type, lr);
    T kw = w * k;
    T out_pass = T(1);
    if (cfg.has_kl_output_clamp) {
      const T oc = T(cfg.kl_output_clamp);
      out_pass = (kw >= -oc && kw <= oc) ? T(1) : T(0);
      kw = dclamp(kw, -oc, oc);
    }
    o.klt = beta * kw;
    const T kappa = cfg.token_level_loss ? kl_mask / t.gvt
                                         : t.sm * t.tmv / (t.kl_row_norm * t.gvs);
    // d kl_t / d cu
    const T dk = kl_deriv<T>(cfg.kl_type, lr) * dlr_pass * T(-1);
    const T dkl = beta * out_pass * ((w_grad ? dw : T(0)) * k + w * dk);
    const T g = kon ? kappa * dkl : T(0);
    if (cfg.has_unfiltered) o.gu = g; else o.gc = o.gc + g;
  }

  // importance weights (loss_functions.py:905-1013) --------------------------
  T w = T(1);
  bool has_w = false;
  o.oob = false;
  if (cfg.need_is) {
    has_w = true;
    w = cfg.sequence_level_is ? t.w_seq : nan_to_zero_all(dexp(pv - gv));
    w = truncate_is(cfg, w, A, t.seq_kept, &o.oob);
  }
  o.w = w;
  const bool use_w = cfg.use_is_correction != 0;

  // actor objective (clipped_pg.py:131-194) ----------------------------------
  const T lo = T(1.0 - cfg.ratio_clip_min);
  const T hi = T(1.0 + cfg.ratio_clip_max);
  T r, rc, dr_dc, drc_dr;
  if (cfg.force_on_policy) {
    r = dexp(c - c);
    rc = r;
    dr_dc = r;
    drc_dr = T(1);
  } else if (!cfg.disable_ppo_ratio) {
    if (cfg.sequence_level_is) {
      r = t.r_seq;
      dr_dc = T(0);  // handled through the sequence-level share
    } else {
      r = dexp(c - pv);
      dr_dc = r;
    }
    rc = dclamp(r, lo, hi);
    drc_dr = (r >= lo && r <= hi) ? T(1) : T(0);
  } else {
    r = c;
    rc = c;
    dr_dc = T(1);
    drc_dr = T(1);
  }
  o.r = r;
  o.rc = rc;
  const T na = -A;
  T cl, dcl_dr = T(0), dcl_dc_direct = T(0);
  if (cfg.use_cispo) {
    cl = (na * rc) * c;
    dcl_dc_direct = na * rc;
  } else {
    const T a1 = na * r, a2 = na * rc;
    cl = a1 > a2 ? a1 : (a1 < a2 ? a2 : a1);
    if (isnan(a1) || isnan(a2)) cl = a1 + a2;
    const T sa = max_share_a(a1, a2);
    dcl_dr = sa * na + (T(1) - sa) * na * drc_dr;
    if (cfg.ratio_clip_c > 0.0 && A < T(0)) {
      const T z = na * T(cfg.ratio_clip_c);
      const T s = cl < z ? T(1) : (cl > z ? T(0) : T(0.5));
      cl = cl < z ? cl : z;
      dcl_dr *= s;
    }
  }
  const T wv = (has_w && use_w) ? w : T(1);
  o.v = wv * cl;
  o.alpha = cfg.token_level_loss ? mask2 / t.gvt : t.sm2 * t.tm2 / (t.actor_row_norm * t.gvs);
  o.gspo = T(0);
  if (cfg.use_cispo) {
    o.gc = o.gc + (on ? o.alpha * wv * dcl_dc_direct : T(0));
  } else if (t.seq_ratio) {
    o.gspo = o.alpha * wv * dcl_dr;
  } else {
    o.gc = o.gc + (on ? o.alpha * wv * dcl_dr * dr_dc : T(0));
  }
  return o;
}

}  // namespace pg
}  // namespace mirl

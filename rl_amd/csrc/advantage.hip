// GRPO group-normalised advantages.
//
// One thread per sample.  A sample's group is every row whose prompt key
// equals its own (exact row equality, as torch.unique(prompts, dim=0) groups
// them); the O(B^2 K) scan is trivial next to the logprob passes (B is the
// number of generations in a microbatch).  Group sums are accumulated in
// double and rounded once to fp32, where the reference uses an fp32
// matrix-vector product; the two agree to the last fp32 ulp of the sum.
//
// Semantics: nemo_rl/algorithms/utils.py:118-234
// (calculate_baseline_and_std_per_prompt) and
// nemo_rl/algorithms/advantage_estimator.py:106-145
// (GRPOAdvantageEstimator.compute_advantage).

#include <cfloat>

#include "common.h"

namespace mirl {
namespace {

__global__ __launch_bounds__(256) void grpo_advantage_kernel(const int64_t* __restrict__ prompts,
                                                             int64_t B, int64_t K, int64_t ps,
                                                             const float* __restrict__ rewards,
                                                             const float* __restrict__ srew,
                                                             const float* __restrict__ valid,
                                                             int loo, int normalize,
                                                             float* __restrict__ adv,
                                                             float* __restrict__ baseline_out,
                                                             float* __restrict__ std_out,
                                                             uint8_t* __restrict__ trivial_out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B) return;
  const int64_t* pi = prompts + i * ps;
  float n = 0.f;
  double srv = 0.0, sqv = 0.0, sq2v = 0.0;
  float cmin = INFINITY, cmax = -INFINITY;
  for (int64_t j = 0; j < B; ++j) {
    const int64_t* pj = prompts + j * ps;
    bool same = true;
    for (int64_t k = 0; k < K; ++k) same = same && (pi[k] == pj[k]);
    if (!same) continue;
    const float vj = valid ? valid[j] : 1.f;
    const float rj = rewards[j];
    const float qj = srew ? srew[j] : rj;
    n += vj;
    if (loo && j == i) continue;
    srv += (double)(rj * vj);
    sqv += (double)(qj * vj);
    sq2v += (double)((qj * qj) * vj);
    if (vj != 0.f) {
      cmin = fminf(cmin, qj);
      cmax = fmaxf(cmax, qj);
    }
  }
  const float ri = rewards[i];
  float base, sd = 0.f;
  bool trivial = true;
  if (n <= 1.f) {
    base = ri;
  } else {
    const float nv = n - (loo ? 1.f : 0.f);
    base = (float)srv / nv;
    const float qbar = srew ? (float)sqv / nv : base;
    const float sq = (float)sq2v / nv;
    trivial = (cmin == cmax);
    sd = sqrtf((sq - qbar * qbar) * (nv / (nv - 1.f)));
    if (isnan(sd)) sd = 0.f;
    else if (isinf(sd)) sd = sd > 0.f ? FLT_MAX : -FLT_MAX;
  }
  float a = ri - base;
  if (normalize && sd > 0.f && !trivial) a = a / (sd + 1e-6f);
  adv[i] = a;
  if (baseline_out) baseline_out[i] = base;
  if (std_out) std_out[i] = sd;
  if (trivial_out) trivial_out[i] = trivial ? 1 : 0;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_grpo_advantage(const int64_t* prompts, int64_t B, int64_t K,
                                   int64_t prompt_stride, const float* rewards,
                                   const float* std_rewards, const float* valid_mask,
                                   int leave_one_out, int normalize,
                                   float* adv, float* baseline, float* std, uint8_t* trivial,
                                   void* stream) {
  clear_error();
  MIRL_REQUIRE(B >= 0 && K > 0, "invalid shape B=%lld K=%lld", (long long)B, (long long)K);
  if (B == 0) return MIRL_OK;
  MIRL_REQUIRE(prompts && rewards && adv, "null pointer argument");
  const unsigned blocks = (unsigned)((B + 255) / 256);
  hipLaunchKernelGGL(grpo_advantage_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), prompts, B, K, prompt_stride, rewards,
                     std_rewards, valid_mask, leave_one_out, normalize, adv, baseline, std, trivial);
  return check_launch("mirl_grpo_advantage");
}

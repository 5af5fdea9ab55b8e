// GRPO group-normalised advantages.
//
// One thread per sample.  A sample's group is every row whose prompt key
// equals its own (exact row equality, as torch.unique(prompts, dim=0) groups
// them), found by a scan over the other samples in ascending order: one thread
// per sample for single-element keys (group ids), one wave per sample for
// longer keys (prompt token rows), where a pair is told apart by its first
// elements in almost every case and rows that agree there are compared 64
// elements at a time with coalesced loads, O(B^2 + B n K) for groups of n.
// Group sums are accumulated in double and rounded once to fp32, where the
// reference uses an fp32 matrix-vector product; the two agree to the last
// fp32 ulp of the sum.
//
// Semantics: nemo_rl/algorithms/utils.py:118-234
// (calculate_baseline_and_std_per_prompt) and
// nemo_rl/algorithms/advantage_estimator.py:106-145
// (GRPOAdvantageEstimator.compute_advantage).

#include <cfloat>

#include "common.h"

namespace mirl {
namespace {

struct AdvArgs {
  const int64_t* prompts;
  int64_t B, K, ps;
  const float* rewards;
  const float* srew;
  const float* valid;
  int loo, normalize;
  float* adv;
  float* baseline_out;
  float* std_out;
  uint8_t* trivial_out;
};

// The advantage of sample i; same(j) tells whether sample j is in i's group.
template <class Same>
__device__ __forceinline__ void sample_advantage(const AdvArgs& A, int64_t i, Same&& same) {
  const int64_t B = A.B;
  const float* __restrict__ rewards = A.rewards;
  const float* __restrict__ srew = A.srew;
  const float* __restrict__ valid = A.valid;
  const int loo = A.loo, normalize = A.normalize;
  float n = 0.f;
  double srv = 0.0, sqv = 0.0, sq2v = 0.0;
  float cmin = INFINITY, cmax = -INFINITY;
  for (int64_t j = 0; j < B; ++j) {
    if (!same(j)) continue;
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
  A.adv[i] = a;
  if (A.baseline_out) A.baseline_out[i] = base;
  if (A.std_out) A.std_out[i] = sd;
  if (A.trivial_out) A.trivial_out[i] = trivial ? 1 : 0;
}

// Rows i and j equal?  The first elements decide most pairs at once; the rest
// is compared with independent loads (no chain of dependent ones).
__device__ __forceinline__ bool same_key(const AdvArgs& A, int64_t i, int64_t j) {
  if (i == j) return true;
  const int64_t* pi = A.prompts + i * A.ps;
  const int64_t* pj = A.prompts + j * A.ps;
  if (pi[0] != pj[0]) return false;
  uint64_t diff = 0;
  for (int64_t k = 1; k < A.K; ++k) diff |= (uint64_t)(pi[k] ^ pj[k]);
  return diff == 0;
}

__global__ __launch_bounds__(256) void grpo_advantage_kernel(AdvArgs A) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= A.B) return;
  sample_advantage(A, i, [&](int64_t j) { return same_key(A, i, j); });
}

// Keys of more than one element: one wave per sample.  The wave walks the
// other samples together (every lane runs the same accumulation in the same
// order, so every lane holds the thread kernel's bits); a row that agrees on
// its first element is compared 64 elements at a time with coalesced loads and
// a ballot.
__global__ __launch_bounds__(256) void grpo_advantage_wave_kernel(AdvArgs A) {
  const int64_t i = (int64_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (i >= A.B) return;  // whole waves leave together
  const int lane = threadIdx.x % kWave;
  const int64_t* pi = A.prompts + i * A.ps;
  const int64_t p0 = pi[0];
  sample_advantage(A, i, [&](int64_t j) {
    if (j == i) return true;
    const int64_t* pj = A.prompts + j * A.ps;
    if (pj[0] != p0) return false;
    uint64_t diff = 0;
    for (int64_t k = 1 + lane; k < A.K; k += kWave) diff |= (uint64_t)(pi[k] ^ pj[k]);
    return __ballot(diff != 0) == 0ull;
  });
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
  AdvArgs a{prompts, B, K, prompt_stride, rewards, std_rewards, valid_mask, leave_one_out, normalize,
            adv, baseline, std, trivial};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K > 1) {
    const unsigned blocks = (unsigned)((B + 3) / 4);  // four samples (waves) per workgroup
    hipLaunchKernelGGL(grpo_advantage_wave_kernel, dim3(blocks), dim3(256), 0, st, a);
  } else {
    const unsigned blocks = (unsigned)((B + 255) / 256);
    hipLaunchKernelGGL(grpo_advantage_kernel, dim3(blocks), dim3(256), 0, st, a);
  }
  return check_launch("mirl_grpo_advantage");
}

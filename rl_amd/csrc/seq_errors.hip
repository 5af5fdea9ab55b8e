// Token-level post-processing of logprobs: masking filtered logprobs outside
// the valid tokens, and the per-sequence multiplicative logprob error.
//
// Semantics (reference nemo_rl/algorithms/utils.py:273-291 and :309-326):
//   mask_filtered_logprobs_outside_tokens:  out = where(mask != 0, lp, 0)
//   compute_seq_logprob_errors, per sequence b with w_s = token_mask[b,s] *
//   sample_mask[b] (fp32 product):
//     count  = sum_s w_s
//     err_s  = (w_s != 0) ? |generation[b,s] - policy[b,s]| : 0
//     errors = (sum_s exp(err_s * w_s) * w_s) / max(count, 1)
//     valid  = count > 0
// A non-finite logprob on a valid token makes that sequence's error
// non-finite (NaN or inf); on a masked token it contributes nothing.  The
// sums run in fp32 in a lane-strided order and a wave tree (torch's own
// reduction order differs; both are fp32 sums of the same terms).

#include "common.h"

namespace mirl {
namespace {

struct Strided2 {
  const float* p;
  int64_t sb, ss;
  __device__ float at(int64_t b, int64_t s) const { return p[b * sb + s * ss]; }
};

__global__ __launch_bounds__(256) void mask_outside_kernel(Strided2 lp, Strided2 mask, float* out,
                                                           int64_t osb, int64_t oss, int64_t S,
                                                           int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const int64_t b = i / S, s = i - b * S;
    out[b * osb + s * oss] = mask.at(b, s) != 0.f ? lp.at(b, s) : 0.f;
  }
}

// One wave per sequence.
__global__ __launch_bounds__(256) void seq_errors_kernel(Strided2 pol, Strided2 gen, Strided2 tm,
                                                         const float* sm, int64_t smb, int64_t B,
                                                         int64_t S, float* errors,
                                                         uint8_t* valid) {
  const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;
  const float smv = sm[b * smb];
  float cnt = 0.f, acc = 0.f;
  for (int64_t s = lane; s < S; s += 64) {
    const float w = tm.at(b, s) * smv;
    cnt += w;
    const float err = (w != 0.f) ? fabsf(gen.at(b, s) - pol.at(b, s)) : 0.f;
    acc += expf(err * w) * w;
  }
  cnt = wave_sum(cnt);
  acc = wave_sum(acc);
  if (lane == 0) {
    errors[b] = acc / fmaxf(cnt, 1.f);
    valid[b] = cnt > 0.f ? 1 : 0;
  }
}

int grid_for(int64_t n) {
  const int64_t blocks = (n + 255) / 256;
  return (int)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_mask_outside_tokens(const float* logprobs, int64_t B, int64_t S, int64_t lp_sb,
                                        int64_t lp_ss, const float* mask, int64_t m_sb,
                                        int64_t m_ss, float* out, int64_t o_sb, int64_t o_ss,
                                        void* stream) {
  clear_error();
  MIRL_REQUIRE(B >= 0 && S >= 0, "invalid shape B=%lld S=%lld", (long long)B, (long long)S);
  const int64_t n = B * S;
  if (n == 0) return MIRL_OK;
  MIRL_REQUIRE(logprobs && mask && out, "null pointer argument");
  hipLaunchKernelGGL(mask_outside_kernel, dim3(grid_for(n)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), Strided2{logprobs, lp_sb, lp_ss},
                     Strided2{mask, m_sb, m_ss}, out, o_sb, o_ss, S, n);
  return check_launch("mirl_mask_outside_tokens");
}

extern "C" int mirl_seq_logprob_errors(const float* policy, int64_t p_sb, int64_t p_ss,
                                       const float* generation, int64_t g_sb, int64_t g_ss,
                                       const float* token_mask, int64_t t_sb, int64_t t_ss,
                                       const float* sample_mask, int64_t s_sb, int64_t B,
                                       int64_t S, float* errors, uint8_t* valid, void* stream) {
  clear_error();
  MIRL_REQUIRE(B >= 0 && S >= 0, "invalid shape B=%lld S=%lld", (long long)B, (long long)S);
  if (B == 0) return MIRL_OK;
  MIRL_REQUIRE(errors && valid && sample_mask, "null pointer argument");
  MIRL_REQUIRE(S == 0 || (policy && generation && token_mask), "null pointer argument");
  hipLaunchKernelGGL(seq_errors_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), Strided2{policy, p_sb, p_ss},
                     Strided2{generation, g_sb, g_ss}, Strided2{token_mask, t_sb, t_ss},
                     sample_mask, s_sb, B, S, errors, valid);
  return check_launch("mirl_seq_logprob_errors");
}

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

// out = mask != 0 ? logprobs : 0, element by element, for an element of W bytes
// (the select copies the value's bits, so any float dtype of that width is exact;
// all-zero bits are +0.0 in every float format).
template <class W>
__global__ __launch_bounds__(256) void mask_outside_kernel(const W* lp, int64_t lsb, int64_t lss,
                                                           Strided2 mask, W* out, int64_t osb,
                                                           int64_t oss, int64_t S, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const int64_t b = i / S, s = i - b * S;
    out[b * osb + s * oss] = mask.at(b, s) != 0.f ? lp[b * lsb + s * lss] : W(0);
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

extern "C" int mirl_mask_outside_tokens(const void* logprobs, int dtype, int64_t B, int64_t S,
                                        int64_t lp_sb, int64_t lp_ss, const float* mask,
                                        int64_t m_sb, int64_t m_ss, void* out, int64_t o_sb,
                                        int64_t o_ss, void* stream) {
  clear_error();
  MIRL_REQUIRE(B >= 0 && S >= 0, "invalid shape B=%lld S=%lld", (long long)B, (long long)S);
  MIRL_REQUIRE(dtype == MIRL_DTYPE_F32 || dtype == MIRL_DTYPE_BF16 || dtype == MIRL_DTYPE_F16 ||
                   dtype == MIRL_DTYPE_F64,
               "unsupported logprobs dtype code %d", dtype);
  const int64_t n = B * S;
  if (n == 0) return MIRL_OK;
  MIRL_REQUIRE(logprobs && mask && out, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Strided2 m{mask, m_sb, m_ss};
  if (dtype == MIRL_DTYPE_F32)
    hipLaunchKernelGGL(mask_outside_kernel<uint32_t>, dim3(grid_for(n)), dim3(256), 0, st,
                       static_cast<const uint32_t*>(logprobs), lp_sb, lp_ss, m,
                       static_cast<uint32_t*>(out), o_sb, o_ss, S, n);
  else if (dtype == MIRL_DTYPE_F64)
    hipLaunchKernelGGL(mask_outside_kernel<uint64_t>, dim3(grid_for(n)), dim3(256), 0, st,
                       static_cast<const uint64_t*>(logprobs), lp_sb, lp_ss, m,
                       static_cast<uint64_t*>(out), o_sb, o_ss, S, n);
  else
    hipLaunchKernelGGL(mask_outside_kernel<uint16_t>, dim3(grid_for(n)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(logprobs), lp_sb, lp_ss, m,
                       static_cast<uint16_t*>(out), o_sb, o_ss, S, n);
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

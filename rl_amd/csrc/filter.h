// Shared definitions of the top-k / top-p filter kernels (topk_filter.hip,
// topk_hist.hip): the per-row result record, the launch parameters, order
// keys of floating-point values and workgroup reductions.
#pragma once

#include <type_traits>

#include "common.h"

namespace mirl {

template <class E>
constexpr int dtype_code() {
  return std::is_same<E, F32>::value ? MIRL_DTYPE_F32
         : std::is_same<E, BF16>::value ? MIRL_DTYPE_BF16 : MIRL_DTYPE_F16;
}

constexpr int kKeepCap = MIRL_FILTER_KEEP_CAP;

// Per-row result of the forward (layout documented as mirl_filter_row_info).
struct RowInfo {
  float m;        // max of the kept values
  float logsum;   // log(sum_kept exp(y - m))
  float v_cut;    // kept <=> y > v_cut || (y == v_cut && j >= i_cut)
  int32_t i_cut;  // < 0: rank form, kept among y == v_cut <=> rank in index order >= -1 - i_cut
  int32_t n_kept;
  int32_t flags;  // bit 0: row must be (re)done by a general path; bit 2: no kept list;
                  // bit 3: a 16-bit top-p cut decided by the exact sequential sum
};
constexpr int kFlagRedo = 1;
constexpr int kFlagNoKeptList = 4;
constexpr int kFlagWalked = 8;
static_assert(sizeof(RowInfo) == sizeof(mirl_filter_row_info), "row info layout");

struct FilterParams {
  const void* logits;
  int64_t R, V, sb, sr;
  const int64_t* target;  // [B, R] view or null
  int64_t tsb, tsr;
  float rT;   // temperature_recip(T): y = dtype(fl32(float(x) * rT))
  int has_t;
  int top_k;  // 0: no top-k
  int has_p;
  float cut;  // fp32(1 - top_p)
  // top-p decided in the 16-bit logits dtype: probabilities rounded to the
  // dtype, their cumulative sum accumulated one element at a time in fp32 and
  // each partial sum rounded to the dtype, compared with thr16 =
  // dtype(fp32(1 - top_p)).  0: decided in fp32 (cumulative sum in double,
  // rounded to fp32, compared with `cut`).
  int dec16;
  float thr16;
  float* out;  // [rows] logprobs or null
  RowInfo* info;
  int32_t* kept_idx;  // [rows, kKeepCap]
  float* kept_p;      // [rows, kKeepCap]
  // top-k export (vocab_topk): [rows, top_k] values and global ids, or null
  float* tk_vals;
  int64_t* tk_idx;
  int64_t tk_base;
  // fp32 two-pass kernel: sum the mass below the cut's bracket exactly in a
  // third pass on every row instead of bounding it (environment variable
  // MIRL_F32_FILTER_EXACT_BELOW=1; tests use it to cover that pass)
  int f32_exact_below;
};

// Order-preserving integer key of a float.  -0.0 maps to the key of +0.0: the
// two compare equal, so a sort treats them as ties ordered by index.
__device__ __forceinline__ uint32_t okey(float y) {
  const uint32_t u = __float_as_uint(y == 0.f ? 0.f : y);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float from_okey(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
__device__ __forceinline__ bool kept_lex(float y, int64_t j, float vc, int32_t ic) {
  return y > vc || (y == vc && j >= (int64_t)ic);
}

// y = dtype(fl32(float(x) * rT)), the logits after the in-place temperature
template <class E>
__device__ __forceinline__ float scaled(float xf, const FilterParams& P) {
  return P.has_t ? round_trip<E>(mul_rn(xf, P.rT)) : xf;
}

// Workgroup reductions over NT threads; `red` holds NT / 64 values.
template <int NT>
__device__ float block_sum_f(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  float r = 0.f;
  for (int k = 0; k < NT / 64; ++k) r += red[k];
  return r;
}
// Sum over NT threads in double; `red` holds NT / 64 doubles.
template <int NT>
__device__ double block_sum_d(double v, double* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  double r = 0.0;
  for (int k = 0; k < NT / 64; ++k) r += red[k];
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ float block_max_f(float v, float* red) {
  v = wave_max(v);
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  float r = red[0];
  for (int k = 1; k < NT / 64; ++k) r = fmaxf(r, red[k]);
  return r;
}
template <int NT>
__device__ int block_sum_i(int v, int* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x % 64, wv = threadIdx.x / 64;
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  int r = 0;
  for (int k = 0; k < NT / 64; ++k) r += red[k];
  return r;
}

// The lowest thread of the workgroup whose flag is set goes into *slot (which
// holds a larger value beforehand) by an LDS minimum.  LDS atomics that many
// lanes aim at one address are serialised (a whole flagged wave costs
// microseconds), so each wave sends one, from its lowest flagged lane.  Every
// thread of the wave calls it.
__device__ __forceinline__ void block_first_flagged(bool f, int* slot) {
  const uint64_t m = __ballot(f);
  if (m != 0u && (int)(threadIdx.x & 63u) == __ffsll((long long)m) - 1)
    atomicMin(slot, (int)threadIdx.x);
}
// Unsigned maximum and minimum over the 64 lanes of a wave.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, off, 64));
  return v;
}

// Cross-lane moves by DPP (no LDS traffic): row_shr:n shifts within rows of 16
// lanes, row_bcast:15 / row_bcast:31 pass a row's last lane on to the next
// row(s).  Lanes with no source, and rows outside ROWMASK, read 0, the
// identity of the sums and unsigned maxima below.
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xf, false);
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint64_t lo = dpp_u32<CTRL, ROWMASK>((uint32_t)u);
  const uint64_t hi = dpp_u32<CTRL, ROWMASK>((uint32_t)(u >> 32));
  return __builtin_bit_cast(double, (hi << 32) | lo);
}
template <int CTRL, int ROWMASK = 0xf, class T>
__device__ __forceinline__ T dpp_move(T v) {
  if constexpr (std::is_same<T, double>::value)
    return dpp_f64<CTRL, ROWMASK>(v);
  else if constexpr (std::is_same<T, float>::value)
    return __uint_as_float(dpp_u32<CTRL, ROWMASK>(__float_as_uint(v)));
  else
    return (T)dpp_u32<CTRL, ROWMASK>((uint32_t)v);
}

// Inclusive scan over the 64 lanes of a wave with op(a, b) (sum, or unsigned
// max): four in-row steps, then the two row broadcasts.
struct OpAdd {
  template <class T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMaxU {
  __device__ __forceinline__ uint32_t operator()(uint32_t a, uint32_t b) const { return max(a, b); }
};
template <class T, class Op = OpAdd>
__device__ __forceinline__ T wave_scan_dpp(T v, Op op = Op()) {
  v = op(v, dpp_move<0x111>(v));
  v = op(v, dpp_move<0x112>(v));
  v = op(v, dpp_move<0x114>(v));
  v = op(v, dpp_move<0x118>(v));
  v = op(v, dpp_move<0x142, 0xa>(v));
  v = op(v, dpp_move<0x143, 0xc>(v));
  return v;
}

// Forward over 16-bit logits by the histogram kernel (topk_hist.hip): every
// row when all_rows != 0, else only the rows whose info.flags bit 0 is set.
int launch_hist_rows(const FilterParams& P, int dtype, int64_t rows, int all_rows,
                     hipStream_t st);

// Rewrites every row whose index cut is in rank form (RowInfo.i_cut < 0) into
// index form (16-bit logits; fp32 rows are always in index form).
int launch_resolve_rows(const FilterParams& P, int dtype, int64_t rows, hipStream_t st);

// Forward over fp32 logits in two passes (topk_f32.hip), every row; rows it
// cannot finish are flagged (info.flags bit 0) for filter_general_kernel.
int launch_f32_rows(const FilterParams& P, int64_t rows, hipStream_t st);

// Largest vocabulary the histogram kernel accepts (its exact-count table
// covers at most 8 values repeated 65536 times or more).
constexpr int64_t kHistMaxV = 9 * 65536 - 1;

}  // namespace mirl

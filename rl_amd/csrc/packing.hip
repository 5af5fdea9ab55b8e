// Packed-sequence glue on the device: packing of per-sample rows along the
// padded sequence boundaries (with the per-sequence roll of next-token
// targets), the roll of packed targets, and the unpacking of packed logprobs to
// [sequences, columns] with its backward.
//
// Semantics: nemo_rl/algorithms/loss/utils.py:355-408 (_pack_input_ids, CP = 1)
// and nemo_rl/distributed/model_utils.py:1116-1139 (target roll inside each
// [cu_seqlens_padded[i], cu_seqlens_padded[i+1]) segment) and :1211-1229
// (unpacking: row i of the output takes packed rows cu[i] .. cu[i+1] - 2, at
// most `cols` of them, zeros after).  The reference runs host loops over the
// sequences; here every packed position (or output slot) is one thread that
// finds its sequence by a binary search of the device copy of the boundaries,
// so the host only uploads the boundary array.
//
// Boundaries are int64 device arrays of n_seq + 1 entries, nondecreasing for
// the results above (the Python layer checks the host copy).  Every read is
// also guarded against the boundary values, so out-of-order or out-of-range
// boundaries give zeros there, never an access outside the buffers.

#include "common.h"

namespace mirl {
namespace {

constexpr int kPackThreads = 256;

// Largest i in [0, n) with b[i] <= p, for b[0] <= p < b[n]: the sequence whose
// segment [b[i], b[i+1]) holds position p (empty segments are skipped).
__device__ __forceinline__ int64_t find_segment(const int64_t* __restrict__ b, int64_t n, int64_t p) {
  int64_t lo = 0, hi = n;  // b[lo] <= p < b[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (b[mid] <= p)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// out[p, e] = x[seq * S + off, e] for the packed position p of sequence seq
// (off = p - cu_pad[seq], rolled by roll_shift inside the padded segment),
// when off < min(cu_q[seq + 1] - cu_q[seq], S); 0 otherwise and outside
// [cu_pad[0], cu_pad[B]).  One thread per (position, element).
template <class T>
__global__ __launch_bounds__(kPackThreads) void pack_kernel(
    const T* __restrict__ x, int64_t B, int64_t S, int64_t row_elems,
    const int64_t* __restrict__ cu_q, const int64_t* __restrict__ cu_pad, int64_t roll_shift,
    T* __restrict__ out, int64_t total) {
  const int64_t n = total * row_elems;
  for (int64_t i = (int64_t)blockIdx.x * kPackThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kPackThreads) {
    const int64_t p = i / row_elems, e = i - p * row_elems;
    T v = T(0);
    if (p >= cu_pad[0] && p < cu_pad[B]) {
      const int64_t seq = find_segment(cu_pad, B, p);
      const int64_t plen = cu_pad[seq + 1] - cu_pad[seq];
      int64_t off = p - cu_pad[seq];
      if (roll_shift != 0 && plen > 0) {
        off = (off - roll_shift) % plen;
        if (off < 0) off += plen;
      }
      const int64_t qlen = cu_q[seq + 1] - cu_q[seq];
      const int64_t copy_len = qlen < S ? qlen : S;
      if (off >= 0 && off < copy_len) v = x[(seq * S + off) * row_elems + e];
    }
    out[i] = v;
  }
}

// out[p] = target[p + 1] inside a segment, target[segment start] at its last
// position, 0 outside [b[0], b[n_seq]).
__global__ __launch_bounds__(kPackThreads) void roll_targets_kernel(
    const int64_t* __restrict__ target, int64_t n, const int64_t* __restrict__ b, int64_t n_seq,
    int64_t* __restrict__ out) {
  for (int64_t p = (int64_t)blockIdx.x * kPackThreads + threadIdx.x; p < n;
       p += (int64_t)gridDim.x * kPackThreads) {
    int64_t v = 0;
    if (p >= b[0] && p < b[n_seq]) {
      const int64_t seq = find_segment(b, n_seq, p);
      const int64_t nxt = p + 1;
      const int64_t src = nxt == b[seq + 1] ? b[seq] : nxt;
      if (src >= 0 && src < n) v = target[src];
    }
    out[p] = v;
  }
}

// out[i, j] = packed[b[i] + j] for j < clip(b[i+1] - b[i] - 1, 0, cols), else 0.
__global__ __launch_bounds__(kPackThreads) void unpack_fwd_kernel(
    const float* __restrict__ packed, int64_t n_rows, const int64_t* __restrict__ b, int64_t n_seq,
    int64_t cols, float* __restrict__ out) {
  const int64_t n = n_seq * cols;
  for (int64_t k = (int64_t)blockIdx.x * kPackThreads + threadIdx.x; k < n;
       k += (int64_t)gridDim.x * kPackThreads) {
    const int64_t i = k / cols, j = k - i * cols;
    const int64_t len = b[i + 1] - b[i] - 1;
    const int64_t src = b[i] + j;
    out[k] = (j < len && src >= 0 && src < n_rows) ? packed[src] : 0.f;
  }
}

// The unpacking's backward: grad_packed[p] = grad_out[seq, p - b[seq]] for the
// packed rows the forward copied, 0 for every other row.
__global__ __launch_bounds__(kPackThreads) void unpack_bwd_kernel(
    const float* __restrict__ grad_out, int64_t n_seq, int64_t cols, const int64_t* __restrict__ b,
    int64_t n_rows, float* __restrict__ grad_packed) {
  for (int64_t p = (int64_t)blockIdx.x * kPackThreads + threadIdx.x; p < n_rows;
       p += (int64_t)gridDim.x * kPackThreads) {
    float v = 0.f;
    if (p >= b[0] && p < b[n_seq]) {
      const int64_t seq = find_segment(b, n_seq, p);
      const int64_t j = p - b[seq];
      const int64_t len = b[seq + 1] - b[seq] - 1;
      if (j >= 0 && j < len && j < cols) v = grad_out[seq * cols + j];
    }
    grad_packed[p] = v;
  }
}

unsigned grid_for(int64_t n) {
  const int64_t blocks = (n + kPackThreads - 1) / kPackThreads;
  return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_pack_sequences(const void* x, int64_t B, int64_t S, int64_t row_elems,
                                   int32_t elem_bytes, const int64_t* cu_seqlens,
                                   const int64_t* cu_seqlens_padded, int64_t roll_shift, void* out,
                                   int64_t total, void* stream) {
  clear_error();
  MIRL_REQUIRE(B >= 1 && S >= 1 && row_elems >= 1 && total >= 0,
               "invalid packing shape B=%lld S=%lld row=%lld total=%lld", (long long)B,
               (long long)S, (long long)row_elems, (long long)total);
  if (total == 0) return MIRL_OK;
  MIRL_REQUIRE(x && cu_seqlens && cu_seqlens_padded && out, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = grid_for(total * row_elems);
#define MIRL_PACK(T)                                                                            \
  hipLaunchKernelGGL(pack_kernel<T>, dim3(grid), dim3(kPackThreads), 0, st,                     \
                     static_cast<const T*>(x), B, S, row_elems, cu_seqlens, cu_seqlens_padded,  \
                     roll_shift, static_cast<T*>(out), total)
  switch (elem_bytes) {
    case 1: MIRL_PACK(uint8_t); break;
    case 2: MIRL_PACK(uint16_t); break;
    case 4: MIRL_PACK(uint32_t); break;
    case 8: MIRL_PACK(uint64_t); break;
    default: MIRL_REQUIRE(false, "element size %d is not 1, 2, 4 or 8 bytes", (int)elem_bytes);
  }
#undef MIRL_PACK
  return check_launch("mirl_pack_sequences");
}

extern "C" int mirl_packed_roll_targets(const int64_t* target, int64_t n, const int64_t* bounds,
                                        int64_t n_seq, int64_t* out, void* stream) {
  clear_error();
  MIRL_REQUIRE(n >= 0 && n_seq >= 0, "invalid shape n=%lld sequences=%lld", (long long)n,
               (long long)n_seq);
  if (n == 0) return MIRL_OK;
  MIRL_REQUIRE(target && bounds && out, "null pointer argument");
  hipLaunchKernelGGL(roll_targets_kernel, dim3(grid_for(n)), dim3(kPackThreads), 0,
                     static_cast<hipStream_t>(stream), target, n, bounds, n_seq, out);
  return check_launch("mirl_packed_roll_targets");
}

extern "C" int mirl_unpack_rows_fwd(const float* packed, int64_t n_rows, const int64_t* bounds,
                                    int64_t n_seq, int64_t cols, float* out, void* stream) {
  clear_error();
  MIRL_REQUIRE(n_rows >= 0 && n_seq >= 0 && cols >= 0, "invalid unpacking shape");
  if (n_seq * cols == 0) return MIRL_OK;
  MIRL_REQUIRE((packed || n_rows == 0) && bounds && out, "null pointer argument");
  hipLaunchKernelGGL(unpack_fwd_kernel, dim3(grid_for(n_seq * cols)), dim3(kPackThreads), 0,
                     static_cast<hipStream_t>(stream), packed, n_rows, bounds, n_seq, cols, out);
  return check_launch("mirl_unpack_rows_fwd");
}

extern "C" int mirl_unpack_rows_bwd(const float* grad_out, int64_t n_seq, int64_t cols,
                                    const int64_t* bounds, int64_t n_rows, float* grad_packed,
                                    void* stream) {
  clear_error();
  MIRL_REQUIRE(n_rows >= 0 && n_seq >= 0 && cols >= 0, "invalid unpacking shape");
  if (n_rows == 0) return MIRL_OK;
  MIRL_REQUIRE(bounds && grad_packed && (grad_out || n_seq * cols == 0), "null pointer argument");
  hipLaunchKernelGGL(unpack_bwd_kernel, dim3(grid_for(n_rows)), dim3(kPackThreads), 0,
                     static_cast<hipStream_t>(stream), grad_out, n_seq, cols, bounds, n_rows,
                     grad_packed);
  return check_launch("mirl_unpack_rows_bwd");
}

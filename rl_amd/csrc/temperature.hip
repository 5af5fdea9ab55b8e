// In-place temperature scaling of logits and its backward.
//
// Semantics (reference nemo_rl/models/automodel/train.py:248-262 and
// nemo_rl/models/megatron/train.py:280-294): logits.div_(T) in the logits
// dtype as torch runs it on the GPU, a product with the reciprocal formed in
// double and rounded once, y = dtype(fl32(float(x) * r)) with r = fl32(1.0 / T)
// (each rounding to nearest even), and the autograd backward of that division,
// grad_x = dtype(fl32(float(g) * r)).  When a second gradient is given, the two
// are first added in the dtype (the autograd engine's accumulation of two
// consumers' gradients): grad_x = dtype(fl32(float(dtype(float(g) + float(g2))) * r)).
//
// Contiguous tensors are walked as one flat array of 16-byte vectors (a scalar
// head up to the first 16-byte boundary and a scalar tail), with nontemporal
// loads and stores; other layouts element by element over [B, R, V].

#include "common.h"

namespace mirl {
namespace {

// The flat kernels walk the array in 4 KB pieces (256 16-byte vectors), one
// per 128-thread workgroup (two vectors per lane, 2 KB apart), with piece
// boundaries on 4 KB addresses: many short workgroups dispatched in order
// keep the reads and writes inside a narrow address window, which mixed
// read/write streams need to approach the HBM rate (a grid-stride loop over
// 2048 resident workgroups measured 4.9 TB/s on bf16 [4, 4096, 151936]).
constexpr int kPieceThreads = 128;
constexpr int kPieceVecs = 256;

// Pieces of the flat kernels: (grid, shift) for an array whose vectors start
// at `first` (shift = vectors of the first piece that lie before the array).
struct Pieces {
  int64_t grid;
  int shift;
};
template <class E>
Pieces pieces_of(const void* base, int64_t n) {
  // the vectors start at the first 16-byte boundary (as RowSpan places them)
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(base);
  int64_t head = (int64_t)(((16u - (a0 & 15u)) & 15u) / sizeof(typename E::raw));
  if (head > n) head = n;
  const int64_t nvec = (n - head) / E::kVec;
  const uintptr_t a = a0 + (uintptr_t)head * sizeof(typename E::raw);
  const int to4k = (int)(((4096u - (a & 4095u)) & 4095u) / 16u);  // vectors before a 4 KB boundary
  const int shift = (kPieceVecs - to4k) & (kPieceVecs - 1);
  return Pieces{(nvec + shift + kPieceVecs - 1) / kPieceVecs, shift};
}

// x[i] <- dtype(fl32(float(x[i]) * r)) over n contiguous elements.
template <class E>
__global__ __launch_bounds__(kPieceThreads) void scale_flat_kernel(void* x, int64_t n, float r,
                                                                   int shift) {
  using raw = typename E::raw;
  raw* p = static_cast<raw*>(x);
  const RowSpan<E> sp(p, n);
  vu4* pv = reinterpret_cast<vu4*>(p + sp.head);
  const int64_t base = (int64_t)blockIdx.x * kPieceVecs + threadIdx.x - shift;
  vu4 q[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * kPieceThreads;
    if (i >= 0 && i < sp.nvec) q[u] = __builtin_nontemporal_load(pv + i);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * kPieceThreads;
    if (i < 0 || i >= sp.nvec) continue;
    float w[E::kVec];
    E::unpack(q[u], w);
#pragma unroll
    for (int k = 0; k < E::kVec; ++k) w[k] = mul_rn(w[k], r);
    __builtin_nontemporal_store(E::pack(w), pv + i);
  }
  if (blockIdx.x == 0) {
    if (threadIdx.x < sp.head) p[threadIdx.x] = E::from_float(mul_rn(E::load(p + threadIdx.x), r));
    if (sp.tail0 + threadIdx.x < n)
      p[sp.tail0 + threadIdx.x] = E::from_float(mul_rn(E::load(p + sp.tail0 + threadIdx.x), r));
  }
}

// out[i] = dtype(fl32(float(dtype(float(g[i]) (+ float(g2[i])))) * r)) over n
// contiguous elements; g, g2 and out share their offset from a 16-byte boundary.
template <class E>
__global__ __launch_bounds__(kPieceThreads) void scale_grad_flat_kernel(const void* g, const void* g2,
                                                                        void* out, int64_t n, float r,
                                                                        int shift) {
  using raw = typename E::raw;
  const raw* a = static_cast<const raw*>(g);
  const raw* b = static_cast<const raw*>(g2);
  raw* o = static_cast<raw*>(out);
  const RowSpan<E> sp(a, n);
  const vu4* av = reinterpret_cast<const vu4*>(a + sp.head);
  const vu4* bv = reinterpret_cast<const vu4*>(b + sp.head);
  vu4* ov = reinterpret_cast<vu4*>(o + sp.head);
  auto one = [&](float x, float y, bool two) {
    const float s = two ? round_trip<E>(x + y) : x;
    return mul_rn(s, r);
  };
  const bool two = b != nullptr;
  const int64_t base = (int64_t)blockIdx.x * kPieceVecs + threadIdx.x - shift;
  vu4 qa[2], qb[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * kPieceThreads;
    if (i >= 0 && i < sp.nvec) {
      qa[u] = __builtin_nontemporal_load(av + i);
      if (two) qb[u] = __builtin_nontemporal_load(bv + i);
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * kPieceThreads;
    if (i < 0 || i >= sp.nvec) continue;
    float w[E::kVec], w2[E::kVec];
    E::unpack(qa[u], w);
    if (two) E::unpack(qb[u], w2);
#pragma unroll
    for (int k = 0; k < E::kVec; ++k) w[k] = one(w[k], two ? w2[k] : 0.f, two);
    __builtin_nontemporal_store(E::pack(w), ov + i);
  }
  if (blockIdx.x == 0) {
    auto at = [&](int64_t j) {
      o[j] = E::from_float(one(E::load(a + j), two ? E::load(b + j) : 0.f, two));
    };
    if (threadIdx.x < sp.head) at(threadIdx.x);
    if (sp.tail0 + threadIdx.x < n) at(sp.tail0 + threadIdx.x);
  }
}

struct Strided3 {
  void* p;
  int64_t sb, sr;
};

// Element-wise over [B, R, V] with row strides (unit stride on V).
template <class E>
__global__ __launch_bounds__(256) void scale_rows_kernel(Strided3 x, const void* g2, int64_t g2_sb,
                                                         int64_t g2_sr, Strided3 out, int64_t R,
                                                         int64_t V, int64_t total, float rr,
                                                         int grad) {
  using raw = typename E::raw;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / V, v = i - row * V;
    const int64_t b = row / R, r = row - b * R;
    const raw* src = static_cast<const raw*>(x.p) + b * x.sb + r * x.sr + v;
    float s = E::load(src);
    if (grad && g2 != nullptr)
      s = round_trip<E>(s + E::load(static_cast<const raw*>(g2) + b * g2_sb + r * g2_sr + v));
    static_cast<raw*>(out.p)[b * out.sb + r * out.sr + v] = E::from_float(mul_rn(s, rr));
  }
}

int grid_for(int64_t work) {
  const int64_t blocks = (work + 255) / 256;
  return (int)(blocks < 8192 ? (blocks > 0 ? blocks : 1) : 8192);
}

bool contiguous(int64_t B, int64_t R, int64_t V, int64_t sb, int64_t sr) {
  return sr == V && (B == 1 || sb == R * V);
}

template <class E>
int run_scale(void* x, int64_t B, int64_t R, int64_t V, int64_t sb, int64_t sr, float r,
              hipStream_t st) {
  const int64_t n = B * R * V;
  if (contiguous(B, R, V, sb, sr)) {
    const Pieces pc = pieces_of<E>(x, n);
    hipLaunchKernelGGL((scale_flat_kernel<E>), dim3((unsigned)(pc.grid > 0 ? pc.grid : 1)),
                       dim3(kPieceThreads), 0, st, x, n, r, pc.shift);
  } else {
    const Strided3 s{x, sb, sr};
    hipLaunchKernelGGL((scale_rows_kernel<E>), dim3(grid_for(n)), dim3(256), 0, st, s, nullptr,
                       int64_t(0), int64_t(0), s, R, V, n, r, 0);
  }
  return check_launch("mirl_temperature_scale");
}

template <class E>
int run_grad(const void* g, int64_t g_sb, int64_t g_sr, const void* g2, int64_t g2_sb,
             int64_t g2_sr, void* out, int64_t o_sb, int64_t o_sr, int64_t B, int64_t R, int64_t V,
             float r, hipStream_t st) {
  const int64_t n = B * R * V;
  const uintptr_t mis = (reinterpret_cast<uintptr_t>(g) & 15u);
  const bool flat = contiguous(B, R, V, g_sb, g_sr) && contiguous(B, R, V, o_sb, o_sr) &&
                    (reinterpret_cast<uintptr_t>(out) & 15u) == mis &&
                    (g2 == nullptr ||
                     (contiguous(B, R, V, g2_sb, g2_sr) && (reinterpret_cast<uintptr_t>(g2) & 15u) == mis));
  if (flat) {
    const Pieces pc = pieces_of<E>(g, n);
    hipLaunchKernelGGL((scale_grad_flat_kernel<E>), dim3((unsigned)(pc.grid > 0 ? pc.grid : 1)),
                       dim3(kPieceThreads), 0, st, g, g2, out, n, r, pc.shift);
  } else {
    const Strided3 a{const_cast<void*>(g), g_sb, g_sr};
    const Strided3 o{out, o_sb, o_sr};
    hipLaunchKernelGGL((scale_rows_kernel<E>), dim3(grid_for(n)), dim3(256), 0, st, a, g2, g2_sb,
                       g2_sr, o, R, V, n, r, 1);
  }
  return check_launch("mirl_temperature_scale_grad");
}

int check_args(int dtype, int64_t B, int64_t R, int64_t V, double temperature) {
  if (dtype != MIRL_DTYPE_F32 && dtype != MIRL_DTYPE_BF16 && dtype != MIRL_DTYPE_F16) {
    set_error("unsupported logits dtype code %d", dtype);
    return MIRL_ERR_UNSUPPORTED;
  }
  MIRL_REQUIRE(B >= 0 && R >= 0 && V >= 0, "invalid shape B=%lld R=%lld V=%lld", (long long)B,
               (long long)R, (long long)V);
  MIRL_REQUIRE(temperature > 0.0, "temperature must be positive, got %g", temperature);
  return MIRL_OK;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int mirl_temperature_scale(void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                                      int64_t stride_b, int64_t stride_r, double temperature,
                                      void* stream) {
  clear_error();
  if (int e = check_args(dtype, B, R, V, temperature)) return e;
  if (B * R * V == 0) return MIRL_OK;
  MIRL_REQUIRE(logits != nullptr, "null pointer argument");
  const float r = temperature_recip(temperature);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32) return run_scale<F32>(logits, B, R, V, stride_b, stride_r, r, st);
  if (dtype == MIRL_DTYPE_BF16) return run_scale<BF16>(logits, B, R, V, stride_b, stride_r, r, st);
  return run_scale<F16>(logits, B, R, V, stride_b, stride_r, r, st);
}

extern "C" int mirl_temperature_scale_grad(const void* grad, int dtype, int64_t B, int64_t R,
                                           int64_t V, int64_t g_stride_b, int64_t g_stride_r,
                                           const void* grad2, int64_t g2_stride_b,
                                           int64_t g2_stride_r, double temperature, void* out,
                                           int64_t o_stride_b, int64_t o_stride_r, void* stream) {
  clear_error();
  if (int e = check_args(dtype, B, R, V, temperature)) return e;
  if (B * R * V == 0) return MIRL_OK;
  MIRL_REQUIRE(grad != nullptr && out != nullptr, "null pointer argument");
  const float r = temperature_recip(temperature);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == MIRL_DTYPE_F32)
    return run_grad<F32>(grad, g_stride_b, g_stride_r, grad2, g2_stride_b, g2_stride_r, out,
                         o_stride_b, o_stride_r, B, R, V, r, st);
  if (dtype == MIRL_DTYPE_BF16)
    return run_grad<BF16>(grad, g_stride_b, g_stride_r, grad2, g2_stride_b, g2_stride_r, out,
                          o_stride_b, o_stride_r, B, R, V, r, st);
  return run_grad<F16>(grad, g_stride_b, g_stride_r, grad2, g2_stride_b, g2_stride_r, out,
                       o_stride_b, o_stride_r, B, R, V, r, st);
}

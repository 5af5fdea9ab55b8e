// Token logprobs straight from hidden states and the output (LM-head) weight:
// the logits tile H[rows] . W[cols]^T is formed on the MFMA units and reduced
// in the same kernel, so the [T, V] logits are never written.
//
// Semantics follow nemo_rl/distributed/model_utils.py:2541-2745
// (from_parallel_hidden_states_to_logprobs, ChunkedDistributedHiddenStatesToLogprobs)
// with a vocab group of size 1:
//   logits    = bf16(H . W^T)                (the reference's bf16 matmul output)
//   logprob_t = (x_t - m) - log(sum_v exp(x_v - m)),  0 for targets outside [vs, ve)
//   backward  G = (onehot(t) - softmax(x)) * g,  dH = G . W,  dW = G^T . H
// The forward kernel writes, per row and per 256-column tile, the tile's
// (max, sum exp(x - max)) and the target logit; a merge kernel combines the
// tiles of a row.  The gradient kernel recomputes a logits tile and writes the
// bf16 G tile (the two GEMMs that consume G are plain library GEMMs).
//
// Tile: 256 rows x 256 columns per 256-thread workgroup, K in steps of 64,
// two LDS stages of 64 KB.  Each wave owns a 128 x 128 quarter as 4 x 4
// v_mfma_f32_32x32x16_bf16 tiles (256 fp32 accumulators per lane).  LDS rows are
// 128 B with their 16-byte chunks XOR-swizzled by (row % 8), so the 32 rows
// read by one MFMA operand load fall in distinct banks.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l holds A[l % 32][k]
// and B[k][l % 32] for k = (l / 32) * 8 + 0..7; accumulator element v of lane l
// is C[(v / 4) * 8 + (l / 32) * 4 + v % 4][l % 32].

#include "common.h"

#pragma clang fp contract(off)

namespace mirl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 256;                 // rows per tile
constexpr int kBN = 256;                 // vocabulary columns per tile
constexpr int kBK = 64;                  // hidden elements per K step
constexpr int kThreads = 256;            // 4 waves in a 2 x 2 arrangement
constexpr int kWM = 128, kWN = 128;      // per-wave quarter
constexpr int kTM = kWM / 32, kTN = kWN / 32;
constexpr int kRowBytes = kBK * 2;       // one tile row in LDS
constexpr int kStageBytes = (kBM + kBN) * kRowBytes;
constexpr int kLoadsPerThread = kBM * kRowBytes / 16 / kThreads;  // 16-byte chunks of A (and of B)
constexpr int kGroupM = 8;               // row tiles sharing a sweep over the vocabulary

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

__device__ __forceinline__ float bf16_round(float f) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f) << 16);
}

enum LceMode { kFwd = 0, kGrad = 1 };

struct LceParams {
  const uint16_t* h;  // [T, Hd] bf16, row stride ldh
  const uint16_t* w;  // [V, Hd] bf16, row stride ldw
  int64_t ldh, ldw;
  int64_t V, Hd;
  int64_t row0, nrows;  // rows handled: [row0, row0 + nrows)
  int64_t bsz;          // row r is (s, b) = (r / bsz, r % bsz)
  const int64_t* target;
  int64_t tsb, tss;
  int64_t vs, ve;
  int64_t n_mt, n_nt;   // row tiles, column tiles
  // forward
  float* part;          // [nrows, n_nt, 2]
  float* xt;            // [nrows]
  // gradient
  const float* stats;   // [T, 2] {max, logsum} by absolute row
  const float* g;
  int64_t gsb, gss;
  uint16_t* G;          // [nrows, V] bf16, row stride ldg
  int64_t ldg;
};

template <int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void lce_tile_kernel(LceParams P) {
  __shared__ __align__(16) unsigned char lds[2 * kStageBytes];
  __shared__ int s_tcol[kBM];
  __shared__ float s_m[kBM], s_ls[kBM], s_g[kBM];
  __shared__ float s_red[2][kBM][2];

  // grouped tile order: kGroupM row tiles sweep the vocabulary together
  const int64_t bid = blockIdx.x;
  const int64_t per_group = (int64_t)kGroupM * P.n_nt;
  const int64_t group = bid / per_group;
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = (P.n_mt - first_m < kGroupM) ? (P.n_mt - first_m) : kGroupM;
  const int64_t in_group = bid - group * per_group;
  const int64_t mt = first_m + in_group % gsize;
  const int64_t nt = in_group / gsize;
  const int64_t m0 = P.row0 + mt * kBM;  // absolute first row
  const int64_t n0 = nt * kBN;
  const int64_t row_end = P.row0 + P.nrows;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // per-row metadata of the tile (kThreads == kBM: one row per thread)
  float my_g = 0.f;
  {
    const int64_t r = m0 + tid;
    int tc = -1;
    float lm = 0.f, ll = 0.f;
    if (r < row_end) {
      const int64_t s = r / P.bsz, b = r - s * P.bsz;
      const int64_t t = P.target[b * P.tsb + s * P.tss];
      const bool tmask = (t < P.vs) || (t >= P.ve) || (t - P.vs >= P.V);
      if (!tmask) {
        const int64_t c = t - P.vs - n0;
        if (c >= 0 && c < kBN) tc = (int)c;
      }
      if (MODE == kGrad) {
        my_g = P.g[b * P.gsb + s * P.gss];
        lm = P.stats[2 * r];
        ll = P.stats[2 * r + 1];
      }
    }
    s_tcol[tid] = tc;
    if (MODE == kGrad) {
      s_g[tid] = my_g;
      s_m[tid] = lm;
      s_ls[tid] = ll;
    }
  }
  if (MODE == kGrad) {
    // (onehot - p) * 0 == 0: a tile whose rows all have a zero upstream
    // gradient is written as zeros without the GEMM.
    if (!__syncthreads_or(my_g != 0.f)) {
      const int cvec = kBN / 8;
      for (int q = tid; q < kBM * cvec; q += kThreads) {
        const int rl = q / cvec, cv = q - rl * cvec;
        const int64_t r = m0 + rl;
        const int64_t c = n0 + cv * 8;
        if (r >= row_end || c >= P.V) continue;
        uint16_t* dst = P.G + (r - P.row0) * P.ldg + c;
        if (c + 8 <= P.V && ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0)) {
          *reinterpret_cast<vu4*>(dst) = vu4{0u, 0u, 0u, 0u};
        } else {
          for (int e = 0; e < 8 && c + e < P.V; ++e) dst[e] = 0;
        }
      }
      return;
    }
  }

  // ---- main loop: acc = H[m0 : m0+256] . W[n0 : n0+256]^T ----
  const int nk = (int)(P.Hd / kBK);
  vu4 ra[kLoadsPerThread], rb[kLoadsPerThread];
  const vu4 zero = vu4{0u, 0u, 0u, 0u};
  auto gload = [&](int kt) {
    const int64_t k0 = (int64_t)kt * kBK;
#pragma unroll
    for (int j = 0; j < kLoadsPerThread; ++j) {
      const int q = tid + j * kThreads;
      const int row = q >> 3, c = q & 7;
      const int64_t ar = m0 + row;
      ra[j] = (ar < row_end) ? *reinterpret_cast<const vu4*>(P.h + ar * P.ldh + k0 + c * 8) : zero;
      const int64_t br = n0 + row;
      rb[j] = (br < P.V) ? *reinterpret_cast<const vu4*>(P.w + br * P.ldw + k0 + c * 8) : zero;
    }
  };
  auto sstore = [&](int stage) {
    unsigned char* base = lds + stage * kStageBytes;
#pragma unroll
    for (int j = 0; j < kLoadsPerThread; ++j) {
      const int q = tid + j * kThreads;
      const int row = q >> 3, c = q & 7;
      *reinterpret_cast<vu4*>(base + lds_off(row, c)) = ra[j];
      *reinterpret_cast<vu4*>(base + kBM * kRowBytes + lds_off(row, c)) = rb[j];
    }
  };

  f32x16 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload(kt + 1);
    const unsigned char* As = lds + (kt & 1) * kStageBytes;
    const unsigned char* Bs = As + kBM * kRowBytes;
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      bf16x8 af[kTM], bfr[kTN];
#pragma unroll
      for (int i = 0; i < kTM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(As + lds_off(wm * kWM + i * 32 + (lane & 31), c));
#pragma unroll
      for (int j = 0; j < kTN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(Bs + lds_off(wn * kWN + j * 32 + (lane & 31), c));
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) sstore((kt + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const int half = lane >> 5;  // which 4-row group of each 8-row band this lane holds
  const int col_lane = lane & 31;
  if (MODE == kFwd) {
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
        float x[kTN];
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          const int cl = wn * kWN + j * 32 + col_lane;
          x[j] = (n0 + cl < P.V) ? bf16_round(acc[i][j][v]) : -INFINITY;
          mx = fmaxf(mx, x[j]);
        }
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float s = 0.f;
        if (mx != -INFINITY) {
#pragma unroll
          for (int j = 0; j < kTN; ++j) s += fast_exp2((x[j] - mx) * kLog2e);
        }
#pragma unroll
        for (int off = 1; off < 32; off <<= 1) s += __shfl_xor(s, off, 64);
        const int tc = s_tcol[rl];
        if (tc >= 0) {
#pragma unroll
          for (int j = 0; j < kTN; ++j)
            if (tc == wn * kWN + j * 32 + col_lane) P.xt[m0 + rl - P.row0] = x[j];
        }
        if (col_lane == 0) {
          s_red[wn][rl][0] = mx;
          s_red[wn][rl][1] = s;
        }
      }
    }
    __syncthreads();
    const int64_t r = m0 + tid;
    if (r < row_end) {
      const float m_a = s_red[0][tid][0], s_a = s_red[0][tid][1];
      const float m_b = s_red[1][tid][0], s_b = s_red[1][tid][1];
      const float M = fmaxf(m_a, m_b);
      float s = 0.f;
      if (M != -INFINITY) {
        if (m_a != -INFINITY) s += s_a * fast_exp2((m_a - M) * kLog2e);
        if (m_b != -INFINITY) s += s_b * fast_exp2((m_b - M) * kLog2e);
      }
      float* dst = P.part + ((r - P.row0) * P.n_nt + nt) * 2;
      dst[0] = M;
      dst[1] = s;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
        const int64_t r = m0 + rl;
        if (r >= row_end) continue;
        const float gv = s_g[rl], M = s_m[rl], LS = s_ls[rl];
        const int tc = s_tcol[rl];
        uint16_t* dst = P.G + (r - P.row0) * P.ldg + n0;
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          const int cl = wn * kWN + j * 32 + col_lane;
          if (n0 + cl >= P.V) continue;
          const float x = bf16_round(acc[i][j][v]);
          const float p = fast_exp2(((x - M) - LS) * kLog2e);
          const float o = (cl == tc) ? (1.f - p) * gv : -p * gv;
          dst[cl] = BF16::from_float(o);
        }
      }
    }
  }
}

// Per row: combine the column-tile partials into the row's max and log-sum-exp,
// then logprob = (x_t - max) - logsum (0 for targets outside the slice).
// One wave per row.
__global__ __launch_bounds__(256) void lce_merge_kernel(
    const float* __restrict__ part, const float* __restrict__ xt, int64_t row0, int64_t nrows,
    int64_t n_nt, int64_t bsz, const int64_t* __restrict__ target, int64_t tsb, int64_t tss,
    int64_t vs, int64_t ve, int64_t V, float* __restrict__ out, int64_t osb, int64_t oss,
    float* __restrict__ stats) {
  const int lane = threadIdx.x & 63;
  const int64_t rl = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (rl >= nrows) return;
  const float* p = part + rl * n_nt * 2;
  float M = -INFINITY;
  for (int64_t j = lane; j < n_nt; j += 64) M = fmaxf(M, p[2 * j]);
  M = wave_max(M);
  float s = 0.f;
  if (M != -INFINITY) {
    for (int64_t j = lane; j < n_nt; j += 64) {
      const float mj = p[2 * j];
      if (mj != -INFINITY) s += p[2 * j + 1] * fast_exp2((mj - M) * kLog2e);
    }
  }
  s = wave_sum(s);
  if (lane == 0) {
    const int64_t r = row0 + rl;
    const int64_t sq = r / bsz, b = r - sq * bsz;
    const int64_t t = target[b * tsb + sq * tss];
    const bool tmask = (t < vs) || (t >= ve) || (t - vs >= V);
    const float logsum = logf(s);
    out[b * osb + sq * oss] = tmask ? 0.f : (xt[rl] - M) - logsum;
    if (stats != nullptr) {
      stats[2 * r] = M;
      stats[2 * r + 1] = logsum;
    }
  }
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int check_common(const void* hidden, int64_t T, int64_t Hd, int64_t ldh, const void* weight,
                 int64_t V, int64_t ldw, const int64_t* target, int64_t bsz) {
  MIRL_REQUIRE(hidden && weight && target, "null pointer argument");
  MIRL_REQUIRE(T >= 0 && V > 0 && Hd > 0 && bsz > 0, "invalid shape T=%lld V=%lld H=%lld B=%lld",
               (long long)T, (long long)V, (long long)Hd, (long long)bsz);
  MIRL_REQUIRE(T % bsz == 0, "row count %lld is not a multiple of the batch size %lld",
               (long long)T, (long long)bsz);
  MIRL_REQUIRE(Hd % kBK == 0, "hidden size %lld must be a multiple of %d", (long long)Hd, kBK);
  MIRL_REQUIRE(ldh % 8 == 0 && ldw % 8 == 0 && ldh >= Hd && ldw >= Hd,
               "row strides (%lld, %lld) must be multiples of 8 elements and >= the hidden size",
               (long long)ldh, (long long)ldw);
  MIRL_REQUIRE((reinterpret_cast<uintptr_t>(hidden) & 15u) == 0 &&
                   (reinterpret_cast<uintptr_t>(weight) & 15u) == 0,
               "hidden states and weight must be 16-byte aligned");
  MIRL_REQUIRE(V < (int64_t(1) << 31) && T < (int64_t(1) << 31), "sizes exceed 2^31-1");
  return MIRL_OK;
}

}  // namespace
}  // namespace mirl

using namespace mirl;

extern "C" int64_t mirl_linear_ce_workspace_elems(int64_t T, int64_t V) {
  if (T <= 0 || V <= 0) return 0;
  return T * ceil_div(V, kBN) * 2 + T;
}

extern "C" int mirl_linear_ce_fwd(const void* hidden, int64_t T, int64_t Hd, int64_t ldh,
                                  const void* weight, int64_t V, int64_t ldw, int64_t bsz,
                                  const int64_t* target, int64_t t_stride_b, int64_t t_stride_s,
                                  int64_t vocab_start, int64_t vocab_end, float* out,
                                  int64_t o_stride_b, int64_t o_stride_s, float* row_stats,
                                  float* workspace, void* stream) {
  clear_error();
  if (int e = check_common(hidden, T, Hd, ldh, weight, V, ldw, target, bsz)) return e;
  if (T == 0) return MIRL_OK;
  MIRL_REQUIRE(out && workspace, "null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  LceParams P{};
  P.h = static_cast<const uint16_t*>(hidden);
  P.w = static_cast<const uint16_t*>(weight);
  P.ldh = ldh;
  P.ldw = ldw;
  P.V = V;
  P.Hd = Hd;
  P.row0 = 0;
  P.nrows = T;
  P.bsz = bsz;
  P.target = target;
  P.tsb = t_stride_b;
  P.tss = t_stride_s;
  P.vs = vocab_start;
  P.ve = vocab_end;
  P.n_mt = ceil_div(T, kBM);
  P.n_nt = ceil_div(V, kBN);
  P.part = workspace;
  P.xt = workspace + T * P.n_nt * 2;
  const int64_t grid = P.n_mt * P.n_nt;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((lce_tile_kernel<kFwd>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  hipLaunchKernelGGL(lce_merge_kernel, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, st, P.part,
                     P.xt, (int64_t)0, T, P.n_nt, bsz, target, t_stride_b, t_stride_s,
                     vocab_start, vocab_end, V, out, o_stride_b, o_stride_s, row_stats);
  return check_launch("mirl_linear_ce_fwd");
}

extern "C" int mirl_linear_ce_grad(const void* hidden, int64_t T, int64_t Hd, int64_t ldh,
                                   const void* weight, int64_t V, int64_t ldw, int64_t bsz,
                                   const int64_t* target, int64_t t_stride_b,
                                   int64_t t_stride_s, int64_t vocab_start, int64_t vocab_end,
                                   const float* row_stats, const float* grad_out,
                                   int64_t g_stride_b, int64_t g_stride_s, int64_t row0,
                                   int64_t nrows, void* grad_logits, int64_t ldg, void* stream) {
  clear_error();
  if (int e = check_common(hidden, T, Hd, ldh, weight, V, ldw, target, bsz)) return e;
  MIRL_REQUIRE(row0 >= 0 && nrows >= 0 && row0 + nrows <= T, "row range [%lld, %lld) outside [0, %lld)",
               (long long)row0, (long long)(row0 + nrows), (long long)T);
  if (nrows == 0) return MIRL_OK;
  MIRL_REQUIRE(row_stats && grad_out && grad_logits, "null pointer argument");
  MIRL_REQUIRE(ldg >= V, "gradient row stride %lld is smaller than V=%lld", (long long)ldg,
               (long long)V);
  hipStream_t st = static_cast<hipStream_t>(stream);
  LceParams P{};
  P.h = static_cast<const uint16_t*>(hidden);
  P.w = static_cast<const uint16_t*>(weight);
  P.ldh = ldh;
  P.ldw = ldw;
  P.V = V;
  P.Hd = Hd;
  P.row0 = row0;
  P.nrows = nrows;
  P.bsz = bsz;
  P.target = target;
  P.tsb = t_stride_b;
  P.tss = t_stride_s;
  P.vs = vocab_start;
  P.ve = vocab_end;
  P.n_mt = ceil_div(nrows, kBM);
  P.n_nt = ceil_div(V, kBN);
  P.stats = row_stats;
  P.g = grad_out;
  P.gsb = g_stride_b;
  P.gss = g_stride_s;
  P.G = static_cast<uint16_t*>(grad_logits);
  P.ldg = ldg;
  const int64_t grid = P.n_mt * P.n_nt;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((lce_tile_kernel<kGrad>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  return check_launch("mirl_linear_ce_grad");
}

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
// 128 B with their 16-byte chunks XOR-swizzled (see lds_off), so the rows read
// by one MFMA operand load fall in distinct banks.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l holds A[l % 32][k]
// and B[k][l % 32] for k = (l / 32) * 8 + 0..7; accumulator element v of lane l
// is C[(v / 4) * 8 + (l / 32) * 4 + v % 4][l % 32].

#include <type_traits>

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
constexpr int kGroupM = 4;               // row tiles sharing a sweep over the vocabulary
constexpr int kXcds = 8;                 // accelerator dies, each with its own L2

// LDS byte offset of 16-byte chunk `chunk` of tile row `row`.  A ds_read_b128
// serves 16 lanes per pass (16 x 16 B = the 64 four-byte banks); an MFMA
// operand read has those lanes on 16 consecutive rows at one chunk, so the
// chunk is XOR-ed with (row / 2) % 8: the 8 even and the 8 odd rows then each
// hit 8 distinct chunks, i.e. 16 distinct bank groups.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// Epilogue layout of a [256][256] bf16 tile in LDS: row-major, 16-byte chunks
// XOR-swizzled by row % 32 (element index).
__device__ __forceinline__ int xs_index(int row, int col) {
  return row * kBN + ((((col >> 3) ^ (row & 31)) << 3) | (col & 7));
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

  // Tile order.  Workgroups are dispatched to the 8 XCDs round-robin
  // (XCD = blockIdx % 8) and each XCD has its own L2, so each XCD takes one
  // contiguous run of a grouped order (kGroupM row tiles sweep the vocabulary
  // together): the ~32 workgroups resident on an XCD then cover about
  // kGroupM row tiles x 8 column tiles and share their H and W reads in L2.
  const int64_t ntiles = P.n_mt * P.n_nt;
  const int64_t per_xcd = (ntiles + kXcds - 1) / kXcds;
  const int64_t gi = (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (gi >= ntiles) return;
  const int64_t per_group = (int64_t)kGroupM * P.n_nt;
  const int64_t group = gi / per_group;
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = (P.n_mt - first_m < kGroupM) ? (P.n_mt - first_m) : kGroupM;
  const int64_t in_group = gi - group * per_group;
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
  //
  // Global -> register loads go through buffer resources covering the tile's
  // valid rows, so rows past the end of H or W read as zero with no branch.
  // Thread t moves the 16-byte chunk (t & 7) of rows (t >> 3) + 32 j, j < 8,
  // of both operands; its LDS slot is fixed up to the row offset 32 j * 128.
  //
  // One K step (64 hidden elements) is four MFMA blocks kk = 0..3 of 16
  // MFMAs.  While block kk runs, the operand fragments of block kk + 1 are read
  // from LDS into the other fragment set; staged global loads are written to
  // the other LDS stage during block 2; the step's barrier comes before block
  // 3, whose MFMAs then cover the LDS reads of the next step's block 0.
  // sched_barrier fences keep that order.
  const int nk = (int)(P.Hd / kBK);
  const int64_t a_rows = (row_end - m0 < kBM) ? (row_end - m0) : kBM;
  const int64_t b_rows = (P.V - n0 < kBN) ? (P.V - n0) : kBN;
  const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.h + m0 * P.ldh), 0, (int)(a_rows * P.ldh * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(P.w + n0 * P.ldw), 0, (int)(b_rows * P.ldw * 2), 0x00020000);
  const int ld_row = tid >> 3, ld_chunk = tid & 7;
  const int voff_a = (int)((ld_row * P.ldh + ld_chunk * 8) * 2);
  const int voff_b = (int)((ld_row * P.ldw + ld_chunk * 8) * 2);
  const int jstride_a = (int)(32 * P.ldh * 2), jstride_b = (int)(32 * P.ldw * 2);
  const int st_off = lds_off(ld_row, ld_chunk);  // + j * 32 rows

  // Two staging register sets: the data of step m lives in set m % 2.
  vu4 ra[2][kLoadsPerThread], rb[2][kLoadsPerThread];
  auto gload_one = [&](int set, int kt, int j) {
    const int k_bytes = kt * kBK * 2;
    ra[set][j] = __builtin_bit_cast(vu4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a, j * jstride_a + k_bytes, 0));
    rb[set][j] = __builtin_bit_cast(vu4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b, j * jstride_b + k_bytes, 0));
  };
  auto sstore_one = [&](int set, unsigned char* base, int j) {
    *reinterpret_cast<vu4*>(base + st_off + j * 32 * kRowBytes) = ra[set][j];
    *reinterpret_cast<vu4*>(base + kBM * kRowBytes + st_off + j * 32 * kRowBytes) = rb[set][j];
  };

  // fragment read offsets: row (wm*128 | wn*128) + i*32 + (lane & 31), chunk kk*2 + (lane >> 5)
  const int frow = lane & 31;
  int frag_off[kBK / 16];
#pragma unroll
  for (int kk = 0; kk < kBK / 16; ++kk) frag_off[kk] = lds_off(frow, kk * 2 + (lane >> 5));
  bf16x8 fa[2][kTM], fb[2][kTN];
  auto fread = [&](int set, const unsigned char* stage, int kk, int idx) {
    // idx < kTM: A fragment idx; else B fragment idx - kTM
    if (idx < kTM)
      fa[set][idx] = *reinterpret_cast<const bf16x8*>(stage + (wm * kWM + idx * 32) * kRowBytes + frag_off[kk]);
    else
      fb[set][idx - kTM] = *reinterpret_cast<const bf16x8*>(
          stage + kBM * kRowBytes + (wn * kWN + (idx - kTM) * 32) * kRowBytes + frag_off[kk]);
  };

  f32x16 acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  auto mfma = [&](int set, int q) {
    const int i = q / kTN, j = q % kTN;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
  };

  // Prologue: step 0 into LDS stage 0, step 1's loads in flight, block 0's fragments.
#pragma unroll
  for (int j = 0; j < kLoadsPerThread; ++j) gload_one(0, 0, j);
#pragma unroll
  for (int j = 0; j < kLoadsPerThread; ++j) sstore_one(0, lds, j);
  if (nk > 1) {
#pragma unroll
    for (int j = 0; j < kLoadsPerThread; ++j) gload_one(1, 1, j);
  }
  __syncthreads();
#pragma unroll
  for (int idx = 0; idx < kTM + kTN; ++idx) fread(0, lds, 0, idx);

  // One K step kt (PAR = kt % 2).  Step kt + 2's loads go into staging set PAR
  // (free since step kt's data went to LDS one step earlier), two pairs per
  // block, a step or more before they are written; blocks 1 and 2 write step
  // kt + 1's data (set PAR ^ 1) to the other LDS stage, one chunk pair every 4
  // MFMAs; block 3 reads the next step's block-0 fragments after the barrier.
  // Spreading the loads and writes keeps the address and LDS data queues from
  // filling, which would stall the single wave of the SIMD and with it the
  // MFMAs queued behind.  Every read of the current stage happens before the
  // step's barrier; the next write into it (step kt + 2's data) comes in the
  // next step's block 1.
  auto step = [&](int kt, auto par_c, auto next_c, auto load_c) {
    constexpr int PAR = decltype(par_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr bool LOAD = decltype(load_c)::value;
    const unsigned char* cur = lds + PAR * kStageBytes;
    unsigned char* nxt = lds + (PAR ^ 1) * kStageBytes;
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
      const int set = kk & 1;
#pragma unroll
      for (int q = 0; q < kTM * kTN; ++q) {
        mfma(set, q);
        if (q < kTM + kTN) fread(set ^ 1, cur, kk + 1, q);
        if constexpr (LOAD) {
          if ((q & 7) == 0) gload_one(PAR, kt + 2, kk * 2 + (q >> 3));
        }
        if constexpr (NEXT) {
          if (kk >= 1 && (q & 3) == 0) sstore_one(PAR ^ 1, nxt, (kk - 1) * 4 + (q >> 2));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kTM * kTN; ++q) {
      mfma(1, q);
      if constexpr (NEXT) {
        if (q < kTM + kTN) fread(0, nxt, 0, q);
      }
      if constexpr (LOAD) {
        if ((q & 7) == 0) gload_one(PAR, kt + 2, 6 + (q >> 3));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  // nk is even (the hidden size is a multiple of 2 * kBK): pairs of steps,
  // then the last pair without the loads that would run past the end.
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    step(kt, I0{}, T_{}, T_{});
    step(kt + 1, I1{}, T_{}, T_{});
  }
  step(kt, I0{}, T_{}, F_{});
  step(kt + 1, I1{}, F_{}, F_{});

  // ---- epilogue: the tile goes through LDS as bf16, one row per thread ----
  //
  // The accumulators of a row are spread over 32 lanes; instead of cross-lane
  // reductions each wave writes its quarter to LDS (row-major [256][256] bf16,
  // 16-byte chunks XOR-swizzled by row % 32) and thread t then walks row t
  // (forward) or copies rows out with 16-byte stores (gradient).  The last
  // step's barrier already ordered every read of the LDS stages before this.
  __syncthreads();
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds);
  const int half = lane >> 5;  // which 4-row group of each 8-row band this lane holds
  const int col_lane = lane & 31;
  if (MODE == kFwd) {
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
      for (int j = 0; j < kTN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
          const int cl = wn * kWN + j * 32 + col_lane;
          xs[xs_index(rl, cl)] = BF16::from_float(acc[i][j][v]);
        }
    __syncthreads();
    const int64_t r = m0 + tid;
    if (r < row_end) {
      const int ncols = (P.V - n0 < kBN) ? (int)(P.V - n0) : kBN;
      const vu4* rowp = reinterpret_cast<const vu4*>(xs + tid * kBN);
      const int sw = tid & 31;
      float M = -INFINITY;
      for (int c = 0; c < kBN / 8; ++c) {
        float w[8];
        BF16::unpack(rowp[c ^ sw], w);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (c * 8 + e < ncols) M = fmaxf(M, w[e]);
      }
      float sum = 0.f;
      if (M != -INFINITY) {
        float s4[4] = {0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < kBN / 8; ++c) {
          float w[8];
          BF16::unpack(rowp[c ^ sw], w);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (c * 8 + e < ncols) s4[e & 3] += fast_exp2((w[e] - M) * kLog2e);
        }
        sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
      }
      float* dst = P.part + ((r - P.row0) * P.n_nt + nt) * 2;
      dst[0] = M;
      dst[1] = sum;
      const int tc = s_tcol[tid];
      if (tc >= 0) P.xt[r - P.row0] = BF16::load(xs + xs_index(tid, tc));
    }
  } else {
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
        const float gv = s_g[rl], M = s_m[rl], LS = s_ls[rl];
        const int tc = s_tcol[rl];
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          const int cl = wn * kWN + j * 32 + col_lane;
          const float x = bf16_round(acc[i][j][v]);
          const float p = fast_exp2(((x - M) - LS) * kLog2e);
          const float o = (cl == tc) ? (1.f - p) * gv : -p * gv;
          xs[xs_index(rl, cl)] = BF16::from_float(o);
        }
      }
    }
    __syncthreads();
    // 32 threads per row, one 16-byte chunk each; 8 rows per pass
    const int c = tid & 31;
    for (int k = 0; k < kBM / 8; ++k) {
      const int rl = (tid >> 5) + 8 * k;
      const int64_t r = m0 + rl;
      const int64_t col0 = n0 + c * 8;
      if (r >= row_end || col0 >= P.V) continue;
      const vu4 q = reinterpret_cast<const vu4*>(xs + rl * kBN)[c ^ (rl & 31)];
      uint16_t* dst = P.G + (r - P.row0) * P.ldg + col0;
      if (col0 + 8 <= P.V && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        *reinterpret_cast<vu4*>(dst) = q;
      } else {
        const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
        for (int e = 0; e < 8 && col0 + e < P.V; ++e)
          dst[e] = (uint16_t)(wv[e >> 1] >> ((e & 1) * 16));
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
  MIRL_REQUIRE(Hd % (2 * kBK) == 0, "hidden size %lld must be a multiple of %d", (long long)Hd, 2 * kBK);
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
  const int64_t grid = ceil_div(P.n_mt * P.n_nt, kXcds) * kXcds;
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
  const int64_t grid = ceil_div(P.n_mt * P.n_nt, kXcds) * kXcds;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((lce_tile_kernel<kGrad>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  return check_launch("mirl_linear_ce_grad");
}

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
// bf16 G tile and its transpose; the two products that consume G run on the
// same tile loop as a plain GEMM.  Row counts may live on the device (the
// backward's active rows): the kernels read them and skip what lies past them,
// so the host never waits for them.
//
// Tile: 256 rows x 256 columns per 256-thread workgroup.  Each wave owns a
// 128 x 128 quarter as 4 x 4 v_mfma_f32_32x32x16_bf16 tiles (256 fp32
// accumulators per lane).  The hidden dimension streams through two LDS stages
// of 64 elements (64 KB each: 256 rows of H and 256 rows of W, 128 B per row),
// filled by direct global->LDS loads (buffer_load_dwordx4 ... lds) one stage
// ahead of the MFMAs: no staging registers and no LDS store instructions sit
// between the loads and the MFMAs, and the only waits are one vmcnt + barrier
// per stage.  Each row of a stage is one 128-byte line of H or W.  A row's
// eight 16-byte chunks are XOR-swizzled by (row / 2) % 8 (see lds_off), so the
// 16 rows read by one pass of an MFMA operand load fall in distinct banks.
//
// MFMA 32x32x16 bf16 lane layout (checked on gfx950): lane l holds A[l % 32][k]
// and B[k][l % 32] for k = (l / 32) * 8 + 0..7; accumulator element v of lane l
// is C[(v / 4) * 8 + (l / 32) * 4 + v % 4][l % 32].

#include <type_traits>

#include "common.h"

#pragma clang fp contract(off)

namespace mirl {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Operand dtype of the logits GEMM (bf16 or fp16): the 32x32x16 MFMA and its
// 8-element fragment.  The two instructions share one lane layout.
template <class E>
struct Mma;
template <>
struct Mma<BF16> {
  typedef __bf16 frag __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma<F16> {
  typedef _Float16 frag __attribute__((ext_vector_type(8)));
  __device__ __forceinline__ static f32x16 run(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
// fp32 operands (plain GEMM only): a 16-byte fragment holds four hidden
// elements of a row, k = (l / 32) * 4 + 0..3, and feeds four
// v_mfma_f32_32x32x2_f32, element e of both fragments to the e-th one.  That
// instruction takes A[l % 32][l / 32] and B[l / 32][l % 32] from lane l, so the
// four together sum the products over the fragment's eight hidden elements
// (element e of the lanes below 32 is k = e, of the others k = 4 + e), in the
// same accumulator layout as the 16-bit instructions.
template <>
struct Mma<F32> {
  typedef float frag __attribute__((ext_vector_type(4)));
  __device__ __forceinline__ static f32x16 run(frag a, frag b, f32x16 c) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0], b[0], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[1], b[1], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[2], b[2], c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[3], b[3], c, 0, 0, 0);
    return c;
  }
};

// 16-bit element bits <-> fp32 for a dtype E (round to nearest even).
template <class E>
__device__ __forceinline__ uint16_t bits_of(float f) {
  return __builtin_bit_cast(uint16_t, E::from_float(f));
}
template <class E>
__device__ __forceinline__ float value_of(uint16_t b) {
  return E::load_raw(__builtin_bit_cast(typename E::raw, b));
}
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kBM = 256;                 // rows per tile
constexpr int kBN = 256;                 // vocabulary columns per tile
constexpr int kSK = 64;                  // 16-bit hidden elements per LDS stage (128 bytes)
constexpr int kStages = 2;
constexpr int kThreads = 256;            // 4 waves in a 2 x 2 arrangement
constexpr int kWaves = kThreads / kWave;
constexpr int kWM = 128, kWN = 128;      // per-wave quarter
constexpr int kTM = kWM / 32, kTN = kWN / 32;
constexpr int kRowBytes = kSK * 2;       // 128 B: one tile row of a stage
constexpr int kKK = kRowBytes / 32;      // fragment steps per stage (two 16-byte chunks each)
constexpr int kHalfBytes = kBM * kRowBytes;    // 32 KB: the H (or W) rows of a stage
constexpr int kStageBytes = 2 * kHalfBytes;    // 64 KB
constexpr int kDmaBytes = kWave * 16;          // one direct load: 64 lanes x 16 B = 8 rows
constexpr int kDmaRows = kDmaBytes / kRowBytes;
constexpr int kDmaPerWave = kHalfBytes / kDmaBytes / kWaves;  // loads of H (and of W) per wave and stage
constexpr int kEpiRows = kStageBytes / (kBN * 2);  // epilogue tile rows held by one stage array
constexpr int kGroupM = 8;               // row tiles sharing a sweep over the vocabulary
constexpr int kXcds = 8;                 // accelerator dies, each with its own L2
static_assert(kBM == kBN, "H and W halves of a stage have the same size");
static_assert(kEpiRows * kStages == kBM, "the epilogue tile fills the stage arrays");
static_assert(kEpiRows == kWM, "a wave's epilogue rows live in one stage array");

// LDS byte offset (within a stage half) of 16-byte chunk `chunk` of tile row
// `row`.  A ds_read_b128 serves 16 lanes per pass (16 x 16 B = the 64
// four-byte banks); an MFMA operand read has those lanes on 16 consecutive rows
// at one chunk.  Two 128-byte rows span the 64 banks, so the chunk is XOR-ed
// with (row / 2) % 8: the 8 even and the 8 odd rows then each hit 8 distinct
// chunks, i.e. 16 distinct bank groups.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * kRowBytes + ((chunk ^ ((row >> 1) & 7)) << 4);
}

// Epilogue layout of the [256][256] bf16 tile: row r lives in stage array
// r / 128 at local row r % 128, row-major, 16-byte chunks XOR-swizzled by
// r % 32 (element index within the array).
__device__ __forceinline__ int xs_index(int row, int col) {
  return (row & (kEpiRows - 1)) * kBN + ((((col >> 3) ^ (row & 31)) << 3) | (col & 7));
}

// s_waitcnt vmcnt(N) lgkmcnt(0), then s_barrier.  The memory clobber keeps the
// compiler from moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

enum LceMode { kFwd = 0, kGrad = 1, kGemm = 2 };

struct LceParams {
  const void* h;  // [T, Hd] of the kernel's E (bf16, fp16; fp32 for the plain GEMM), row stride ldh
  const void* w;  // [V, Hd] of the same dtype, row stride ldw
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
  uint16_t* Gt;         // or null: G transposed, [V, ldgt] bf16 (column r - row0 of row v)
  int64_t ldgt;
  // plain GEMM (kGemm): C = A . B^T with A = h [nrows, Hd], B = w [V, Hd]; the
  // hidden dimension is split into n_ks ranges of kb_len (C holds n_ks
  // partial products [n_ks][nrows][ldc]), or Cb receives bf16(C) (n_ks = 1)
  int64_t n_ks, kb_len;
  float* C;
  uint16_t* Cb;        // bf16 output, fp16 with cb_f16
  int cb_f16;
  int64_t ldc, ldcb;
  int accumulate;       // C += A . B^T instead of C = A . B^T (n_ks = 1)
  // device count (or null): c = *count - count_off.  kFwd/kGrad and count_axis
  // 0: rows r >= c are absent (not read, not written); count_axis 1 (kGemm):
  // the reduction stops at round_up(c, 128).  With both C and Cb, the output
  // is Cb = bf16(A . B^T (+ C when accumulate)) if *count <= final_at and C
  // otherwise; an empty reduction with accumulate set writes nothing.
  const int64_t* count;
  int64_t count_off;
  int count_axis;
  int64_t final_at;
};

template <int MODE, class E>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void lce_tile_kernel(LceParams P) {
  using frag = typename Mma<E>::frag;
  static_assert(MODE == kGemm || sizeof(typename E::raw) == 2, "fp32 operands: plain GEMM only");
  constexpr int kES = (int)sizeof(typename E::raw);  // bytes per element
  constexpr int kSKE = kRowBytes / kES;              // hidden elements per stage
  // Two arrays rather than one, so that the compiler tracks the direct loads
  // into each stage on their own and an LDS read waits only for its stage.
  __shared__ __align__(1024) unsigned char st0[kStageBytes];
  __shared__ __align__(1024) unsigned char st1[kStageBytes];
  __shared__ int s_tcol[kBM];
  __shared__ float s_m[kBM], s_ls[kBM], s_g[kBM];
  auto stage_ptr = [&](int s) -> unsigned char* { return s == 0 ? st0 : st1; };

  // Tile order.  Workgroups are dispatched to the 8 XCDs round-robin
  // (XCD = blockIdx % 8) and each XCD has its own L2, so each XCD takes one
  // contiguous run of a grouped order (kGroupM row tiles sweep the vocabulary
  // together): the ~32 workgroups resident on an XCD then cover about
  // kGroupM row tiles x 4 column tiles and share their H and W reads in L2.
  // (A plain GEMM's hidden-dimension splits are the outermost index.)
  // A device count of rows shortens the row range; the tile order then covers
  // only the row tiles that hold rows (so every XCD keeps its share of the
  // work) and the workgroups past them return at once.
  int64_t row_end = P.row0 + P.nrows;
  int64_t k_end = P.Hd;
  bool to_bf16 = P.Cb != nullptr;
  if (P.count != nullptr) {
    const int64_t c = *P.count - P.count_off;
    if (MODE != kGemm || P.count_axis == 0) {
      if (c < row_end) row_end = c;
    } else {
      constexpr int64_t kstep = kStages * kSKE;
      const int64_t ke = c <= 0 ? 0 : (c + kstep - 1) / kstep * kstep;
      if (ke < k_end) k_end = ke;
      if (ke == 0 && P.accumulate) return;
      if (P.C != nullptr && P.Cb != nullptr) to_bf16 = *P.count <= P.final_at;
    }
  }
  if (row_end <= P.row0) return;
  const int64_t n_mt = (row_end - P.row0 + kBM - 1) / kBM;  // <= P.n_mt
  const int64_t tiles2 = n_mt * P.n_nt;
  const int64_t ntiles = tiles2 * (MODE == kGemm ? P.n_ks : 1);
  const int64_t per_xcd = (ntiles + kXcds - 1) / kXcds;
  // (the grid holds per_xcd workgroups per XCD only without a count)
  if ((int64_t)(blockIdx.x / kXcds) >= per_xcd) return;
  const int64_t gi0 = (int64_t)(blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
  if (gi0 >= ntiles) return;
  const int64_t ks = gi0 / tiles2;
  const int64_t gi = gi0 - ks * tiles2;
  const int64_t per_group = (int64_t)kGroupM * P.n_nt;
  const int64_t group = gi / per_group;
  const int64_t first_m = group * kGroupM;
  const int64_t gsize = (n_mt - first_m < kGroupM) ? (n_mt - first_m) : kGroupM;
  const int64_t in_group = gi - group * per_group;
  const int64_t mt = first_m + in_group % gsize;
  const int64_t nt = in_group / gsize;
  const int64_t m0 = P.row0 + mt * kBM;  // absolute first row
  const int64_t n0 = nt * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // per-row metadata of the tile (kThreads == kBM: one row per thread)
  float my_g = 0.f;
  if constexpr (MODE != kGemm) {
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
      if (P.Gt != nullptr && n0 + tid < P.V) {
        uint16_t* dt = P.Gt + (n0 + tid) * P.ldgt + (m0 - P.row0);
        for (int r8 = 0; r8 < kBM / 8; ++r8) *reinterpret_cast<vu4*>(dt + r8 * 8) = vu4{0u, 0u, 0u, 0u};
      }
      return;
    }
  }

  // ---- main loop: acc = H[m0 : m0+256] . W[n0 : n0+256]^T ----
  //
  // Direct loads go through buffer resources covering the tile's valid rows.
  // The row offset is in the VGPR offset, which the range check covers, so rows
  // past the end of H or W read as zero with no branch; the SGPR offset carries
  // only the stage's hidden offset, which stays inside a valid row.
  //
  // One direct load moves 8 rows x 128 B: lane l writes LDS bytes
  // [16 l, 16 l + 16) of the load's 1 KB block, i.e. row l / 8, slot l % 8, so
  // it fetches global chunk (l % 8) ^ ((row / 2) % 8) of that row (the inverse
  // of the lds_off swizzle).  Each wave issues kDmaPerWave loads of H and of W
  // per stage.
  // this tile's range of the hidden dimension (the whole of it but for split GEMMs)
  const int64_t kbase = (MODE == kGemm) ? ks * P.kb_len : 0;
  const int64_t krest = k_end - kbase < 0 ? 0 : k_end - kbase;
  const int64_t klen = (MODE == kGemm) ? (krest < P.kb_len ? krest : P.kb_len) : P.Hd;
  const int nst = (int)(klen / kSKE);  // a multiple of kStages (0: an empty reduction)
  if (MODE == kGemm && nst == 0) {
    // an empty reduction range (a reduction-length count, or a split past it):
    // the product is zero; handled here, before the accumulators exist
    for (int q = threadIdx.x; q < kBM * kBN; q += kThreads) {
      const int64_t row = m0 + q / kBN, col = n0 + q % kBN;
      if (row >= row_end || col >= P.V) continue;
      if (to_bf16) {
        const float o = (P.accumulate && P.C != nullptr) ? P.C[row * P.ldc + col] : 0.f;
        P.Cb[row * P.ldcb + col] = P.cb_f16 ? bits_of<F16>(o) : bits_of<BF16>(o);
      } else if (!P.accumulate) {
        P.C[(ks * P.nrows + row) * P.ldc + col] = 0.f;
      }
    }
    return;
  }
  const int64_t a_rows = (row_end - m0 < kBM) ? (row_end - m0) : kBM;
  const int64_t b_rows = (P.V - n0 < kBN) ? (P.V - n0) : kBN;
  const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(P.h) + (m0 * P.ldh + kbase) * kES), 0,
      (int)((a_rows * P.ldh - kbase) * kES), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(static_cast<const char*>(P.w) + (n0 * P.ldw + kbase) * kES), 0,
      (int)((b_rows * P.ldw - kbase) * kES), 0x00020000);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int voff_a[kDmaPerWave], voff_b[kDmaPerWave];
#pragma unroll
  for (int i = 0; i < kDmaPerWave; ++i) {
    const int row = (wave * kDmaPerWave + i) * kDmaRows + (lane >> 3);
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    voff_a[i] = (int)(row * P.ldh * kES) + chunk * 16;
    voff_b[i] = (int)(row * P.ldw * kES) + chunk * 16;
  }
  // load q of stage data t: q < kDmaPerWave is an H block, else a W block
  auto dma = [&](unsigned char* stage, int t, int q) {
    const int soff = t * kRowBytes;
    if (q < kDmaPerWave) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc_a, (lds_ptr_t)(stage + (wave_u * kDmaPerWave + q) * kDmaBytes), 16, voff_a[q], soff, 0, 0);
    } else {
      const int qb = q - kDmaPerWave;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc_b, (lds_ptr_t)(stage + kHalfBytes + (wave_u * kDmaPerWave + qb) * kDmaBytes), 16,
          voff_b[qb], soff, 0, 0);
    }
  };

  // fragment read offsets: row (wm*128 | wn*128) + i*32 + (lane & 31), chunk kk*2 + (lane >> 5)
  const int frow = lane & 31;
  int frag_off[kKK];
#pragma unroll
  for (int kk = 0; kk < kKK; ++kk) frag_off[kk] = lds_off(frow, kk * 2 + (lane >> 5));
  frag fa[2][kTM], fb[2][kTN];
  auto fread = [&](int set, const unsigned char* stage, int kk, int idx) {
    // idx < kTM: A fragment idx; else B fragment idx - kTM
    if (idx < kTM)
      fa[set][idx] = *reinterpret_cast<const frag*>(stage + (wm * kWM + idx * 32) * kRowBytes + frag_off[kk]);
    else
      fb[set][idx - kTM] = *reinterpret_cast<const frag*>(
          stage + kHalfBytes + (wn * kWN + (idx - kTM) * 32) * kRowBytes + frag_off[kk]);
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
    acc[i][j] = Mma<E>::run(fa[set][i], fb[set][j], acc[i][j]);
  };

  constexpr int kL = 2 * kDmaPerWave;  // direct loads per wave and stage
  static_assert(kL == kTM * kTN, "one direct load per MFMA of block 3");
  // Prologue: stage data 0 and 1 in flight; wait for 0 and read its block-0 fragments.
#pragma unroll
  for (int q = 0; q < kL; ++q) dma(st0, 0, q);
#pragma unroll
  for (int q = 0; q < kL; ++q) dma(st1, 1, q);
  wait_vm_barrier<kL>();
#pragma unroll
  for (int idx = 0; idx < kTM + kTN; ++idx) fread(0, st0, 0, idx);

  // One stage t (S = t % 2): four MFMA blocks kk = 0..3 of 16 MFMAs (16 hidden
  // elements each for 16-bit operands; for fp32, 8 elements in four instructions).  While block kk runs on fragment set kk % 2, block kk + 1's
  // fragments are read into the other set.  Before block 3 this wave waits for
  // its loads of stage data t + 1 (the only ones in flight) and the workgroup
  // barrier makes every wave's loads visible and ends every read of stage S
  // (block 3's fragments were read during block 2).  Block 3 then reads the
  // next stage's block-0 fragments and issues the direct loads of stage data
  // t + 2 into stage S: a full stage ahead of their use.
  auto step = [&](int t, auto s_c, auto next_c, auto load_c) {
    constexpr int S = decltype(s_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    constexpr bool LOAD = decltype(load_c)::value;
    unsigned char* cur = stage_ptr(S);
    const unsigned char* nxt = stage_ptr(S ^ 1);
#pragma unroll
    for (int kk = 0; kk < 3; ++kk) {
#pragma unroll
      for (int q = 0; q < kTM * kTN; ++q) {
        mfma(kk & 1, q);
        if (q < kTM + kTN) fread((kk + 1) & 1, cur, kk + 1, q);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (NEXT) wait_vm_barrier<0>();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < kTM * kTN; ++q) {
      mfma(1, q);
      if constexpr (NEXT) {
        if (q < kTM + kTN) fread(0, nxt, 0, q);
      }
      if constexpr (LOAD) dma(cur, t + 2, q);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;
  int t = 0;
  for (; t < nst - kStages; t += kStages) {
    step(t, S0{}, T_{}, T_{});
    step(t + 1, S1{}, T_{}, T_{});
  }
  step(t, S0{}, T_{}, F_{});
  step(t + 1, S1{}, F_{}, F_{});

  if constexpr (MODE == kGemm) {
    // ---- plain GEMM: the accumulators go straight to C ----
    // accumulator v of lane l in MFMA tile (i, j) is C[(v / 4) * 8 + (l / 32) * 4 + v % 4][l % 32];
    // lanes 0-31 (32-63) store 32 consecutive columns of one row
    const int half_g = lane >> 5, col_g = lane & 31;
    // a bf16 output over an fp32 running sum: the sum is completed in C first,
    // then each thread rounds the elements it wrote
    const bool via_c = to_bf16 && P.accumulate && P.C != nullptr;
    // every accumulator inside the output, one loop per kind of store: a
    // single loop choosing its store per element grew past what the compiler
    // unrolls and put the 256 accumulators on the stack (1088 bytes per lane)
    auto each = [&](auto&& put) {
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = m0 + wm * kWM + i * 32 + (v >> 2) * 8 + half_g * 4 + (v & 3);
            const int64_t col = n0 + wn * kWN + j * 32 + col_g;
            if (row < row_end && col < P.V) put(row, col, acc[i][j][v]);
          }
    };
    if (to_bf16 && !via_c) {
      if (P.cb_f16)
        each([&](int64_t row, int64_t col, float o) { P.Cb[row * P.ldcb + col] = bits_of<F16>(o); });
      else
        each([&](int64_t row, int64_t col, float o) { P.Cb[row * P.ldcb + col] = bits_of<BF16>(o); });
    } else if (P.accumulate) {
      each([&](int64_t row, int64_t col, float o) { P.C[(ks * P.nrows + row) * P.ldc + col] += o; });
    } else {
      each([&](int64_t row, int64_t col, float o) { P.C[(ks * P.nrows + row) * P.ldc + col] = o; });
    }
    if (via_c) {
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = m0 + wm * kWM + i * 32 + (v >> 2) * 8 + half_g * 4 + (v & 3);
            const int64_t col = n0 + wn * kWN + j * 32 + col_g;
            if (row < row_end && col < P.V) {
              const float o = P.C[row * P.ldc + col];
              P.Cb[row * P.ldcb + col] = P.cb_f16 ? bits_of<F16>(o) : bits_of<BF16>(o);
            }
          }
    }
  } else {
  // ---- epilogue: the tile goes through LDS as bf16, one row per thread ----
  //
  // The accumulators of a row are spread over 32 lanes; instead of cross-lane
  // reductions each wave writes its quarter to LDS (row-major [256][256] bf16
  // over the two stage arrays, 16-byte chunks XOR-swizzled by row % 32) and
  // thread t then walks row t (forward) or copies rows out with 16-byte stores
  // (gradient).  Every direct load has landed (the last wait was vmcnt(0)); the
  // barrier orders every wave's last fragment reads before the stores.
  wait_vm_barrier<0>();
  const int half = lane >> 5;  // which 4-row group of each 8-row band this lane holds
  const int col_lane = lane & 31;
  const int wm_u = wave_u >> 1;
  // the epilogue rows of this wave's quarter live in stage array wm
  auto xq = [&](int) { return reinterpret_cast<uint16_t*>(stage_ptr(wm_u)); };
  if (MODE == kFwd) {
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      uint16_t* xs = xq(i);
#pragma unroll
      for (int j = 0; j < kTN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
          const int cl = wn * kWN + j * 32 + col_lane;
          xs[xs_index(rl, cl)] = bits_of<E>(acc[i][j][v]);
        }
    }
    __syncthreads();
    const int64_t r = m0 + tid;
    if (r < row_end) {
      // row tid is local row tid % 128 of stage array tid / 128
      const uint16_t* xs = reinterpret_cast<const uint16_t*>(stage_ptr(wm_u));
      const int ncols = (P.V - n0 < kBN) ? (int)(P.V - n0) : kBN;
      const vu4* rowp = reinterpret_cast<const vu4*>(xs + (tid & (kEpiRows - 1)) * kBN);
      const int sw = tid & 31;
      float M = -INFINITY, sum = 0.f;
      // two passes (max, then sum of exp); the column bound is only checked in
      // the last, partial column tile
      auto walk = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        for (int c = 0; c < kBN / 8; ++c) {
          float w[8];
          E::unpack(rowp[c ^ sw], w);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (FULL || c * 8 + e < ncols) M = fmaxf(M, w[e]);
        }
        if (M != -INFINITY) {
          float s4[4] = {0.f, 0.f, 0.f, 0.f};
          for (int c = 0; c < kBN / 8; ++c) {
            float w[8];
            E::unpack(rowp[c ^ sw], w);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (FULL || c * 8 + e < ncols) s4[e & 3] += fast_exp2((w[e] - M) * kLog2e);
          }
          sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
        }
      };
      if (ncols == kBN)
        walk(std::true_type{});
      else
        walk(std::false_type{});
      float* dst = P.part + ((r - P.row0) * P.n_nt + nt) * 2;
      dst[0] = M;
      dst[1] = sum;
      const int tc = s_tcol[tid];
      if (tc >= 0) P.xt[r - P.row0] = value_of<E>(xs[xs_index(tid, tc)]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
      uint16_t* xs = xq(i);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int rl = wm * kWM + i * 32 + (v >> 2) * 8 + half * 4 + (v & 3);
        const float gv = s_g[rl], M = s_m[rl], LS = s_ls[rl];
        const int tc = s_tcol[rl];
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
          const int cl = wn * kWN + j * 32 + col_lane;
          const float x = round_trip<E>(acc[i][j][v]);  // the logit in the operand dtype
          const float p = fast_exp2(((x - M) - LS) * kLog2e);
          const float o = (cl == tc) ? (1.f - p) * gv : -p * gv;
          xs[xs_index(rl, cl)] = bits_of<BF16>(o);  // G is bf16 for either operand dtype
        }
      }
    }
    __syncthreads();
    // 32 threads per row, one 16-byte chunk each; 8 rows per pass
    const int c = tid & 31;
#pragma unroll 4
    for (int k = 0; k < kBM / 8; ++k) {
      const int rl = (tid >> 5) + 8 * k;
      const int64_t r = m0 + rl;
      const int64_t col0 = n0 + c * 8;
      if (r >= row_end || col0 >= P.V) continue;
      const uint16_t* xs = reinterpret_cast<const uint16_t*>(stage_ptr(rl / kEpiRows));
      const vu4 q = reinterpret_cast<const vu4*>(xs + (rl & (kEpiRows - 1)) * kBN)[c ^ (rl & 31)];
      uint16_t* dst = P.G + (r - P.row0) * P.ldg + col0;
      if (col0 + 8 <= P.V && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
        *reinterpret_cast<vu4*>(dst) = q;
      } else {
        const uint32_t wv[4] = {q.x, q.y, q.z, q.w};
        for (int e = 0; e < 8 && col0 + e < P.V; ++e)
          dst[e] = (uint16_t)(wv[e >> 1] >> ((e & 1) * 16));
      }
    }
    if (P.Gt != nullptr) {
      // the transposed tile: thread t writes column t of the tile as 256
      // consecutive elements of G^T row n0 + t (rows of G past its end are
      // zeros, which the caller's padded reduction length relies on)
      const int64_t col = n0 + tid;
      if (col < P.V) {
        uint16_t* dst = P.Gt + col * P.ldgt + (m0 - P.row0);
        const uint16_t* x0 = reinterpret_cast<const uint16_t*>(stage_ptr(0));
        const uint16_t* x1 = reinterpret_cast<const uint16_t*>(stage_ptr(1));
#pragma unroll 4
        for (int r8 = 0; r8 < kBM / 8; ++r8) {
          uint32_t wv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int ra = r8 * 8 + 2 * e, rb = ra + 1;
            const uint32_t lo = (ra < kEpiRows ? x0 : x1)[xs_index(ra, tid)];
            const uint32_t hi = (rb < kEpiRows ? x0 : x1)[xs_index(rb, tid)];
            wv[e] = lo | (hi << 16);
          }
          *reinterpret_cast<vu4*>(dst + r8 * 8) = vu4{wv[0], wv[1], wv[2], wv[3]};
        }
      }
    }
  }
  }  // the fused epilogues
}

// dst[c][r] = bf16(src[r][c]) for r < R, c < C, and dst[c][r] = 0 for
// R <= r < Rp (src of dtype ES, bf16 or fp16; dst rows of stride ldd >= Rp),
// R = min(R, *count) when count is given.  64 x 64 tiles through LDS, moved
// as 16-byte pieces (eight elements of a row in, eight of a column out) where
// the pointers, strides and tile edges allow, element by element elsewhere.
template <class ES>
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ src,
                                                             int64_t R, int64_t C, int64_t lds,
                                                             uint16_t* __restrict__ dst,
                                                             int64_t ldd, int64_t Rp,
                                                             int64_t n_ct,
                                                             const int64_t* __restrict__ count) {
  // row pitch 66 elements (33 words): the eight rows 8 apart that a wave's
  // column reads touch start in different LDS banks
  constexpr int kP = 66;
  __shared__ uint16_t tile[64 * kP];
  if (count != nullptr && *count < R) R = *count;
  const int64_t tr = blockIdx.x / n_ct, tc = blockIdx.x - tr * n_ct;
  const int64_t r0 = tr * 64, c0 = tc * 64;
  const bool vin = ((lds & 7) | (reinterpret_cast<uintptr_t>(src) & 15)) == 0;
  const bool vout = ((ldd & 7) | (reinterpret_cast<uintptr_t>(dst) & 15)) == 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = (int)threadIdx.x + 256 * k, lr = idx >> 3, cg = (idx & 7) * 8;
    const int64_t r = r0 + lr, c = c0 + cg;
    uint32_t w[4];
    if (vin && r < R && c + 8 <= C) {
      const vu4 q = *reinterpret_cast<const vu4*>(src + r * lds + c);
      w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = (r < R && c + 2 * j < C) ? src[r * lds + c + 2 * j] : 0u;
        const uint32_t hi = (r < R && c + 2 * j + 1 < C) ? src[r * lds + c + 2 * j + 1] : 0u;
        w[j] = lo | (hi << 16);
      }
    }
    if constexpr (std::is_same<ES, F16>::value) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)bits_of<BF16>(value_of<F16>((uint16_t)(w[j] & 0xffffu))) |
               ((uint32_t)bits_of<BF16>(value_of<F16>((uint16_t)(w[j] >> 16))) << 16);
    }
    // (lr * 66 + cg) elements = a whole number of 4-byte words
    uint32_t* t32 = reinterpret_cast<uint32_t*>(tile + lr * kP + cg);
#pragma unroll
    for (int j = 0; j < 4; ++j) t32[j] = w[j];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int idx = (int)threadIdx.x + 256 * k, lc = idx >> 3, rg = (idx & 7) * 8;
    const int64_t c = c0 + lc, r = r0 + rg;
    if (c >= C) continue;
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)tile[(rg + 2 * j) * kP + lc] | ((uint32_t)tile[(rg + 2 * j + 1) * kP + lc] << 16);
    uint16_t* d = dst + c * ldd + r;
    if (vout && r + 8 <= Rp) {
      *reinterpret_cast<vu4*>(d) = vu4{w[0], w[1], w[2], w[3]};
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (r + i < Rp) d[i] = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
    }
  }
}

// dst[c][r] = src[r][c] for r < R, c < C, and dst[c][r] = 0 for R <= r < Rp
// (fp32; dst rows of stride ldd >= Rp), R = min(R, *count - count_off) when
// count is given.  64 x 64 tiles through LDS, moved as 16-byte pieces (four
// elements of a row in, four of a column out) where the pointers, strides and
// tile edges allow, element by element elsewhere.
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ src, int64_t R,
                                                            int64_t C, int64_t lds,
                                                            float* __restrict__ dst, int64_t ldd,
                                                            int64_t Rp, int64_t n_ct,
                                                            const int64_t* __restrict__ count,
                                                            int64_t count_off) {
  // row pitch 65 words: a wave's row pieces and column reads each fall in
  // distinct LDS banks
  constexpr int kP = 65;
  __shared__ float tile[64 * kP];
  if (count != nullptr) {
    const int64_t c = *count - count_off;
    if (c < R) R = c < 0 ? 0 : c;
  }
  const int64_t tr = blockIdx.x / n_ct, tc = blockIdx.x - tr * n_ct;
  const int64_t r0 = tr * 64, c0 = tc * 64;
  const bool vin = ((lds & 3) | (reinterpret_cast<uintptr_t>(src) & 15)) == 0;
  const bool vout = ((ldd & 3) | (reinterpret_cast<uintptr_t>(dst) & 15)) == 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = (int)threadIdx.x + 256 * k, lr = idx >> 4, cg = (idx & 15) * 4;
    const int64_t r = r0 + lr, c = c0 + cg;
    float w[4];
    if (vin && r < R && c + 4 <= C) {
      const float4 q = *reinterpret_cast<const float4*>(src + r * lds + c);
      w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (r < R && c + j < C) ? src[r * lds + c + j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) tile[lr * kP + cg + j] = w[j];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = (int)threadIdx.x + 256 * k, lc = idx >> 4, rg = (idx & 15) * 4;
    const int64_t c = c0 + lc, r = r0 + rg;
    if (c >= C) continue;
    float w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = tile[(rg + i) * kP + lc];
    float* d = dst + c * ldd + r;
    if (vout && r + 4 <= Rp) {
      *reinterpret_cast<float4*>(d) = make_float4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (r + i < Rp) d[i] = w[i];
    }
  }
}

// out[r(m)][n] = EO(sum over s of part[s][m][n]) (EO bf16, fp16 or fp32), summed in split order,
// with r(m) = out_rows[m] when a row map is given (rows mapped outside
// [0, out_nrows) are skipped) and m otherwise; with a count, rows
// m >= *count - count_off are written as zeros without reading.  VEC
// consecutive elements per thread (N and ld multiples of VEC).
template <int VEC, class EO>
__global__ __launch_bounds__(256) void sum_splits_kernel(const float* __restrict__ part,
                                                         int64_t n_ks, int64_t M, int64_t N,
                                                         int64_t ld, void* __restrict__ out,
                                                         int64_t ldo,
                                                         const int64_t* __restrict__ out_rows,
                                                         int64_t out_nrows,
                                                         const int64_t* __restrict__ count,
                                                         int64_t count_off) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VEC;
  if (i >= M * N) return;
  const int64_t m = i / N, n = i - m * N;
  int64_t r = m;
  if (out_rows != nullptr) {
    r = out_rows[m];
    if (r < 0 || r >= out_nrows) return;
  }
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  if (count == nullptr || m < *count - count_off) {
    for (int64_t s = 0; s < n_ks; ++s) {
      const float* src = part + (s * M + m) * ld + n;
      if constexpr (VEC == 4) {
        const float4 q = *reinterpret_cast<const float4*>(src);
        acc[0] += q.x;
        acc[1] += q.y;
        acc[2] += q.z;
        acc[3] += q.w;
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += src[e];
      }
    }
  }
  if constexpr (std::is_same<EO, F32>::value) {
    float* dst = static_cast<float*>(out) + r * ldo + n;
    if constexpr (VEC == 4) {
      *reinterpret_cast<float4*>(dst) = float4{acc[0], acc[1], acc[2], acc[3]};
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e] = acc[e];
    }
  } else {
    uint16_t* dst = static_cast<uint16_t*>(out) + r * ldo + n;
    if constexpr (VEC == 4) {
      const uint32_t lo = (uint32_t)bits_of<EO>(acc[0]) | ((uint32_t)bits_of<EO>(acc[1]) << 16);
      const uint32_t hi = (uint32_t)bits_of<EO>(acc[2]) | ((uint32_t)bits_of<EO>(acc[3]) << 16);
      *reinterpret_cast<uint2*>(dst) = uint2{lo, hi};
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e] = bits_of<EO>(acc[e]);
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
  MIRL_REQUIRE(Hd % (kStages * kSK) == 0, "hidden size %lld must be a multiple of %d", (long long)Hd,
               kStages * kSK);
  MIRL_REQUIRE(ldh < (int64_t(1) << 22) && ldw < (int64_t(1) << 22),
               "row strides (%lld, %lld) must be below 2^22 elements", (long long)ldh, (long long)ldw);
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

static bool lce_dtype_ok(int dtype) { return dtype == MIRL_DTYPE_BF16 || dtype == MIRL_DTYPE_F16; }

extern "C" int mirl_linear_ce_fwd(const void* hidden, int dtype, int64_t T, int64_t Hd, int64_t ldh,
                                  const void* weight, int64_t V, int64_t ldw, int64_t bsz,
                                  const int64_t* target, int64_t t_stride_b, int64_t t_stride_s,
                                  int64_t vocab_start, int64_t vocab_end, float* out,
                                  int64_t o_stride_b, int64_t o_stride_s, float* row_stats,
                                  float* workspace, void* stream) {
  clear_error();
  MIRL_REQUIRE(lce_dtype_ok(dtype), "hidden states and weight must be bf16 or fp16 (dtype code %d)",
               dtype);
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
  if (dtype == MIRL_DTYPE_BF16)
    hipLaunchKernelGGL((lce_tile_kernel<kFwd, BF16>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((lce_tile_kernel<kFwd, F16>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  hipLaunchKernelGGL(lce_merge_kernel, dim3((unsigned)ceil_div(T, 4)), dim3(256), 0, st, P.part,
                     P.xt, (int64_t)0, T, P.n_nt, bsz, target, t_stride_b, t_stride_s,
                     vocab_start, vocab_end, V, out, o_stride_b, o_stride_s, row_stats);
  return check_launch("mirl_linear_ce_fwd");
}

extern "C" int mirl_linear_ce_grad(const void* hidden, int dtype, int64_t T, int64_t Hd, int64_t ldh,
                                   const void* weight, int64_t V, int64_t ldw, int64_t bsz,
                                   const int64_t* target, int64_t t_stride_b,
                                   int64_t t_stride_s, int64_t vocab_start, int64_t vocab_end,
                                   const float* row_stats, const float* grad_out,
                                   int64_t g_stride_b, int64_t g_stride_s, int64_t row0,
                                   int64_t nrows, void* grad_logits, int64_t ldg,
                                   void* grad_logits_t, int64_t ldgt, const int64_t* row_count,
                                   void* stream) {
  clear_error();
  MIRL_REQUIRE(lce_dtype_ok(dtype), "hidden states and weight must be bf16 or fp16 (dtype code %d)",
               dtype);
  if (int e = check_common(hidden, T, Hd, ldh, weight, V, ldw, target, bsz)) return e;
  MIRL_REQUIRE(row0 >= 0 && nrows >= 0 && row0 + nrows <= T, "row range [%lld, %lld) outside [0, %lld)",
               (long long)row0, (long long)(row0 + nrows), (long long)T);
  if (nrows == 0) return MIRL_OK;
  MIRL_REQUIRE(row_stats && grad_out && grad_logits, "null pointer argument");
  MIRL_REQUIRE(ldg >= V, "gradient row stride %lld is smaller than V=%lld", (long long)ldg,
               (long long)V);
  // the transposed tiles cover whole 256-row tiles, written as 16-byte vectors
  MIRL_REQUIRE(grad_logits_t == nullptr ||
                   (ldgt >= ceil_div(nrows, kBM) * kBM && ldgt % 8 == 0 &&
                    (reinterpret_cast<uintptr_t>(grad_logits_t) & 15u) == 0),
               "transposed gradient: row stride %lld must cover %lld rows in whole 256-row tiles, "
               "be a multiple of 8 elements and start 16-byte aligned",
               (long long)ldgt, (long long)nrows);
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
  P.Gt = static_cast<uint16_t*>(grad_logits_t);
  P.ldgt = ldgt;
  P.count = row_count;
  const int64_t grid = ceil_div(P.n_mt * P.n_nt, kXcds) * kXcds;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  if (dtype == MIRL_DTYPE_BF16)
    hipLaunchKernelGGL((lce_tile_kernel<kGrad, BF16>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  else
    hipLaunchKernelGGL((lce_tile_kernel<kGrad, F16>), dim3((unsigned)grid), dim3(kThreads), 0, st, P);
  return check_launch("mirl_linear_ce_grad");
}

extern "C" int mirl_gemm_bf16_abt(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                                  int64_t N, int64_t K, int64_t k_splits, float* C, int64_t ldc,
                                  int accumulate, void* Cb, int64_t ldcb, int cb_dtype,
                                  const int64_t* count, int64_t count_off, int count_axis,
                                  int64_t final_at, void* stream) {
  clear_error();
  MIRL_REQUIRE(Cb == nullptr || lce_dtype_ok(cb_dtype), "the 16-bit output must be bf16 or fp16 (dtype code %d)",
               cb_dtype);
  MIRL_REQUIRE(M >= 0 && N >= 0 && K > 0 && k_splits >= 1, "invalid shape M=%lld N=%lld K=%lld splits=%lld",
               (long long)M, (long long)N, (long long)K, (long long)k_splits);
  if (M == 0 || N == 0) return MIRL_OK;
  MIRL_REQUIRE(A && B && (C || Cb), "null pointer argument");
  const int64_t kstep = (int64_t)kStages * kSK;
  MIRL_REQUIRE(K % kstep == 0, "reduction length %lld must be a multiple of %lld", (long long)K,
               (long long)kstep);
  const int64_t kb = ceil_div(ceil_div(K, k_splits), kstep) * kstep;
  const int64_t n_ks = ceil_div(K, kb);
  MIRL_REQUIRE(n_ks == k_splits,
               "%lld splits of K=%lld in ranges of %lld leave %lld non-empty (choose a split count "
               "that divides into whole 128-element ranges)",
               (long long)k_splits, (long long)K, (long long)kb, (long long)n_ks);
  MIRL_REQUIRE(count_axis == MIRL_COUNT_ROWS || count_axis == MIRL_COUNT_K, "invalid count axis %d",
               count_axis);
  const bool both = C != nullptr && Cb != nullptr;
  MIRL_REQUIRE(!both || (count != nullptr && count_axis == MIRL_COUNT_K && n_ks == 1),
               "an fp32 and a bf16 output together take a reduction-length count and one split");
  MIRL_REQUIRE(Cb == nullptr || (n_ks == 1 && (!accumulate || both)),
               "a bf16 output takes one split and accumulates only over the fp32 output");
  MIRL_REQUIRE(!accumulate || n_ks == 1, "accumulation takes one split");
  MIRL_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K,
               "row strides (%lld, %lld) must be multiples of 8 elements and >= K", (long long)lda,
               (long long)ldb);
  MIRL_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15u) == 0 && (reinterpret_cast<uintptr_t>(B) & 15u) == 0,
               "operands must be 16-byte aligned");
  // buffer ranges of one 256-row tile are 32-bit byte counts
  MIRL_REQUIRE(kBM * lda * 2 < (int64_t(1) << 31) && kBN * ldb * 2 < (int64_t(1) << 31),
               "row strides (%lld, %lld) too large", (long long)lda, (long long)ldb);
  MIRL_REQUIRE(M < (int64_t(1) << 31) && N < (int64_t(1) << 31), "sizes exceed 2^31-1");
  MIRL_REQUIRE(C == nullptr || ldc >= N, "output row stride %lld is smaller than N=%lld",
               (long long)ldc, (long long)N);
  MIRL_REQUIRE(Cb == nullptr || ldcb >= N, "output row stride %lld is smaller than N=%lld",
               (long long)ldcb, (long long)N);
  LceParams P{};
  P.h = static_cast<const uint16_t*>(A);
  P.w = static_cast<const uint16_t*>(B);
  P.ldh = lda;
  P.ldw = ldb;
  P.V = N;
  P.Hd = K;
  P.row0 = 0;
  P.nrows = M;
  P.n_mt = ceil_div(M, kBM);
  P.n_nt = ceil_div(N, kBN);
  P.n_ks = n_ks;
  P.kb_len = kb;
  P.C = C;
  P.Cb = static_cast<uint16_t*>(Cb);
  P.cb_f16 = cb_dtype == MIRL_DTYPE_F16;
  P.ldc = ldc;
  P.ldcb = ldcb;
  P.accumulate = accumulate;
  P.count = count;
  P.count_off = count_off;
  P.count_axis = count_axis;
  P.final_at = final_at;
  const int64_t grid = ceil_div(P.n_mt * P.n_nt * n_ks, kXcds) * kXcds;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((lce_tile_kernel<kGemm, BF16>), dim3((unsigned)grid), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), P);
  return check_launch("mirl_gemm_bf16_abt");
}

extern "C" int mirl_sum_splits_bf16(const float* part, int64_t k_splits, int64_t M, int64_t N,
                                    int64_t ld, void* out, int64_t ldo, int out_dtype,
                                    const int64_t* out_rows, int64_t out_nrows,
                                    const int64_t* count, int64_t count_off, void* stream) {
  clear_error();
  MIRL_REQUIRE(lce_dtype_ok(out_dtype) || out_dtype == MIRL_DTYPE_F32,
               "the output must be bf16, fp16 or fp32 (dtype code %d)", out_dtype);
  MIRL_REQUIRE(M >= 0 && N >= 0 && k_splits >= 1 && ld >= N && ldo >= N, "invalid shape");
  if (M == 0 || N == 0) return MIRL_OK;
  MIRL_REQUIRE(part && out, "null pointer argument");
  MIRL_REQUIRE(out_rows == nullptr || out_nrows >= 0, "invalid output row count");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uintptr_t out_align = out_dtype == MIRL_DTYPE_F32 ? 15u : 7u;  // 4 elements
  const bool vec4 = N % 4 == 0 && ld % 4 == 0 && ldo % 4 == 0 &&
                    (reinterpret_cast<uintptr_t>(part) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & out_align) == 0;
  auto launch = [&](auto vec_c, auto eo) {
    constexpr int VEC = decltype(vec_c)::value;
    using EO = decltype(eo);
    hipLaunchKernelGGL((sum_splits_kernel<VEC, EO>), dim3((unsigned)ceil_div(M * N / VEC, 256)),
                       dim3(256), 0, st, part, k_splits, M, N, ld, out, ldo, out_rows, out_nrows,
                       count, count_off);
  };
  using V4 = std::integral_constant<int, 4>;
  using V1 = std::integral_constant<int, 1>;
  if (out_dtype == MIRL_DTYPE_BF16) {
    if (vec4) launch(V4{}, BF16{}); else launch(V1{}, BF16{});
  } else if (out_dtype == MIRL_DTYPE_F16) {
    if (vec4) launch(V4{}, F16{}); else launch(V1{}, F16{});
  } else {
    if (vec4) launch(V4{}, F32{}); else launch(V1{}, F32{});
  }
  return check_launch("mirl_sum_splits_bf16");
}

extern "C" int mirl_transpose_bf16(const void* src, int src_dtype, int64_t R, int64_t C,
                                   int64_t lds, void* dst, int64_t ldd, int64_t R_pad,
                                   const int64_t* count, void* stream) {
  clear_error();
  MIRL_REQUIRE(lce_dtype_ok(src_dtype), "the source must be bf16 or fp16 (dtype code %d)", src_dtype);
  MIRL_REQUIRE(R >= 0 && C >= 0 && R_pad >= R && lds >= C && ldd >= R_pad, "invalid shape");
  if (C == 0 || R_pad == 0) return MIRL_OK;
  MIRL_REQUIRE(src && dst, "null pointer argument");
  const int64_t n_rt = ceil_div(R_pad, 64), n_ct = ceil_div(C, 64);
  MIRL_REQUIRE(n_rt * n_ct < (int64_t(1) << 31), "too many tiles");
  auto launch = [&](auto es) {
    using ES = decltype(es);
    hipLaunchKernelGGL((transpose_bf16_kernel<ES>), dim3((unsigned)(n_rt * n_ct)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(src), R, C,
                       lds, static_cast<uint16_t*>(dst), ldd, R_pad, n_ct, count);
  };
  if (src_dtype == MIRL_DTYPE_BF16) launch(BF16{}); else launch(F16{});
  return check_launch("mirl_transpose_bf16");
}

extern "C" int mirl_gemm_f32_abt(const float* A, int64_t lda, const float* B, int64_t ldb, int64_t M,
                                 int64_t N, int64_t K, int64_t k_splits, float* C, int64_t ldc,
                                 int accumulate, const int64_t* count, int64_t count_off,
                                 int count_axis, void* stream) {
  clear_error();
  MIRL_REQUIRE(M >= 0 && N >= 0 && K > 0 && k_splits >= 1, "invalid shape M=%lld N=%lld K=%lld splits=%lld",
               (long long)M, (long long)N, (long long)K, (long long)k_splits);
  if (M == 0 || N == 0) return MIRL_OK;
  MIRL_REQUIRE(A && B && C, "null pointer argument");
  const int64_t kstep = (int64_t)kStages * (kRowBytes / 4);
  MIRL_REQUIRE(K % kstep == 0, "reduction length %lld must be a multiple of %lld", (long long)K,
               (long long)kstep);
  const int64_t kb = ceil_div(ceil_div(K, k_splits), kstep) * kstep;
  const int64_t n_ks = ceil_div(K, kb);
  MIRL_REQUIRE(n_ks == k_splits,
               "%lld splits of K=%lld in ranges of %lld leave %lld non-empty (choose a split count "
               "that divides into whole 64-element ranges)",
               (long long)k_splits, (long long)K, (long long)kb, (long long)n_ks);
  MIRL_REQUIRE(count_axis == MIRL_COUNT_ROWS || count_axis == MIRL_COUNT_K, "invalid count axis %d",
               count_axis);
  MIRL_REQUIRE(!accumulate || n_ks == 1, "accumulation takes one split");
  MIRL_REQUIRE(lda % 4 == 0 && ldb % 4 == 0 && lda >= K && ldb >= K,
               "row strides (%lld, %lld) must be multiples of 4 elements and >= K", (long long)lda,
               (long long)ldb);
  MIRL_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15u) == 0 && (reinterpret_cast<uintptr_t>(B) & 15u) == 0,
               "operands must be 16-byte aligned");
  // buffer ranges of one 256-row tile are 32-bit byte counts
  MIRL_REQUIRE(kBM * lda * 4 < (int64_t(1) << 31) && kBN * ldb * 4 < (int64_t(1) << 31),
               "row strides (%lld, %lld) too large", (long long)lda, (long long)ldb);
  MIRL_REQUIRE(M < (int64_t(1) << 31) && N < (int64_t(1) << 31), "sizes exceed 2^31-1");
  MIRL_REQUIRE(ldc >= N, "output row stride %lld is smaller than N=%lld", (long long)ldc, (long long)N);
  LceParams P{};
  P.h = A;
  P.w = B;
  P.ldh = lda;
  P.ldw = ldb;
  P.V = N;
  P.Hd = K;
  P.row0 = 0;
  P.nrows = M;
  P.n_mt = ceil_div(M, kBM);
  P.n_nt = ceil_div(N, kBN);
  P.n_ks = n_ks;
  P.kb_len = kb;
  P.C = C;
  P.Cb = nullptr;
  P.ldc = ldc;
  P.accumulate = accumulate;
  P.count = count;
  P.count_off = count_off;
  P.count_axis = count_axis;
  P.final_at = 0;
  const int64_t grid = ceil_div(P.n_mt * P.n_nt * n_ks, kXcds) * kXcds;
  MIRL_REQUIRE(grid < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL((lce_tile_kernel<kGemm, F32>), dim3((unsigned)grid), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), P);
  return check_launch("mirl_gemm_f32_abt");
}

extern "C" int mirl_transpose_f32(const float* src, int64_t R, int64_t C, int64_t lds, float* dst,
                                  int64_t ldd, int64_t R_pad, const int64_t* count, int64_t count_off,
                                  void* stream) {
  clear_error();
  MIRL_REQUIRE(R >= 0 && C >= 0 && R_pad >= R && lds >= C && ldd >= R_pad, "invalid shape");
  if (C == 0 || R_pad == 0) return MIRL_OK;
  MIRL_REQUIRE(src && dst, "null pointer argument");
  const int64_t n_rt = ceil_div(R_pad, 64), n_ct = ceil_div(C, 64);
  MIRL_REQUIRE(n_rt * n_ct < (int64_t(1) << 31), "too many tiles");
  hipLaunchKernelGGL(transpose_f32_kernel, dim3((unsigned)(n_rt * n_ct)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), src, R, C, lds, dst, ldd, R_pad, n_ct, count,
                     count_off);
  return check_launch("mirl_transpose_f32");
}

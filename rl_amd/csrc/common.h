// Shared device and host helpers for libmirl (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <type_traits>
#include <string>

#include "../../include/mirl.h"

namespace mirl {

// Native 16-byte vector (clang ext vector, usable with the nontemporal builtins).
typedef uint32_t vu4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// host-side error state
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
void clear_error();

#define MIRL_REQUIRE(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      ::mirl::set_error(__VA_ARGS__);           \
      return MIRL_ERR_INVALID_ARGUMENT;         \
    }                                           \
  } while (0)

// Returns MIRL_ERR_HIP with the runtime's message when the last launch failed.
int check_launch(const char* what);

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The reference's in-place temperature, logits.div_(T), runs on the GPU, where
// torch divides a tensor by a Python scalar as a product with the reciprocal
// formed in double and rounded once to fp32: y = dtype(fl32(float(x) * r)),
// r = fl32(1.0 / T); autograd's backward of that division does the same to the
// gradient.  The host forms r with temperature_recip.
inline float temperature_recip(double T) { return (float)(1.0 / T); }

// fl32(x * r) as a product rounded on its own: contraction is off in this
// scope, so the multiply is never fused with an add that consumes it, and the
// empty asm makes the fp32 product opaque, so that a narrowing to fp16 that
// follows rounds that product (two roundings, as torch's vectorised kernel
// does) instead of being folded with the multiply into one mixed-precision
// instruction that rounds the exact product once.
__device__ __forceinline__ float mul_rn(float x, float r) {
#pragma clang fp contract(off)
  float p = x * r;
  asm("" : "+v"(p));
  return p;
}

// Element loaders: raw storage type -> fp32.
struct F32 {
  using raw = float;
  static constexpr int kVec = 4;  // elements per 16-byte vector
  static constexpr uint32_t kNegInf2 = 0xFF800000u;  // one 32-bit word of -inf elements
  // one word of -2^100 elements: very low, finite, and x*log2e is exact in fp32
  static constexpr uint32_t kLowPad2 = 0xF1800000u;
  __device__ __forceinline__ static float load(const raw* p) { return *p; }
  __device__ __forceinline__ static float load_raw(raw r) { return r; }
  __device__ __forceinline__ static void unpack(const vu4& q, float (&v)[kVec]) {
    v[0] = __uint_as_float(q.x);
    v[1] = __uint_as_float(q.y);
    v[2] = __uint_as_float(q.z);
    v[3] = __uint_as_float(q.w);
  }
  __device__ __forceinline__ static raw from_float(float f) { return f; }
  __device__ __forceinline__ static vu4 pack(const float (&v)[kVec]) {
    return vu4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
               __float_as_uint(v[3])};
  }
};

// bfloat16 stored as uint16_t bits.  Widening is exact (a shift); narrowing uses
// the gfx950 v_cvt_pk_bf16_f32 instruction (round to nearest even, NaN kept).
struct BF16 {
  using raw = uint16_t;
  static constexpr int kVec = 8;
  static constexpr uint32_t kNegInf2 = 0xFF80FF80u;
  static constexpr uint32_t kLowPad2 = 0xF180F180u;  // -2^100 (see F32)
  __device__ __forceinline__ static float widen(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
  }
  __device__ __forceinline__ static float load(const raw* p) { return widen(*p); }
  __device__ __forceinline__ static float load_raw(raw r) { return widen(r); }
  __device__ __forceinline__ static void unpack(const vu4& q, float (&v)[kVec]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = __uint_as_float(w[k] << 16);
      v[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    bf16x2 r;
    r.x = (__bf16)lo;
    r.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ __forceinline__ static raw from_float(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
  }
  __device__ __forceinline__ static vu4 pack(const float (&v)[kVec]) {
    return vu4{pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7])};
  }
};

struct F16 {
  using raw = _Float16;
  static constexpr int kVec = 8;
  static constexpr uint32_t kNegInf2 = 0xFC00FC00u;
  static constexpr uint32_t kLowPad2 = 0xF800F800u;  // -2^15 (see F32)
  __device__ __forceinline__ static float load(const raw* p) { return (float)*p; }
  __device__ __forceinline__ static float load_raw(raw r) { return (float)r; }
  __device__ __forceinline__ static void unpack(const vu4& q, float (&v)[kVec]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      h2 h = __builtin_bit_cast(h2, w[k]);
      v[2 * k] = (float)h.x;
      v[2 * k + 1] = (float)h.y;
    }
  }
  // The value is narrowed as an fp32 register holds it: the empty asm keeps
  // the compiler from folding a product that feeds the narrowing into one
  // mixed-precision fma (v_fma_mix), which rounds the exact product to fp16
  // once and so differs from fl16(fl32(a * b)) where fl32(a * b) falls
  // exactly between two fp16 values.
  __device__ __forceinline__ static raw from_float(float f) {
    asm("" : "+v"(f));
    return (_Float16)f;
  }
  __device__ __forceinline__ static vu4 pack(const float (&v)[kVec]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float a = v[2 * k], b = v[2 * k + 1];
      asm("" : "+v"(a), "+v"(b));
      h2 h;
      h.x = (_Float16)a;
      h.y = (_Float16)b;
      w[k] = __builtin_bit_cast(uint32_t, h);
    }
    return vu4{w[0], w[1], w[2], w[3]};
  }
};

// Splits a row at `p` into a scalar head (up to the next 16-byte boundary), a
// body of aligned 16-byte vectors and a scalar tail.
template <class E>
struct RowSpan {
  int64_t head, nvec, tail0;
  __device__ __forceinline__ RowSpan(const void* p, int64_t V) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    head = (int64_t)(((16u - (a & 15u)) & 15u) / sizeof(typename E::raw));
    if (head > V) head = V;
    nvec = (V - head) / E::kVec;
    tail0 = head + nvec * E::kVec;
  }
};

// fp32 value rounded to the element type and widened back.
template <class E>
__device__ __forceinline__ float round_trip(float f) {
  return E::load_raw(E::from_float(f));
}

// Two fp32 values rounded to the element type and widened back (one
// conversion instruction for both in bf16).
template <class E>
__device__ __forceinline__ void round_trip2(float& a, float& b) {
  if constexpr (std::is_same<E, BF16>::value) {
    const uint32_t w = BF16::pack2(a, b);
    a = __uint_as_float(w << 16);
    b = __uint_as_float(w & 0xffff0000u);
  } else {
    a = round_trip<E>(a);
    b = round_trip<E>(b);
  }
}

// Wave-wide reductions (64 lanes) through cross-lane shuffles.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace mirl

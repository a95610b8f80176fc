// fmx_common.hpp -- shared device/host helpers of the MI355X MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fmx {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr int kGroup = 64;  // quantisation group (elements)

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even. On gfx950 the device path is one v_cvt_pk_bf16_f32.
__device__ inline uint16_t f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

__device__ inline float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Single round-to-nearest-even from fp64 to bf16, on the integer image of the
// double: keep the top 8 significand bits of a normal result, or scale the
// value onto bf16's subnormal grid (exact power-of-two multiply, then rint).
__device__ inline uint16_t f64_to_bf16(double d) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(d));
  const uint16_t sign = static_cast<uint16_t>((u >> 48) & 0x8000u);
  const uint64_t a = u & 0x7fffffffffffffffull;
  if (a > 0x7ff0000000000000ull) return 0x7fc0u;                     // NaN
  if (a >= 0x47f0000000000000ull) return sign | 0x7f80u;             // >= 2^128: inf
  if (a < 0x3810000000000000ull) {                                   // < 2^-126
    const double n = rint(fabs(d) * 0x1p133);                        // 0..128
    return sign | static_cast<uint16_t>(n);
  }
  const uint64_t r = (a + 0x00000fffffffffffull + ((a >> 45) & 1u)) >> 45;
  return sign | static_cast<uint16_t>(r - (static_cast<uint64_t>(1023 - 127) << 7));
}

// e^r for the router softmax. Cody-Waite reduction by ln2 (fdlibm's split
// constants), degree-13 Taylor polynomial of e^t on |t| <= ln2/2 by Horner
// with explicit fma, scaling by 2^n. Uses IEEE basic operations only, so the
// CPU restatement that follows the same steps produces the same bits.
__device__ inline double exp_det(double r) {
  if (r != r) return r;
  if (r > 709.0) return __builtin_huge_val();
  if (r < -690.0) return 0.0;
  const double log2e = 1.4426950408889634074;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  const double n = rint(r * log2e);
  double t = __builtin_fma(-n, ln2_hi, r);
  t = __builtin_fma(-n, ln2_lo, t);
  double p = 1.0 / 6227020800.0;
  p = __builtin_fma(p, t, 1.0 / 479001600.0);
  p = __builtin_fma(p, t, 1.0 / 39916800.0);
  p = __builtin_fma(p, t, 1.0 / 3628800.0);
  p = __builtin_fma(p, t, 1.0 / 362880.0);
  p = __builtin_fma(p, t, 1.0 / 40320.0);
  p = __builtin_fma(p, t, 1.0 / 5040.0);
  p = __builtin_fma(p, t, 1.0 / 720.0);
  p = __builtin_fma(p, t, 1.0 / 120.0);
  p = __builtin_fma(p, t, 1.0 / 24.0);
  p = __builtin_fma(p, t, 1.0 / 6.0);
  p = __builtin_fma(p, t, 0.5);
  p = __builtin_fma(p, t, 1.0);
  p = __builtin_fma(p, t, 1.0);
  return ldexp(p, static_cast<int>(n));
}

// bf16(sigmoid(v)) for a bf16-valued v, computed in fp64 and rounded once.
__device__ inline float sigmoid_bf16(float v) {
  const double s = 1.0 / (1.0 + exp(-static_cast<double>(v)));
  return bf16_to_f32(f64_to_bf16(s));
}

// bf16(sigmoid(v)) from fp32 hardware exp2 and reciprocal (a few ulp of
// fp32, far below the bf16 rounding step).
__device__ inline float sigmoid_bf16_fast(float v) {
  const float e = __builtin_amdgcn_exp2f(-v * 1.4426950408889634f);
  return round_bf16(__builtin_amdgcn_rcpf(1.0f + e));
}

// MLX's compiled SwiGLU on bf16 arrays: multiply(multiply(g, sigmoid(g)), u),
// every op rounded to bf16 (server/src/model.cpp:14-25).
__device__ inline uint16_t swiglu_bf16(float g_bf, float u_bf) {
  const float sg = sigmoid_bf16_fast(g_bf);
  const float t = round_bf16(g_bf * sg);
  return f32_to_bf16(t * u_bf);
}

// ---- float16 activations (a float16 checkpoint, model.cpp:208-214)

__host__ __device__ inline float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// round to nearest even (the conversion instruction's default mode)
__device__ inline uint16_t f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f)); }

__device__ inline float round_f16(float f) { return f16_to_f32(f32_to_f16(f)); }

// Single round-to-nearest-even from fp64 to fp16, on the integer image of
// the double: keep the top 10 fraction bits of a normal result, or scale the
// value onto fp16's subnormal grid (exact power-of-two multiply, then rint);
// from 65520 (the midpoint past the largest finite value) it is infinite.
__device__ inline uint16_t f64_to_f16(double d) {
  const uint64_t u = static_cast<uint64_t>(__double_as_longlong(d));
  const uint16_t sign = static_cast<uint16_t>((u >> 48) & 0x8000u);
  const uint64_t a = u & 0x7fffffffffffffffull;
  if (a > 0x7ff0000000000000ull) return sign | 0x7e00u;               // NaN
  if (a >= 0x40effe0000000000ull) return sign | 0x7c00u;              // >= 65520: inf
  if (a < 0x3f10000000000000ull)                                      // < 2^-14: subnormal
    return sign | static_cast<uint16_t>(rint(fabs(d) * 0x1p24));      // 0..1024
  const uint64_t r = (a + 0x000001ffffffffffull + ((a >> 42) & 1u)) >> 42;
  return sign | static_cast<uint16_t>(r - (static_cast<uint64_t>(1023 - 15) << 10));
}

// fp16(sigmoid(v)) for an fp16-valued v, computed in fp64 and rounded once
__device__ inline float sigmoid_f16(float v) {
  const double s = 1.0 / (1.0 + exp(-static_cast<double>(v)));
  return f16_to_f32(f64_to_f16(s));
}

// MLX's compiled SwiGLU on float16 arrays: every op rounded to fp16
__device__ inline uint16_t swiglu_f16(float g_h, float u_h) {
  const float e = __builtin_amdgcn_exp2f(-g_h * 1.4426950408889634f);
  const float sg = round_f16(__builtin_amdgcn_rcpf(1.0f + e));
  const float t = round_f16(g_h * sg);
  return f32_to_f16(t * u_h);
}

// The activation dtype's loads and roundings: Act<false> bf16, Act<true>
// fp16; lo / hi load the low / high element of a 32-bit pair
template <bool F16>
struct Act {
  static __device__ inline float ld(uint16_t h) { return bf16_to_f32(h); }
  static __device__ inline float lo(uint32_t v) { return __uint_as_float(v << 16); }
  static __device__ inline float hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
  static __device__ inline uint16_t st(float f) { return f32_to_bf16(f); }
  static __device__ inline float rnd(float f) { return round_bf16(f); }
  static __device__ inline uint16_t from64(double d) { return f64_to_bf16(d); }
  static __device__ inline float sigmoid(float v) { return sigmoid_bf16(v); }
  static __device__ inline uint16_t swiglu(float g, float u) { return swiglu_bf16(g, u); }
};
template <>
struct Act<true> {
  static __device__ inline float ld(uint16_t h) { return f16_to_f32(h); }
  static __device__ inline float lo(uint32_t v) { return f16_to_f32(static_cast<uint16_t>(v)); }
  static __device__ inline float hi(uint32_t v) { return f16_to_f32(static_cast<uint16_t>(v >> 16)); }
  static __device__ inline uint16_t st(float f) { return f32_to_f16(f); }
  static __device__ inline float rnd(float f) { return round_f16(f); }
  static __device__ inline uint16_t from64(double d) { return f64_to_f16(d); }
  static __device__ inline float sigmoid(float v) { return sigmoid_f16(v); }
  static __device__ inline uint16_t swiglu(float g, float u) { return swiglu_f16(g, u); }
};

// Octet permutation of activation rows ("P8 layout"). Within each run of 8
// consecutive elements, element i is stored at slot p8_slot(i):
// 0,4,1,5,2,6,3,7 -> slots 0..7. A packed weight word's nibble pairs
// (q_i, q_{i+4}) then line up with consecutive bf16 pairs of the activation.
__host__ __device__ inline int p8_slot(int i) { return i < 4 ? 2 * i : 2 * (i - 4) + 1; }

__host__ __device__ inline int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace fmx

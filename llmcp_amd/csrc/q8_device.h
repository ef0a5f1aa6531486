// q8_device.h -- device-side scalar math shared by the gfx950 kernels:
// f16/bf16 conversions and the linear activations.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <utility>

namespace llmcp_q8 {

// Activation codes of include/llmcp_q8.h (llmcp_q8_activation).
enum DeviceActivation { ACT_NONE = 0, ACT_SILU = 1, ACT_SIGMOID = 2, ACT_SOFTPLUS = 3 };

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ __forceinline__ uint16_t float_to_half_bits(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);  // v_cvt_f16_f32: RNE
}

// bf16 -> f32 is exact (bf16ToFloat, Quantization.cpp:25-30).
__device__ __forceinline__ float bf16_to_float(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

// f32 -> bf16 round to nearest even (arith.truncf on a bf16 result type);
// NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t float_to_bf16(float v) {
  const uint32_t x = __builtin_bit_cast(uint32_t, v);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

// RN(1 / s) for s in [2^-125, 2^126]: v_rcp_f32 plus one Newton step with
// FMA is exact there (checked exhaustively on gfx950 by the device
// self-test).  Outside that range -- where 1/s is subnormal or overflows --
// only IEEE division is exact; recip_in_range reports which case holds.
__device__ __forceinline__ bool recip_in_range(float s) {
  return s >= 0x1p-125f && s <= 0x1p126f;
}
__device__ __forceinline__ float recip_fast(float s) {
  const float y = __builtin_amdgcn_rcpf(s);
  const float e = __builtin_fmaf(-s, y, 1.0f);
  return __builtin_fmaf(e, y, y);
}

// exp(x) in f64 for x in [-110, 100] (NaN passes through): k = rint(x/ln2),
// r = x - k*ln2 with ln2 in two parts (k*hi is exact, so r carries an error
// of one rounding), then Taylor terms to r^13 (truncation < 2^-57 for
// |r| <= ln2/2) by Horner with FMA, scaled by 2^k.  About 1 ulp.  Written
// out rather than calling the math library's exp(double): with the
// coefficients as FMA addends the compiler keeps them in SGPRs, where the
// library's form re-copied each one into VGPRs per evaluation.
__device__ __forceinline__ double exp_f64_reduced(double x) {
  const double k = __builtin_rint(x * 1.4426950408889634);
  double r = __builtin_fma(k, -0.6931471803691238, x);
  r = __builtin_fma(k, -1.9082149292705877e-10, r);
  double p = 1.6059043836821613e-10;
  p = __builtin_fma(p, r, 2.08767569878681e-09);
  p = __builtin_fma(p, r, 2.505210838544172e-08);
  p = __builtin_fma(p, r, 2.755731922398589e-07);
  p = __builtin_fma(p, r, 2.7557319223985893e-06);
  p = __builtin_fma(p, r, 2.48015873015873e-05);
  p = __builtin_fma(p, r, 0.0001984126984126984);
  p = __builtin_fma(p, r, 0.001388888888888889);
  p = __builtin_fma(p, r, 0.008333333333333333);
  p = __builtin_fma(p, r, 0.041666666666666664);
  p = __builtin_fma(p, r, 0.16666666666666666);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  return __builtin_ldexp(p, (int)k);
}

// The activations of applyMatmulActivation (MatmulLoweringCommon.cpp:78-103),
// each MLIR op rounded to f32 in turn.  math.exp and the log of softplus
// are evaluated in f64 and rounded once to f32 (the CPU oracle does the same
// with the host libm).  exp saturates outside [-110, 100], where the f32 result is 0 or
// inf either way.  The device self-test (llmcp_q8_selftest_exp) lists every
// float input whose exp lies near a rounding midpoint, the only inputs on
// which two exp(double) evaluations accurate to 2^-46 can round differently.
__device__ __forceinline__ float exp_f32(float v) {
  const float x = v > 100.0f ? 100.0f : (v < -110.0f ? -110.0f : v);
  return (float)exp_f64_reduced((double)x);
}
// 1 / (1 + e) with e >= 0: the denominator is in [1, 2^126] unless v < -87.3
// (or NaN), so recip_fast gives the IEEE quotient; a wave holding any other
// denominator divides in every lane (a uniform branch).
__device__ __forceinline__ float sigmoid_f32(float v) {
  const float d = 1.0f + exp_f32(-v);
  if (__builtin_amdgcn_ballot_w64(!(d <= 0x1p126f)) == 0) return recip_fast(d);
  return 1.0f / d;
}
__device__ __forceinline__ float silu_f32(float v) {
  return v * sigmoid_f32(v);
}
// softplus = math.log1p(math.exp(v)); the reference's --convert-math-to-llvm
// lowers log1p(y) to log(1 + y) with an f32 add (llmcp-compile.cpp:186), so
// the sum is rounded to f32 before the logarithm.  log is evaluated in f64
// and rounded once, like exp.
__device__ __forceinline__ float softplus_f32(float v) {
  const float s = 1.0f + exp_f32(v);
  return (float)log((double)s);
}
// activate() over an array in straight-line code (no per-element branch, so
// exp's constants stay in SGPRs across the elements), with one wave-uniform
// choice of the sigmoid's reciprocal for all of them.
template <int N>
__device__ __forceinline__ void activate_array(float (&v)[N], int act) {
  if (act == ACT_SILU || act == ACT_SIGMOID) {
    float d[N];
    bool slow = false;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      d[i] = 1.0f + exp_f32(-v[i]);
      slow |= !(d[i] <= 0x1p126f);
    }
    if (__builtin_amdgcn_ballot_w64(slow) == 0) {
#pragma unroll
      for (int i = 0; i < N; ++i) d[i] = recip_fast(d[i]);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i) d[i] = 1.0f / d[i];
    }
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = act == ACT_SILU ? v[i] * d[i] : d[i];
  } else if (act == ACT_SOFTPLUS) {
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = softplus_f32(v[i]);
  }
}
__device__ __forceinline__ float activate(float v, int act) {
  switch (act) {
    case ACT_SILU: return silu_f32(v);
    case ACT_SIGMOID: return sigmoid_f32(v);
    case ACT_SOFTPLUS: return softplus_f32(v);
    default: return v;
  }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0 .. N-1,
// so that every private-array index in the body is a constant.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace llmcp_q8

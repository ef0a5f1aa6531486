// q8_device.h -- device-side scalar math shared by the gfx950 kernels:
// f16/bf16 conversions and the linear activations.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

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

// The activations of applyMatmulActivation (MatmulLoweringCommon.cpp:78-103),
// each MLIR op rounded to f32 in turn.  math.exp / math.log1p are evaluated
// in f64 and rounded once (the CPU oracle does the same).
__device__ __forceinline__ float exp_f32(float v) {
  return (float)exp((double)v);
}
__device__ __forceinline__ float sigmoid_f32(float v) {
  const float e = exp_f32(-v);
  return 1.0f / (1.0f + e);
}
__device__ __forceinline__ float silu_f32(float v) {
  return v * sigmoid_f32(v);
}
__device__ __forceinline__ float softplus_f32(float v) {
  const float e = exp_f32(v);
  return (float)log1p((double)e);
}
__device__ __forceinline__ float activate(float v, int act) {
  switch (act) {
    case ACT_SILU: return silu_f32(v);
    case ACT_SIGMOID: return sigmoid_f32(v);
    case ACT_SOFTPLUS: return softplus_f32(v);
    default: return v;
  }
}

}  // namespace llmcp_q8

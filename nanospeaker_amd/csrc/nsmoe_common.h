// Shared device helpers for the nanoSpeaker MoE HIP kernels (gfx950 / CDNA4).
//
// Element types travel as raw 16- or 32-bit storage; conversions to and from fp32 are
// written out so rounding is round-to-nearest-even, the same as torch's CPU casts.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsmoe {

// Data-type codes shared with the C ABI (include/nsmoe.h).
enum DType : int { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };

// Gate activations, numbered as the reference's KERNEL_ACTIVATIONS
// (src/model/moe_kernel.py:75): silu/swish 0, gelu 1, relu 2, sigmoid 3, tanh 4.
enum Act : int { ACT_SILU = 0, ACT_GELU = 1, ACT_RELU = 2, ACT_SIGMOID = 3, ACT_TANH = 4 };

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

// ---- scalar conversions ------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f(uint16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

__device__ __forceinline__ uint16_t f_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float f16_to_f(uint16_t v) {
  _Float16 h;
  __builtin_memcpy(&h, &v, 2);
  return (float)h;
}

__device__ __forceinline__ uint16_t f_to_f16(float f) {
  _Float16 h = (_Float16)f;
  uint16_t v;
  __builtin_memcpy(&v, &h, 2);
  return v;
}

template <int DT> struct Elem;
template <> struct Elem<DT_BF16> {
  using T = uint16_t;
  __device__ static float to_f(T v) { return bf16_to_f(v); }
  __device__ static T from_f(float f) { return f_to_bf16(f); }
};
template <> struct Elem<DT_F16> {
  using T = uint16_t;
  __device__ static float to_f(T v) { return f16_to_f(v); }
  __device__ static T from_f(float f) { return f_to_f16(f); }
};
template <> struct Elem<DT_F32> {
  using T = float;
  __device__ static float to_f(T v) { return v; }
  __device__ static T from_f(float f) { return f; }
};

// ---- gate activations in fp32 (reference: src/model/moe_kernel.py:223-250) ----------

__device__ __forceinline__ float sigmoid_f(float g) { return 1.0f / (1.0f + expf(-g)); }

__device__ __forceinline__ float act_fwd(float g, int act) {
  switch (act) {
    case ACT_SILU: return g * sigmoid_f(g);
    case ACT_GELU: return 0.5f * g * (1.0f + erff(g * 0.7071067811865476f));
    case ACT_RELU: return g > 0.0f ? g : 0.0f;
    case ACT_SIGMOID: return sigmoid_f(g);
    default: return tanhf(g);
  }
}

// d act / d g, the closed forms of moe_kernel.py:237-250.
__device__ __forceinline__ float act_bwd(float g, int act) {
  switch (act) {
    case ACT_SILU: {
      float s = sigmoid_f(g);
      return s * (1.0f + g * (1.0f - s));
    }
    case ACT_GELU:
      return 0.5f * (1.0f + erff(g * 0.7071067811865476f)) +
             g * 0.3989422804014327f * expf(-0.5f * g * g);
    case ACT_RELU: return g > 0.0f ? 1.0f : 0.0f;
    case ACT_SIGMOID: {
      float s = sigmoid_f(g);
      return s * (1.0f - s);
    }
    default: {
      float t = tanhf(g);
      return 1.0f - t * t;
    }
  }
}

// ---- wave helpers ---------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace nsmoe

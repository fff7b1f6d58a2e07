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

// Inclusive prefix sum over the wave's 64 lanes: Hillis-Steele inside each 16-lane row
// (DPP row_shr 1, 2, 4, 8), then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then rows 0-1's total into rows 2 and 3 (row_bcast:31).  Lanes a DPP
// move does not write read 0 (the `old` operand).
__device__ __forceinline__ int wave_scan_incl(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return v;
}

// ---- compile-time activations for the expert epilogues ----------------------------------
//
// Same closed forms as act_fwd / act_bwd (moe_kernel.py:223-250), selected at compile time
// so an epilogue carries no per-element dispatch.  The logistic function uses the
// hardware exp2 and reciprocal (a few ulp in fp32), far inside the bf16 / fp16 output
// rounding and the fp32 kernels' 1e-5 tolerance; erf and its derivative keep the accurate
// library forms.
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

template <int ACT>
__device__ __forceinline__ float act_fwd_t(float g) {
  if constexpr (ACT == ACT_SILU) return g * fast_sigmoid(g);
  else if constexpr (ACT == ACT_GELU) return 0.5f * g * (1.0f + erff(g * 0.7071067811865476f));
  else if constexpr (ACT == ACT_RELU) return g > 0.0f ? g : 0.0f;
  else if constexpr (ACT == ACT_SIGMOID) return fast_sigmoid(g);
  else return 2.0f * fast_sigmoid(2.0f * g) - 1.0f;  // tanh g = 2 sigma(2g) - 1
}

// act(g) and act'(g) together (they share the logistic term).
template <int ACT>
__device__ __forceinline__ void act_both_t(float g, float& a, float& da) {
  if constexpr (ACT == ACT_SILU) {
    const float s = fast_sigmoid(g);
    a = g * s;
    da = s * (1.0f + g * (1.0f - s));
  } else if constexpr (ACT == ACT_GELU) {
    const float c = 0.5f * (1.0f + erff(g * 0.7071067811865476f));
    a = g * c;
    da = c + g * 0.3989422804014327f * __expf(-0.5f * g * g);
  } else if constexpr (ACT == ACT_RELU) {
    a = g > 0.0f ? g : 0.0f;
    da = g > 0.0f ? 1.0f : 0.0f;
  } else if constexpr (ACT == ACT_SIGMOID) {
    const float s = fast_sigmoid(g);
    a = s;
    da = s * (1.0f - s);
  } else {
    const float t = 2.0f * fast_sigmoid(2.0f * g) - 1.0f;
    a = t;
    da = 1.0f - t * t;
  }
}

// Calls f.template operator()<ACT>() with the run-time activation id as a constant.
template <class F>
__device__ __forceinline__ void with_act(int act, F&& f) {
  switch (act) {
    case ACT_SILU: f.template operator()<ACT_SILU>(); break;
    case ACT_GELU: f.template operator()<ACT_GELU>(); break;
    case ACT_RELU: f.template operator()<ACT_RELU>(); break;
    case ACT_SIGMOID: f.template operator()<ACT_SIGMOID>(); break;
    default: f.template operator()<ACT_TANH>(); break;
  }
}

// ---- packed conversions (hardware round-to-nearest-even) --------------------------------

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;

// Two fp32 values as two 16-bit elements of type DT in one dword (low half = lo).
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  uint32_t u;
  if constexpr (DT == DT_BF16) {
    const bf16x2_t b = __builtin_convertvector(f32x2{lo, hi}, bf16x2_t);
    __builtin_memcpy(&u, &b, 4);
  } else {
    const f16x2_t h = __builtin_convertvector(f32x2{lo, hi}, f16x2_t);
    __builtin_memcpy(&u, &h, 4);
  }
  return u;
}

// N fp32 values rounded to DT: bf16 two at a time through the packed hardware conversion
// (round-to-nearest-even, as f_to_bf16, on every value but NaN, which stays a NaN), the
// other types one at a time.
template <int DT, int N>
__device__ __forceinline__ void round_to(const float (&v)[N], typename Elem<DT>::T (&o)[N]) {
  if constexpr (DT == DT_BF16 && N % 2 == 0) {
#pragma unroll
    for (int q = 0; q < N / 2; ++q) {
      const uint32_t u = pack2<DT>(v[2 * q], v[2 * q + 1]);
      __builtin_memcpy(&o[2 * q], &u, 4);
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) o[e] = Elem<DT>::from_f(v[e]);
  }
}

// Element e (0 or 1) of a dword holding two 16-bit elements, as fp32.
template <int DT>
__device__ __forceinline__ float unpack2(uint32_t u, int e) {
  const uint16_t v = (uint16_t)(e ? (u >> 16) : (u & 0xffffu));
  if constexpr (DT == DT_BF16) return bf16_to_f(v);
  else return f16_to_f(v);
}

// ---- wave helpers ---------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace nsmoe

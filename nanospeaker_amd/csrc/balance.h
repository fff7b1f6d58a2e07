// Wave-level reductions and the last level of the balance loss, shared by the router
// (route.hip) and the dispatch (dispatch.hip, which can fold the loss into its launch).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nsmoe {

// ---- wave primitives -----------------------------------------------------------------

__device__ __forceinline__ int rl(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float rlf(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Butterfly inside each 16-lane row (xor 1, xor 2, half-row mirror, row mirror: every
// lane of a row ends with the same value, by commutativity), then the four rows in order.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = op(v, dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = op(v, dpp<0x141>(v));  // row_half_mirror
  v = op(v, dpp<0x140>(v));  // row_mirror
  return op(op(rlf(v, 0), rlf(v, 16)), op(rlf(v, 32), rlf(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
  return wave_reduce(v, [](float a, float b) { return a + b; });
}

__device__ __forceinline__ float wave_max(float v) {
  return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

// ---- balance loss, last level --------------------------------------------------------------
//
// aux = coef * E * sum_e f_e * P_e with f_e = counts_e / max(sum counts, 1) and
// P_e = (sum over the partial blocks of column e) / T (router.py:100-111).  1024 threads:
// thread (q, e) with q = tid / 128 sums partial blocks q, q + 8, q + 16, ... of expert e in
// that order; the 8 slices are then added in q order.  counts may be in global or LDS
// memory.
struct BalanceLds {
  float q[8][128];
  float part[2][2];
};

__device__ __forceinline__ void balance_loss_block(const float* __restrict__ partial, int64_t nblk,
                                                   const int32_t* counts, int64_t T, int E,
                                                   float coef, float* __restrict__ aux,
                                                   BalanceLds& L) {
  const int tid = threadIdx.x, e = tid & 127, q = tid >> 7;
  if (e < E) {
    // Slice q holds partials q, q + 8, q + 16, ... of expert e; they are fetched 32 at a
    // time (all loads in flight together) and added in that order.
    constexpr int DEPTH = 32;
    float acc = 0.0f;
    for (int64_t b0 = q; b0 < nblk; b0 += 8 * DEPTH) {
      float v[DEPTH];
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) {
        const int64_t b = b0 + 8 * u;
        v[u] = b < nblk ? partial[b * E + e] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < DEPTH; ++u) acc += v[u];
    }
    L.q[q][e] = acc;
  }
  __syncthreads();
  if (tid < 128) {
    const int lane = tid & 63, wave = tid >> 6;
    float col = 0.0f, c = 0.0f;
    if (e < E) {
#pragma unroll
      for (int qq = 0; qq < 8; ++qq) col += L.q[qq][e];
      c = (float)counts[e];
    }
    const float num = wave_sum(c * col), den = wave_sum(c);
    if (lane == 0) {
      L.part[wave][0] = num;
      L.part[wave][1] = den;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const float n = L.part[0][0] + L.part[1][0];
    const float dsum = fmaxf(L.part[0][1] + L.part[1][1], 1.0f);
    aux[0] = coef * (float)E * (n / dsum / (float)T);
  }
}

}  // namespace nsmoe

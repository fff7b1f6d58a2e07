// The block's RMSNorm + residual backward (norm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nsmoe {

constexpr int NORM_MAX_D = 1024;  // model width of the backward kernel (two chunks per lane)
constexpr int NORM_ROWS = 32;     // token rows per norm_bwd workgroup (one dw partial each)

struct NormBwdArgs {
  const void* x;       // [T, d] the residual stream (the block's input before the norm)
  const float* rstd;   // [T] the forward's rsqrt(mean(x^2) + eps)
  const void* w;       // [d] the norm's gain
  const void* dxn;     // [T, d] gradient of the normalised input (the block's dx)
  const void* g;       // [T, d] gradient of the sublayer's output (the residual's share)
  void* dx;            // [T, d] out: g + the norm's backward of dxn
  float* partial;      // [ceil(T / NORM_ROWS), d] workspace: column sums per workgroup
  void* dw;            // [d] out: the gain's gradient
  int64_t T;
  int d;
};

size_t norm_bwd_partial_bytes(int64_t T, int d);
int norm_bwd_launch(int dtype, const NormBwdArgs& a, hipStream_t s);

}  // namespace nsmoe

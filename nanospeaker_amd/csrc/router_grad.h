// The router GEMM's backward on the block path (router_grad.hip): arguments and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace nsmoe {

// dx[t] = sum of the token's expert dX rows + glogits[t] W^T  (combine_dx_kernel)
struct CombineDxArgs {
  const void* rows;      // [rows_total, d] expert dX rows (routed slots, then shared)
  const int32_t* inv;    // [T, k] slot of each pair, -1 when dropped
  const void* glogits;   // [T, ep] d(logits), zero in the pad columns
  const void* w;         // the router weight [d, E] packed as RouterWPack (nks = cdiv(ep, 32))
  void* dx;              // [T, d] output
  int64_t T, l_cap;
  int d, k, S, E, ep;
};

// W.grad = x^T glogits  (router_dw_kernel, then the reduce inside combine_dx's launch)
struct RouterDwArgs {
  const void* x;         // [T, d]
  const void* glogits;   // [T, ep]
  float* partial;        // [cdiv(T, RDW_RC), d, ep] fp32 scratch (router_dw_partial_bytes)
  void* dw;              // [d, E] output
  int64_t T;
  int d, E, ep;
};

// The fused path takes 16-bit types, d % 16 == 0 and E % 4 == 0, E <= 128.
bool router_grad_supported(int dtype, int d, int E);
// Row pitch of d(logits) on this path: E rounded up to 8 (16-byte rows).
int router_logits_pitch(int E);
size_t router_dw_partial_bytes(int64_t T, int d, int E);
// combine_dx; with rdw set the same launch also reduces router_dw_kernel's partials into
// rdw->dw (router_dw_launch must have run before it on the stream), and with dwr set
// (nbx > 0) the experts' dW split-K reduce (experts_bwd_launch's defer_reduce; the dW
// launch must have run before it on the stream).
struct DwReduceArgs;
int combine_dx_launch(int dtype, const CombineDxArgs& a, const RouterDwArgs* rdw,
                      hipStream_t stream, const DwReduceArgs* dwr = nullptr);
// The router dW's partials (router_dw_kernel) alone.
int router_dw_launch(int dtype, const RouterDwArgs& a, hipStream_t stream);

}  // namespace nsmoe

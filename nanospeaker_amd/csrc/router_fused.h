// The fused router (router.hip): x W_r, softmax, top-k, gates, per-chunk expert
// histograms and the balance loss's column sums, for 16-bit blocks.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pack_tile.h"

namespace nsmoe {

constexpr int RT_TOK = 32;              // tokens per router workgroup (= dispatch chunk / k)
constexpr int RT_MAXK = 16;             // largest top_k (one selected expert per row lane)
constexpr int RT_MAX_STEPS = 18;        // k-steps of 32 held in registers: d <= 576
constexpr int RT_MAX_E = 80;            // experts: up to 5 MFMA column blocks

struct RouterArgs {
  const void* x;         // [T, d] tokens
  const void* w;         // [d, E] router weight
  const float* bias;     // [E] offset added to the GEMM's fp32 output, or NULL
  int64_t T;
  int d, E, k, flags;    // flags: NSMOE_ROUTE_PROBS | NSMOE_ROUTE_NORMALIZE
  void* logits;          // [T, E] out: the rounded GEMM output (in the block's dtype)
  float* probs;          // [T, E] out, training branch
  void* topk_w;          // [T, k] out
  int64_t* topk_idx;     // [T, k] out
  // workspace (router_fused_args):
  int32_t* hist;         // [chunks, E] experts chosen by each workgroup's tokens
  float* colsum;         // [chunks, E] column sums of probs (training), or NULL
  // RMSNorm ahead of the router (norm_w non-NULL): x is the residual stream, and the
  // router runs on xn = x rsqrt(mean(x^2) + eps) norm_w (ln.py:30-36, F.rms_norm's fp32
  // arithmetic, one rounding to the dtype), which it writes to xn [T, d] with the
  // per-token rsqrt to rstd [T] (fp32).
  const void* norm_w;    // [d] in the block's dtype
  float norm_eps;
  void* xn;
  float* rstd;
  // With pack_on, the 16-bit expert-weight pack (PackPairArgs' wave items) runs in the
  // 16-wave form's last RT_PACK_WAVES waves of every workgroup (the ones the selection
  // leaves idle), beside the selection and the exact pass, instead of in a launch of its
  // own (router_fused_can_pack).
  PackPairArgs pack;
  int pack_on;
};
constexpr int RT_PACK_WAVES = 4;

inline int64_t router_fused_chunks(int64_t T) { return (T + RT_TOK - 1) / RT_TOK; }

// Whether the fused router takes this shape: bf16/fp16, d % 32 == 0, d <= 576,
// E % 4 == 0, E <= RT_MAX_E, top_k <= RT_MAXK.
bool router_fused_supported(int dtype, int d, int E, int k);
// Workspace of the fused router (histograms, column sums) and its carving.
size_t router_fused_ws_bytes(int64_t T, int E);
RouterArgs router_fused_args(void* ws, int64_t T, int E);
// The router's launch (router_fwd_kernel) on stream s.
int router_fused_launch(const RouterArgs& a, int dtype, hipStream_t s);
// Whether the router launch for T tokens can take a weight pack of `items` wave items
// (RouterArgs::pack_on): its 16-wave form, with few enough items per packing wave.
bool router_fused_can_pack(int64_t T, int64_t items);

}  // namespace nsmoe

// The MoE block's kernel path in one call per direction.
//
// Reference: MoEBlock.forward (src/model/moe.py:345-418) on its kernel branch -- the
// router tail (src/model/router.py:79-98), dispatch and experts (fused_moe_forward,
// src/model/moe_kernel.py:785-803), the shared experts (moe.py:310-329) and the balance
// loss (router.py:100-111) -- and its backward.  These entry points only sequence the
// per-stage ones (nsmoe_route_fwd, nsmoe_dispatch, nsmoe_pack_weights,
// nsmoe_experts_fwd, nsmoe_balance_loss and their backwards) over buffers carved from
// two caller allocations, so a framework pays one host call per direction instead of
// one per stage.
//
// `saved` holds what the forward produces and the backward reads again (routing, the
// dispatch buffers, the packed weights); its layout is reported by
// nsmoe_block_saved_layout.  `workspace` is scratch for one call.
#include <string.h>

#include "experts_common.h"
#include "pack.h"
#include "../../include/nsmoe.h"

namespace nsmoe {

static size_t al256(size_t b) { return (b + 255) & ~(size_t)255; }

struct BlockLayout {
  size_t off[NSMOE_BLOCK_NSAVED];
  size_t total;
};

static BlockLayout block_layout(const nsmoe_experts_args* a, int32_t flags) {
  const size_t T = (size_t)a->n_tokens, E = (size_t)a->n_experts, k = (size_t)a->top_k;
  const size_t es = a->dtype == DT_F32 ? 4 : 2;
  const int64_t m = (int64_t)(T * k);
  const size_t l_cap = (size_t)nsmoe_dispatch_l_cap(m, (int32_t)E);
  const PackGeom pg = pack_geom(a->dtype, a->d_model, a->d_hidden, a->n_experts, a->n_shared);
  const size_t sizes[NSMOE_BLOCK_NSAVED] = {
      T * k * es,                                   // topk_w
      T * k * 8,                                    // topk_idx
      (flags & NSMOE_ROUTE_PROBS) ? T * E * 4 : 0,  // probs
      l_cap * 4,                                    // sorted_ids
      (l_cap / (size_t)nsmoe_align_m()) * 4,        // expert_ids
      (E + 1) * 4,                                  // pad_offsets
      E * 4,                                        // counts
      4,                                            // n_post_pad
      T * k * 4,                                    // inv
      pg.in_bytes,                                  // packed W_in
      pg.out_bytes,                                 // packed W_out
  };
  BlockLayout L;
  size_t o = 0;
  for (int i = 0; i < NSMOE_BLOCK_NSAVED; ++i) {
    L.off[i] = o;
    o += al256(sizes[i]);
  }
  L.total = o;
  return L;
}

// Points a copy of the caller's args at the routing state inside `saved`.
static nsmoe_experts_args with_routing(const nsmoe_experts_args* a, const BlockLayout& L,
                                       char* saved) {
  nsmoe_experts_args b = *a;
  b.l_cap = nsmoe_dispatch_l_cap(a->n_tokens * a->top_k, a->n_experts);
  b.topk_w = saved + L.off[NSMOE_SAVED_TOPK_W];
  b.sorted_ids = (const int32_t*)(saved + L.off[NSMOE_SAVED_SORTED_IDS]);
  b.pad_offsets = (const int32_t*)(saved + L.off[NSMOE_SAVED_PAD_OFFSETS]);
  b.counts = (const int32_t*)(saved + L.off[NSMOE_SAVED_COUNTS]);
  b.w_in_packed = saved + L.off[NSMOE_SAVED_W_IN_PACKED];
  b.w_out_packed = saved + L.off[NSMOE_SAVED_W_OUT_PACKED];
  return b;
}

static size_t fwd_ws_parts(const nsmoe_experts_args* b, size_t* dsp, size_t* exp, size_t* bal) {
  const int64_t m = b->n_tokens * b->top_k;
  *dsp = al256(nsmoe_dispatch_workspace_size(m, b->n_experts));
  *exp = al256(nsmoe_experts_fwd_workspace_size(b));
  *bal = al256(nsmoe_balance_loss_workspace_size(b->n_tokens, b->n_experts));
  return *dsp + *exp + *bal;
}

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_block_saved_layout(const nsmoe_experts_args* a, int32_t route_flags,
                                        size_t* offsets, size_t* total_bytes) {
  NSMOE_REQUIRE(a && offsets && total_bytes, "block_saved_layout: NULL pointer");
  NSMOE_REQUIRE(a->n_tokens >= 0 && a->n_experts >= 1 && a->top_k >= 1,
                "block_saved_layout: bad dimensions");
  const BlockLayout L = block_layout(a, route_flags);
  memcpy(offsets, L.off, sizeof(L.off));
  *total_bytes = L.total;
  return NSMOE_OK;
}

extern "C" size_t nsmoe_block_fwd_workspace_size(const nsmoe_experts_args* a,
                                                 int32_t route_flags) {
  if (!a) return 0;
  nsmoe_experts_args b = *a;
  b.l_cap = nsmoe_dispatch_l_cap(a->n_tokens * a->top_k, a->n_experts);
  (void)route_flags;
  size_t dsp, exp, bal;
  return fwd_ws_parts(&b, &dsp, &exp, &bal);
}

extern "C" int nsmoe_block_fwd(const nsmoe_experts_args* a, const void* logits,
                               int32_t route_flags, float aux_coef, void* saved, void* out,
                               float* aux, void* workspace, size_t workspace_bytes,
                               void* stream) {
  NSMOE_REQUIRE(a && saved && out, "block_fwd: NULL pointer");
  NSMOE_REQUIRE(!(route_flags & NSMOE_ROUTE_PROBS) || aux, "block_fwd: NULL aux");
  if (a->n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(logits, "block_fwd: NULL logits");
  const BlockLayout L = block_layout(a, route_flags);
  char* sv = (char*)saved;
  nsmoe_experts_args b = with_routing(a, L, sv);
  size_t dsp, exp, bal;
  const size_t need = fwd_ws_parts(&b, &dsp, &exp, &bal);
  if (!workspace || workspace_bytes < need) {
    set_error("block_fwd: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  char* ws = (char*)workspace;
  const int32_t E = a->n_experts, k = a->top_k;
  const int64_t T = a->n_tokens, m = T * k;
  float* probs = (route_flags & NSMOE_ROUTE_PROBS) ? (float*)(sv + L.off[NSMOE_SAVED_PROBS])
                                                   : nullptr;
  int64_t* topk_idx = (int64_t*)(sv + L.off[NSMOE_SAVED_TOPK_IDX]);
  int32_t* inv = (int32_t*)(sv + L.off[NSMOE_SAVED_INV]);
  NSMOE_TRY(nsmoe_route_fwd(logits, T, E, k, route_flags, a->dtype, (void*)b.topk_w, topk_idx,
                            probs, stream));
  NSMOE_TRY(nsmoe_dispatch(topk_idx, m, E, (int32_t*)b.sorted_ids,
                           (int32_t*)(sv + L.off[NSMOE_SAVED_EXPERT_IDS]),
                           (int32_t*)b.pad_offsets, (int32_t*)b.counts,
                           (int32_t*)(sv + L.off[NSMOE_SAVED_N_POST_PAD]), inv, ws, dsp, stream));
  NSMOE_TRY(nsmoe_pack_weights(&b, (void*)b.w_in_packed, (void*)b.w_out_packed, stream));
  NSMOE_TRY(nsmoe_experts_fwd(&b, inv, out, ws + dsp, exp, stream));
  if (route_flags & NSMOE_ROUTE_PROBS)
    NSMOE_TRY(nsmoe_balance_loss(probs, b.counts, T, E, aux_coef, aux, ws + dsp + exp, bal,
                                 stream));
  return NSMOE_OK;
}

extern "C" size_t nsmoe_block_bwd_workspace_size(const nsmoe_experts_args* a,
                                                 int32_t route_flags) {
  if (!a) return 0;
  nsmoe_experts_args b = *a;
  b.l_cap = nsmoe_dispatch_l_cap(a->n_tokens * a->top_k, a->n_experts);
  (void)route_flags;
  const size_t es = a->dtype == DT_F32 ? 4 : 2;
  return al256((size_t)a->n_tokens * a->top_k * es) + nsmoe_experts_bwd_workspace_size(&b);
}

extern "C" int nsmoe_block_bwd(const nsmoe_experts_args* a, const void* logits,
                               int32_t route_flags, float aux_coef, const void* saved,
                               const void* grad_out, const float* grad_aux,
                               const nsmoe_experts_grads* grads, void* grad_logits,
                               void* workspace, size_t workspace_bytes, void* stream) {
  NSMOE_REQUIRE(a && saved && grad_out && grads && grad_logits, "block_bwd: NULL pointer");
  if (a->n_tokens == 0) return NSMOE_OK;
  const BlockLayout L = block_layout(a, route_flags);
  char* sv = (char*)saved;
  nsmoe_experts_args b = with_routing(a, L, sv);
  const size_t es = a->dtype == DT_F32 ? 4 : 2;
  const size_t tw_bytes = al256((size_t)a->n_tokens * a->top_k * es);
  const size_t need = tw_bytes + nsmoe_experts_bwd_workspace_size(&b);
  if (!workspace || workspace_bytes < need) {
    set_error("block_bwd: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  char* ws = (char*)workspace;
  nsmoe_experts_grads g = *grads;
  g.dtopk_w = ws;  // the gate gradient stays internal: it feeds the router backward
  NSMOE_TRY(nsmoe_experts_bwd(&b, (const int32_t*)(sv + L.off[NSMOE_SAVED_INV]), grad_out, &g,
                              ws + tw_bytes, workspace_bytes - tw_bytes, stream));
  const bool probs = route_flags & NSMOE_ROUTE_PROBS;
  const void* src = probs ? (const void*)(sv + L.off[NSMOE_SAVED_PROBS]) : logits;
  NSMOE_REQUIRE(src, "block_bwd: NULL logits (eval branch)");
  return nsmoe_route_bwd(src, (const int64_t*)(sv + L.off[NSMOE_SAVED_TOPK_IDX]), ws, a->dtype,
                         nullptr, probs ? grad_aux : nullptr, probs && grad_aux ? b.counts : nullptr,
                         aux_coef, a->n_tokens, a->n_experts, a->top_k, route_flags, grad_logits,
                         stream);
}

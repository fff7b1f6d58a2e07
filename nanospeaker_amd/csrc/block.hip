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
// `saved` holds what the forward produces and the backward reads again (gates, probs and
// the dispatch buffers); its layout is reported by nsmoe_block_saved_layout.  The expert
// ids and routing counts are separate caller buffers, because callers keep them past the
// step, and the packed weights are the caller's too, so a caller can keep them across
// calls while the weights do not change.  `workspace` is scratch for one call.
#include <string.h>

#include "dw_reduce.h"
#include "experts_common.h"
#include "norm.h"
#include "pack.h"
#include "pack_tile.h"
#include "router_fused.h"
#include "router_grad.h"
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
  nsmoe_experts_args b = *a;
  b.l_cap = (int64_t)l_cap;
  const size_t act = (flags & NSMOE_BLOCK_SAVE_ACT) ? experts_save_act_bytes(&b) : 0;
  const bool norm = flags & NSMOE_BLOCK_NORM;
  const size_t d = (size_t)a->d_model;
  const size_t sizes[NSMOE_BLOCK_NSAVED] = {
      T * k * es,                                   // topk_w
      (flags & NSMOE_ROUTE_PROBS) ? T * E * 4 : 0,  // probs
      l_cap * 4,                                    // sorted_ids
      (l_cap / (size_t)nsmoe_align_m()) * 4,        // expert_ids
      (E + 1) * 4,                                  // pad_offsets
      4,                                            // n_post_pad
      T * k * 4,                                    // inv
      act,                                          // pre-activations (SAVE_ACT)
      norm ? T * d * es : 0,                        // normalised input (NORM)
      norm ? T * 4 : 0,                             // rstd (NORM)
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

// The saved pre-activations, or NULL when the layout has none.
static char* act_part(const BlockLayout& L, char* saved, int32_t flags) {
  const bool has = (flags & NSMOE_BLOCK_SAVE_ACT) && L.off[NSMOE_SAVED_ACT] < L.total;
  return has ? saved + L.off[NSMOE_SAVED_ACT] : nullptr;
}

// Points a copy of the caller's args at the routing state inside `saved` and at the
// routing counts.
static nsmoe_experts_args with_routing(const nsmoe_experts_args* a, const BlockLayout& L,
                                       char* saved, const int32_t* counts) {
  nsmoe_experts_args b = *a;
  b.l_cap = nsmoe_dispatch_l_cap(a->n_tokens * a->top_k, a->n_experts);
  b.topk_w = saved + L.off[NSMOE_SAVED_TOPK_W];
  b.sorted_ids = (const int32_t*)(saved + L.off[NSMOE_SAVED_SORTED_IDS]);
  b.pad_offsets = (const int32_t*)(saved + L.off[NSMOE_SAVED_PAD_OFFSETS]);
  b.counts = counts;
  return b;
}

// Forward workspace: the dispatch's histograms (unfused router), the router's partials
// (the balance loss's column sums, or the fused router's histograms, tie lists and column
// sums) and the experts' per-row outputs.
static size_t fwd_ws_parts(const nsmoe_experts_args* b, size_t* dsp, size_t* exp, size_t* rt) {
  const int64_t m = b->n_tokens * b->top_k;
  *dsp = al256(nsmoe_dispatch_workspace_size(m, b->n_experts));
  *exp = al256(nsmoe_experts_fwd_workspace_size(b));
  const size_t bal = al256(nsmoe_balance_loss_workspace_size(b->n_tokens, b->n_experts));
  const size_t fused = al256(router_fused_ws_bytes(b->n_tokens, b->n_experts));
  *rt = bal > fused ? bal : fused;
  return *dsp + *exp + *rt;
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
  size_t dsp, exp, rt;
  return fwd_ws_parts(&b, &dsp, &exp, &rt);
}

extern "C" int nsmoe_block_fwd(const nsmoe_experts_args* a, const nsmoe_block_norm* norm,
                               const void* w_router,
                               const float* logit_bias, void* logits, int32_t route_flags,
                               float aux_coef, void* saved, int64_t* topk_idx, int32_t* counts,
                               void* out, float* aux, void* workspace, size_t workspace_bytes,
                               void* stream) {
  NSMOE_REQUIRE(a && saved && out && topk_idx && counts && logits, "block_fwd: NULL pointer");
  NSMOE_REQUIRE(!(route_flags & NSMOE_ROUTE_PROBS) || aux, "block_fwd: NULL aux");
  NSMOE_REQUIRE(a->w_in_packed && a->w_out_packed, "block_fwd: NULL packed weights");
  NSMOE_REQUIRE(w_router || !logit_bias, "block_fwd: logit_bias needs the fused router");
  NSMOE_REQUIRE(!norm == !(route_flags & NSMOE_BLOCK_NORM),
                "block_fwd: pass the norm together with NSMOE_BLOCK_NORM");
  NSMOE_REQUIRE(!norm || (norm->weight && w_router), "block_fwd: the norm needs its weight "
                "and the fused router (w_router)");
  NSMOE_REQUIRE(!w_router || router_fused_supported(a->dtype, (int)a->d_model, a->n_experts,
                                                    a->top_k),
                "block_fwd: the fused router takes bf16/fp16, d %% 32 == 0, d <= 576, "
                "E %% 4 == 0, E <= 80 and top_k <= 16 (d %d, E %d, k %d)", (int)a->d_model,
                a->n_experts,
                a->top_k);
  if (a->n_tokens == 0) return NSMOE_OK;
  const BlockLayout L = block_layout(a, route_flags);
  char* sv = (char*)saved;
  nsmoe_experts_args b = with_routing(a, L, sv, counts);
  // With the norm, everything past the router reads the normalised rows it stores.
  if (norm) b.x = sv + L.off[NSMOE_SAVED_XN];
  size_t dsp, exp, rtb;
  const size_t need = fwd_ws_parts(&b, &dsp, &exp, &rtb);
  if (!workspace || workspace_bytes < need) {
    set_error("block_fwd: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  char* ws = (char*)workspace;
  char* ws_rt = ws + dsp + exp;
  const int32_t E = a->n_experts, k = a->top_k;
  const int64_t T = a->n_tokens, m = T * k;
  float* probs = (route_flags & NSMOE_ROUTE_PROBS) ? (float*)(sv + L.off[NSMOE_SAVED_PROBS])
                                                   : nullptr;
  int32_t* inv = (int32_t*)(sv + L.off[NSMOE_SAVED_INV]);
  int32_t* eids = (int32_t*)(sv + L.off[NSMOE_SAVED_EXPERT_IDS]);
  int32_t* npp = (int32_t*)(sv + L.off[NSMOE_SAVED_N_POST_PAD]);
  // The weight packing (when asked for) does not depend on the routing: it runs on the
  // side stream while the latency-bound routing and dispatch kernels run on the caller's.
  hipStream_t s = (hipStream_t)stream;
  const bool pack = route_flags & NSMOE_BLOCK_PACK;
  // On the fused-router path the 16-bit packs run inside the dispatch's place launch, in
  // workgroups of their own beside the placing ones (dispatch_place_launch), unless the
  // side stream is asked for.
  PackPairArgs pk{};
  const bool pack_in_place =
      pack && w_router && !option(OPT_SIDE_STREAM) &&
      pack_pair_args(a->dtype, b.w_in, b.w_out, b.w_sh_in, b.w_sh_out, (int)b.n_experts,
                     (int)b.n_shared, (int)b.d_model, (int)b.d_hidden, (void*)b.w_in_packed,
                     (void*)b.w_out_packed, &pk);
  hipStream_t s_pack = pack && !pack_in_place ? side_fork(s, kSideSlotPack) : s;
  int rc = pack && !pack_in_place
               ? nsmoe_pack_weights(&b, (void*)b.w_in_packed, (void*)b.w_out_packed, s_pack)
               : NSMOE_OK;
  if (pack_in_place) {  // nsmoe_pack_weights' own checks
    NSMOE_REQUIRE(b.w_in && b.w_out, "block_fwd: NULL expert weights");
    NSMOE_REQUIRE(b.n_shared == 0 || (b.w_sh_in && b.w_sh_out),
                  "block_fwd: shared weights missing");
  }
  if (w_router) {
    // Router GEMM + tail + the dispatch's histograms in the router's two launches; the
    // dispatch is then its place pass alone, with the balance loss in one more workgroup.
    RouterArgs r = router_fused_args(ws_rt, T, E);
    r.x = a->x;
    r.w = w_router;
    r.bias = logit_bias;
    r.T = T;
    r.d = (int)a->d_model;
    r.E = E;
    r.k = k;
    r.flags = route_flags & (NSMOE_ROUTE_PROBS | NSMOE_ROUTE_NORMALIZE);
    r.logits = logits;
    r.probs = probs;
    r.topk_w = (void*)b.topk_w;
    r.topk_idx = topk_idx;
    if (!probs) r.colsum = nullptr;
    // The pack rides in the router's launch where that launch can take it, else in the
    // place launch.
    const bool pack_in_router =
        pack_in_place && router_fused_can_pack(T, pk.items_in + pk.items_out);
    if (pack_in_router) {
      r.pack = pk;
      r.pack_on = 1;
    }
    if (norm) {
      r.norm_w = norm->weight;
      r.norm_eps = norm->eps;
      r.xn = sv + L.off[NSMOE_SAVED_XN];
      r.rstd = (float*)(sv + L.off[NSMOE_SAVED_RSTD]);
    }
    if (rc == NSMOE_OK) rc = router_fused_launch(r, a->dtype, s);
    BalanceArgs fold{r.colsum, router_fused_chunks(T), T, aux_coef, aux};
    if (rc == NSMOE_OK)
      rc = dispatch_place_launch(topk_idx, m, E, r.hist, router_fused_chunks(T), RT_TOK * k,
                                 (int32_t*)b.sorted_ids, eids, (int32_t*)b.pad_offsets, counts,
                                 npp, inv, probs ? &fold : nullptr, s,
                                 pack_in_place && !pack_in_router ? &pk : nullptr, a->dtype,
                                 probs ? nullptr : aux);
  } else {
    // In training the route kernel also leaves the balance loss's per-workgroup column
    // sums of probs in the workspace, so probs is not read back for the loss.
    float* colsum = probs ? (float*)ws_rt : nullptr;
    if (rc == NSMOE_OK)
      rc = route_fwd_launch(logits, T, E, k, route_flags, a->dtype, (void*)b.topk_w,
                            topk_idx, probs, colsum, s);
    // In training the balance loss is one more workgroup of the dispatch's second launch.
    BalanceArgs fold{colsum, balance_partial_count(T), T, aux_coef, aux};
    if (rc == NSMOE_OK)
      rc = dispatch_launch(topk_idx, m, E, (int32_t*)b.sorted_ids, eids,
                           (int32_t*)b.pad_offsets, counts, npp, inv, ws, dsp,
                           probs ? &fold : nullptr, s, probs ? nullptr : aux);
  }
  const int jrc = side_join(s, s_pack, kSideSlotPack);  // joined on every path
  NSMOE_TRY(rc);
  NSMOE_TRY(jrc);
  return experts_fwd_launch(&b, inv, out, ws + dsp, exp, act_part(L, sv, route_flags), s,
                            norm ? a->x : nullptr);
}

namespace nsmoe {

// Backward workspace: the gate gradient (T x k), the expert backward's workspace, and on
// the fused router path d(logits) at pitch ep plus the router dW partials.
struct BwdWs {
  size_t tw, exp, gl, part, wpk, dxn, npart, total;
};

static BwdWs bwd_ws(const nsmoe_experts_args* b, bool router, bool norm) {
  const size_t es = b->dtype == DT_F32 ? 4 : 2;
  BwdWs w;
  w.tw = 0;
  w.exp = al256((size_t)b->n_tokens * b->top_k * es);
  w.gl = w.exp + al256(nsmoe_experts_bwd_workspace_size(b));
  w.part = w.gl;
  w.wpk = w.gl;
  w.total = w.gl;
  if (router) {
    const int ep = router_logits_pitch(b->n_experts);
    w.part = w.gl + al256((size_t)b->n_tokens * ep * es);
    w.wpk = w.part + al256(router_dw_partial_bytes(b->n_tokens, b->d_model, b->n_experts));
    w.total = w.wpk + al256(router_w_pack_bytes((int)b->d_model, (ep + 31) / 32));
  }
  // With the norm: the block's input gradient before the norm's backward, and the gain's
  // per-workgroup column sums.
  w.dxn = w.npart = w.total;
  if (norm) {
    w.npart = w.dxn + al256((size_t)b->n_tokens * b->d_model * es);
    w.total = w.npart + al256(norm_bwd_partial_bytes(b->n_tokens, (int)b->d_model));
  }
  return w;
}

}  // namespace nsmoe

namespace nsmoe {
int block_bwd_router(const nsmoe_experts_args* a, const nsmoe_experts_args& b,
                     const BlockLayout& L, char* sv, const int64_t* topk_idx,
                     const void* logits, int32_t route_flags, float aux_coef,
                     const float* grad_aux, const nsmoe_experts_grads* grads,
                     const void* w_router, void* grad_w_router, void* grad_logits, char* ws,
                     const BwdWs& W, const int32_t* inv, bool fuse, void* dx, hipStream_t s,
                     const DwReduceArgs* dwr);
}  // namespace nsmoe

extern "C" size_t nsmoe_block_bwd_workspace_size(const nsmoe_experts_args* a,
                                                 int32_t route_flags, int32_t fuse_router) {
  if (!a) return 0;
  nsmoe_experts_args b = *a;
  b.l_cap = nsmoe_dispatch_l_cap(a->n_tokens * a->top_k, a->n_experts);
  return bwd_ws(&b, fuse_router != 0, route_flags & NSMOE_BLOCK_NORM).total;
}

extern "C" int nsmoe_block_bwd(const nsmoe_experts_args* a, const nsmoe_block_norm* norm,
                               const void* logits,
                               int32_t route_flags, float aux_coef, const void* saved,
                               const int64_t* topk_idx, const int32_t* counts,
                               const void* grad_out, const float* grad_aux,
                               const nsmoe_experts_grads* grads, const void* w_router,
                               void* grad_w_router, void* grad_logits, void* workspace,
                               size_t workspace_bytes, void* stream) {
  NSMOE_REQUIRE(a && saved && topk_idx && counts && grad_out && grads,
                "block_bwd: NULL pointer");
  NSMOE_REQUIRE(a->w_in_packed, "block_bwd: NULL packed W_in");
  const bool fuse = w_router != nullptr;
  NSMOE_REQUIRE(fuse ? grad_w_router != nullptr : grad_logits != nullptr,
                "block_bwd: NULL %s", fuse ? "grad_w_router" : "grad_logits");
  NSMOE_REQUIRE(!fuse || router_grad_supported(a->dtype, (int)a->d_model, a->n_experts),
                "block_bwd: the fused router backward takes bf16/fp16, d %% 16 == 0, "
                "E %% 4 == 0 and E <= 128 (d %d, E %d)", (int)a->d_model, a->n_experts);
  NSMOE_REQUIRE(!norm == !(route_flags & NSMOE_BLOCK_NORM),
                "block_bwd: pass the norm together with NSMOE_BLOCK_NORM");
  NSMOE_REQUIRE(!norm || (norm->weight && norm->grad_weight && fuse),
                "block_bwd: the norm needs its weight, grad_weight and the fused router");
  if (a->n_tokens == 0) return NSMOE_OK;
  const BlockLayout L = block_layout(a, route_flags);
  char* sv = (char*)saved;
  nsmoe_experts_args b = with_routing(a, L, sv, counts);
  if (norm) b.x = sv + L.off[NSMOE_SAVED_XN];
  const BwdWs W = bwd_ws(&b, fuse, norm != nullptr);
  if (!workspace || workspace_bytes < W.total) {
    set_error("block_bwd: workspace %zu B < %zu B", workspace_bytes, W.total);
    return NSMOE_EWORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const int32_t* inv = (const int32_t*)(sv + L.off[NSMOE_SAVED_INV]);
  nsmoe_experts_grads g = *grads;
  g.dtopk_w = ws + W.tw;  // the gate gradient stays internal: it feeds the router backward
  // dW runs on the side stream beside everything below; joined before returning.
  hipStream_t s_dw = s;
  // On the fused-router path the experts' dW split-K reduce rides in combine_dx's launch.
  DwReduceArgs dwr{};
  NSMOE_TRY(experts_bwd_launch(&b, inv, grad_out, &g, ws + W.exp, W.gl - W.exp, !fuse, s, &s_dw,
                               act_part(L, sv, route_flags), fuse ? &dwr : nullptr));
  // With the norm the combine's dx is the normalised input's gradient: it goes to the
  // workspace, and the norm's backward turns it into grads->dx.
  void* dxn = norm ? (void*)(ws + W.dxn) : grads->dx;
  int rc = block_bwd_router(a, b, L, sv, topk_idx, logits, route_flags, aux_coef, grad_aux,
                            grads, w_router, grad_w_router, grad_logits, ws, W, inv, fuse, dxn,
                            s, &dwr);
  if (rc == NSMOE_OK && norm) {
    NormBwdArgs n;
    n.x = a->x;
    n.rstd = (const float*)(sv + L.off[NSMOE_SAVED_RSTD]);
    n.w = norm->weight;
    n.dxn = dxn;
    n.g = grad_out;
    n.dx = grads->dx;
    n.partial = (float*)(ws + W.npart);
    n.dw = norm->grad_weight;
    n.T = a->n_tokens;
    n.d = (int)a->d_model;
    rc = norm_bwd_launch(a->dtype, n, s);
  }
  const int jrc = side_join(s, s_dw, kSideSlotDw);
  NSMOE_TRY(rc);
  return jrc;
}

namespace nsmoe {

// The router's part of the block backward, after the experts' (block.hip's
// nsmoe_block_bwd): d(logits) from the gate gradient, then dx and W_router's gradient.
int block_bwd_router(const nsmoe_experts_args* a, const nsmoe_experts_args& b,
                     const BlockLayout& L, char* sv, const int64_t* topk_idx,
                     const void* logits, int32_t route_flags, float aux_coef,
                     const float* grad_aux, const nsmoe_experts_grads* grads,
                     const void* w_router, void* grad_w_router, void* grad_logits, char* ws,
                     const BwdWs& W, const int32_t* inv, bool fuse, void* dx, hipStream_t s,
                     const DwReduceArgs* dwr) {
  const bool probs = route_flags & NSMOE_ROUTE_PROBS;
  const void* src = probs ? (const void*)(sv + L.off[NSMOE_SAVED_PROBS]) : logits;
  NSMOE_REQUIRE(src, "block_bwd: NULL logits (eval branch)");
  const int E = a->n_experts;
  const int ldg = fuse ? router_logits_pitch(E) : E;
  void* gl = fuse ? (void*)(ws + W.gl) : grad_logits;
  // With the router GEMM fused, the same launch packs W for combine_dx's router term.
  const RouterWPack pack{w_router, ws + W.wpk, (int)a->d_model, E, (ldg + 31) / 32};
  NSMOE_TRY(route_bwd_launch(src, topk_idx,
                             ws + W.tw, a->dtype, nullptr, probs ? grad_aux : nullptr,
                             probs && grad_aux ? b.counts : nullptr, aux_coef, a->n_tokens, E,
                             a->top_k, route_flags, gl, ldg, s, fuse ? &pack : nullptr));
  if (!fuse) return NSMOE_OK;
  CombineDxArgs c;
  c.rows = ws + W.exp + experts_bwd_dxrows_offset(&b);
  c.inv = inv;
  c.glogits = gl;
  c.w = ws + W.wpk;
  c.dx = dx;
  c.T = a->n_tokens;
  c.l_cap = b.l_cap;
  c.d = (int)a->d_model;
  c.k = a->top_k;
  c.S = a->n_shared;
  c.E = E;
  c.ep = ldg;
  // The router dW's partials first; their reduce rides in the combine_dx launch.
  RouterDwArgs r;
  r.x = b.x;
  r.glogits = gl;
  r.partial = (float*)(ws + W.part);
  r.dw = grad_w_router;
  r.T = a->n_tokens;
  r.d = (int)a->d_model;
  r.E = E;
  r.ep = ldg;
  NSMOE_TRY(router_dw_launch(a->dtype, r, s));
  return combine_dx_launch(a->dtype, c, &r, s, dwr);
}

}  // namespace nsmoe

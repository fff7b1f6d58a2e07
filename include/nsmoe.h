/*
 * nsmoe.h -- C ABI of libnsmoe.so, the MI355X (gfx950) HIP implementation of
 * nanoSpeaker's dropless MoE hot path: router tail, dispatch, grouped SwiGLU experts
 * (routed + shared), combine and the full backward.
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated; tensors are dense row-major.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).  Calls only
 *     enqueue work: no host synchronisation, no device allocation.  Scratch memory is a
 *     caller-provided `workspace` sized by the matching *_workspace_size query.
 *   - Return value: 0 on success, non-zero on error; nsmoe_last_error() then holds a
 *     message (thread-local).  1 = invalid argument, 2 = HIP launch error,
 *     3 = workspace too small.
 *   - dtype codes: 0 = bf16, 1 = fp16, 2 = fp32 (NSMOE_BF16 / NSMOE_F16 / NSMOE_F32).
 *   - activation codes match the reference's KERNEL_ACTIVATIONS
 *     (src/model/moe_kernel.py:75): 0 silu/swish, 1 gelu (erf), 2 relu, 3 sigmoid,
 *     4 tanh.
 *
 * Each entry point names the reference interface it replaces.
 */
#ifndef NSMOE_H_
#define NSMOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NSMOE_BF16 0
#define NSMOE_F16 1
#define NSMOE_F32 2

/* ---- library housekeeping ---------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). */
const char* nsmoe_last_error(void);

/* Number of kernels this process has launched through the library (monotonic). */
uint64_t nsmoe_launch_count(void);

/* ABI version of this header. */
int32_t nsmoe_abi_version(void);

/* Measurement hooks (no counterpart in the reference; used by bench.py).  When enabled,
 * the library records a HIP event pair on the launch stream around each launch of its
 * main kernels ("pack", "route_fwd", "dispatch", "expert_fwd", "combine",
 * "expert_bwd", "expert_dx", "dw" (or "dw_in" and "dw_out" where they run apart),
 * "combine_dx", "router_dw", "route_bwd", "norm_bwd", "attn_k_prep", "attn_fwd", "ce_rows", "norm_fwd") until
 * `capacity` pairs are used.
 * nsmoe_timing_read waits for the recorded events of one kernel and returns their
 * summed duration.  capacity 0 disables timing and frees the events. */
int nsmoe_timing_enable(int32_t capacity);
int nsmoe_timing_read(const char* kernel_name, double* total_ms, int64_t* launches);

/* Tuning options (no counterpart in the reference; for tests and measurements).  Each is
 * process-wide, starts at 0 (= the library's own choice) and applies to calls made after
 * it is set.  Names and accepted values:
 *   "side_stream"    1: run the weight packing and the dW stage of an eager block call on
 *                    a second stream, forked and joined with events (default: every
 *                    kernel on the caller's stream, which costs less host time)
 *   "fwd_rows"       rows per tile of the 16-bit forward expert kernel: 32, 64 or 96
 *   "fwd_dist"       its weight prefetch distance in k-steps: 2, 3 or 6 (6 with 32-row
 *                    tiles only); a distance that does not divide both GEMMs' k-steps is
 *                    not taken
 *   "bwd_rows"       rows per tile of the GLU-backward kernel: 48, 64, 80 or 96 (96
 *                    only when the forward saved the pre-activations)
 *   "bwd_dist"       its prefetch distance: 2, 3 or 4 (4 only with the pre-activations
 *                    saved); a distance that does not divide the k-steps is not taken
 *   "dx_rows"        rows per tile of the dX kernel: 64 or 96
 *   "dx_dist"        its prefetch distance: 2, 3 or 4
 *   "xcd_run"        tiles of one group dealt to one XCD in a row: 1 .. 1024
 *   "dw_stages"      LDS ring stages of the dW kernel: 2, 3 or 4 (default 2)
 *   "router_waves"   waves per workgroup of the fused router: 16 (one workgroup per CU,
 *                    the router weight copied whole) or 8 (two per CU, the weight in parts);
 *                    default 8 once the grid has more workgroups than the device has CUs
 *   "pack_in_place"  1: a training block call packs the expert weights in the dispatch's
 *                    place launch (default: in the router's launch where its 16-wave form
 *                    runs with enough workgroups, else in the place launch)
 * A value that does not fit a shape falls back to the library's choice for that call.
 * nsmoe_set_option returns 1 for an unknown name or a value out of range (0 always
 * restores the default); nsmoe_get_option returns -1 for an unknown name. */
int nsmoe_set_option(const char* name, int64_t value);
int64_t nsmoe_get_option(const char* name);

/* ---- router tail ----------------------------------------------------------------------
 * Replaces the softmax / topk / renormalise / cast tail of TopKRouter.forward
 * (src/model/router.py:79-98); the logits GEMM `(x @ W)` (router.py:69) is the caller's.
 *   logits    [n_tokens, n_experts]: fp32, or -- with NSMOE_ROUTE_LOGITS16 -- the 16-bit
 *             GEMM output in w_dtype, widened in the kernel exactly as router.py:69's
 *             .float() widens it.
 *   flags     NSMOE_ROUTE_PROBS: training branch (router.py:79-81): probs =
 *             softmax(logits) is written to `probs` [n_tokens, n_experts] fp32 and the
 *             top-k runs on it; otherwise top-k runs on the logits (router.py:86-92).
 *             NSMOE_ROUTE_NORMALIZE: normalize_weights.
 *             NSMOE_ROUTE_LOGITS16: logits (and, in the backward, the eval branch's
 *             `src` and grad_logits) are stored in w_dtype (bf16 / fp16 only).
 *   topk_w    [n_tokens, top_k] in w_dtype; topk_idx [n_tokens, top_k] int64, in the
 *             order CPU torch.topk returns them, ties included.
 * Limits: 1 <= top_k <= n_experts <= 128.
 */
#define NSMOE_ROUTE_PROBS 1
#define NSMOE_ROUTE_NORMALIZE 2
#define NSMOE_ROUTE_LOGITS16 4
int nsmoe_route_fwd(const void* logits, int64_t n_tokens, int32_t n_experts, int32_t top_k,
                    int32_t flags, int32_t w_dtype, void* topk_w, int64_t* topk_idx,
                    float* probs, void* stream);

/* Backward of nsmoe_route_fwd to d(logits) [n_tokens, n_experts] (torch autograd through
 * router.py:79-98).  `src` is the probs of the forward (fp32) when flags has
 * NSMOE_ROUTE_PROBS, else the logits.  d(probs) is the sum of two optional terms:
 *   grad_probs  [n_tokens, n_experts] fp32, any upstream gradient of probs (or NULL);
 *   the balance loss aux = aux_coef * E * sum_e f_e * mean_t probs[t, e] with
 *   f = aux_counts / max(sum aux_counts, 1) (router.py:100-111; f is constant), given
 *   its upstream gradient grad_aux (device fp32 scalar) and aux_counts [n_experts] int32
 *   -- both NULL to leave it out.  grad_logits is fp32, or w_dtype under
 *   NSMOE_ROUTE_LOGITS16. */
int nsmoe_route_bwd(const void* src, const int64_t* topk_idx, const void* grad_topk_w,
                    int32_t w_dtype, const float* grad_probs, const float* grad_aux,
                    const int32_t* aux_counts, float aux_coef, int64_t n_tokens,
                    int32_t n_experts, int32_t top_k, int32_t flags, void* grad_logits,
                    void* stream);

/* Balance loss TopKRouter.balance_loss (router.py:100-111):
 *   aux[0] = coef * n_experts * sum_e (counts[e] / max(sum counts, 1)) * mean_t probs[t, e]
 * probs [n_tokens, n_experts] fp32, counts [n_experts] int32, aux [1] fp32 (device).
 * Deterministic (fixed summation order).  workspace >=
 * nsmoe_balance_loss_workspace_size(n_tokens, n_experts) bytes. */
size_t nsmoe_balance_loss_workspace_size(int64_t n_tokens, int32_t n_experts);
int nsmoe_balance_loss(const float* probs, const int32_t* counts, int64_t n_tokens,
                       int32_t n_experts, float coef, float* aux, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---- dispatch -------------------------------------------------------------------------
 * Replaces moe_dispatch (src/model/moe_kernel.py:180-218) with the permutation of
 * MoEBlock._plan (src/model/moe.py:208-223): pairs p = t * top_k + j are sorted by
 * expert, stably, so each expert's run is in increasing p.
 *   topk_idx     [n_pairs] int64 expert ids (ids outside [0, n_experts) are ignored and
 *                get inv = -1)
 *   sorted_ids   [l_cap] int32: pair id per slot, sentinel n_pairs in pad slots
 *   expert_ids   [l_cap / align_m] int32: owner expert of each aligned block (0 past the
 *                data)
 *   pad_offsets  [n_experts + 1] int32: run starts, each run padded to align_m slots
 *   counts       [n_experts] int32: routing counts
 *   n_post_pad   [1] int32: padded total
 *   inv          [n_pairs] int32: slot of each pair
 * l_cap = nsmoe_dispatch_l_cap(n_pairs, n_experts); workspace >=
 * nsmoe_dispatch_workspace_size(n_pairs, n_experts) bytes.  n_experts <= 1024.
 */
int64_t nsmoe_align_m(void);
int64_t nsmoe_dispatch_l_cap(int64_t n_pairs, int32_t n_experts);
size_t nsmoe_dispatch_workspace_size(int64_t n_pairs, int32_t n_experts);
int nsmoe_dispatch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                   int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                   int32_t* counts, int32_t* n_post_pad, int32_t* inv, void* workspace,
                   size_t workspace_bytes, void* stream);

/* nsmoe_dispatch without a workspace: no counterpart in the reference.  For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, outputs and kernels as
 * nsmoe_dispatch; the scratch is a 4 MiB array owned by the library on each device (held
 * until the process ends), so it takes calls whose nsmoe_dispatch_workspace_size is at
 * most 4 MiB -- up to 14,128,128 pairs at 76 experts, 262,144 at 1024 -- and rejects
 * larger ones with error 1.  It allocates nothing.  Every call on a device shares that
 * device's array: calls that overlap on one device (two streams, two threads) race.
 * The first call on each device resolves the array's address and must not be made under
 * HIP graph capture (error 1 if it is); later calls, captured or not, reuse it. */
int nsmoe_dispatch_noalloc(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                           int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                           int32_t* counts, int32_t* n_post_pad, int32_t* inv, void* stream);

/* ---- experts --------------------------------------------------------------------------
 * Routed experts (moe_experts, src/model/moe_kernel.py:558-617) plus, when n_shared > 0,
 * the always-on shared experts (MoEBlock._shared, src/model/moe.py:310-329) folded in
 * as extra groups over every token at gate 1.
 *
 * Row space: routed rows are the dispatch slots [0, l_cap); shared expert s owns rows
 * l_cap + s * n_tokens + t.  rows_total = l_cap + n_shared * n_tokens.
 *
 * Limits: d_hidden <= 256; n_experts + n_shared <= 1024.
 */
typedef struct nsmoe_experts_args {
  int32_t dtype;       /* element type of x, weights, biases, topk_w and outputs */
  int32_t activation;
  int64_t n_tokens;    /* T */
  int32_t d_model;     /* d */
  int32_t d_hidden;    /* H; w_in is [E, d, 2H] with gate columns [0, H), up [H, 2H) */
  int32_t n_experts;   /* E (routed) */
  int32_t n_shared;    /* S */
  int32_t top_k;       /* k */
  int32_t reserved0;
  int64_t l_cap;       /* length of sorted_ids */

  const void* x;        /* [T, d] */
  const void* w_in;     /* [E, d, 2H] */
  const void* w_out;    /* [E, H, d] */
  const void* b_in;     /* [E, 2H] or NULL */
  const void* b_out;    /* [E, d] or NULL */
  const void* w_sh_in;  /* [S, d, 2H] (NULL when S == 0) */
  const void* w_sh_out; /* [S, H, d] */
  const void* b_sh_in;  /* [S, 2H] or NULL */
  const void* b_sh_out; /* [S, d] or NULL */
  const void* topk_w;   /* [T, k] gate weights */

  const int32_t* sorted_ids;  /* dispatch outputs (nsmoe_dispatch) */
  const int32_t* pad_offsets;
  const int32_t* counts;

  const void* w_in_packed;   /* nsmoe_pack_weights outputs: required by the forward */
  const void* w_out_packed;  /* (both) and the backward (w_in_packed) */
} nsmoe_experts_args;

/* Weight repacking (no counterpart in the reference: the layout its Triton kernels read
 * through tl.dot is the plain stack).  Rewrites w_in / w_sh_in and w_out / w_sh_out into
 * MFMA fragment order so the grouped GEMMs load each 16 x 32 weight fragment with one
 * coalesced load.  Run once per weight update (every forward in training); the backward
 * reuses the forward's w_in_packed.  w_out_packed may be NULL to pack W_in only.
 * nsmoe_pack_sizes reports the two buffer sizes in bytes. */
int nsmoe_pack_sizes(const nsmoe_experts_args* args, size_t* w_in_bytes, size_t* w_out_bytes);
int nsmoe_pack_weights(const nsmoe_experts_args* args, void* w_in_packed, void* w_out_packed,
                       void* stream);

/* Forward: out [T, d] = sum_j topk_w[t, j] * expert_{idx[t, j]}(x[t]) + sum_s shared_s(x[t]).
 *   inv    [T * k] int32 from nsmoe_dispatch.
 * workspace >= nsmoe_experts_fwd_workspace_size(args) (the per-row expert outputs). */
size_t nsmoe_experts_fwd_workspace_size(const nsmoe_experts_args* args);
int nsmoe_experts_fwd(const nsmoe_experts_args* args, const int32_t* inv, void* out,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Backward (_moe_experts_bwd, src/model/moe_kernel.py:626-739, plus the shared experts).
 * The gate/up pre-activations are recomputed inside the backward's tiles (fp32, never
 * stored), as the reference recomputes them (moe_kernel.py:663-672).
 *   grad_out  [T, d]
 *   dx        [T, d]; dw_in / dw_out like w_in / w_out; dw_sh_in / dw_sh_out like the
 *             shared weights (NULL when S == 0); dtopk_w [T, k]
 *   db_in, db_out, db_sh_in, db_sh_out: bias gradients, each NULL when not wanted.
 * dtopk_w is the full derivative of (h W_out + b_out) * w with respect to w, so it
 * includes <grad_out, b_out> when the experts have an output bias.
 * workspace >= nsmoe_experts_bwd_workspace_size(args). */
typedef struct nsmoe_experts_grads {
  void* dx;
  void* dw_in;
  void* dw_out;
  void* dw_sh_in;
  void* dw_sh_out;
  void* dtopk_w;
  void* db_in;
  void* db_out;
  void* db_sh_in;
  void* db_sh_out;
} nsmoe_experts_grads;

size_t nsmoe_experts_bwd_workspace_size(const nsmoe_experts_args* args);
int nsmoe_experts_bwd(const nsmoe_experts_args* args, const int32_t* inv,
                      const void* grad_out, const nsmoe_experts_grads* grads,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- the whole block, one call per direction ------------------------------------------
 * MoEBlock.forward's kernel branch (src/model/moe.py:345-418: the router, router.py:56-98,
 * fused_moe_forward moe_kernel.py:785-803 with the shared experts moe.py:310-329, balance
 * loss router.py:100-111) and its backward, as a sequence of kernels over caller buffers.
 *
 * The router GEMM (router.py:69):
 *   forward, w_router [d, E] non-NULL: computed here, fused with the router tail and the
 *     dispatch's histogram pass (bf16/fp16, d % 32 == 0, d <= 576, E % 4 == 0,
 *     E <= 80, top_k <= 16).  `logits` [T, E] (args dtype) receives x W_r with fp32 accumulation,
 *     plus logit_bias [E] fp32 when given (a harness hook with no counterpart in the
 *     reference router, which has no bias; NULL in MoEBlock), rounded to the dtype.
 *   forward, w_router NULL: `logits` holds the caller's GEMM output; logit_bias must be
 *     NULL.
 *   backward: either done here (w_router given: dx gets d(logits) W^T, grad_w_router gets
 *     x^T d(logits)) or left to the caller (w_router NULL: grad_logits receives d(logits)).
 *
 * `args` carries dims, dtype, activation, x, weights, biases and the packed weights
 * (w_in_packed, w_out_packed: nsmoe_pack_weights layout, both required by the forward,
 * w_in_packed by the backward); its routing pointers (topk_w, sorted_ids, pad_offsets,
 * counts) and l_cap are ignored -- the calls place them in `saved`.  With
 * NSMOE_BLOCK_PACK in route_flags the forward first packs the weights into
 * w_in_packed / w_out_packed itself (with the router weight passed and the "side_stream"
 * option off, inside the router's or the place launch; otherwise in a launch of its own,
 * on a second stream beside the routing kernels when that option is set);
 * without it they must hold the current weights already, so a caller that keeps the
 * packs while the weights do not change skips that pass.
 *
 * `saved` (nsmoe_block_saved_layout: total bytes and the offset of each part) is written
 * by the forward and read by the backward: topk_w [T, k] (args dtype), probs [T, E] fp32
 * (train branch only), the dispatch buffers of nsmoe_dispatch and, with
 * NSMOE_BLOCK_SAVE_ACT in route_flags, the experts' pre-activations x W_in + b_in (args
 * dtype, [gate | up] for the dispatch's l_cap rows and each shared expert's T rows rounded
 * up to 16, stored in 16 x 16 blocks in the expert kernels' register order: opaque to the
 * caller).  With them saved the backward does not recompute x W_in, which is two
 * thirds of its expert GEMM work; the reference recomputes them in its backward
 * (moe_kernel.py:663-672) and rounds them to the same dtype.  The part is empty (and the
 * flag has no effect) where the register-tiled expert kernels do not apply: 16-bit
 * types, d % 64 == 0, H % 16 == 0, H <= 128.  Pass the same route_flags to the forward,
 * the backward and the layout and workspace queries.  The expert ids
 * topk_idx [T, k] int64 and the routing counts [E] int32 are separate caller buffers
 * (MoEBlock keeps both after the step), written by the forward and read by the backward.
 *
 * Forward: out [T, d]; aux [1] fp32 = the balance loss (train branch, route_flags has
 * NSMOE_ROUTE_PROBS).  In the eval branch a non-NULL aux receives four zero bytes (the
 * branch's zero loss in any dtype up to 4 bytes wide, written by the dispatch's launch so
 * the caller needs no fill of its own); NULL leaves it to the caller.  Backward: grads as nsmoe_experts_bwd
 * (dtopk_w is ignored: the gate gradient goes straight into the router backward);
 * grad_aux (device fp32 scalar) may be NULL.  `logits` is needed again by the backward in
 * the eval branch.
 *   w_router [d, E] non-NULL (bf16/fp16, d % 16 == 0, E % 4 == 0, E <= 128): grads->dx
 *     is the whole input gradient (experts + router), grad_w_router [d, E] receives the
 *     router weight's gradient, grad_logits is unused; the workspace is
 *     nsmoe_block_bwd_workspace_size(args, route_flags, 1).
 *   w_router NULL: grads->dx holds the experts' part only, grad_logits [T, E] receives
 *     d(logits) as nsmoe_route_bwd writes it, grad_w_router is unused; workspace
 *     nsmoe_block_bwd_workspace_size(args, route_flags, 0).
 *
 * The RMSNorm and residual around the block (`norm` non-NULL, NSMOE_BLOCK_NORM in
 * route_flags; both or neither): the FFN half of the reference's Block.forward,
 *   out = x + MoEBlock(RMSNorm(x))          (src/model/nanospeaker.py:169, ln.py:30-36)
 * with args->x the residual stream.  RMSNorm is F.rms_norm's arithmetic: fp32
 * rstd = 1 / sqrt(mean(x^2) + eps), xn = (x rstd) weight rounded once to the dtype.  The
 * router kernel normalises the rows as it loads them and keeps xn and rstd in `saved`
 * (the experts and the backward read xn); the combine adds x to the block's output,
 * each rounded to the dtype as the separate ops round them.  The backward's grads->dx is
 * the gradient of x through both paths, and norm->grad_weight [d] receives the gain's
 * gradient.  Needs the fused router (w_router given, shapes as above).  Callers without
 * the norm pass NULL.
 */
typedef struct nsmoe_block_norm {
  const void* weight;  /* [d] RMSNorm gain, args dtype */
  void* grad_weight;   /* [d] backward output, args dtype */
  float eps;
  int32_t reserved;
} nsmoe_block_norm;

#define NSMOE_BLOCK_NORM 32
#define NSMOE_BLOCK_PACK 8
#define NSMOE_BLOCK_SAVE_ACT 16

#define NSMOE_SAVED_TOPK_W 0
#define NSMOE_SAVED_PROBS 1
#define NSMOE_SAVED_SORTED_IDS 2
#define NSMOE_SAVED_EXPERT_IDS 3
#define NSMOE_SAVED_PAD_OFFSETS 4
#define NSMOE_SAVED_N_POST_PAD 5
#define NSMOE_SAVED_INV 6
#define NSMOE_SAVED_ACT 7
#define NSMOE_SAVED_XN 8   /* NSMOE_BLOCK_NORM: [T, d] normalised input (args dtype) */
#define NSMOE_SAVED_RSTD 9 /* NSMOE_BLOCK_NORM: [T] fp32 */
#define NSMOE_BLOCK_NSAVED 10

int nsmoe_block_saved_layout(const nsmoe_experts_args* args, int32_t route_flags,
                             size_t* offsets /* [NSMOE_BLOCK_NSAVED] */, size_t* total_bytes);
size_t nsmoe_block_fwd_workspace_size(const nsmoe_experts_args* args, int32_t route_flags);
int nsmoe_block_fwd(const nsmoe_experts_args* args, const nsmoe_block_norm* norm,
                    const void* w_router,
                    const float* logit_bias, void* logits, int32_t route_flags, float aux_coef,
                    void* saved, int64_t* topk_idx, int32_t* counts, void* out, float* aux,
                    void* workspace, size_t workspace_bytes, void* stream);
size_t nsmoe_block_bwd_workspace_size(const nsmoe_experts_args* args, int32_t route_flags,
                                      int32_t fuse_router);
int nsmoe_block_bwd(const nsmoe_experts_args* args, const nsmoe_block_norm* norm,
                    const void* logits, int32_t route_flags,
                    float aux_coef, const void* saved, const int64_t* topk_idx,
                    const int32_t* counts, const void* grad_out, const float* grad_aux,
                    const nsmoe_experts_grads* grads, const void* w_router,
                    void* grad_w_router, void* grad_logits, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- RMSNorm forward (the decoder around the block) -------------------------------------
 * RMSNorm.forward (src/model/ln.py:30-36, F.rms_norm) for the norms the block's kernels do
 * not take: the attention's pre-norm (nanospeaker.py:168) and the final norm
 * (nanospeaker.py:231).  y [n_rows, d] = (x rstd) weight rounded once to the dtype, fp32
 * rstd = 1 / sqrt(mean(x^2) + eps), written to rstd [n_rows] when it is not NULL.
 * 16-bit types; d a multiple of 8, at most 1024; 16-byte aligned x, weight, y. */
int nsmoe_rms_norm(int32_t dtype, const void* x, const void* weight, float eps,
                   int64_t n_rows, int32_t d, void* y, float* rstd, void* stream);

/* ---- prefill attention (the decoder around the block) --------------------------------
 * Replaces the middle of OptimizedMultiHeadAttention.forward on its SDPA path
 * (src/model/mha.py:258-287, masks mha.py:49-66): the per-head RMSNorm of Q and K
 * (qk_norm=True; F.rms_norm, src/model/ln.py:30-36), the rotary embedding
 * (src/model/rope.py, rotate-half over the whole head, p = 1; the rotation in the dtype
 * from fp32 tables cast to it) at positions 0 .. seq_len - 1, and causal attention with an
 * optional sliding window over grouped-query heads (query head h reads key/value head
 * h / (n_heads / n_kv_heads)), scale 1 / sqrt(64).
 *   qkv  [batch * seq_len, ld]: each token's n_heads query heads, then n_kv_heads key
 *        heads, then n_kv_heads value heads, 64 elements each (the projection
 *        Z [W_q | W_k | W_v]).  The key heads are normalised and rotated IN PLACE.
 *   out  [batch * seq_len, n_heads * 64]: the attention output, ready for W_O.
 *   cos, sin [seq_len, 32] fp32: cos / sin(pos * base^(-2 j / 64)) (rope.py's table).
 *   q_gamma, k_gamma [64]: the two RMSNorm gains, args dtype.
 * 16-bit types; head_dim 64; n_heads / n_kv_heads in 1..4.  window = keys a query sees,
 * itself included (mha.py:63); 0 or >= seq_len is full causal attention.
 */
typedef struct nsmoe_attn_args {
  int32_t dtype;       /* NSMOE_BF16 or NSMOE_F16 */
  int32_t n_heads;     /* Hq */
  int32_t n_kv_heads;  /* Hkv */
  int32_t head_dim;    /* 64 */
  int64_t batch;
  int64_t seq_len;
  int32_t ld;          /* qkv row pitch in elements (a multiple of 8) */
  int32_t window;
  float eps;           /* the RMSNorms' epsilon */
  int32_t reserved;
  void* qkv;
  const void* q_gamma;
  const void* k_gamma;
  const float* cos;
  const float* sin;
  void* out;
} nsmoe_attn_args;

int nsmoe_attn_prefill(const nsmoe_attn_args* args, void* stream);

/* ---- cross-entropy over the tied head's logits ----------------------------------------
 * The loss part of NanoSpeaker.forward with targets (src/model/nanospeaker.py:236-250:
 * F.cross_entropy((h @ embed.weight.T).float(), y), mean over the targets that are not
 * ignore_index; the reference fuses it with the head GEMM through
 * LigerFusedLinearCrossEntropyLoss).  The GEMMs around it stay library GEMMs.
 *   logits [n_rows, ld] (vocab columns used), 16-bit; target [n_rows] int64.
 *   loss [n_rows] fp32: logsumexp(row) - row[target] in fp32 (0 for ignore_index, NaN for a
 *        target outside [0, vocab)).
 *   grad NULL, or [n_rows, ld] (may be `logits` itself): (softmax(row) - onehot(target)) / n
 *        rounded to the dtype, n = *n_valid (int64, device memory: the number of targets
 *        that are not ignore_index); zero rows for ignored targets.
 * vocab a multiple of 8, at most 65536; ld a multiple of 8; 16-byte aligned rows.
 */
int nsmoe_cross_entropy_rows(int32_t dtype, const void* logits, int64_t ld, int64_t n_rows,
                             int32_t vocab, const int64_t* target, int64_t ignore_index,
                             const int64_t* n_valid, float* loss, void* grad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NSMOE_H_ */

// Definitions shared by the grouped-expert kernels (experts.hip, experts_async.hip).
#pragma once

#include "gemm_core.h"
#include "nsmoe_capi_internal.h"

namespace nsmoe {

constexpr int BM = 64;      // rows per tile
constexpr int NT = 256;     // threads per workgroup
constexpr int DW_RC = 768;  // rows per dW chunk (work items of similar size)
constexpr int NP2 = 192;  // output columns per pass of the second GEMMs
constexpr int XCD_RUN = 16;  // default tiles per XCD run of the token-tile kernels

struct ExpParams {
  const void* x;
  const void* w_in;
  const void* w_out;
  const void* b_in;
  const void* b_out;
  const void* w_sh_in;
  const void* w_sh_out;
  const void* b_sh_in;
  const void* b_sh_out;
  const void* topk_w;
  const int32_t* sorted_ids;
  const int32_t* offs;
  const int32_t* counts;
  int64_t T;
  int64_t l_cap;
  int d, H, E, S, k, act;
  int fast;
  // Token-tile kernels: runs of xcd_run consecutive tiles are dealt round-robin over the
  // XCDs (0: each XCD takes one contiguous eighth of the grid).
  int xcd_run;
  // fragment-order weight packs (pack.hip): W_in for GEMM1, W_out for GEMM2
  const char* p_in;
  const char* p_out;
  int in_kb, in_nb, out_kb, out_nb;
  // forward output rows
  void* y;
  // The pre-activations a1 = x W_in + b_in in 16 x 16 blocks (act_block): written by the
  // forward when a1_out is set, read by the backward (instead of being recomputed) when
  // a1_in is set.
  void* a1_out;
  const void* a1_in;
  // backward
  const void* dout;
  void* da1;
  void* hbuf;
  void* dxrow;
  void* dtw;
  // dW
  void* dw_a;      // dW_in or dW_out (routed)
  void* dw_sh;     // shared counterpart
  float* partial;  // fp32 partials
  void* db;        // bias grad (routed)
  void* db_sh;     // bias grad (shared)
};

__device__ __forceinline__ int tile_of_block(const ExpParams& p) {
  return p.xcd_run > 0 ? xcd_deal(blockIdx.x, gridDim.x, p.xcd_run)
                       : xcd_remap(blockIdx.x, gridDim.x);
}

__device__ __forceinline__ int rows_of(const ExpParams& p, int g) {
  return g < p.E ? p.counts[g] : (int)p.T;
}
__device__ __forceinline__ int64_t row_start(const ExpParams& p, int g) {
  return g < p.E ? (int64_t)p.offs[g] : p.l_cap + (int64_t)(g - p.E) * p.T;
}
template <class T>
__device__ __forceinline__ const T* per_group(const void* routed, const void* shared, int g,
                                              int E, int64_t stride) {
  return g < E ? (const T*)routed + (int64_t)g * stride
               : (const T*)shared + (int64_t)(g - E) * stride;
}

// The saved pre-activations (ExpParams::a1_out / a1_in) are stored in blocks of 16 rows x
// 16 columns, 512 contiguous bytes each: lane l = 16 q + r of a wave holds row r, columns
// 4 q .. 4 q + 3 of the block (the MFMA accumulator layout), so each 8-byte store or load
// of a wave covers one whole block.  A row block holds the 2H / 16 column blocks of 16
// rows [gate 0 .. H | up 0 .. H]; the row blocks are the routed groups' in dispatch order
// (pad_offsets are multiples of 16), then each shared group's ceil(T / 16).
// act_block(p, g, r) is the row block of local rows r .. r + 15 of group g (r % 16 == 0).
__device__ __forceinline__ int64_t act_block(const ExpParams& p, int g, int r) {
  const int64_t start = g < p.E ? (int64_t)p.offs[g]
                                : p.l_cap + (int64_t)(g - p.E) * ((p.T + 15) / 16 * 16);
  return (start + r) / 16;
}

// Token, gate weight and pair id of local row `r` of group g (slot = row_start + r).
template <int DT>
__device__ __forceinline__ void row_info(const ExpParams& p, int g, int64_t slot, int r,
                                         int& tok, float& w, int& pair) {
  if (g < p.E) {
    pair = p.sorted_ids[slot];
    tok = pair / p.k;
    w = Elem<DT>::to_f(((const typename Elem<DT>::T*)p.topk_w)[pair]);
  } else {
    pair = -1;
    tok = r;
    w = 1.0f;
  }
}

// Copies `rows` rows of an LDS tile out to global rows dst + (slot0 + m) * ld, columns
// [0, n_a) from LDS columns [0, n_a) and, if n_b > 0, global columns [n_a, n_a + n_b)
// from LDS columns [lds_b, lds_b + n_b).
template <int DT>
__device__ __forceinline__ void copy_out(const char* tile, int pitch, int rows,
                                         typename Elem<DT>::T* dst, int64_t ld, int64_t col0,
                                         int n_a, int lds_b, int n_b, bool fast) {
  using G = Geo<DT>;
  using T = typename G::T;
  const int ncols = n_a + n_b;
  if (fast) {
    const int vpr = ncols / G::VE;
    for (int i = threadIdx.x; i < rows * vpr; i += NT) {
      const int m = i / vpr, c = (i % vpr) * G::VE;
      const int lc = c < n_a ? c : lds_b + (c - n_a);
      *(u32x4*)(dst + m * ld + col0 + c) = *(const u32x4*)(tile + m * pitch + lc * G::ES);
    }
  } else {
    for (int i = threadIdx.x; i < rows * ncols; i += NT) {
      const int m = i / ncols, c = i % ncols;
      const int lc = c < n_a ? c : lds_b + (c - n_a);
      dst[m * ld + col0 + c] = *(const T*)(tile + m * pitch + lc * G::ES);
    }
  }
}


// Row chunks of group g in the dW work decomposition.
__device__ __forceinline__ int dw_chunks(int rows) {
  const int c = (rows + DW_RC - 1) / DW_RC;
  return c < 1 ? 1 : c;  // an empty group still owns one (all-zero) chunk
}

// Async (direct-to-LDS) variants for 16-bit types and d_hidden <= 128; each returns
// NSMOE_OK after launching, or -1 when the shape is not one they take.
int launch_fwd_async(int dtype, const ExpParams& p, int nbw, int64_t grid, hipStream_t s);
// Both dW modes in one launch (q_in: dW_in, q_out: dW_out pointers and partials).
int launch_dw_pair_async(int dtype, const ExpParams& q_in, const ExpParams& q_out,
                         int64_t groups_chunks, hipStream_t s);
// Backward tiles: part 0 the GLU backward (fills p.da1, p.hbuf and p.dtw), part 1 the dX
// rows from p.da1 (fills p.dxrow).  Both parts take or refuse the same shapes.
int launch_bwd_async(int dtype, const ExpParams& p, int nbw, int64_t grid, int part,
                     hipStream_t s);

}  // namespace nsmoe

struct nsmoe_experts_args;
struct nsmoe_experts_grads;

namespace nsmoe {
struct DwReduceArgs;  // dw_reduce.h
// nsmoe_experts_bwd; with combine = false the per-row dX stay in the workspace at
// experts_bwd_dxrows_offset(a) (rows as the forward's row space) and grads->dx is unused.
// The dW stage runs on the side stream (side_fork slot kSideSlotDw); with side_out != NULL
// a successful call leaves that stream in *side_out for the caller to join with
// side_join(stream, *side_out, kSideSlotDw), otherwise it is joined before returning.
// act_in: the forward's saved pre-activations (experts_fwd_launch's act_out), or NULL to
// recompute them.
// defer_reduce: when set and dW runs on `stream`, the dW split-K reduce is not launched
// but described there (nbx > 0) for a later launch on the stream to run (combine_dx's);
// nbx = 0 when it ran here.
int experts_bwd_launch(const ::nsmoe_experts_args* a, const int32_t* inv, const void* grad_out,
                       const ::nsmoe_experts_grads* grads, void* workspace,
                       size_t workspace_bytes, bool combine, hipStream_t stream,
                       hipStream_t* side_out, const void* act_in = nullptr,
                       DwReduceArgs* defer_reduce = nullptr);
size_t experts_bwd_dxrows_offset(const ::nsmoe_experts_args* a);
// nsmoe_experts_fwd that also writes the pre-activations a1 = x W_in + b_in (act_block's
// layout) to act_out when experts_save_act_bytes(a) > 0 -- the backward then reads them
// instead of recomputing -- and with resid [T, d] non-NULL returns resid + the block
// output (each rounded to the dtype) in out.
int experts_fwd_launch(const ::nsmoe_experts_args* a, const int32_t* inv, void* out,
                       void* workspace, size_t workspace_bytes, void* act_out,
                       hipStream_t stream, const void* resid = nullptr);
// Bytes of the saved pre-activations for this shape (a->l_cap set), 0 where the kernels
// that write and read them do not apply (16-bit types, d % 64 == 0, H % 16 == 0, H <= 128
// and the step-count parities of the register-tiled forward and backward).
size_t experts_save_act_bytes(const ::nsmoe_experts_args* a);
}  // namespace nsmoe

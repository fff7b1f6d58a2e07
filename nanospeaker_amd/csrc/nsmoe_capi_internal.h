// Host-side plumbing shared by the C-ABI entry points: error strings, launch checks and
// a launch counter the tests read to prove the HIP path ran.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <atomic>
#include <string>

namespace nsmoe {

enum Status : int { NSMOE_OK = 0, NSMOE_EINVAL = 1, NSMOE_EHIP = 2, NSMOE_EWORKSPACE = 3 };

void set_error(const char* fmt, ...);
void note_launch();

// Checks the launch that was just enqueued; records an error string on failure.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return NSMOE_EHIP;
  }
  note_launch();
  return NSMOE_OK;
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace nsmoe

#define NSMOE_REQUIRE(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      ::nsmoe::set_error(__VA_ARGS__);    \
      return ::nsmoe::NSMOE_EINVAL;       \
    }                                     \
  } while (0)

#define NSMOE_TRY(expr)                   \
  do {                                    \
    int _rc = (expr);                     \
    if (_rc != 0) return _rc;             \
  } while (0)

namespace nsmoe {
// Process-wide tuning options (nsmoe_set_option); 0 means the library's own choice.
enum OptionId : int {
  OPT_SIDE_STREAM = 0,
  OPT_FWD_ROWS,
  OPT_FWD_DIST,
  OPT_BWD_ROWS,
  OPT_BWD_DIST,
  OPT_DX_ROWS,
  OPT_DX_DIST,
  OPT_XCD_RUN,
  OPT_DW_STAGES,
  OPT_ROUTER_WAVES,
  OPT_PACK_IN_PLACE,
  OPT_COUNT
};
int64_t option(OptionId id);
}  // namespace nsmoe

namespace nsmoe {
// Fork/join onto the calling thread's side stream for the current device (capi.hip).
// side_fork returns the side stream, ordered after the work already on `s`, or `s` itself
// when no side stream is available; side_join orders `s` after the side stream's work
// (a no-op when side == s).  Slots 0 .. 3 each own a fork and a join event.
hipStream_t side_fork(hipStream_t s, int slot);
int side_join(hipStream_t s, hipStream_t side, int slot);
// Slots in use: the block forward's weight packing and the experts backward's dW.
constexpr int kSideSlotPack = 0;
constexpr int kSideSlotDw = 1;

// dst[0, n) = value, as a kernel (graph-capture safe, unlike hipMemsetAsync).
int fill_i32(int32_t* dst, int64_t n, int32_t value, hipStream_t stream);
}  // namespace nsmoe

namespace nsmoe {
// Optional per-kernel timing with HIP events recorded on the launch stream (enabled by
// nsmoe_timing_enable; used by the benchmark to time its dominant kernel live).
// KernelTimer brackets one launch: construct before the launch, stop() after it.
class KernelTimer {
 public:
  KernelTimer(const char* name, hipStream_t stream);
  void stop();

 private:
  int slot_;
  hipStream_t stream_;
};
}  // namespace nsmoe

namespace nsmoe {
// Router entry points with the options the block path uses (route.hip).
// route_fwd_launch: nsmoe_route_fwd, plus optional per-workgroup column sums of probs
// ([balance_partial_count(n_tokens), n_experts] fp32) for balance_final_launch.
int route_fwd_launch(const void* logits, int64_t n_tokens, int32_t n_experts, int32_t top_k,
                     int32_t flags, int32_t w_dtype, void* topk_w, int64_t* topk_idx,
                     float* probs, float* prob_colsum, hipStream_t stream);
// The router weight W [d, E] (16-bit) packed as MFMA A-operand fragments for the router
// term of combine_dx: fragment (mb, ks) = rows 16 mb .. + 15, k columns 32 ks .. + 31 (zero
// past E or d) sits at bytes ((mb * nks + ks) * 64 + lane) * 16, lane l holding row
// 16 mb + l % 16, columns 32 ks + 8 (l / 16) .. + 7.
struct RouterWPack {
  const void* w;
  void* pk;
  int d, E, nks;
};
inline size_t router_w_pack_bytes(int d, int nks) { return (size_t)((d + 15) / 16) * nks * 1024; }
// route_bwd_launch: nsmoe_route_bwd with grad_logits rows of pitch ldg (pad columns zero);
// with `pack` non-NULL (16-bit types) the launch also writes that pack, in extra workgroups.
int route_bwd_launch(const void* src, const int64_t* topk_idx, const void* grad_w,
                     int32_t w_dtype, const float* grad_probs, const float* grad_aux,
                     const int32_t* aux_counts, float aux_coef, int64_t n_tokens,
                     int32_t n_experts, int32_t top_k, int32_t flags, void* grad_logits,
                     int32_t ldg, hipStream_t stream, const RouterWPack* pack = nullptr);
int64_t balance_partial_count(int64_t n_tokens);
// The balance loss folded into the dispatch (dispatch_launch): column-sum partials of probs
// from route_fwd_launch ([nblk = balance_partial_count(T), E] fp32), T, coef -> aux[0].
struct BalanceArgs {
  const float* partial;
  int64_t nblk;
  int64_t T;
  float coef;
  float* aux;
};
// nsmoe_dispatch, plus the balance loss in one extra workgroup of its second launch when
// bal is non-NULL (E <= 128).
int dispatch_launch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                    int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                    int32_t* counts, int32_t* n_post_pad, int32_t* inv, void* workspace,
                    size_t workspace_bytes, const BalanceArgs* bal, void* stream,
                    float* zero_out = nullptr);
// The place pass of the dispatch from per-chunk histograms [n_chunks, E] made elsewhere
// (chunk c = pairs [c chunk_pairs, (c + 1) chunk_pairs)); E <= 128, chunk_pairs <= 1024.
struct PackPairArgs;
// With pack non-NULL (16-bit pack_dtype, pack_pair_args), the same launch also packs both
// weight stacks in workgroups of its own beside the placement ones.
int dispatch_place_launch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                          const int32_t* hist, int64_t n_chunks, int chunk_pairs,
                          int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                          int32_t* counts, int32_t* n_post_pad, int32_t* inv,
                          const BalanceArgs* bal, hipStream_t stream,
                          const PackPairArgs* pack = nullptr, int pack_dtype = 0,
                          float* zero_out = nullptr);
int balance_final_launch(const float* partial, int64_t n_tokens, int32_t n_experts,
                         const int32_t* counts, float coef, float* aux, hipStream_t stream);
}  // namespace nsmoe

// Router tail on device: softmax, top-k selection with torch-CPU tie order, gate
// renormalisation, the matching backward to d(logits), and the balance loss.
//
// Reference: TopKRouter.forward (src/model/router.py:69-98) and balance_loss
// (router.py:100-111).  The logits GEMM `x @ W` (router.py:69) and the optional
// exploration noise (router.py:76-77) stay with the caller; this file takes the logits.
//
// Forward layout: one token row per wavefront at a time; each workgroup owns RF_ROWS
// rows (RF_RPW per wave), whose probs it also sums per expert for the balance loss.  A lane holds row elements lane and lane + 64.
// Row max / sum are DPP butterflies inside each 16-lane row, combined across the four
// rows through v_readlane in a fixed order.
//
// Selection has to reproduce torch's CPU topk bit for bit, ties included: the order of
// equal keys is whatever libstdc++'s nth_element / sort / partial_sort leave (see
// ATen/native/TopKImpl.h:44-94).
//   * Fast path: k rounds of a wave-wide arg-max.  If every round's maximum is unique
//     among the values still in play (no NaN, no tie inside the top k, none at its
//     boundary), the sorted top k is unique, so any selection returns CPU topk's answer.
//   * Exact path, for rows with a tie that matters: the routines below restate those
//     published algorithms (introselect with median-of-three, unguarded Hoare partition,
//     heap select, insertion sort, introsort) on the row as the wave holds it in
//     registers.  Every access takes a wave-uniform index (a v_readlane, or a lane
//     compare-and-select for a store), so the sequential algorithm runs in uniform (scalar) control flow
//     with register latency instead of one lane walking the row through LDS.
#include "balance.h"
#include "nsmoe_capi_internal.h"
#include "nsmoe_common.h"
#include "topk_exact.h"

namespace nsmoe {

constexpr int ROUTE_MAX_EXPERTS = 128;       // two row elements per lane
constexpr int RF_WAVES = 16;                 // route_fwd: waves per workgroup
constexpr int RF_RPW = 1;                    // route_fwd: rows per wave (one row per wave
                                             // measured fastest: a tie row's exact path
                                             // then delays no other row)
constexpr int RF_ROWS = RF_WAVES * RF_RPW;   // rows per route_fwd workgroup = rows per
                                             // balance-loss partial
constexpr int ROUTE_WAVES = 4;               // route_bwd: rows (waves) per workgroup
constexpr int ROUTE_THREADS = 64 * ROUTE_WAVES;

// ---- forward ---------------------------------------------------------------------------
//
// flags bit 0 (want_probs): training branch, probs = softmax(logits) and the selection
//   runs on probs (router.py:79-81); probs [T, E] is written out.
// flags bit 1 (normalize):  normalize_weights.
// Without want_probs the selection runs on the logits and the gates are
// softmax(topk logits) (normalize) or softmax(logits)[idx] (router.py:83-92).
// With want_probs and normalize and k > 1 the gates are p / sum(p) (router.py:96-97).
// flags bit 2 (logits16): the logits are stored in the gate dtype DT (the bf16 / fp16 GEMM
//   output that router.py:69 widens with .float()); they are widened here on load.
// prob_colsum (optional, want_probs only): [gridDim.x, E] sums of probs over the
//   workgroup's RF_ROWS rows, in a fixed order -- the first level of the balance loss's
//   mean over tokens.
template <int DT>
__global__ void __launch_bounds__(RF_WAVES * 64)
route_fwd_kernel(const void* __restrict__ logits, int64_t T, int E, int k, int flags,
                 typename Elem<DT>::T* __restrict__ topk_w, int64_t* __restrict__ topk_idx,
                 float* __restrict__ probs, float* __restrict__ prob_colsum) {
  __shared__ float s_col[RF_WAVES][ROUTE_MAX_EXPERTS];
  __shared__ int2 s_pos[RF_WAVES][TOPK_SWAP_SLOTS];  // exact path: swap slots
  using OutT = typename Elem<DT>::T;
  // readfirstlane: the compiler then knows the wave index, and every row condition
  // below, is wave-uniform (scalar branches, not exec masks).
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;
  const bool has0 = lane < E, has1 = lane + 64 < E;
  const int64_t row0 = (int64_t)blockIdx.x * RF_ROWS + wave;  // the wave's rows: row0 + j W

  // Phase 0: every row's logits in flight at once (branch-free: lanes past E and rows
  // past T read a valid element and are masked afterwards).  On gfx9 vmcnt counts stores
  // as well, so nothing is loaded after the first store.
  uint32_t raw[RF_RPW][2];
#pragma unroll
  for (int j = 0; j < RF_RPW; ++j) {
    const int64_t row = min(row0 + (int64_t)j * RF_WAVES, T - 1);
    const int c0 = has0 ? lane : 0, c1 = has1 ? lane + 64 : 0;
    if constexpr (DT != DT_F32) {
      if (flags & 4) {
        const OutT* lrow = (const OutT*)logits + row * E;
        raw[j][0] = lrow[c0];
        raw[j][1] = lrow[c1];
        continue;
      }
    }
    const float* lrow = (const float*)logits + row * E;
    raw[j][0] = __float_as_uint(lrow[c0]);
    raw[j][1] = __float_as_uint(lrow[c1]);
  }
  // Widened right away, so the one wait for the loads comes before the first store.
  float val[RF_RPW][2];
#pragma unroll
  for (int j = 0; j < RF_RPW; ++j) {
    float v0, v1;
    if (DT != DT_F32 && (flags & 4)) {
      v0 = Elem<DT>::to_f((OutT)raw[j][0]);
      v1 = Elem<DT>::to_f((OutT)raw[j][1]);
    } else {
      v0 = __uint_as_float(raw[j][0]);
      v1 = __uint_as_float(raw[j][1]);
    }
    val[j][0] = has0 ? v0 : -INFINITY;
    val[j][1] = has1 ? v1 : -INFINITY;
    // pins the values (and so the load wait) here, ahead of every store below
    asm volatile("" : "+v"(val[j][0]), "+v"(val[j][1]));
  }

  auto write_out = [&](int64_t row, float s0, float s1, int d0, int d1, float m,
                       float row_inv_sum) {
    write_route_row<DT>(row, k, lane, want_probs, normalize, s0, s1, d0, d1, m, row_inv_sum,
                        topk_w, topk_idx);
  };

  // Phase A: softmax, probs, column sums and the fast selection for every row; rows with
  // a tie that matters are marked for phase B with their keys kept in registers.
  float key[RF_RPW][2], rmax[RF_RPW], rinv[RF_RPW];
  unsigned exact_rows = 0;  // wave-uniform bit set
  float col0 = 0.0f, col1 = 0.0f;  // this wave's sums of probs, elements lane, lane + 64
#pragma unroll
  for (int j = 0; j < RF_RPW; ++j) {
    const int64_t row = row0 + (int64_t)j * RF_WAVES;
    key[j][0] = key[j][1] = 0.0f;
    rmax[j] = rinv[j] = 0.0f;
    if (row >= T) continue;  // wave-uniform
    const float v0 = val[j][0], v1 = val[j][1];
    // Row max (NaN-propagating, like torch's softmax) and sum of exp.
    const bool nan_here = (has0 && __builtin_isnan(v0)) || (has1 && __builtin_isnan(v1));
    const bool any_nan = __ballot(nan_here) != 0ull;
    float m = wave_max(fmaxf(v0, v1));
    if (any_nan) m = __uint_as_float(0x7fc00000u);
    float row_inv_sum = 0.0f;
    float k0 = v0, k1 = v1;
    if (want_probs || !normalize) {
      const float e0 = has0 ? expf(v0 - m) : 0.0f;
      const float e1 = has1 ? expf(v1 - m) : 0.0f;
      row_inv_sum = 1.0f / wave_sum(e0 + e1);
      if (want_probs) {
        k0 = e0 * row_inv_sum;
        k1 = e1 * row_inv_sum;
        float* prow = probs + row * E;
        if (has0) prow[lane] = k0;
        if (has1) prow[lane + 64] = k1;
        col0 += has0 ? k0 : 0.0f;
        col1 += has1 ? k1 : 0.0f;
      }
    }
    key[j][0] = k0;
    key[j][1] = k1;
    rmax[j] = m;
    rinv[j] = row_inv_sum;
    float s0 = 0.0f, s1 = 0.0f;
    int d0 = 0, d1 = 0;
    bool exact = any_nan;
    if (!exact) {
      bool av0 = has0, av1 = has1;
      for (int t = 0; t < k; ++t) {
        const float c = fmaxf(av0 ? k0 : -INFINITY, av1 ? k1 : -INFINITY);
        const float mx = wave_max(c);
        const unsigned long long b0 = __ballot(av0 && k0 == mx);
        const unsigned long long b1 = __ballot(av1 && k1 == mx);
        if (__popcll(b0) + __popcll(b1) != 1) {
          exact = true;
          break;
        }
        const int src = b0 ? __ffsll((long long)b0) - 1 : __ffsll((long long)b1) - 1 + 64;
        if (lane == (src & 63)) {
          if (src < 64) av0 = false;
          else av1 = false;
        }
        if (lane == (t & 63)) {
          if (t < 64) { s0 = mx; d0 = src; }
          else { s1 = mx; d1 = src; }
        }
      }
    }
    if (exact) exact_rows |= 1u << j;
    else write_out(row, s0, s1, d0, d1, m, row_inv_sum);
  }

  // Phase B: the exact restatement for the marked rows.
  for (int j = 0; j < RF_RPW; ++j) {
    if (!(exact_rows & (1u << j))) continue;  // wave-uniform
    float k0 = 0.0f, k1 = 0.0f, m = 0.0f, inv = 0.0f;
#pragma unroll
    for (int u = 0; u < RF_RPW; ++u)
      if (u == j) {
        k0 = key[u][0];
        k1 = key[u][1];
        m = rmax[u];
        inv = rinv[u];
      }
    RegRow r{(int)ord_key(k0), (int)ord_key(k1), lane, lane + 64, lane};
    topk_select(r, E, k, s_pos[wave]);
    // The selected values, bit for bit, from the row as loaded (element id of output j).
    const int a0 = (r.i0 & 63) * 4, a1 = (r.i1 & 63) * 4;
    const float lo0 = __int_as_float(__builtin_amdgcn_ds_bpermute(a0, __float_as_int(k0)));
    const float hi0 = __int_as_float(__builtin_amdgcn_ds_bpermute(a0, __float_as_int(k1)));
    const float lo1 = __int_as_float(__builtin_amdgcn_ds_bpermute(a1, __float_as_int(k0)));
    const float hi1 = __int_as_float(__builtin_amdgcn_ds_bpermute(a1, __float_as_int(k1)));
    write_out(row0 + (int64_t)j * RF_WAVES, r.i0 < 64 ? lo0 : hi0, r.i1 < 64 ? lo1 : hi1, r.i0,
              r.i1, m, inv);
  }

  if (prob_colsum) {  // uniform: every wave reaches the barrier
    s_col[wave][lane] = col0;
    s_col[wave][lane + 64] = col1;
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < RF_WAVES; ++w) s += s_col[w][e];
      prob_colsum[(int64_t)blockIdx.x * E + e] = s;
    }
  }
}

// ---- backward --------------------------------------------------------------------------
//
// d(logits) for the same three branches, in fp32, one row per wave:
//   train: w = p_sel / S (normalize, k > 1)  ->  dp_j = (dw_j - sum_i dw_i w_i) / S
//          dprobs = grad_probs (aux loss, may be absent) + scatter(dp)
//          dlogits = p * (dprobs - sum_e p_e dprobs_e)
//   eval normalize:   w = softmax(l_sel) -> dl_sel = w * (dw - sum w dw)
//   eval !normalize:  w = softmax(l)[idx] -> softmax backward of scatter(dw)
// `src` holds probs for the train branch and logits otherwise.  Ids outside [0, E)
// (not produced by route_fwd) give the row a zero gradient.
// The balance loss aux = coef E sum_e f_e mean_t p[t, e] (router.py:110-111, f constant)
// adds d aux / d p[t, e] = grad_aux coef E f_e / T to d(probs), computed here from the
// counts (aux_counts non-NULL) instead of being materialised as a [T, E] tensor.
// flags bit 2 (logits16): in the eval branches `src` is stored in DT, and grad_logits is
// written in DT (the gradient of router.py:69's .float()); otherwise both are fp32.
// grad_logits rows have pitch ldg >= E; the pad columns are written as zeros.
// One 16-byte chunk of the router-weight pack (RouterWPack) per thread, chunk c.
template <int DT>
__device__ __forceinline__ void router_w_pack_chunk(const RouterWPack& pk, int64_t c) {
  using T = typename Elem<DT>::T;
  const int lane = (int)(c & 63);
  const int64_t f = c >> 6;
  const int ks = (int)(f % pk.nks), mb = (int)(f / pk.nks);
  const int m = mb * 16 + (lane & 15), n = ks * 32 + 8 * (lane >> 4);
  const T* w = (const T*)pk.w + (int64_t)m * pk.E;
  T v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = m < pk.d && n + e < pk.E ? w[n + e] : T(0);
  uint4 o;
  __builtin_memcpy(&o, v, 16);
  *(uint4*)((char*)pk.pk + c * 16) = o;
}

template <int DT>
__global__ void __launch_bounds__(ROUTE_THREADS)
route_bwd_kernel(const void* __restrict__ src, const int64_t* __restrict__ topk_idx,
                 const typename Elem<DT>::T* __restrict__ grad_w,
                 const float* __restrict__ grad_probs, const float* __restrict__ grad_aux,
                 const int32_t* __restrict__ aux_counts, float aux_coef, int64_t T, int E,
                 int k, int flags, void* __restrict__ grad_logits_v, int ldg, RouterWPack pk,
                 int64_t row_blocks) {
  extern __shared__ float lds_f[];
  if ((int64_t)blockIdx.x >= row_blocks) {  // the extra workgroups: the router-weight pack
    if constexpr (DT != DT_F32) {
      const int64_t c = ((int64_t)blockIdx.x - row_blocks) * ROUTE_THREADS + threadIdx.x;
      if (c < (int64_t)((pk.d + 15) / 16) * pk.nks * 64) router_w_pack_chunk<DT>(pk, c);
    }
    return;
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROUTE_WAVES + wave;
  if (row >= T) return;  // no workgroup barriers below: each wave works alone
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;
  float* sv = lds_f + wave * 2 * E;  // the row's src values
  float* sg = sv + E;                // running d(probs) or d(logits) row
  const bool has0 = lane < E, has1 = lane + 64 < E;
  const bool w16 = (flags & 4) != 0;
  using ET = typename Elem<DT>::T;
  float x0 = 0.0f, x1 = 0.0f;
  if (w16 && !want_probs) {
    const ET* srow = (const ET*)src + row * E;
    if (has0) x0 = Elem<DT>::to_f(srow[lane]);
    if (has1) x1 = Elem<DT>::to_f(srow[lane + 64]);
  } else {
    const float* srow = (const float*)src + row * E;
    if (has0) x0 = srow[lane];
    if (has1) x1 = srow[lane + 64];
  }
  float g0 = 0.0f, g1 = 0.0f;
  if (grad_probs && want_probs) {
    const float* gp = grad_probs + row * E;
    if (has0) g0 = gp[lane];
    if (has1) g1 = gp[lane + 64];
  }
  if (aux_counts && grad_aux && want_probs) {
    const float c0 = has0 ? (float)aux_counts[lane] : 0.0f;
    const float c1 = has1 ? (float)aux_counts[lane + 64] : 0.0f;
    const float scale = grad_aux[0] * aux_coef * (float)E / fmaxf(wave_sum(c0 + c1), 1.0f) /
                        (float)T;
    g0 += c0 * scale;
    g1 += c1 * scale;
  }
  // d(logits) is stored through these (fp32, or DT under logits16 in the eval branches).
  auto put = [&](int e, float v) {
    if (w16) ((ET*)grad_logits_v)[row * ldg + e] = Elem<DT>::from_f(v);
    else ((float*)grad_logits_v)[row * ldg + e] = v;
  };
  // Pad columns [E, ldg) of the row are zero (ldg - E < 64: lanes past E hold them).
  if (!has0 && lane < ldg) put(lane, 0.0f);
  if (!has1 && lane + 64 < ldg) put(lane + 64, 0.0f);
  if (has0) { sv[lane] = x0; sg[lane] = want_probs ? g0 : 0.0f; }
  if (has1) { sv[lane + 64] = x1; sg[lane + 64] = want_probs ? g1 : 0.0f; }
  const bool o0 = lane < k, o1 = lane + 64 < k;
  int64_t i0 = o0 ? topk_idx[row * k + lane] : 0, i1 = o1 ? topk_idx[row * k + lane + 64] : 0;
  const bool bad = (o0 && (i0 < 0 || i0 >= E)) || (o1 && (i1 < 0 || i1 >= E));
  if (__ballot(bad) != 0ull) {
    if (has0) put(lane, 0.0f);
    if (has1) put(lane + 64, 0.0f);
    return;
  }
  const float d0 = o0 ? Elem<DT>::to_f(grad_w[row * k + lane]) : 0.0f;
  const float d1 = o1 ? Elem<DT>::to_f(grad_w[row * k + lane + 64]) : 0.0f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float s_0 = o0 ? sv[i0] : 0.0f, s_1 = o1 ? sv[i1] : 0.0f;  // selected src values

  float p0, p1;  // softmax probabilities of this lane's row elements
  if (want_probs) {
    const bool renorm = normalize && k > 1;
    float a0 = d0, a1 = d1;
    if (renorm) {
      const float S = wave_sum(s_0 + s_1);
      const float dot = wave_sum(d0 * (s_0 / S) + d1 * (s_1 / S));
      a0 = (d0 - dot) / S;
      a1 = (d1 - dot) / S;
    }
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] += a0;  // ids in a row are distinct: no two lanes hit one slot
    if (o1) sg[i1] += a1;
    p0 = x0;
    p1 = x1;
  } else if (normalize) {
    const float mk = wave_max(fmaxf(o0 ? s_0 : -INFINITY, o1 ? s_1 : -INFINITY));
    const float e0 = o0 ? expf(s_0 - mk) : 0.0f, e1 = o1 ? expf(s_1 - mk) : 0.0f;
    const float inv = 1.0f / wave_sum(e0 + e1);
    const float w0 = e0 * inv, w1 = e1 * inv;
    const float dot = wave_sum(w0 * d0 + w1 * d1);
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] = w0 * (d0 - dot);
    if (o1) sg[i1] = w1 * (d1 - dot);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (has0) put(lane, sg[lane]);
    if (has1) put(lane + 64, sg[lane + 64]);
    return;
  } else {
    const float m = wave_max(fmaxf(has0 ? x0 : -INFINITY, has1 ? x1 : -INFINITY));
    const float e0 = has0 ? expf(x0 - m) : 0.0f, e1 = has1 ? expf(x1 - m) : 0.0f;
    const float inv = 1.0f / wave_sum(e0 + e1);
    p0 = e0 * inv;
    p1 = e1 * inv;
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] += d0;
    if (o1) sg[i1] += d1;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float q0 = has0 ? sg[lane] : 0.0f, q1 = has1 ? sg[lane + 64] : 0.0f;
  const float pd = wave_sum((has0 ? p0 * q0 : 0.0f) + (has1 ? p1 * q1 : 0.0f));
  if (has0) put(lane, p0 * (q0 - pd));
  if (has1) put(lane + 64, p1 * (q1 - pd));
}

// ---- balance loss (router.py:100-111) ----------------------------------------------------
//
// aux = coef * E * sum_e f_e * mean_t probs[t, e],  f = counts / max(sum counts, 1).
// Level 1 sums probs over each run of RF_ROWS rows per expert: route_fwd does it on the
// way (prob_colsum), or balance_partial_kernel from a probs tensor.  Level 2
// (balance_final_kernel) adds the partials in a fixed order and forms the scalar, so the
// result is deterministic.
//
// balance_partial_kernel: 256 threads per RF_ROWS rows; thread (h, e) sums the rows
// h * RF_ROWS / 2 + [0, RF_ROWS / 2) of column e with all loads independent, and the
// two halves are added in order.
__global__ void __launch_bounds__(256)
balance_partial_kernel(const float* __restrict__ probs, int64_t T, int E,
                       float* __restrict__ partial) {
  constexpr int HALF = RF_ROWS / 2;
  __shared__ float s_half[ROUTE_MAX_EXPERTS];
  const int e = threadIdx.x & 127, h = threadIdx.x >> 7;
  const int64_t r0 = (int64_t)blockIdx.x * RF_ROWS + h * HALF;
  float v[HALF];
#pragma unroll
  for (int u = 0; u < HALF; ++u)
    v[u] = (e < E && r0 + u < T) ? probs[(r0 + u) * E + e] : 0.0f;
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < HALF; ++u) s += v[u];
  if (h == 1) s_half[e] = s;
  __syncthreads();
  if (h == 0 && e < E) partial[(int64_t)blockIdx.x * E + e] = s + s_half[e];
}

// 1024 threads: the whole balance loss from the column-sum partials (balance_loss_block).
__global__ void __launch_bounds__(1024)
balance_final_kernel(const float* __restrict__ partial, int64_t nblk, const int32_t* counts,
                     int64_t T, int E, float coef, float* __restrict__ aux) {
  __shared__ BalanceLds lds;
  balance_loss_block(partial, nblk, counts, T, E, coef, aux, lds);
}

}  // namespace nsmoe

using namespace nsmoe;

namespace nsmoe {

int route_fwd_launch(const void* logits, int64_t n_tokens, int32_t n_experts, int32_t top_k,
                     int32_t flags, int32_t w_dtype, void* topk_w, int64_t* topk_idx,
                     float* probs, float* prob_colsum, hipStream_t s) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_fwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_fwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_fwd: top_k %d outside [1, %d]",
                top_k, n_experts);
  NSMOE_REQUIRE(!(flags & 1) || probs, "route_fwd: probs requested but NULL");
  NSMOE_REQUIRE(!(flags & 4) || w_dtype != DT_F32, "route_fwd: 16-bit logits need a 16-bit dtype");
  NSMOE_REQUIRE(!prob_colsum || (flags & 1), "route_fwd: column sums need probs");
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(logits && topk_w && topk_idx, "route_fwd: NULL pointer");
  const dim3 grid((unsigned)cdiv(n_tokens, RF_ROWS)), block(RF_WAVES * 64);
  KernelTimer timer("route_fwd", s);
  switch (w_dtype) {
    case DT_BF16:
      route_fwd_kernel<DT_BF16><<<grid, block, 0, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (uint16_t*)topk_w, topk_idx, probs, prob_colsum);
      break;
    case DT_F16:
      route_fwd_kernel<DT_F16><<<grid, block, 0, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (uint16_t*)topk_w, topk_idx, probs, prob_colsum);
      break;
    case DT_F32:
      route_fwd_kernel<DT_F32><<<grid, block, 0, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (float*)topk_w, topk_idx, probs, prob_colsum);
      break;
    default:
      NSMOE_REQUIRE(false, "route_fwd: unknown dtype %d", w_dtype);
  }
  timer.stop();
  return check_launch("route_fwd_kernel");
}

int64_t balance_partial_count(int64_t n_tokens) { return cdiv(n_tokens, RF_ROWS); }

int balance_final_launch(const float* partial, int64_t n_tokens, int32_t n_experts,
                         const int32_t* counts, float coef, float* aux, hipStream_t s) {
  const int64_t nblk = n_tokens > 0 ? balance_partial_count(n_tokens) : 0;
  balance_final_kernel<<<1, 1024, 0, s>>>(partial, nblk, counts, n_tokens, n_experts, coef,
                                          aux);
  return check_launch("balance_final_kernel");
}

}  // namespace nsmoe

extern "C" int nsmoe_route_fwd(const void* logits, int64_t n_tokens, int32_t n_experts,
                               int32_t top_k, int32_t flags, int32_t w_dtype, void* topk_w,
                               int64_t* topk_idx, float* probs, void* stream) {
  return route_fwd_launch(logits, n_tokens, n_experts, top_k, flags, w_dtype, topk_w,
                          topk_idx, probs, nullptr, (hipStream_t)stream);
}

namespace nsmoe {

int route_bwd_launch(const void* src, const int64_t* topk_idx, const void* grad_w,
                     int32_t w_dtype, const float* grad_probs, const float* grad_aux,
                     const int32_t* aux_counts, float aux_coef, int64_t n_tokens,
                     int32_t n_experts, int32_t top_k, int32_t flags, void* grad_logits,
                     int32_t ldg, hipStream_t s, const RouterWPack* pack) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_bwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_bwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_bwd: bad top_k %d", top_k);
  NSMOE_REQUIRE(ldg >= n_experts && ldg - n_experts < 64, "route_bwd: bad row pitch %d", ldg);
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(src && topk_idx && grad_w && grad_logits, "route_bwd: NULL pointer");
  NSMOE_REQUIRE(!(flags & 4) || w_dtype != DT_F32, "route_bwd: 16-bit logits need a 16-bit dtype");
  NSMOE_REQUIRE(!pack || (w_dtype != DT_F32 && pack->w && pack->pk && pack->d > 0 &&
                          pack->nks > 0 && pack->nks * 32 >= pack->E),
                "route_bwd: bad router-weight pack");
  const int64_t row_blocks = cdiv(n_tokens, ROUTE_WAVES);
  const int64_t pack_blocks =
      pack ? cdiv((int64_t)((pack->d + 15) / 16) * pack->nks * 64, ROUTE_THREADS) : 0;
  const RouterWPack pk = pack ? *pack : RouterWPack{nullptr, nullptr, 0, 0, 1};
  dim3 grid((unsigned)(row_blocks + pack_blocks)), block(ROUTE_THREADS);
  size_t lds = (size_t)n_experts * ROUTE_WAVES * sizeof(float) * 2;
  KernelTimer timer("route_bwd", s);
  switch (w_dtype) {
    case DT_BF16:
      route_bwd_kernel<DT_BF16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits, ldg, pk, row_blocks);
      break;
    case DT_F16:
      route_bwd_kernel<DT_F16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits, ldg, pk, row_blocks);
      break;
    case DT_F32:
      route_bwd_kernel<DT_F32><<<grid, block, lds, s>>>(src, topk_idx, (const float*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits, ldg, pk, row_blocks);
      break;
    default:
      NSMOE_REQUIRE(false, "route_bwd: unknown dtype %d", w_dtype);
  }
  timer.stop();
  return check_launch("route_bwd_kernel");
}

}  // namespace nsmoe

extern "C" int nsmoe_route_bwd(const void* src, const int64_t* topk_idx, const void* grad_w,
                               int32_t w_dtype, const float* grad_probs, const float* grad_aux,
                               const int32_t* aux_counts, float aux_coef, int64_t n_tokens,
                               int32_t n_experts, int32_t top_k, int32_t flags,
                               void* grad_logits, void* stream) {
  return route_bwd_launch(src, topk_idx, grad_w, w_dtype, grad_probs, grad_aux, aux_counts,
                          aux_coef, n_tokens, n_experts, top_k, flags, grad_logits, n_experts,
                          (hipStream_t)stream);
}

extern "C" size_t nsmoe_balance_loss_workspace_size(int64_t n_tokens, int32_t n_experts) {
  if (n_tokens <= 0 || n_experts <= 0) return 0;
  return (size_t)balance_partial_count(n_tokens) * (size_t)n_experts * sizeof(float);
}

extern "C" int nsmoe_balance_loss(const float* probs, const int32_t* counts, int64_t n_tokens,
                                  int32_t n_experts, float coef, float* aux, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "balance_loss: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "balance_loss: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(aux && counts, "balance_loss: NULL pointer");
  hipStream_t s = (hipStream_t)stream;
  if (n_tokens == 0)
    // mean over no rows is NaN in torch (router.py:111 on an empty batch); the block never
    // calls this with T = 0, but keep the definition total.
    return balance_final_launch(nullptr, 0, n_experts, counts, coef, aux, s);
  NSMOE_REQUIRE(probs && workspace, "balance_loss: NULL pointer");
  const size_t need = nsmoe_balance_loss_workspace_size(n_tokens, n_experts);
  if (workspace_bytes < need) {
    set_error("balance_loss: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  balance_partial_kernel<<<(unsigned)balance_partial_count(n_tokens), 256, 0, s>>>(
      probs, n_tokens, n_experts, (float*)workspace);
  NSMOE_TRY(check_launch("balance_partial_kernel"));
  return balance_final_launch((const float*)workspace, n_tokens, n_experts, counts, coef, aux,
                              s);
}

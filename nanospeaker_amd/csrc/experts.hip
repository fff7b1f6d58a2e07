// Grouped SwiGLU experts on gfx950 MFMA: forward, combine and the full backward.
//
// Reference: moe_experts / _moe_experts_bwd (src/model/moe_kernel.py:558-739) for the
// routed experts, MoEBlock._shared (src/model/moe.py:310-329) for the shared ones.  The
// shared experts are folded in as extra groups: group g < E is routed expert g over its
// dispatch slots, group E + s is shared expert s over every token at gate 1.
//
// Kernels (one workgroup = 4 waves, tiles of 64 rows of one group):
//   expert_fwd   GEMM1 x[tok] @ W_in[g] with the gate and up halves in two accumulator
//                sets, bias + act(gate) * up in registers, h kept in LDS (bf16) and fed
//                straight into GEMM2 h @ W_out[g]; + b_out, * gate weight, stored per row.
//   combine      out[t] = sum_j y[inv[t, j]] + sum_s y[shared_s, t], in fp32.
//   expert_bwd   recomputes a1 = x[tok] @ W_in[g] (fp32, in registers) alongside
//                G = dout[tok] @ W_out[g]^T, runs the GLU backward in the epilogue (dA1,
//                the hidden h, the gate gradient), then dA1 @ W_in[g]^T from LDS into
//                per-row dX rows (reduced by `combine`).
//   dw           dW_in[g] = x^T dA1 and dW_out[g] = h^T (w * dout) over the group's rows,
//                split into row chunks of DW_RC; groups with several chunks write fp32
//                partials that dw_reduce sums in chunk order (deterministic, no atomics).
//   bias_grad    per-group column sums for the optional biases.
#include <algorithm>

#include "dw_reduce.h"
#include "experts_common.h"
#include "pack.h"
#include "../../include/nsmoe.h"

namespace nsmoe {

// ============================ forward ====================================================
//
// One workgroup = 4 waves = one 64-row tile of one group.  GEMM1 [64, d] x [d, gate|up]:
// the gathered token rows go through swizzled LDS (shared by the waves), the packed W_in
// fragments come straight from L2 into registers one k-step ahead.  Wave w owns gate
// column blocks [w * NBW, +NBW) and the up blocks at the same columns, so act(gate) * up
// is lane-local.  h (rounded to the element type, as the reference stores it) stays in
// LDS and feeds GEMM2 [64, H] x [H, d] against packed W_out in 192-column passes
// (48 columns per wave); + b_out, * gate weight, then the rows go out through LDS.

template <int DT, int NBW>
__global__ void __launch_bounds__(NT) expert_fwd_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  constexpr int HPMAX = 64 * NBW;
  constexpr int SA = BM * G::ROWB;
  constexpr int HP_PITCH = HPMAX * G::ES + 16;
  constexpr int Y_PITCH = NP2 * G::ES + 16;
  __shared__ __attribute__((aligned(16))) char s_a[2][SA];
  __shared__ __attribute__((aligned(16))) char s_h[BM * HP_PITCH];
  __shared__ __attribute__((aligned(16))) char s_y[BM * Y_PITCH];
  __shared__ int s_tok[BM];
  __shared__ float s_w[BM];
  __shared__ int s_loc[3];

  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + BM - 1) / BM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * BM;
  const int rows = min(BM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  if (tid < BM) {
    int tok = -1, pair;
    float w = 0.0f;
    if (tid < rows) row_info<DT>(p, g, slot0 + tid, m0 + tid, tok, w, pair);
    s_tok[tid] = tok;
    s_w[tid] = w;
  }
  __syncthreads();

  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const bool fast = p.fast;
  const T* X = (const T*)p.x;
  auto rowA = [&](int r) -> const T* {
    const int t = s_tok[r];
    return t >= 0 ? X + (int64_t)t * d : nullptr;
  };
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB;

  // ---- GEMM1 ----
  DirectStage<DT, BM, NT> stA;
  f32x4 accg[4][NBW], accu[4][NBW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) accg[i][j] = accu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  Frag b0[2 * NBW], b1[2 * NBW];
  auto loadB = [&](Frag* b, int kb) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int jb = wave * NBW + j;
      b[j] = frag_pk<DT>(P1, jb, kb, p.in_kb);
      b[NBW + j] = frag_pk<DT>(P1, HPMAX / 16 + jb, kb, p.in_kb);
    }
  };
  const int nk = p.in_kb;
  auto step = [&](int kc, const Frag* use, Frag* nxt) {
    const bool more = kc + 1 < nk;
    if (more) {
      stA.load(rowA, (kc + 1) * G::KC, d, fast);
      loadB(nxt, kc + 1);
    }
    Frag af[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = frag_sw<DT>(s_a[kc & 1], i * 16);
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        M::run(accg[i][j], af[i], use[j]);
        M::run(accu[i][j], af[i], use[NBW + j]);
      }
    if (more) stA.store(s_a[(kc + 1) & 1]);
    __syncthreads();
  };
  stA.load(rowA, 0, d, fast);
  loadB(b0, 0);
  stA.store(s_a[0]);
  __syncthreads();
  for (int kc = 0; kc < nk; kc += 2) {
    step(kc, b0, b1);
    if (kc + 1 < nk) step(kc + 1, b1, b0);
  }

  // ---- GEMM1 epilogue: bias, h = act(gate) * up into LDS ----
  const T* bin = (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int n = (wave * NBW + j) * 16 + lc;
    const bool nv = n < H;
    const float bgv = (nv && bin) ? Elem<DT>::to_f(bin[n]) : 0.0f;
    const float buv = (nv && bin) ? Elem<DT>::to_f(bin[H + n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = i * 16 + lg * 4 + r;
        const float gv = accg[i][j][r] + bgv, uv = accu[i][j][r] + buv;
        const float hv = nv ? act_fwd(gv, p.act) * uv : 0.0f;
        *(T*)(s_h + m * HP_PITCH + n * G::ES) = Elem<DT>::from_f(hv);
      }
  }
  __syncthreads();

  // ---- GEMM2: [BM, H] x [H, d] in passes of NP2 columns, + b_out, * gate ----
  const char* P4 = p.p_out + (int64_t)g * p.out_nb * p.out_kb * G::PKB;
  const T* bout = (g < p.E ? p.b_out : p.b_sh_out)
                      ? per_group<T>(p.b_out, p.b_sh_out, g, p.E, d) : nullptr;
  const int nk2 = p.out_kb;
  T* Y = (T*)p.y;
  for (int n0 = 0; n0 < d; n0 += NP2) {
    f32x4 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nbase = n0 / 16 + wave * 3;
    auto loadB2 = [&](Frag* b, int kb) {
#pragma unroll
      for (int j = 0; j < 3; ++j)
        b[j] = nbase + j < p.out_nb ? frag_pk<DT>(P4, nbase + j, kb, p.out_kb) : M::zero();
    };
    Frag c0[3], c1[3];
    loadB2(c0, 0);
    for (int kk = 0; kk < nk2; ++kk) {
      Frag* use = (kk & 1) ? c1 : c0;
      Frag* nxt = (kk & 1) ? c0 : c1;
      if (kk + 1 < nk2) loadB2(nxt, kk + 1);
      Frag af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = frag_at<DT>(s_h, HP_PITCH, i * 16, kk * G::ROWB);
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) M::run(acc[i][j], af[i], use[j]);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int nl = wave * 48 + j * 16 + lc;
      const int n = n0 + nl;
      const float bo = (bout && n < d) ? Elem<DT>::to_f(bout[n]) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = i * 16 + lg * 4 + r;
          *(T*)(s_y + m * Y_PITCH + nl * G::ES) = Elem<DT>::from_f((acc[i][j][r] + bo) * s_w[m]);
        }
    }
    __syncthreads();
    copy_out<DT>(s_y, Y_PITCH, rows, Y + slot0 * d, d, n0, min(NP2, d - n0), 0, 0, fast);
    __syncthreads();
  }
}

// ============================ combine ====================================================
// out[t] = sum_j rows[inv[t * k + j]] + sum_s rows[l_cap + s * T + t], fp32 accumulation
// in the order routed j = 0 .. k - 1, then shared s = 0 .. S - 1.  With `resid` the sum,
// rounded to the dtype, is added to resid[t] and rounded again: the block output plus the
// residual stream, as `x + ffn(norm(x))` computes it (nanospeaker.py:169).
constexpr int COMBINE_KMAX = 8;  // top_k and shared-expert counts of the gather fast path
constexpr int COMBINE_SMAX = 2;
template <int DT>
__global__ void __launch_bounds__(NT)
combine_kernel(const typename Elem<DT>::T* __restrict__ rows, const int32_t* __restrict__ inv,
               int64_t ntok, int d, int k, int S, int64_t l_cap,
               typename Elem<DT>::T* __restrict__ out, int fast,
               const typename Elem<DT>::T* __restrict__ resid) {
  using G = Geo<DT>;
  using TT = typename G::T;
  // The rounded block output plus the residual, rounded again.
  auto plus_resid = [&](TT (&o)[G::VE], int64_t off) __attribute__((always_inline)) {
    if (!resid) return;
    u32x4 rv = *(const u32x4*)(resid + off);
    TT r[G::VE];
    __builtin_memcpy(r, &rv, 16);
    float sum[G::VE];
#pragma unroll
    for (int e = 0; e < G::VE; ++e) sum[e] = Elem<DT>::to_f(r[e]) + Elem<DT>::to_f(o[e]);
    round_to<DT>(sum, o);
  };
  if (fast && k <= COMBINE_KMAX && S <= COMBINE_SMAX && ntok * (d / G::VE) < INT32_MAX) {
    // Every slot index is loaded first, then every row chunk: all of a thread's loads
    // are in flight together instead of one dependent pair per row.
    const int vpr = d / G::VE;
    const int n = (int)(ntok * vpr);
    for (int i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) {
      const int t = i / vpr;
      const int c = (i - t * vpr) * G::VE;
      int32_t sl[COMBINE_KMAX];
#pragma unroll
      for (int j = 0; j < COMBINE_KMAX; ++j) sl[j] = j < k ? inv[(int64_t)t * k + j] : -1;
      u32x4 v[COMBINE_KMAX + COMBINE_SMAX];
#pragma unroll
      for (int j = 0; j < COMBINE_KMAX; ++j) {
        v[j] = u32x4{0u, 0u, 0u, 0u};
        if (sl[j] >= 0) v[j] = *(const u32x4*)(rows + (int64_t)sl[j] * d + c);
      }
#pragma unroll
      for (int q = 0; q < COMBINE_SMAX; ++q) {
        v[COMBINE_KMAX + q] = u32x4{0u, 0u, 0u, 0u};
        if (q < S) v[COMBINE_KMAX + q] = *(const u32x4*)(rows + (l_cap + (int64_t)q * ntok + t) * d + c);
      }
      float acc[G::VE];
#pragma unroll
      for (int e = 0; e < G::VE; ++e) acc[e] = 0.0f;
#pragma unroll
      for (int j = 0; j < COMBINE_KMAX + COMBINE_SMAX; ++j) {
        TT tmp[G::VE];
        __builtin_memcpy(tmp, &v[j], 16);
#pragma unroll
        for (int e = 0; e < G::VE; ++e) acc[e] += Elem<DT>::to_f(tmp[e]);
      }
      TT o[G::VE];
      round_to<DT>(acc, o);
      plus_resid(o, (int64_t)t * d + c);
      u32x4 ov;
      __builtin_memcpy(&ov, o, 16);
      *(u32x4*)(out + (int64_t)t * d + c) = ov;
    }
  } else if (fast) {
    const int vpr = d / G::VE;
    const int64_t n = ntok * vpr;
    for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
      const int64_t t = i / vpr;
      const int c = (int)(i % vpr) * G::VE;
      float acc[G::VE];
#pragma unroll
      for (int e = 0; e < G::VE; ++e) acc[e] = 0.0f;
      for (int j = 0; j < k; ++j) {
        const int32_t s = inv[t * k + j];
        if (s < 0) continue;
        u32x4 v = *(const u32x4*)(rows + (int64_t)s * d + c);
        TT tmp[G::VE];
        __builtin_memcpy(tmp, &v, 16);
#pragma unroll
        for (int e = 0; e < G::VE; ++e) acc[e] += Elem<DT>::to_f(tmp[e]);
      }
      for (int s = 0; s < S; ++s) {
        u32x4 v = *(const u32x4*)(rows + (l_cap + (int64_t)s * ntok + t) * d + c);
        TT tmp[G::VE];
        __builtin_memcpy(tmp, &v, 16);
#pragma unroll
        for (int e = 0; e < G::VE; ++e) acc[e] += Elem<DT>::to_f(tmp[e]);
      }
      TT o[G::VE];
      round_to<DT>(acc, o);
      plus_resid(o, t * d + c);
      u32x4 ov;
      __builtin_memcpy(&ov, o, 16);
      *(u32x4*)(out + t * d + c) = ov;
    }
  } else {
    const int64_t n = ntok * d;
    for (int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
      const int64_t t = i / d;
      const int c = (int)(i % d);
      float acc = 0.0f;
      for (int j = 0; j < k; ++j) {
        const int32_t s = inv[t * k + j];
        if (s >= 0) acc += Elem<DT>::to_f(rows[(int64_t)s * d + c]);
      }
      for (int s = 0; s < S; ++s)
        acc += Elem<DT>::to_f(rows[(l_cap + (int64_t)s * ntok + t) * d + c]);
      TT o = Elem<DT>::from_f(acc);
      if (resid) o = Elem<DT>::from_f(Elem<DT>::to_f(resid[t * d + c]) + Elem<DT>::to_f(o));
      out[t * d + c] = o;
    }
  }
}

// ============================ backward: recompute, GLU backward, dX rows ==================
//
// Phase 1 runs three GEMMs over the same 64 gathered token rows and K = d in one loop:
//   a1 = x[tok] @ W_in[g]      (gate and up, the forward's pre-activations, recomputed
//                               in fp32 registers instead of being saved and re-read)
//   G  = dout[tok] @ W_out[g]^T
// x and dout rows go through swizzled LDS; packed W_in fragments and the rows of W_out
// (contiguous along d, the contraction index) come straight from L2.  Wave w owns hidden
// columns {(w * NBW + j) * 16 ..}: the gate, up and G accumulators of one (row, column)
// sit in the same lane and register, so the GLU backward is lane-local:
//   h = act(g) * u,  dtopk_w += G * h,  d_gate = w G u act'(g),  d_up = w G act(g).
// dA1 = [d_gate | d_up] goes to LDS (bf16) for phase 3 and to HBM for dW_in; w * h goes
// to HBM for dW_out (= sum (w h)^T dout).  The gate gradient also takes <dout[tok], b_out[g]> when the expert
// has an output bias (the derivative of (h W_out + b_out) * w with respect to w).
// Phase 3: dX rows = dA1 @ W_in[g]^T (W_in's rows are contiguous along 2H, the
// contraction index), in passes of NP2 columns; reduced per token by `combine`.
template <int DT, int NBW>
__global__ void __launch_bounds__(NT) expert_bwd_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  constexpr int HPMAX = 64 * NBW;
  constexpr int SA = BM * G::ROWB;
  constexpr int DA_PITCH = 2 * HPMAX * G::ES + 16;
  constexpr int Y_PITCH = NP2 * G::ES + 16;
  __shared__ __attribute__((aligned(16))) char s_ax[2][SA];
  __shared__ __attribute__((aligned(16))) char s_ad[2][SA];
  __shared__ __attribute__((aligned(16))) char s_da[BM * DA_PITCH];
  __shared__ __attribute__((aligned(16))) char s_y[BM * Y_PITCH];
  __shared__ int s_tok[BM];
  __shared__ int s_pair[BM];
  __shared__ float s_w[BM];
  __shared__ float s_dtw[5][BM];
  __shared__ int s_loc[3];

  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + BM - 1) / BM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * BM;
  const int rows = min(BM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  if (tid < BM) {
    int tok = -1, pair = -1;
    float w = 0.0f;
    if (tid < rows) row_info<DT>(p, g, slot0 + tid, m0 + tid, tok, w, pair);
    s_tok[tid] = tok;
    s_pair[tid] = pair;
    s_w[tid] = w;
    s_dtw[4][tid] = 0.0f;
  }
  __syncthreads();

  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const bool fast = p.fast;
  const T* X = (const T*)p.x;
  const T* DO = (const T*)p.dout;
  const T* Win = per_group<T>(p.w_in, p.w_sh_in, g, p.E, (int64_t)d * twoH);
  const T* Wout = per_group<T>(p.w_out, p.w_sh_out, g, p.E, (int64_t)H * d);
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB;
  auto rowX = [&](int r) -> const T* {
    const int t = s_tok[r];
    return t >= 0 ? X + (int64_t)t * d : nullptr;
  };
  auto rowD = [&](int r) -> const T* {
    const int t = s_tok[r];
    return t >= 0 ? DO + (int64_t)t * d : nullptr;
  };
  auto rowWo = [&](int n) -> const T* { return n < H ? Wout + (int64_t)n * d : nullptr; };

  // ---- phase 1: a1 = x W_in, G = dout W_out^T ----
  DirectStage<DT, BM, NT> stX, stD;
  f32x4 accg[4][NBW], accu[4][NBW], accG[4][NBW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
      accg[i][j] = accu[i][j] = accG[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  Frag b0[3 * NBW], b1[3 * NBW];
  auto loadB = [&](Frag* b, int kb) {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int jb = wave * NBW + j;
      b[j] = frag_pk<DT>(P1, jb, kb, p.in_kb);
      b[NBW + j] = frag_pk<DT>(P1, HPMAX / 16 + jb, kb, p.in_kb);
      b[2 * NBW + j] = frag_rows<DT>(rowWo, jb * 16, kb * G::KC, d, fast);
    }
  };
  const int nk = p.in_kb;
  auto step = [&](int kc, const Frag* use, Frag* nxt) {
    const bool more = kc + 1 < nk;
    if (more) {
      stX.load(rowX, (kc + 1) * G::KC, d, fast);
      stD.load(rowD, (kc + 1) * G::KC, d, fast);
      loadB(nxt, kc + 1);
    }
    Frag ax[4], ad[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      ax[i] = frag_sw<DT>(s_ax[kc & 1], i * 16);
      ad[i] = frag_sw<DT>(s_ad[kc & 1], i * 16);
    }
#pragma unroll
    for (int j = 0; j < NBW; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        M::run(accg[i][j], ax[i], use[j]);
        M::run(accu[i][j], ax[i], use[NBW + j]);
        M::run(accG[i][j], ad[i], use[2 * NBW + j]);
      }
    if (more) {
      stX.store(s_ax[(kc + 1) & 1]);
      stD.store(s_ad[(kc + 1) & 1]);
    }
    __syncthreads();
  };
  stX.load(rowX, 0, d, fast);
  stD.load(rowD, 0, d, fast);
  loadB(b0, 0);
  stX.store(s_ax[0]);
  stD.store(s_ad[0]);
  __syncthreads();
  for (int kc = 0; kc < nk; kc += 2) {
    step(kc, b0, b1);
    if (kc + 1 < nk) step(kc + 1, b1, b0);
  }

  // ---- phase 2: GLU backward, lane-local ----
  const T* bin = (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
  T* HB = (T*)p.hbuf;
  float part[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) part[i][r] = 0.0f;
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int n = (wave * NBW + j) * 16 + lc;
    const bool nv = n < H;
    const float bgv = (nv && bin) ? Elem<DT>::to_f(bin[n]) : 0.0f;
    const float buv = (nv && bin) ? Elem<DT>::to_f(bin[H + n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = i * 16 + lg * 4 + r;
        const bool v = m < rows && nv;
        float dg = 0.0f, du = 0.0f;
        if (v) {
          const float gg = accg[i][j][r] + bgv, uu = accu[i][j][r] + buv;
          const float Gv = accG[i][j][r];
          const float a = act_fwd(gg, p.act);
          const float hv = a * uu;
          part[i][r] += Gv * hv;
          const float dh = s_w[m] * Gv;
          dg = dh * uu * act_bwd(gg, p.act);
          du = dh * a;
          HB[(slot0 + m) * H + n] = Elem<DT>::from_f(s_w[m] * hv);
        }
        *(T*)(s_da + m * DA_PITCH + n * G::ES) = Elem<DT>::from_f(dg);
        *(T*)(s_da + m * DA_PITCH + (HPMAX + n) * G::ES) = Elem<DT>::from_f(du);
      }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = part[i][r];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      v += __shfl_xor(v, 8, 64);
      if (lc == 0) s_dtw[wave][i * 16 + lg * 4 + r] = v;
    }
  // <dout[tok], b_out[g]>: four lanes per row, strided over d.
  if (g < p.E && p.b_out) {
    const T* bo = (const T*)p.b_out + (int64_t)g * d;
    const int m = tid >> 2, q = tid & 3;
    float v = 0.0f;
    if (m < rows) {
      const T* dr = DO + (int64_t)s_tok[m] * d;
      for (int c = q; c < d; c += 4) v += Elem<DT>::to_f(dr[c]) * Elem<DT>::to_f(bo[c]);
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    if (q == 0 && m < rows) s_dtw[4][m] = v;
  }
  __syncthreads();
  if (g < p.E && tid < rows) {
    const float s = s_dtw[0][tid] + s_dtw[1][tid] + s_dtw[2][tid] + s_dtw[3][tid] + s_dtw[4][tid];
    ((T*)p.dtw)[s_pair[tid]] = Elem<DT>::from_f(s);
  }
  copy_out<DT>(s_da, DA_PITCH, rows, (T*)p.da1 + slot0 * twoH, twoH, 0, H, HPMAX, H, fast);

  // ---- phase 3: dX rows = dA1 @ W_in[g]^T in passes of NP2 columns ----
  // k chunk q: half = q / nkh (0 gate, 1 up); LDS columns half * HPMAX + kk, source
  // columns half * H + kk of W_in's rows.
  const int nkh = (H + G::KC - 1) / G::KC;
  const int nk3 = 2 * nkh;
  auto rowWi = [&](int n) -> const T* { return n < d ? Win + (int64_t)n * twoH : nullptr; };
  T* DX = (T*)p.dxrow;
  for (int n0 = 0; n0 < d; n0 += NP2) {
    f32x4 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int nw = n0 + wave * 48;
    auto loadB3 = [&](Frag* b, int q) {
      const int half = q / nkh, kk = (q % nkh) * G::KC;
#pragma unroll
      for (int j = 0; j < 3; ++j)
        b[j] = frag_rows<DT>(rowWi, nw + j * 16, half * H + kk, half * H + H, fast);
    };
    Frag c0[3], c1[3];
    loadB3(c0, 0);
    for (int q = 0; q < nk3; ++q) {
      Frag* use = (q & 1) ? c1 : c0;
      Frag* nxt = (q & 1) ? c0 : c1;
      if (q + 1 < nk3) loadB3(nxt, q + 1);
      const int half = q / nkh, kk = (q % nkh) * G::KC;
      const int kbyte = (half * HPMAX + kk) * G::ES;
      Frag af[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = frag_at<DT>(s_da, DA_PITCH, i * 16, kbyte);
#pragma unroll
      for (int j = 0; j < 3; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) M::run(acc[i][j], af[i], use[j]);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int nl = wave * 48 + j * 16 + lc;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = i * 16 + lg * 4 + r;
          *(T*)(s_y + m * Y_PITCH + nl * G::ES) = Elem<DT>::from_f(acc[i][j][r]);
        }
    }
    __syncthreads();
    copy_out<DT>(s_y, Y_PITCH, rows, DX + slot0 * d, d, n0, min(NP2, d - n0), 0, 0, fast);
    __syncthreads();
  }
}

// ============================ backward: dW ===============================================
// MODE 0: dW_in[g]  [d, 2H] = sum_r x[tok_r]^T dA1[slot_r]
// MODE 1: dW_out[g] [H, d]  = sum_r (w_r h[slot_r])^T dout[tok_r]   (the backward stores
//                                                                     w * h per row)
// The contraction runs over the group's rows, which are contiguous along the output
// index in memory, so both operands are staged transposed (TransStage) into swizzled
// LDS: KCH chunks of 32 rows per barrier, the A and B chunks of a stage staged by
// disjoint thread ranges so every wave shares the transposes.  The row -> token lookups
// of the work item's rows are read once into LDS.  Tile BMo x BNo =
// (WGM * TM * 16) x (WGN * TN * 16).

template <int MODE> struct DwShape;
template <> struct DwShape<0> {  // dW_in: 64 x 128 tiles, waves side by side along N
  static constexpr int WGM = 1, WGN = 4, TM = 4, TN = 2;
};
template <> struct DwShape<1> {  // dW_out: 128 x 64 tiles, waves stacked along M
  static constexpr int WGM = 4, WGN = 1, TM = 2, TN = 4;
};

// Transposed staging of one dW stage: KCH chunks of the A tile (BMA columns) and of the
// B tile (BNB columns), VE x VE blocks spread over the workgroup's threads (a thread keeps
// registers for its own PER blocks only).  Same transpose, rotation and swizzle as
// TransStage.
template <int DT, int BMA, int BNB, int KCH>
struct DwStager {
  using G = Geo<DT>;
  using T = typename G::T;
  static constexpr int VE = G::VE;
  static constexpr int KB = G::KC / VE;
  static constexpr int NBA = KB * (BMA / VE), NBB = KB * (BNB / VE);
  static constexpr int TOT = KCH * (NBA + NBB);
  static constexpr int PER = (TOT + NT - 1) / NT;
  static constexpr int TA = BMA * G::ROWB, TB = BNB * G::ROWB;
  u32x4 v[PER][VE];

  struct Role {
    bool on, is_a;
    int q, kb, nb;
  };
  __device__ __forceinline__ static Role role(int i) {
    const int b = (int)threadIdx.x + i * NT;
    Role r{b < TOT, false, 0, 0, 0};
    if (!r.on) return r;
    int blk;
    if (b < KCH * NBA) {
      r.is_a = true;
      r.q = b / NBA;
      blk = b % NBA;
    } else {
      const int b2 = b - KCH * NBA;
      r.q = b2 / NBB;
      blk = b2 % NBB;
    }
    r.kb = blk % KB;
    r.nb = blk / KB;
    return r;
  }

  template <class RowA, class RowB>
  __device__ __forceinline__ void load(RowA rowA, RowB rowB, int k0, int klim, int m0, int Md,
                                       int n0, int Nd, bool fast) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const Role ro = role(i);
      const int col = (ro.is_a ? m0 : n0) + ro.nb * VE;
      const int lim = ro.is_a ? Md : Nd;
#pragma unroll
      for (int r = 0; r < VE; ++r) {
        v[i][r] = u32x4{0u, 0u, 0u, 0u};
        const int k = k0 + ro.q * G::KC + ro.kb * VE + r;
        if (!ro.on || k >= klim) continue;
        const T* src = ro.is_a ? rowA(k) : rowB(k);
        T tmp[VE];
        if (fast) {
          if (col < lim) {
            u32x4 raw = *(const u32x4*)(src + col);
            __builtin_memcpy(tmp, &raw, 16);
          } else {
#pragma unroll
            for (int e = 0; e < VE; ++e) tmp[e] = T(0);
          }
        } else {
#pragma unroll
          for (int e = 0; e < VE; ++e) tmp[e] = (col + e < lim) ? src[col + e] : T(0);
        }
        __builtin_memcpy(&v[i][r], tmp, 16);
      }
    }
  }

  __device__ __forceinline__ void store(char* stage) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const Role ro = role(i);
      if (!ro.on) continue;
      char* tile = stage + (ro.is_a ? ro.q * TA : KCH * TA + ro.q * TB);
      if constexpr (G::ES == 2) {
        store_trans8<DT>(v[i], tile, ro.nb, ro.kb);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4 o{v[i][0][c], v[i][1][c], v[i][2][c], v[i][3][c]};
          *(u32x4*)(tile + sw_off<DT>(ro.nb * 4 + c, ro.kb)) = o;
        }
      }
    }
  }
};

template <int DT, int MODE>
__global__ void __launch_bounds__(NT) dw_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using Mm = Mma<DT>;
  using S = DwShape<MODE>;
  constexpr int BMo = S::WGM * S::TM * 16, BNo = S::WGN * S::TN * 16;
  constexpr int KCH = 2;  // 32-row chunks per stage
  using Stager = DwStager<DT, BMo, BNo, KCH>;
  constexpr int TA = Stager::TA, TB = Stager::TB;
  constexpr int STAGE = KCH * (TA + TB);
  __shared__ __attribute__((aligned(16))) char s_stage[2][STAGE];
  __shared__ int s_tok[DW_RC];
  __shared__ int s_loc[3];

  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const int Md = MODE == 0 ? d : H;
  const int Nd = MODE == 0 ? twoH : d;
  const int tn = (Nd + BNo - 1) / BNo, ntiles = ((Md + BMo - 1) / BMo) * tn;
  const int item = xcd_remap(blockIdx.x, gridDim.x);
  Located loc;
  if (!locate(item, p.E + p.S, [&](int g) { return dw_chunks(rows_of(p, g)) * ntiles; },
              [&](int g) {
                const int c = dw_chunks(rows_of(p, g));
                return c > 1 ? c : 0;
              },
              s_loc, loc))
    return;
  const int g = loc.g;
  const int rows_g = rows_of(p, g);
  const int nch = dw_chunks(rows_g);
  const int chunk = loc.local / ntiles, t = loc.local % ntiles;
  const int m0 = (t / tn) * BMo, n0 = (t % tn) * BNo;
  const int r0 = chunk * DW_RC, r1 = min(rows_g, r0 + DW_RC);
  const int64_t rs = row_start(p, g);
  const bool fast = p.fast;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wm = wave / S::WGN, wn = wave % S::WGN;

  for (int r = r0 + tid; r < r1; r += NT)
    s_tok[r - r0] = g < p.E ? p.sorted_ids[rs + r] / p.k : r;
  __syncthreads();

  const T* X = (const T*)p.x;
  const T* DA = (const T*)p.da1;
  const T* HB = (const T*)p.hbuf;
  const T* DO = (const T*)p.dout;
  auto rowA = [&](int r) -> const T* {
    if (MODE == 0) return X + (int64_t)s_tok[r - r0] * d;
    return HB + (rs + r) * H;
  };
  auto rowB = [&](int r) -> const T* {
    if (MODE == 0) return DA + (rs + r) * twoH;
    return DO + (int64_t)s_tok[r - r0] * d;
  };

  Stager stg;
  auto load = [&](int k0) { stg.load(rowA, rowB, k0, r1, m0, Md, n0, Nd, fast); };
  auto store = [&](int b) { stg.store(s_stage[b]); };
  f32x4 acc[S::TM][S::TN];
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int KS = KCH * G::KC;
  const int ns = (r1 - r0 + KS - 1) / KS;
  if (ns > 0) {
    load(r0);
    store(0);
    __syncthreads();
    for (int st = 0; st < ns; ++st) {
      const int cur = st & 1;
      const bool more = st + 1 < ns;
      if (more) load(r0 + (st + 1) * KS);
#pragma unroll
      for (int q = 0; q < KCH; ++q) {
        const char* ta = s_stage[cur] + q * TA;
        const char* tb = s_stage[cur] + KCH * TA + q * TB;
        typename Mm::Frag af[S::TM], bf[S::TN];
#pragma unroll
        for (int i = 0; i < S::TM; ++i) af[i] = frag_sw<DT>(ta, (wm * S::TM + i) * 16);
#pragma unroll
        for (int j = 0; j < S::TN; ++j) bf[j] = frag_sw<DT>(tb, (wn * S::TN + j) * 16);
#pragma unroll
        for (int i = 0; i < S::TM; ++i)
#pragma unroll
          for (int j = 0; j < S::TN; ++j) Mm::run(acc[i][j], af[i], bf[j]);
      }
      if (more) store(cur ^ 1);
      __syncthreads();
    }
  }
  const int64_t mn = (int64_t)Md * Nd;
  T* dst = nullptr;
  float* pdst = nullptr;
  if (nch == 1) {
    dst = g < p.E ? (T*)p.dw_a + (int64_t)g * mn : (T*)p.dw_sh + (int64_t)(g - p.E) * mn;
  } else {
    pdst = p.partial + (int64_t)(loc.aux + chunk) * mn;
  }
#pragma unroll
  for (int i = 0; i < S::TM; ++i)
#pragma unroll
    for (int j = 0; j < S::TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + (wm * S::TM + i) * 16 + lg * 4 + r;
        const int n = n0 + (wn * S::TN + j) * 16 + lc;
        if (m < Md && n < Nd) {
          if (dst) dst[(int64_t)m * Nd + n] = Elem<DT>::from_f(acc[i][j][r]);
          else pdst[(int64_t)m * Nd + n] = acc[i][j][r];
        }
      }
}

// The dW split-K reduce (dw_reduce.h): one group per grid row, or both modes over the
// multi-chunk groups in one launch.  grid = (dwr_blocks, rows).
template <int DT, int MODE>
__global__ void __launch_bounds__(NT) dw_reduce_kernel(ExpParams p) {
  dw_reduce_group<DT, MODE>(p, blockIdx.y, blockIdx.x, gridDim.x);
}

template <int DT>
__global__ void __launch_bounds__(NT) dw_reduce_pair_kernel(DwReduceArgs r) {
  dw_reduce_pair_row<DT>(r, blockIdx.x, blockIdx.y);
}

// Rows of routed groups in dw_reduce_pair_kernel's grid: one per routed group when an
// average routed group comes near a chunk (many of them then have several), else one row
// for all of them.
static int dw_reduce_routed_rows(const nsmoe_experts_args* a) {
  return a->n_tokens * a->top_k > (int64_t)a->n_experts * (DW_RC * 9 / 10) ? a->n_experts : 1;
}

// Workgroups per group of the dW reduce: one 16-byte vector of the larger dW per thread,
// so every thread issues its chunk loads once.
static unsigned dwr_blocks(const nsmoe_experts_args* a) {
  const int64_t big = (int64_t)a->d_model * 2 * a->d_hidden;  // dW_in, the larger of the two
  return (unsigned)std::min<int64_t>(cdiv(cdiv(big, 4), NT), 1024);
}

// Bias gradients: WHICH 0 -> db_in[g] = sum_r dA1[slot_r]; 1 -> db_out[g] = sum_r w_r dout[tok_r].
template <int DT, int WHICH>
__global__ void __launch_bounds__(NT) bias_grad_kernel(ExpParams p) {
  using T = typename Elem<DT>::T;
  const int g = blockIdx.y;
  T* dst = g < p.E ? (T*)p.db : (T*)p.db_sh;
  if (!dst) return;
  const int ncols = WHICH == 0 ? 2 * p.H : p.d;
  const int col = blockIdx.x * NT + threadIdx.x;
  if (col >= ncols) return;
  const int rows = rows_of(p, g);
  const int64_t rs = row_start(p, g);
  float s = 0.0f;
  for (int r = 0; r < rows; ++r) {
    if (WHICH == 0) {
      s += Elem<DT>::to_f(((const T*)p.da1)[(rs + r) * ncols + col]);
    } else {
      int tok, pair;
      float w;
      row_info<DT>(p, g, rs + r, r, tok, w, pair);
      s += w * Elem<DT>::to_f(((const T*)p.dout)[(int64_t)tok * p.d + col]);
    }
  }
  dst[(int64_t)(g < p.E ? g : g - p.E) * ncols + col] = Elem<DT>::from_f(s);
}

// ============================ host side ==================================================

static int elem_size(int dt) { return dt == DT_F32 ? 4 : 2; }

static size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

static int64_t rows_total(const nsmoe_experts_args* a) {
  return a->l_cap + (int64_t)a->n_shared * a->n_tokens;
}

static int nbw_for(const nsmoe_experts_args* a) {
  const int hp = (a->d_hidden + 15) / 16 * 16;
  if (hp <= 64) return 1;
  if (hp <= 128) return 2;
  return 4;
}

static int validate_dims(const nsmoe_experts_args* a) {
  NSMOE_REQUIRE(a, "experts: NULL args");
  NSMOE_REQUIRE(a->dtype == DT_BF16 || a->dtype == DT_F16 || a->dtype == DT_F32,
                "experts: unknown dtype %d", a->dtype);
  NSMOE_REQUIRE(a->activation >= 0 && a->activation <= 4, "experts: unknown activation %d",
                a->activation);
  NSMOE_REQUIRE(a->n_tokens >= 0 && a->d_model >= 1 && a->d_hidden >= 1 && a->n_experts >= 1 &&
                    a->n_shared >= 0 && a->top_k >= 1 && a->top_k <= a->n_experts,
                "experts: bad dimensions");
  NSMOE_REQUIRE(a->d_hidden <= (a->dtype == DT_F32 ? 128 : 256),
                "experts: d_hidden %d above the kernel limit", a->d_hidden);
  NSMOE_REQUIRE(a->n_experts + a->n_shared <= 1024, "experts: too many groups");
  NSMOE_REQUIRE(a->n_tokens * a->top_k < (int64_t)INT32_MAX / 2 &&
                    rows_total(a) < (int64_t)INT32_MAX / 2,
                "experts: too many rows");
  return NSMOE_OK;
}

static int validate(const nsmoe_experts_args* a) {
  NSMOE_TRY(validate_dims(a));
  NSMOE_REQUIRE(a->n_shared == 0 || (a->w_sh_in && a->w_sh_out),
                "experts: shared weights missing");
  return NSMOE_OK;
}

static bool aligned16(const void* q) { return ((uintptr_t)q & 15u) == 0; }

static ExpParams make_params(const nsmoe_experts_args* a) {
  ExpParams p{};
  p.x = a->x;
  p.w_in = a->w_in;
  p.w_out = a->w_out;
  p.b_in = a->b_in;
  p.b_out = a->b_out;
  p.w_sh_in = a->w_sh_in;
  p.w_sh_out = a->w_sh_out;
  p.b_sh_in = a->b_sh_in;
  p.b_sh_out = a->b_sh_out;
  p.topk_w = a->topk_w;
  p.sorted_ids = a->sorted_ids;
  p.offs = a->pad_offsets;
  p.counts = a->counts;
  p.p_in = (const char*)a->w_in_packed;
  p.p_out = (const char*)a->w_out_packed;
  const PackGeom pg = pack_geom(a->dtype, a->d_model, a->d_hidden, a->n_experts, a->n_shared);
  p.in_kb = pg.in_kb;
  p.in_nb = pg.in_nb;
  p.out_kb = pg.out_kb;
  p.out_nb = pg.out_nb;
  p.T = a->n_tokens;
  p.l_cap = a->l_cap;
  p.d = a->d_model;
  p.H = a->d_hidden;
  p.E = a->n_experts;
  p.S = a->n_shared;
  p.k = a->top_k;
  p.act = a->activation;
  // Weight fragments and staged rows read 8 (2-byte types) or 4..8 (fp32) contiguous
  // elements per lane: the vector paths need d and H to be multiples of 8.
  p.fast = (a->d_model % 8 == 0) && (a->d_hidden % 8 == 0) && aligned16(a->x) &&
           aligned16(a->w_in) && aligned16(a->w_out) &&
           (a->n_shared == 0 || (aligned16(a->w_sh_in) && aligned16(a->w_sh_out)));
  const int64_t run = option(OPT_XCD_RUN);
  p.xcd_run = run ? (int)run : XCD_RUN;
  return p;
}

static int64_t fwd_grid(const nsmoe_experts_args* a) {
  const int64_t M = a->n_tokens * a->top_k;
  const int64_t nonempty = M < a->n_experts ? M : a->n_experts;
  return cdiv(M, BM) + nonempty + (int64_t)a->n_shared * cdiv(a->n_tokens, BM);
}

static int64_t dw_groups_chunks(const nsmoe_experts_args* a) {
  const int64_t M = a->n_tokens * a->top_k;
  return a->n_experts + cdiv(M, DW_RC) + (int64_t)a->n_shared * (cdiv(a->n_tokens, DW_RC) + 1);
}

static int64_t dw_partial_chunks(const nsmoe_experts_args* a) {
  const int64_t M = a->n_tokens * a->top_k;
  return 2 * cdiv(M, DW_RC) + 1 + (int64_t)a->n_shared * (cdiv(a->n_tokens, DW_RC) + 1);
}

template <int DT>
static int launch_fwd_tiles(const ExpParams& p, int nbw, int64_t grid, hipStream_t s) {
  if (grid <= 0) return NSMOE_OK;
  const int rc = launch_fwd_async(DT, p, nbw, grid, s);
  if (rc != -1) return rc;
  KernelTimer timer("expert_fwd", s);
  if (nbw == 1) expert_fwd_kernel<DT, 1><<<(unsigned)grid, NT, 0, s>>>(p);
  else if (nbw == 2) expert_fwd_kernel<DT, 2><<<(unsigned)grid, NT, 0, s>>>(p);
  else if constexpr (DT != DT_F32) expert_fwd_kernel<DT, 4><<<(unsigned)grid, NT, 0, s>>>(p);
  timer.stop();
  return check_launch("expert_fwd_kernel");
}

template <int DT>
static int launch_combine(const void* rows, const int32_t* inv, int64_t T, int d, int k, int S,
                          int64_t l_cap, void* out, bool fast, hipStream_t s,
                          const void* resid = nullptr) {
  using TT = typename Elem<DT>::T;
  if (T <= 0) return NSMOE_OK;
  const int ve = 16 / (int)sizeof(TT);
  const int64_t work = fast ? T * (d / ve) : T * d;
  int64_t blocks = cdiv(work, NT);
  if (blocks > 65535) blocks = 65535;
  KernelTimer timer("combine", s);
  combine_kernel<DT><<<(unsigned)blocks, NT, 0, s>>>((const TT*)rows, inv, T, d, k, S, l_cap,
                                                      (TT*)out, fast ? 1 : 0,
                                                      (const TT*)resid);
  timer.stop();
  return check_launch("combine_kernel");
}

// Whether the register-tiled forward and backward both take this shape (launch_fwd_async,
// launch_bwd_async): the pre-activations are then saved by the one and read by the other.
static bool save_act_shape(const nsmoe_experts_args* a) {
  if (a->dtype != DT_BF16 && a->dtype != DT_F16) return false;
  const int d = a->d_model, H = a->d_hidden;
  if (nbw_for(a) > 2 || d % 64 != 0 || H % 16 != 0) return false;
  const PackGeom pg = pack_geom(a->dtype, d, H, a->n_experts, a->n_shared);
  const int npass = (d + NP2 - 1) / NP2;
  return (npass * pg.out_kb) % 2 == 0 && (npass * (2 * H / 32)) % 2 == 0 && pg.in_kb >= 4;
}

template <int DT>
static int experts_fwd_impl(const nsmoe_experts_args* a, const int32_t* inv, void* out, void* ws,
                            void* act_out, const void* resid, hipStream_t s) {
  ExpParams p = make_params(a);
  p.y = ws;
  // Saved only where the forward kernel that writes them runs (which needs p.fast); the
  // backward's decision (experts_bwd_impl) is the same function of the same arguments.
  p.a1_out = act_out && p.fast && save_act_shape(a) ? act_out : nullptr;
  const bool fast = p.fast && aligned16(out) && aligned16(resid);
  NSMOE_TRY(launch_fwd_tiles<DT>(p, nbw_for(a), fwd_grid(a), s));
  return launch_combine<DT>(ws, inv, a->n_tokens, a->d_model, a->top_k, a->n_shared, a->l_cap,
                            out, fast, s, resid);
}

struct BwdLayout {
  size_t da1, hbuf, dxrow, p_in, p_out, total;
};

static BwdLayout bwd_layout(const nsmoe_experts_args* a) {
  const size_t es = elem_size(a->dtype);
  const size_t rt = (size_t)rows_total(a);
  const size_t d = a->d_model, H = a->d_hidden;
  const size_t pc = (size_t)dw_partial_chunks(a);
  BwdLayout L;
  size_t off = 0;
  L.da1 = off;
  off += align256(rt * 2 * H * es);
  L.hbuf = off;
  off += align256(rt * H * es);
  L.dxrow = off;
  off += align256(rt * d * es);
  L.p_in = off;
  off += align256(pc * d * 2 * H * 4);
  L.p_out = off;
  off += align256(pc * H * d * 4);
  L.total = off;
  return L;
}

// dW_in / dW_out (and the bias gradients) of every group from the backward's dA1 and w h
// rows, on stream s.
template <int DT>
static int experts_dw(const nsmoe_experts_args* a, const ExpParams& p,
                      const nsmoe_experts_grads* gr, char* ws, const BwdLayout& L,
                      hipStream_t s, DwReduceArgs* defer) {
  const int G = a->n_experts + a->n_shared;
  const int d = a->d_model, H = a->d_hidden;
  const int64_t gc = dw_groups_chunks(a);
  ExpParams q_in = p, q_out = p;
  q_in.dw_a = gr->dw_in;
  q_in.dw_sh = gr->dw_sh_in;
  q_in.partial = (float*)(ws + L.p_in);
  q_out.dw_a = gr->dw_out;
  q_out.dw_sh = gr->dw_sh_out;
  q_out.partial = (float*)(ws + L.p_out);
  const int prc = launch_dw_pair_async(DT, q_in, q_out, gc, s);
  if (prc != -1) {
    NSMOE_TRY(prc);
    const int rr = dw_reduce_routed_rows(a);
    const DwReduceArgs r{q_in, q_out, rr, (int)dwr_blocks(a), 2 * (a->n_shared + rr)};
    if (defer) {  // the caller's later launch runs it
      *defer = r;
    } else {
      dw_reduce_pair_kernel<DT><<<dim3((unsigned)r.nbx, (unsigned)r.rows), NT, 0, s>>>(r);
      NSMOE_TRY(check_launch("dw_reduce_pair_kernel"));
    }
  } else {
    {  // dW_in
      const ExpParams& q = q_in;
      const int64_t ntiles = cdiv(d, 64) * cdiv(2 * H, 128);
      KernelTimer timer("dw_in", s);
      dw_kernel<DT, 0><<<(unsigned)(gc * ntiles), NT, 0, s>>>(q);
      timer.stop();
      NSMOE_TRY(check_launch("dw_kernel<in>"));
      dim3 rg(dwr_blocks(a), (unsigned)G);
      dw_reduce_kernel<DT, 0><<<rg, NT, 0, s>>>(q);
      NSMOE_TRY(check_launch("dw_reduce_kernel<in>"));
    }
    {  // dW_out
      const ExpParams& q = q_out;
      const int64_t ntiles = cdiv(H, 128) * cdiv(d, 64);
      KernelTimer timer("dw_out", s);
      dw_kernel<DT, 1><<<(unsigned)(gc * ntiles), NT, 0, s>>>(q);
      timer.stop();
      NSMOE_TRY(check_launch("dw_kernel<out>"));
      dim3 rg(dwr_blocks(a), (unsigned)G);
      dw_reduce_kernel<DT, 1><<<rg, NT, 0, s>>>(q);
      NSMOE_TRY(check_launch("dw_reduce_kernel<out>"));
    }
  }
  if (gr->db_in || gr->db_sh_in) {
    ExpParams q = p;
    q.db = gr->db_in;
    q.db_sh = gr->db_sh_in;
    dim3 bg((unsigned)cdiv(2 * H, NT), (unsigned)G);
    bias_grad_kernel<DT, 0><<<bg, NT, 0, s>>>(q);
    NSMOE_TRY(check_launch("bias_grad_kernel<in>"));
  }
  if (gr->db_out || gr->db_sh_out) {
    ExpParams q = p;
    q.db = gr->db_out;
    q.db_sh = gr->db_sh_out;
    dim3 bg((unsigned)cdiv(d, NT), (unsigned)G);
    bias_grad_kernel<DT, 1><<<bg, NT, 0, s>>>(q);
    NSMOE_TRY(check_launch("bias_grad_kernel<out>"));
  }
  return NSMOE_OK;
}

// combine = false leaves the per-row dX in the workspace (bwd_layout(a).dxrow) for the
// caller to reduce, and gr->dx is not written.  dW runs on the calling thread's side stream
// (forked after the GLU backward) beside the dX rows on s; with side_out the caller gets
// that stream and must join it (side_join(s, *side_out, kSideSlotDw)), else it is joined
// here.
template <int DT>
static int experts_bwd_impl(const nsmoe_experts_args* a, const int32_t* inv, const void* dout,
                            const nsmoe_experts_grads* gr, char* ws, bool combine,
                            hipStream_t s, hipStream_t* side_out, const void* act_in,
                            DwReduceArgs* defer) {
  const BwdLayout L = bwd_layout(a);
  ExpParams p = make_params(a);
  // The forward wrote them under the same condition (p.fast here before dout's alignment
  // is folded in); a backward that then takes another kernel recomputes them instead.
  p.a1_in = act_in && p.fast && save_act_shape(a) ? act_in : nullptr;
  const int nbw = nbw_for(a);
  const int64_t grid = fwd_grid(a);
  p.dout = dout;
  p.da1 = ws + L.da1;
  p.hbuf = ws + L.hbuf;
  p.dxrow = ws + L.dxrow;
  p.dtw = gr->dtopk_w;
  p.fast = p.fast && aligned16(dout);
  const int arc = launch_bwd_async(DT, p, nbw, grid, 0, s);
  if (arc != -1) {
    NSMOE_TRY(arc);
  } else if (grid > 0) {
    KernelTimer timer("expert_bwd", s);
    if (nbw == 1) expert_bwd_kernel<DT, 1><<<(unsigned)grid, NT, 0, s>>>(p);
    else if (nbw == 2) expert_bwd_kernel<DT, 2><<<(unsigned)grid, NT, 0, s>>>(p);
    else if constexpr (DT != DT_F32) expert_bwd_kernel<DT, 4><<<(unsigned)grid, NT, 0, s>>>(p);
    timer.stop();
    NSMOE_TRY(check_launch("expert_bwd_kernel"));
  }
  hipStream_t s2 = side_fork(s, kSideSlotDw);
  // The reduce is handed to the caller only while dW runs on s itself (its partials are
  // then complete before any later launch on s).
  if (defer) defer->nbx = 0;
  int rc = experts_dw<DT>(a, p, gr, ws, L, s2, s2 == s ? defer : nullptr);
  if (rc == NSMOE_OK && arc != -1) rc = launch_bwd_async(DT, p, nbw, grid, 1, s);
  if (rc == NSMOE_OK && combine)
    rc = launch_combine<DT>(ws + L.dxrow, inv, a->n_tokens, a->d_model, a->top_k, a->n_shared,
                            a->l_cap, gr->dx, p.fast && aligned16(gr->dx), s);
  if (rc == NSMOE_OK && side_out) {
    *side_out = s2;
    return NSMOE_OK;
  }
  const int jrc = side_join(s, s2, kSideSlotDw);  // joined on every other path
  NSMOE_TRY(rc);
  return jrc;
}

}  // namespace nsmoe

using namespace nsmoe;

extern "C" size_t nsmoe_experts_fwd_workspace_size(const nsmoe_experts_args* a) {
  if (!a) return 0;
  return align256((size_t)rows_total(a) * a->d_model * elem_size(a->dtype));
}

extern "C" int nsmoe_experts_fwd(const nsmoe_experts_args* a, const int32_t* inv, void* out,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return experts_fwd_launch(a, inv, out, workspace, workspace_bytes, nullptr,
                            (hipStream_t)stream);
}

namespace nsmoe {

size_t experts_save_act_bytes(const nsmoe_experts_args* a) {
  if (!a || !save_act_shape(a)) return 0;
  // act_block's row blocks: the dispatch's l_cap rows (a multiple of 16), then each shared
  // group's T rows rounded up to 16.
  const int64_t rows = a->l_cap + (int64_t)a->n_shared * cdiv(a->n_tokens, 16) * 16;
  return (size_t)rows * 2 * a->d_hidden * elem_size(a->dtype);
}

int experts_fwd_launch(const nsmoe_experts_args* a, const int32_t* inv, void* out,
                       void* workspace, size_t workspace_bytes, void* act_out, hipStream_t s,
                       const void* resid) {
  NSMOE_TRY(validate(a));
  if (a->n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(a->x && a->w_in && a->w_out && a->topk_w && a->sorted_ids && a->pad_offsets &&
                    a->counts && inv && out, "experts_fwd: NULL pointer");
  NSMOE_REQUIRE(a->w_in_packed && a->w_out_packed,
                "experts_fwd: packed weights missing (nsmoe_pack_weights)");
  const size_t need = nsmoe_experts_fwd_workspace_size(a);
  if (workspace_bytes < need || !workspace) {
    set_error("experts_fwd: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  switch (a->dtype) {
    case DT_BF16: return experts_fwd_impl<DT_BF16>(a, inv, out, workspace, act_out, resid, s);
    case DT_F16: return experts_fwd_impl<DT_F16>(a, inv, out, workspace, act_out, resid, s);
    default: return experts_fwd_impl<DT_F32>(a, inv, out, workspace, act_out, resid, s);
  }
}

}  // namespace nsmoe

extern "C" size_t nsmoe_experts_bwd_workspace_size(const nsmoe_experts_args* a) {
  if (!a) return 0;
  return bwd_layout(a).total;
}

namespace nsmoe {

int experts_bwd_launch(const nsmoe_experts_args* a, const int32_t* inv, const void* grad_out,
                       const nsmoe_experts_grads* grads, void* workspace,
                       size_t workspace_bytes, bool combine, hipStream_t s,
                       hipStream_t* side_out, const void* act_in, DwReduceArgs* defer) {
  NSMOE_TRY(validate(a));
  NSMOE_REQUIRE(grads, "experts_bwd: NULL grads");
  if (a->n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(a->x && a->w_in && a->w_out && a->topk_w && a->sorted_ids && a->pad_offsets &&
                    a->counts && inv && grad_out && (grads->dx || !combine) &&
                    grads->dw_in && grads->dw_out && grads->dtopk_w,
                "experts_bwd: NULL pointer");
  NSMOE_REQUIRE(a->n_shared == 0 || (grads->dw_sh_in && grads->dw_sh_out),
                "experts_bwd: shared weight gradients missing");
  NSMOE_REQUIRE(a->w_in_packed, "experts_bwd: packed W_in missing (nsmoe_pack_weights)");
  const size_t need = bwd_layout(a).total;
  if (workspace_bytes < need || !workspace) {
    set_error("experts_bwd: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  switch (a->dtype) {
    case DT_BF16:
      return experts_bwd_impl<DT_BF16>(a, inv, grad_out, grads, (char*)workspace, combine, s,
                                       side_out, act_in, defer);
    case DT_F16:
      return experts_bwd_impl<DT_F16>(a, inv, grad_out, grads, (char*)workspace, combine, s,
                                       side_out, act_in, defer);
    default:
      return experts_bwd_impl<DT_F32>(a, inv, grad_out, grads, (char*)workspace, combine, s,
                                       side_out, act_in, defer);
  }
}

size_t experts_bwd_dxrows_offset(const nsmoe_experts_args* a) { return bwd_layout(a).dxrow; }

}  // namespace nsmoe

extern "C" int nsmoe_experts_bwd(const nsmoe_experts_args* a, const int32_t* inv,
                                 const void* grad_out, const nsmoe_experts_grads* grads,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return experts_bwd_launch(a, inv, grad_out, grads, workspace, workspace_bytes, true,
                            (hipStream_t)stream, nullptr);
}

extern "C" int nsmoe_pack_sizes(const nsmoe_experts_args* a, size_t* w_in_bytes,
                                size_t* w_out_bytes) {
  NSMOE_TRY(validate_dims(a));
  NSMOE_REQUIRE(w_in_bytes && w_out_bytes, "pack_sizes: NULL output");
  const PackGeom pg = pack_geom(a->dtype, a->d_model, a->d_hidden, a->n_experts, a->n_shared);
  *w_in_bytes = pg.in_bytes;
  *w_out_bytes = pg.out_bytes;
  return NSMOE_OK;
}

extern "C" int nsmoe_pack_weights(const nsmoe_experts_args* a, void* w_in_packed,
                                  void* w_out_packed, void* stream) {
  NSMOE_TRY(validate(a));
  NSMOE_REQUIRE(a->w_in && w_in_packed, "pack_weights: NULL W_in or destination");
  NSMOE_REQUIRE(!w_out_packed || a->w_out, "pack_weights: NULL W_out");
  NSMOE_REQUIRE(a->n_shared == 0 || (a->w_sh_in && (!w_out_packed || a->w_sh_out)),
                "pack_weights: shared weights missing");
  return pack_weights(a->dtype, a->w_in, w_out_packed ? a->w_out : nullptr, a->w_sh_in,
                      a->w_sh_out, a->n_experts, a->n_shared, a->d_model, a->d_hidden,
                      w_in_packed, w_out_packed, (hipStream_t)stream);
}

// The router GEMM's backward, fused into the block's backward (16-bit types).
//
// Reference: TopKRouter.forward computes logits = x @ W (src/model/router.py:69); its
// backward is dx += d(logits) W^T and dW = x^T d(logits) (torch autograd).  Here:
//
//   combine_dx_kernel   dx[t] = sum_j rows[inv[t, j]] + sum_s rows[shared_s, t]
//                               + d(logits)[t] W^T
//     The expert half is the combine of the expert backward's dX rows (the reference's
//     index_add_ over the routed and shared experts, moe.py:395-418); the router half is
//     one MFMA pass per 16-token x 64-column tile, staged through LDS and added in the
//     same fp32 sum, so dx is written once.
//   router_dw_kernel    fp32 partials of x^T d(logits) over chunks of RDW_RC tokens
//                       (split over tokens: the output is only d x E)
//   router dW reduce    the partials summed in chunk order -> W.grad in the module dtype,
//                       as extra workgroups of the combine_dx launch that follows
//                       router_dw_kernel
//
// d(logits) arrives from route_bwd with a row pitch `ep` = E rounded up to 8 (16-byte rows,
// zero in the pad columns), which both kernels read as MFMA operands directly.
#include "dw_reduce.h"
#include "experts_common.h"
#include "router_grad.h"

namespace nsmoe {

constexpr int CDX_TOK = 64;   // tokens per combine_dx workgroup (16 per wave)
constexpr int CDX_COLS = 64;  // columns of dx per combine_dx workgroup
constexpr int CDX_PITCH = CDX_COLS + 4;  // fp32 LDS row pitch (4 banks of skew per row)
constexpr int CDX_KMAX = 8;   // top_k and shared counts of the gather fast path
constexpr int CDX_SMAX = 2;
constexpr int CDX_KS = 4;    // k-steps of 32 experts in the router term (E <= 128)
constexpr int RDW_RC = 160;   // tokens per router_dw chunk: 5 k-steps
constexpr int RDW_BMT = 64;   // columns of x (rows of W) per router_dw tile
constexpr int RDW_BNT = 128;  // experts per router_dw tile (all of them: E <= 128)
// router_dw ring stages: one more than a chunk's k-steps, so every copy of the chunk is
// requested before the first MFMA (one memory round trip per workgroup instead of one per
// two steps); 6 stages of 12 KiB, two workgroups per CU.  At T = 8192, d = 576: 52 chunks
// x 9 column tiles = 468 workgroups, one round on 256 CUs.  Measured against 128, 256 and
// 320 tokens per chunk (11.1 against 13.1, 16.9 and 12.5 us launch to launch), with the
// reduce's extra partials costing 0.6 us in the combine_dx launch.
constexpr int RDW_S = RDW_RC / 32 + 1;
constexpr int RDW_LOADS = 8;  // router_dw_reduce: partials in flight per lane

// W.grad[m][n] = sum over the chunks of partial[c][m][n], n < E.  Four lanes per 4-wide
// output group: lane q sums chunks q, q + 4, q + 8, ... (RDW_LOADS of them in flight at a
// time, in that order), then the four lane sums are added as (q0 + q1) + (q2 + q3): a fixed
// order, so the result does not vary between runs.
// Workgroup `blk` of the reduce (NT threads); workgroups past the output do nothing.
template <int DT>
__device__ __forceinline__ void router_dw_reduce_block(const RouterDwArgs& a, int nchunks,
                                                       int64_t blk) {
  using T = typename Elem<DT>::T;
  const int n4 = a.ep / 4;
  const int64_t i = (blk * NT + threadIdx.x) >> 2;
  const int q = threadIdx.x & 3;
  const bool live = i < (int64_t)a.d * n4;
  const int m = live ? (int)(i / n4) : 0, n = live ? (int)(i % n4) * 4 : 0;
  const int64_t mn = (int64_t)a.d * a.ep;
  const float* src = a.partial + (int64_t)m * a.ep + n;
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int c0 = q; c0 < nchunks; c0 += 4 * RDW_LOADS) {
    f32x4 v[RDW_LOADS];
#pragma unroll
    for (int u = 0; u < RDW_LOADS; ++u) {
      const int c = c0 + 4 * u;
      v[u] = live && c < nchunks ? *(const f32x4*)(src + (int64_t)c * mn) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int u = 0; u < RDW_LOADS; ++u) acc += v[u];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x1 = __shfl_xor(acc[e], 1, 64);  // (q0 + q1), (q2 + q3), in lane order
    const float s01 = (q & 1) ? x1 + acc[e] : acc[e] + x1;
    const float x2 = __shfl_xor(s01, 2, 64);
    acc[e] = (q & 2) ? x2 + s01 : s01 + x2;
  }
  if (live && q == 0 && n < a.E)
    *(uint2*)((T*)a.dw + (int64_t)m * a.E + n) =
        make_uint2(pack2<DT>(acc[0], acc[1]), pack2<DT>(acc[2], acc[3]));
}

inline int64_t router_dw_reduce_blocks(int d, int ep) { return cdiv((int64_t)d * ep, NT); }

// ---- combine_dx ----------------------------------------------------------------------------
//
// Wave w of the workgroup owns tokens t0 + 16 w .. + 15 and columns m0 .. m0 + 63.
// Router term, transposed: D[m][t] = sum_n W[m][n] g[t][n] with A = W rows (contiguous in
// n), B = g rows (contiguous in n): each lane ends with 4 consecutive columns m of one
// token, written to the wave's LDS tile [16 tokens][64 columns] in fp32.  Epilogue: lane
// (token l / 4, columns 16 (l % 4) .. + 15) adds its tile entries to the token's k + S
// expert rows (two 16-byte loads per row) and stores dx with two 16-byte stores.
// W arrives packed in fragment order (RouterWPack: one 16-byte load per lane per fragment,
// zero past E).
//
// With `rdw` set, workgroups past the token tiles (blockIdx.x >= tx) are the router dW's
// reduce instead: its fp32 partials summed in chunk order into W.grad, streaming beside
// the combine rather than as a launch of its own.  Workgroups from wx on are the experts'
// dW split-K reduce (dw_reduce.h) when dwr.nbx > 0: the token tiles cover about half of
// the CUs, and the reduce streams on the others instead of in a launch of its own.
template <int DT, int KM>
__global__ void __launch_bounds__(NT, KM <= 6 ? 4 : 3)
combine_dx_kernel(CombineDxArgs a, RouterDwArgs rdw, int rchunks, int tx, DwReduceArgs dwr,
                  int wx) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  __shared__ __attribute__((aligned(16))) float s_acc[4][16][CDX_PITCH];
  __shared__ __attribute__((aligned(1024))) char s_w[4 * CDX_KS][1024];  // the W tile
  if ((int)blockIdx.x >= wx) {  // uniform: an experts' dW reduce workgroup
    const int64_t f = (int64_t)(blockIdx.x - wx) * gridDim.y + blockIdx.y;
    const int y = (int)(f / dwr.nbx), bx = (int)(f - (int64_t)y * dwr.nbx);
    if (y < dwr.rows) dw_reduce_pair_row<DT>(dwr, bx, y);
    return;
  }
  if ((int)blockIdx.x >= tx) {  // uniform: a router dW reduce workgroup
    router_dw_reduce_block<DT>(rdw, rchunks,
                               (int64_t)(blockIdx.x - tx) * gridDim.y + blockIdx.y);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t0 = (int64_t)blockIdx.x * CDX_TOK + 16 * wave;
  const int m0 = blockIdx.y * CDX_COLS;
  const char* WP = (const char*)a.w;
  const T* gl = (const T*)a.glogits;
  const int nks = (a.ep + 31) / 32;
  const T* R = (const T*)a.rows;
  // This lane's share of the sum: token t, columns c0 .. c0 + 15.
  const int tt = lane >> 2, c0 = m0 + 16 * (lane & 3);
  const int64_t t = t0 + tt;
  const bool live = t < a.T && c0 < a.d;

  // Load order: the router term's operands (the workgroup's W tile by LDS-DMA, this
  // wave's g fragments), the slot indices, then the expert rows.  vmcnt retires in order:
  // the wait for the slot indices covers the router operands, and the MFMAs then run
  // while the rows are still in flight.
  const int64_t tb = t0 + (lane & 15);  // this lane's token for the B operand
  {
    // Wave w copies the W fragments of row block w: LDS block w * nks + ks.
    const int mbg = m0 / 16 + wave;
    const uint32_t dst = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)&s_w[0][0] +
                         wave * nks * 1024;
    for (int ks = 0; ks < nks; ++ks) {
      const void* src = mbg * 16 < a.d ? (const void*)(WP + ((int64_t)(mbg * nks + ks) * 64 + lane) * 16)
                                      : (const void*)((const char*)g_zero_kib + lane * 16);
      async_copy16_to(src, dst + ks * 1024);
    }
  }
  Frag gb[CDX_KS];
#pragma unroll
  for (int ks = 0; ks < CDX_KS; ++ks) {
    const int n = 32 * ks + 8 * (lane >> 4);
    gb[ks] = M::zero();
    if (ks < nks && tb < a.T && n < a.ep) gb[ks].v = *(const u32x4*)(gl + tb * a.ep + n);
  }
  // Up to KM routed rows and CDX_SMAX shared rows per token in registers (the fast path).
  constexpr int NR = KM + CDX_SMAX;
  const bool fast = a.k <= KM && a.S <= CDX_SMAX;
  int32_t r[NR];  // row indices (the launcher checks that they fit 31 bits)
#pragma unroll
  for (int j = 0; j < KM; ++j) r[j] = fast && live && j < a.k ? a.inv[t * a.k + j] : -1;
#pragma unroll
  for (int q = 0; q < CDX_SMAX; ++q)
    r[KM + q] = fast && live && q < a.S ? (int32_t)(a.l_cap + (int64_t)q * a.T + t) : -1;
  wait_vmcnt<0>();  // the W copies, g and the slot indices
  barrier_dma();    // every wave's W copies
  u32x4 v[NR][2];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    v[j][0] = v[j][1] = u32x4{0u, 0u, 0u, 0u};
    if (r[j] >= 0) {
      const u32x4* src = (const u32x4*)(R + (int64_t)r[j] * a.d + c0);
      v[j][0] = src[0];
      v[j][1] = src[1];
    }
  }

  f32x4 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < CDX_KS; ++ks) {
    if (ks < nks) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        M::run(acc[mb], M::load(&s_w[0][0] + (mb * nks + ks) * 1024 + lane * 16), gb[ks]);
    }
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
    *(f32x4*)&s_acc[wave][lane & 15][16 * mb + 4 * (lane >> 4)] = acc[mb];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  if (!live) return;  // no barriers below
  float sum[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const f32x4 x = *(const f32x4*)&s_acc[wave][tt][16 * (lane & 3) + 4 * q];
#pragma unroll
    for (int e = 0; e < 4; ++e) sum[4 * q + e] = x[e];
  }
  auto add = [&](const u32x4& v0, const u32x4& v1) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sum[2 * e] += unpack2<DT>(v0[e], 0);
      sum[2 * e + 1] += unpack2<DT>(v0[e], 1);
      sum[8 + 2 * e] += unpack2<DT>(v1[e], 0);
      sum[8 + 2 * e + 1] += unpack2<DT>(v1[e], 1);
    }
  };
  if (fast) {
#pragma unroll
    for (int j = 0; j < NR; ++j) add(v[j][0], v[j][1]);
  } else {
    auto add_row = [&](int64_t rr) {
      const u32x4* src = (const u32x4*)(R + rr * a.d + c0);
      add(src[0], src[1]);
    };
    for (int j = 0; j < a.k; ++j) {
      const int32_t sj = a.inv[t * a.k + j];
      if (sj >= 0) add_row(sj);
    }
    for (int sh = 0; sh < a.S; ++sh) add_row(a.l_cap + (int64_t)sh * a.T + t);
  }
  u32x4 o0, o1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o0[e] = pack2<DT>(sum[2 * e], sum[2 * e + 1]);
    o1[e] = pack2<DT>(sum[8 + 2 * e], sum[8 + 2 * e + 1]);
  }
  u32x4* dst = (u32x4*)((T*)a.dx + t * a.d + c0);
  dst[0] = o0;
  dst[1] = o1;
}

// ---- router dW -------------------------------------------------------------------------
//
// D[n][m] = sum_t g[t][n] x[t][m] over one chunk of RDW_RC tokens, for one 64-column tile
// of x and all (<= 128) experts.  Both operands are contiguous along the output index, so
// they are staged row-major in LDS by lane-linear LDS-DMA copies (chunk swizzle on the
// source side) and read as MFMA operands with ds_read_b64_tr_b16 -- the dW scheme of the
// expert kernels, on dense rows.  Each lane ends with 4 consecutive n of one m and stores
// them as one 16-byte fp32 partial.
template <int ROWB>
__device__ __forceinline__ int rdw_swz(int r) {
  static_assert(ROWB % 128 == 0, "rows of whole 128-byte lines");
  if constexpr (ROWB % 256 == 0) return ((r & 3) | (((r >> 3) & 1) << 2)) << 1;
  else return (((r >> 1) ^ (r >> 2)) & 3) << 1;
}

template <int DT>
__global__ void __launch_bounds__(NT) router_dw_kernel(RouterDwArgs a) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  constexpr int WM = 2, WN = 2;
  constexpr int TMB = RDW_BMT / 16 / WM, TNB = RDW_BNT / 16 / WN;  // blocks per wave
  constexpr int QROWB = RDW_BMT * 2, PROWB = RDW_BNT * 2;           // LDS row bytes
  constexpr int QCPR = RDW_BMT / 8, PCPR = RDW_BNT / 8;             // 16-byte chunks per row
  constexpr int QBYTES = G::KC * QROWB, PBYTES = G::KC * PROWB;
  constexpr int QBLK = QBYTES / 1024, PBLK = PBYTES / 1024;         // 1 KiB copy blocks
  constexpr int STAGE = QBYTES + PBYTES;
  constexpr int NBLK = QBLK + PBLK;
  static_assert(NBLK % 4 == 0, "copy blocks split evenly over the 4 waves");
  constexpr int LOADS = NBLK / 4;
  constexpr int S = RDW_S;
  __shared__ __attribute__((aligned(1024))) char s_ring[S][STAGE];

  // A 1-D grid: the column tiles of one token chunk are consecutive items, dealt to one XCD
  // together (xcd_deal), so the chunk's d(logits) rows, which every tile of the chunk reads,
  // come into that XCD's L2 once.
  const int ntx = (a.d + RDW_BMT - 1) / RDW_BMT;
  const int item = xcd_deal((int)blockIdx.x, (int)gridDim.x, ntx);
  const int chunk = item / ntx;
  const int m0 = (item - chunk * ntx) * RDW_BMT;
  const int64_t r0 = (int64_t)chunk * RDW_RC;
  const int nr = (int)min<int64_t>(RDW_RC, a.T - r0);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const T* X = (const T*)a.x + r0 * a.d + m0;
  const T* GL = (const T*)a.glogits + r0 * a.ep;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const int nsteps = (nr + G::KC - 1) / G::KC;

  auto issue = [&](int s) {
    char* st = s_ring[s % S];
    const int k0 = s * G::KC;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const int b = wave + 4 * u;  // wave-uniform block index
      const void* src = zero;
      if (b < QBLK) {
        const int q = b * 64 + lane, row = q / QCPR, cp = q % QCPR;
        const int c = cp ^ rdw_swz<QROWB>(row);
        if (k0 + row < nr && m0 + c * 8 < a.d) src = X + (int64_t)(k0 + row) * a.d + c * 8;
      } else {
        const int q = (b - QBLK) * 64 + lane, row = q / PCPR, cp = q % PCPR;
        const int c = cp ^ rdw_swz<PROWB>(row);
        if (k0 + row < nr && c * 8 < a.ep) src = GL + (int64_t)(k0 + row) * a.ep + c * 8;
      }
      async_copy16(src, st + b * 1024);
    }
  };
  auto wait_for = [&](int s) {
    if (s + S - 2 < nsteps) wait_vmcnt<(S - 2) * LOADS>();
    else wait_step<S>(s, nsteps, [&](int) { return LOADS; });
  };
  // Transposed fragment of 16 columns (col0 .. col0 + 15) of a 32-row tile.
  auto frag_tr = [&](const char* tile, auto rowb_tag, int col0) -> Frag {
    constexpr int RB = decltype(rowb_tag)::value;
    const int i = lane & 15, gq = lane >> 4;
    const int col = col0 + 4 * (i & 3);
    const int c = col >> 3, cb = (col & 7) * 2;
    const int ra = 8 * gq + (i >> 2), rb = ra + 4;
    const uint2 lo = lds_read_tr16(tile + ra * RB + ((c ^ rdw_swz<RB>(ra)) << 4) + cb);
    const uint2 hi = lds_read_tr16(tile + rb * RB + ((c ^ rdw_swz<RB>(rb)) << 4) + cb);
    Frag f;
    f.v = u32x4{lo.x, lo.y, hi.x, hi.y};
    return f;
  };

  f32x4 acc[TNB][TMB];
#pragma unroll
  for (int j = 0; j < TNB; ++j)
#pragma unroll
    for (int i = 0; i < TMB; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S - 1 && s < nsteps; ++s) issue(s);
  for (int s = 0; s < nsteps; ++s) {
    wait_for(s);
    barrier_lds();
    if (s + S - 1 < nsteps) issue(s + S - 1);
    const char* st = s_ring[s % S];
    Frag qf[TMB], pf[TNB];
#pragma unroll
    for (int i = 0; i < TMB; ++i)
      qf[i] = frag_tr(st, std::integral_constant<int, QROWB>{}, (wm * TMB + i) * 16);
#pragma unroll
    for (int j = 0; j < TNB; ++j)
      pf[j] = frag_tr(st + QBYTES, std::integral_constant<int, PROWB>{}, (wn * TNB + j) * 16);
#pragma unroll
    for (int j = 0; j < TNB; ++j)
#pragma unroll
      for (int i = 0; i < TMB; ++i) M::run(acc[j][i], pf[j], qf[i]);
  }
  wait_vmcnt<0>();

  float* part = a.partial + (int64_t)chunk * a.d * a.ep;
#pragma unroll
  for (int j = 0; j < TNB; ++j) {
    const int n = (wn * TNB + j) * 16 + lg * 4;
    if (n >= a.ep) continue;  // ep % 8 == 0
#pragma unroll
    for (int i = 0; i < TMB; ++i) {
      const int m = m0 + (wm * TMB + i) * 16 + lc;
      if (m < a.d) *(f32x4*)(part + (int64_t)m * a.ep + n) = acc[j][i];
    }
  }
}

// ---- launchers ------------------------------------------------------------------------------

bool router_grad_supported(int dtype, int d, int E) {
  return (dtype == DT_BF16 || dtype == DT_F16) && d % 16 == 0 && E % 4 == 0 &&
         E <= RDW_BNT;
}

int router_logits_pitch(int E) { return (E + 7) / 8 * 8; }

size_t router_dw_partial_bytes(int64_t T, int d, int E) {
  return (size_t)cdiv(T, RDW_RC) * (size_t)d * (size_t)router_logits_pitch(E) * sizeof(float);
}

int combine_dx_launch(int dtype, const CombineDxArgs& a, const RouterDwArgs* rdw,
                      hipStream_t s, const DwReduceArgs* dwr) {
  NSMOE_REQUIRE(router_grad_supported(dtype, a.d, a.E) && a.ep == router_logits_pitch(a.E),
                "combine_dx: unsupported shape (d %d, E %d, pitch %d)", a.d, a.E, a.ep);
  NSMOE_REQUIRE(!rdw || (rdw->d == a.d && rdw->ep == a.ep && rdw->T == a.T && rdw->partial &&
                         rdw->dw),
                "combine_dx: the folded router dW reduce takes the same shape");
  if (a.T == 0) return NSMOE_OK;
  NSMOE_REQUIRE(a.l_cap + (int64_t)a.S * a.T < INT32_MAX, "combine_dx: %lld rows exceed 2^31",
                (long long)(a.l_cap + (int64_t)a.S * a.T));
  const int64_t tx = cdiv(a.T, CDX_TOK), ty = cdiv(a.d, CDX_COLS);
  const int64_t rx = rdw ? cdiv(router_dw_reduce_blocks(a.d, a.ep), ty) : 0;
  // The experts' dW reduce workgroups, flattened over the grid's columns.
  const bool red = dwr && dwr->nbx > 0 && dwr->rows > 0;
  const int64_t wx = tx + rx;
  const int64_t dx_extra = red ? cdiv((int64_t)dwr->nbx * dwr->rows, ty) : 0;
  NSMOE_REQUIRE(wx + dx_extra < INT32_MAX, "combine_dx: %lld tokens", (long long)a.T);
  const dim3 grid((unsigned)(wx + dx_extra), (unsigned)ty);
  DwReduceArgs dr{};
  if (red) dr = *dwr;
  const RouterDwArgs r = rdw ? *rdw : RouterDwArgs{};
  const int rchunks = rdw ? (int)cdiv(a.T, RDW_RC) : 0;
  KernelTimer timer("combine_dx", s);
  if (a.k <= 6) {
    if (dtype == DT_BF16)
      combine_dx_kernel<DT_BF16, 6><<<grid, NT, 0, s>>>(a, r, rchunks, (int)tx, dr,
                                                               (int)wx);
    else combine_dx_kernel<DT_F16, 6><<<grid, NT, 0, s>>>(a, r, rchunks, (int)tx, dr,
                                                               (int)wx);
  } else {
    if (dtype == DT_BF16)
      combine_dx_kernel<DT_BF16, CDX_KMAX><<<grid, NT, 0, s>>>(a, r, rchunks, (int)tx, dr,
                                                               (int)wx);
    else combine_dx_kernel<DT_F16, CDX_KMAX><<<grid, NT, 0, s>>>(a, r, rchunks, (int)tx, dr,
                                                               (int)wx);
  }
  timer.stop();
  return check_launch("combine_dx_kernel");
}

int router_dw_launch(int dtype, const RouterDwArgs& a, hipStream_t s) {
  NSMOE_REQUIRE(router_grad_supported(dtype, a.d, a.E) && a.ep == router_logits_pitch(a.E),
                "router_dw: unsupported shape (d %d, E %d, pitch %d)", a.d, a.E, a.ep);
  if (a.T == 0) return NSMOE_OK;
  const int64_t nchunks = cdiv(a.T, RDW_RC);
  NSMOE_REQUIRE(nchunks < 65536, "router_dw: %lld tokens", (long long)a.T);
  const unsigned grid = (unsigned)(cdiv(a.d, RDW_BMT) * nchunks);
  KernelTimer timer("router_dw", s);
  if (dtype == DT_BF16) router_dw_kernel<DT_BF16><<<grid, NT, 0, s>>>(a);
  else router_dw_kernel<DT_F16><<<grid, NT, 0, s>>>(a);
  timer.stop();
  return check_launch("router_dw_kernel");
}

}  // namespace nsmoe

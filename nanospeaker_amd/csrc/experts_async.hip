// Grouped SwiGLU experts with an asynchronous operand pipeline (gfx950, 16-bit types).
//
// Same arithmetic, tiles and outputs as the register-staged kernels in experts.hip
// (reference: moe_experts, src/model/moe_kernel.py:558-623, and MoEBlock._shared,
// src/model/moe.py:310-329); what changes is how operands reach LDS.  Every k-step's
// operands -- the 64 gathered token rows (32 elements each) and each wave's packed weight
// fragments -- are copied global -> LDS by global_load_lds_dwordx4 into an S-stage ring,
// S - 1 steps ahead of the MFMAs, so a workgroup keeps S - 1 steps of loads in flight
// without holding them in registers.  One barrier per step: it publishes the step's
// copies and frees the ring slot the next issue overwrites.
//
// Taken for bf16 / fp16 when d and H are multiples of 8, the operands are 16-byte aligned
// and H <= 128 (the ring and the h tile fit one workgroup's LDS); other shapes use the
// register-staged kernels.
#include <stdlib.h>

#include <type_traits>
#include <utility>

#include "experts_common.h"

namespace nsmoe {

// One 16-row block of a wave's 48-column slice of a 192-column pass, from the packed MFMA
// accumulators: lo[j] / hi[j] hold columns cw + 16 j + 4 lg .. + 1 / + 2 .. + 3 of row
// row0 + lc (lane 16 lg + lc).  Blocks 0 and 1 are regrouped across lanes (two permlane
// swaps per dword) so that lane (lc, lg) holds columns cw + 8 lg .. + 7 of its row;
// permlane32_swap(b0, b1) gives rows (b0.r0, b0.r1, b1.r0, b1.r1) and (b0.r2, b0.r3, b1.r2,
// b1.r3), permlane16_swap of those (b0.r0, b0.r2, b1.r0, b1.r2) and (b0.r1, b0.r3, b1.r1,
// b1.r3).  That 64-byte row segment and block 2's 32 bytes (columns cw + 32 + 4 lg ..) are
// then moved to the quad-major lane order (bperm_to_quads), so each quad of lanes writes
// one row's contiguous bytes: a 16-byte store and an 8-byte store per lane.  cw is
// wave-uniform; rows at or past `rows` and columns at or past d are not written.
template <int DT>
__device__ __forceinline__ void store_block48(const uint32_t (&lo)[3], const uint32_t (&hi)[3],
                                              typename Elem<DT>::T* Y, int d, int row0,
                                              int rows, int cw, int lane) {
  using T = typename Elem<DT>::T;
  if (cw + 32 <= d) {
    const auto l32 = __builtin_amdgcn_permlane32_swap(lo[0], lo[1], false, false);
    const auto h32 = __builtin_amdgcn_permlane32_swap(hi[0], hi[1], false, false);
    const auto l16 = __builtin_amdgcn_permlane16_swap(l32[0], l32[1], false, false);
    const auto h16 = __builtin_amdgcn_permlane16_swap(h32[0], h32[1], false, false);
    const int qa = bperm_to_quads(lane);
    const u32x4 v = bperm4(qa, u32x4{l16[0], h16[0], l16[1], h16[1]});
    const uint32_t b2lo = bperm(qa, lo[2]), b2hi = bperm(qa, hi[2]);
    const int m = row0 + (lane >> 2), c = lane & 3;
    if (m < rows) {
      T* yrow = Y + (int64_t)m * d;
      *(u32x4*)(yrow + cw + c * 8) = v;
      if (cw + 32 < d) *(uint2*)(yrow + cw + 32 + c * 4) = make_uint2(b2lo, b2hi);
    }
  } else if (cw < d) {
    const int m = row0 + (lane & 15);
    if (m < rows) *(uint2*)(Y + (int64_t)m * d + cw + (lane >> 4) * 4) = make_uint2(lo[0], hi[0]);
  }
}

// ============================ forward ====================================================
//
// One workgroup = 4 waves = one 64-row tile of one group.
//   steps [0, nk1):              GEMM1 k-block s: B = token rows (ring), A = packed W_in
//                                gate and up fragments of the wave's hidden columns (ring)
//   steps [nk1, nk1 + npass*nk2): GEMM2 pass q / nk2, k-block q % nk2: B = h (LDS),
//                                A = 3 packed W_out fragments per wave (ring)
// GEMM2's first fragments are already in flight while GEMM1 finishes.
//
// Both GEMMs run transposed (weights as the MFMA's A operand, token rows as B), so each
// lane ends with 4 consecutive output columns of one row: h reaches LDS with one 8-byte
// store per 16 x 16 block and y reaches HBM with one 8-byte store per block, no staging.
template <int DT, int NBW, int S>
__global__ void __launch_bounds__(NT, 2) expert_fwd_async_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  constexpr int HPMAX = 64 * NBW;
  constexpr int A_BYTES = BM * G::ROWB;  // 64 rows x 32 elements = 4 KiB = one copy per lane
  constexpr int NB1 = 2 * NBW;           // GEMM1 fragments per wave per step
  constexpr int NB2 = 3;                 // GEMM2 fragments per wave per step
  constexpr int NBMAX = NB1 > NB2 ? NB1 : NB2;
  constexpr int WB = NBMAX * G::PKB;     // one wave's fragment area
  constexpr int STAGE = A_BYTES + 4 * WB;
  // 4 dwords of skew per row: the 8-byte h stores of 32 lanes (16 rows x 2 column groups)
  // and the 16-byte fragment reads of 16 rows each hit distinct banks.
  constexpr int HP_PITCH = HPMAX * G::ES + 16;
  __shared__ __attribute__((aligned(1024))) char s_ring[S][STAGE];
  __shared__ __attribute__((aligned(16))) char s_h[BM * HP_PITCH];
  __shared__ int s_tok[BM];
  __shared__ float s_w[BM];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + BM - 1) / BM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * BM;
  const int rows = min(BM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (tid < BM) {
    int tok = -1, pair;
    float w = 0.0f;
    if (tid < rows) row_info<DT>(p, g, slot0 + tid, m0 + tid, tok, w, pair);
    s_tok[tid] = tok;
    s_w[tid] = w;
  }
  __syncthreads();

  const int d = p.d, H = p.H, twoH = 2 * p.H;
  // This lane's share of a step's token tile: LDS chunk tid = row ar, slot (tid & 3),
  // which holds the row's global chunk ac (the swizzle applied on the source side).
  const int ar = tid >> 2, ac = (tid & 3) ^ swz<DT>(ar);
  const int atok = s_tok[ar];
  const T* arow = atok >= 0 ? (const T*)p.x + (int64_t)atok * d + ac * G::VE : nullptr;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB + lane * G::FRAGB;
  const char* P4 = p.p_out + (int64_t)g * p.out_nb * p.out_kb * G::PKB + lane * G::FRAGB;
  const int nk1 = p.in_kb, nk2 = p.out_kb;
  const int npass = (d + NP2 - 1) / NP2;
  const int nsteps = nk1 + npass * nk2;

  auto loads_of = [&](int s) { return s < nk1 ? 1 + NB1 : NB2; };
  auto issue = [&](int s) {
    char* st = s_ring[s % S];
    char* bw = st + A_BYTES + wave * WB;
    if (s < nk1) {
      const int k0 = s * G::KC;
      const bool av = arow && k0 + ac * G::VE < d;
      async_copy16(av ? (const void*)(arow + k0) : (const void*)zero, st + wave * 1024);
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int jb = wave * NBW + j;
        async_copy16(P1 + ((int64_t)jb * nk1 + s) * G::PKB, bw + j * G::PKB);
        async_copy16(P1 + ((int64_t)(HPMAX / 16 + jb) * nk1 + s) * G::PKB,
                     bw + (NBW + j) * G::PKB);
      }
    } else {
      const int q = s - nk1, pass = q / nk2, kb = q - pass * nk2;
      const int nbase = pass * (NP2 / 16) + wave * 3;
#pragma unroll
      for (int j = 0; j < NB2; ++j) {
        const int nb = nbase + j;
        const char* src = nb < p.out_nb ? P4 + ((int64_t)nb * nk2 + kb) * G::PKB : zero;
        async_copy16(src, bw + j * G::PKB);
      }
    }
  };
  // vmcnt wait that completes step s (steps s + 1 .. s + S - 2 stay in flight).
  auto wait_for = [&](int s) {
    if (s + S - 2 < nk1) wait_vmcnt<(S - 2) * (1 + NB1)>();
    else if (s >= nk1 && s + S - 2 < nsteps) wait_vmcnt<(S - 2) * NB2>();
    else wait_step<S>(s, nsteps, loads_of);
  };

  for (int s = 0; s < S - 1 && s < nsteps; ++s) issue(s);

  // ---- GEMM1 (transposed): acc[i][j] = W_in[:, cols of block j]^T x[rows of block i]^T ----
  f32x4 accg[4][NBW], accu[4][NBW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) accg[i][j] = accu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < nk1; ++s) {
    wait_for(s);
    barrier_lds();
    if (s + S - 1 < nsteps) issue(s + S - 1);
    const char* st = s_ring[s % S];
    const char* bw = st + A_BYTES + wave * WB + lane * G::FRAGB;
    Frag xf[4], wg[NBW], wu[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      wg[j] = M::load(bw + j * G::PKB);
      wu[j] = M::load(bw + (NBW + j) * G::PKB);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) xf[i] = frag_sw<DT>(st, i * 16);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        M::run(accg[i][j], wg[j], xf[i]);
        M::run(accu[i][j], wu[j], xf[i]);
      }
  }

  // ---- GEMM1 epilogue: bias, h = act(gate) * up -> LDS (published by the next barrier) ----
  // Lane (lc, lg) of block (i, j) holds row m = i*16 + lc, hidden columns n0 .. n0 + 3.
  const T* bin = (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
  with_act(p.act, [&]<int ACT>() {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int n0 = (wave * NBW + j) * 16 + lg * 4;
      float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
      if (bin) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n0 + r < H) {
            bg[r] = Elem<DT>::to_f(bin[n0 + r]);
            bu[r] = Elem<DT>::to_f(bin[H + n0 + r]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float hv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          hv[r] = n0 + r < H ? act_fwd_t<ACT>(accg[i][j][r] + bg[r]) * (accu[i][j][r] + bu[r])
                             : 0.0f;
        const uint32_t lo = pack2<DT>(hv[0], hv[1]), hi = pack2<DT>(hv[2], hv[3]);
        *(uint2*)(s_h + (i * 16 + lc) * HP_PITCH + n0 * G::ES) = make_uint2(lo, hi);
      }
    }
  });

  // ---- GEMM2 (transposed): y^T = W_out^T h^T, + b_out, * gate, 8-byte row stores ----
  const T* bout = (g < p.E ? p.b_out : p.b_sh_out)
                      ? per_group<T>(p.b_out, p.b_sh_out, g, p.E, d) : nullptr;
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wrow[i] = s_w[i * 16 + lc];
  T* Y = (T*)p.y + slot0 * d;
  for (int pass = 0; pass < npass; ++pass) {
    f32x4 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nk2; ++kb) {
      const int s = nk1 + pass * nk2 + kb;
      wait_for(s);
      barrier_lds();
      if (s + S - 1 < nsteps) issue(s + S - 1);
      const char* bw = s_ring[s % S] + A_BYTES + wave * WB + lane * G::FRAGB;
      Frag hf[4], wf[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) wf[j] = M::load(bw + j * G::PKB);
#pragma unroll
      for (int i = 0; i < 4; ++i) hf[i] = frag_at<DT>(s_h, HP_PITCH, i * 16, kb * G::ROWB);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) M::run(acc[i][j], wf[j], hf[i]);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int n0 = (pass * (NP2 / 16) + wave * 3 + j) * 16 + lg * 4;
      if (n0 >= d) continue;
      float bo[4] = {0.f, 0.f, 0.f, 0.f};
      if (bout) {
        const uint2 b = *(const uint2*)(bout + n0);
        bo[0] = unpack2<DT>(b.x, 0);
        bo[1] = unpack2<DT>(b.x, 1);
        bo[2] = unpack2<DT>(b.y, 0);
        bo[3] = unpack2<DT>(b.y, 1);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = i * 16 + lc;
        if (m < rows) {
          const float w = wrow[i];
          const uint32_t lo = pack2<DT>((acc[i][j][0] + bo[0]) * w, (acc[i][j][1] + bo[1]) * w);
          const uint32_t hi = pack2<DT>((acc[i][j][2] + bo[2]) * w, (acc[i][j][3] + bo[3]) * w);
          *(uint2*)(Y + (int64_t)m * d + n0) = make_uint2(lo, hi);
        }
      }
    }
  }
  wait_vmcnt<0>();  // nothing may be in flight when the workgroup retires
}

// expert_fwd_reg: the same arithmetic as expert_fwd_async_kernel on tiles of MB 16-row
// blocks (MB = 4: 64 rows, MB = 6: 96 rows), with the weights -- private to each wave --
// loaded from L2 straight into registers two k-steps ahead (two fragment sets in flight),
// and only the token tile (shared by the 4 waves) copied through the LDS ring.  GEMM2
// reads h from LDS and its weights from registers.
//
// Every tile streams its group's whole weight stack through the CU once, so the weight
// bytes per MFMA fall as the tile grows: 96-row tiles move 2/3 of the weight bytes per row
// of 64-row tiles, and at T = 8192 their ~720 tiles fit the machine's resident workgroup
// slots in one round where ~1060 64-row tiles take two.
//
// Output: MB = 4 assembles each 192-column pass of y in LDS (over the token ring, idle by
// then) and stores whole 384-byte row segments in 16-byte stores; MB = 6 keeps its LDS at
// 3 workgroups per CU and stores 8 bytes per lane straight from the accumulators.
//
// Step s issues, after its MFMAs, the weights of step s + 2 and then the token copies of
// step s + 2 (one per wave for 64 rows; for 96 rows a second, on half the lanes); step s
// therefore waits (vmcnt) until only what step s - 1 issued is in flight, which also
// covers the weights of step s (issued just before the copies).  Every load is
// unconditional (out-of-range fragments read a zero page), so the compiler's own waits
// for the weight registers are exact or stricter and leave the next step's loads in flight.
// Shapes: d % 64 == 0 (an even number of GEMM1 steps) and an even number of GEMM2 steps.
template <int DT, int NBW, int MB, int D>
__global__ void __launch_bounds__(NT, MB > 2 && (MB == 6 || D == 3) ? 3 : 2)
expert_fwd_reg_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  // 32-row tiles are for small problems (decode): few rows per group, so the tile streams
  // the group's weights with a deeper prefetch instead of more rows.
  static_assert(MB == 2 || MB == 4 || MB == 6, "32-, 64- or 96-row tiles");
  static_assert(D == 2 || D == 3 || (MB == 2 && D == 6), "prefetch distance");
  constexpr int TM = MB * 16;            // tile rows
  constexpr int S = D + 1;               // token-tile ring stages
  // Token copies per wave per step: 4 16-byte slots per row, 256 per full copy; a tile
  // whose slot count is an odd multiple of 128 ends with a copy on half of each wave.
  constexpr int XC = (TM * 4 + NT - 1) / NT;
  constexpr bool XHALF = (TM * 4) % NT != 0;
  static_assert((TM * 4) % NT == 0 || (TM * 4) % NT == NT / 2, "whole or half copies");
  constexpr bool STAGE_Y = MB == 4;
  constexpr int HPMAX = 64 * NBW;
  constexpr int A_BYTES = TM * G::ROWB;  // TM rows x 32 elements
  constexpr int NB1 = 2 * NBW;           // GEMM1 fragments per wave per step
  constexpr int NB2 = 3;                 // GEMM2 fragments per wave per step
  constexpr int NBMAX = NB1 > NB2 ? NB1 : NB2;
  constexpr int HP_PITCH = HPMAX * G::ES + 16;
  constexpr int Y_PITCH = NP2 * G::ES + 16;  // staged y rows: one pass's 192 columns
  constexpr int Y_BYTES = STAGE_Y ? TM * Y_PITCH : 0;
  constexpr int RING_BYTES = S * A_BYTES > Y_BYTES ? S * A_BYTES : Y_BYTES;
  __shared__ __attribute__((aligned(1024))) char s_ring_raw[RING_BYTES];
  char (*s_ring)[A_BYTES] = (char (*)[A_BYTES])s_ring_raw;
  char* s_y = s_ring_raw;  // GEMM2 output staging, after GEMM1 is done with the ring
  __shared__ __attribute__((aligned(16))) char s_h[TM * HP_PITCH];
  __shared__ int s_tok[TM];
  __shared__ float s_w[TM];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + TM - 1) / TM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * TM;
  const int rows = min(TM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  // The first saved pre-activation block of the tile, read here with the other group
  // offsets: inside the epilogue the load of offs[g] would come after the block stores
  // and the GEMM2 weight loads, and waiting for it would wait for all of them.
  const int64_t a1_blk0 = p.a1_out ? act_block(p, g, m0) : 0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB + lane * G::FRAGB;
  const char* P4 = p.p_out + (int64_t)g * p.out_nb * p.out_kb * G::PKB + lane * G::FRAGB;
  const int nk1 = p.in_kb, nk2 = p.out_kb;
  const int npass = (d + NP2 - 1) / NP2;
  const int n2 = npass * nk2;

  // A step's weight fragments, as a value (fragment sets passed by reference end up in
  // scratch memory).
  struct WSet {
    Frag f[NBMAX];
  };
  auto load_w1 = [&](int s) __attribute__((always_inline)) -> WSet {  // s < nk1
    WSet w;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int jb = wave * NBW + j;
      w.f[j] = M::load(P1 + ((int64_t)jb * nk1 + s) * G::PKB);
      w.f[NBW + j] = M::load(P1 + ((int64_t)(HPMAX / 16 + jb) * nk1 + s) * G::PKB);
    }
#pragma unroll
    for (int j = NB1; j < NBMAX; ++j) w.f[j] = M::zero();
    return w;
  };
  auto load_w2 = [&](int q) __attribute__((always_inline)) -> WSet {  // q < n2
    const int pass = q / nk2, kb = q - pass * nk2;
    const int nbase = pass * (NP2 / 16) + wave * 3;
    WSet w;
#pragma unroll
    for (int j = 0; j < NB2; ++j) {
      const int nb = nbase + j;
      w.f[j] = M::load(nb < p.out_nb ? P4 + ((int64_t)nb * nk2 + kb) * G::PKB : zero);
    }
#pragma unroll
    for (int j = NB2; j < NBMAX; ++j) w.f[j] = M::zero();
    return w;
  };

  // The first two weight sets depend only on the group: they are in flight while the
  // rows' tokens are looked up.  The gate weights are loaded before the token copies are
  // issued and reach LDS after GEMM1 (GEMM2's epilogue reads them), so waiting for them
  // never waits for a copy.
  WSet wset[D];
#pragma unroll
  for (int j = 0; j < D; ++j) wset[j] = load_w1(j);
  const bool routed = g < p.E;
  int pair = -1;
  if (tid < TM) {
    int tok = -1;
    if (tid < rows) {
      if (routed) {
        pair = p.sorted_ids[slot0 + tid];
        tok = pair / p.k;
      } else {
        tok = m0 + tid;
      }
    }
    s_tok[tid] = tok;
  }
  __syncthreads();
  float gate_w = 0.0f;
  if (tid < rows)
    gate_w = routed ? Elem<DT>::to_f(((const T*)p.topk_w)[pair]) : 1.0f;
  // Token copies: copy slot c (16 bytes) holds chunk (c % 4) ^ swz(r) of row r = c / 4.
  // Full copy x of wave w fills slots 256 x + 64 w + lane (rows 64 x + tid / 4); a final
  // half copy fills slots 256 x + 32 w + lane (lanes < 32), rows 64 x + 8 w + lane / 4.
  const T* arow[XC];
  int acol[XC];
#pragma unroll
  for (int x = 0; x < XC; ++x) {
    const bool half = XHALF && x == XC - 1;
    const int r = half ? 64 * x + wave * 8 + (lane >> 2) : 64 * x + (tid >> 2);
    acol[x] = (lane & 3) ^ swz<DT>(r);
    const int t = (!half || lane < 32) && r < TM ? s_tok[r] : -1;
    arow[x] = t >= 0 ? (const T*)p.x + (int64_t)t * d + acol[x] * G::VE : nullptr;
  }
  auto issue_x = [&](int s) __attribute__((always_inline)) {
    const int k0 = s * G::KC;
#pragma unroll
    for (int x = 0; x < XC; ++x) {
      const bool av = arow[x] && k0 + acol[x] * G::VE < d;
      const void* src = av ? (const void*)(arow[x] + k0) : (const void*)zero;
      if (XHALF && x == XC - 1) {
        if (lane < 32) async_copy16(src, s_ring[s % S] + 4096 * x + wave * 512);
      } else {
        async_copy16(src, s_ring[s % S] + 4096 * x + wave * 1024);
      }
    }
  };

  // ---- GEMM1 (transposed): acc[i][j] = W_in[:, cols of block j]^T x[rows of block i]^T ----
  f32x4 accg[MB][NBW], accu[MB][NBW];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j) accg[i][j] = accu[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto g1mma = [&](int s, const WSet& w) __attribute__((always_inline)) {
    barrier_dma();
    const char* st = s_ring[s % S];
    // Token fragments in groups of (at most) 4 row blocks, to bound the live registers.
    constexpr int XG = MB > 4 ? 2 : MB;
#pragma unroll
    for (int i0 = 0; i0 < MB; i0 += XG) {
      Frag xf[XG];
#pragma unroll
      for (int i = 0; i < XG; ++i) xf[i] = frag_sw<DT>(st, (i0 + i) * 16);
#pragma unroll
      for (int i = 0; i < XG; ++i)
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          M::run(accg[i0 + i][j], w.f[j], xf[i]);
          M::run(accu[i0 + i][j], w.f[NBW + j], xf[i]);
        }
    }
  };

#pragma unroll
  for (int j = 0; j < D; ++j) issue_x(j);
  // Every prologue load but step D - 1's copies.  The steady-state count below assumes
  // that step s's copies are followed only by the loads of steps s + 1 .. s + D - 1 in
  // issue order; the prologue issues all D weight sets ahead of the copies, so for steps
  // below D - 1 that holds only once their copies are already complete.
  wait_vmcnt<XC>();
  int s = 0;
  for (; s + D < nk1; s += D) {  // steady state: the steps D ahead are GEMM1 steps
#pragma unroll
    for (int j = 0; j < D; ++j) {
      wait_vmcnt<(D - 1) * (NB1 + XC)>();  // step s + j's weights and copies have landed
      g1mma(s + j, wset[j]);
      wset[j] = load_w1(s + j + D);
      issue_x(s + j + D);
    }
  }
  // The last D GEMM1 steps prefetch GEMM2's first D weight sets: before step s + j, the
  // GEMM1 loads of steps s + j + 1 .. s + D - 1 and the GEMM2 sets 0 .. j - 1 may be
  // outstanding.
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wait_vmcnt_dyn((D - 1 - j) * (NB1 + XC) + j * NB2);  // a constant once unrolled
    g1mma(s + j, wset[j]);
    wset[j] = load_w2(j);
  }

  if (tid < TM) s_w[tid] = gate_w;  // published by the barrier after the epilogue
  // ---- GEMM1 epilogue: bias, h = act(gate) * up -> LDS --------------------------------------
  const T* bin = (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
  with_act(p.act, [&]<int ACT>() {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int n0 = (wave * NBW + j) * 16 + lg * 4;
      float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
      if (bin) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (n0 + r < H) {
            bg[r] = Elem<DT>::to_f(bin[n0 + r]);
            bu[r] = Elem<DT>::to_f(bin[H + n0 + r]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        if (p.a1_out) {
          // The pre-activations [gate | up] (bias included, rounded to the element type)
          // for the backward, which then does not recompute them: one 512-byte 16 x 16
          // block per wave and store (act_block).  Saving requires H % 16 == 0, so a
          // column block is all in or all out.
          const int jb = wave * NBW + j;
          if (i * 16 + lc < rows && jb * 16 < H) {
            T* blk = (T*)p.a1_out + (a1_blk0 + i) * (twoH / 16) * 256 + lane * 4;
            *(uint2*)(blk + jb * 256) =
                make_uint2(pack2<DT>(accg[i][j][0] + bg[0], accg[i][j][1] + bg[1]),
                           pack2<DT>(accg[i][j][2] + bg[2], accg[i][j][3] + bg[3]));
            *(uint2*)(blk + (H / 16 + jb) * 256) =
                make_uint2(pack2<DT>(accu[i][j][0] + bu[0], accu[i][j][1] + bu[1]),
                           pack2<DT>(accu[i][j][2] + bu[2], accu[i][j][3] + bu[3]));
          }
        }
        float hv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          hv[r] = n0 + r < H ? act_fwd_t<ACT>(accg[i][j][r] + bg[r]) * (accu[i][j][r] + bu[r])
                             : 0.0f;
        const uint32_t lo = pack2<DT>(hv[0], hv[1]), hi = pack2<DT>(hv[2], hv[3]);
        *(uint2*)(s_h + (i * 16 + lc) * HP_PITCH + n0 * G::ES) = make_uint2(lo, hi);
      }
    }
  });
  // h published: its ds_write stores complete, then a bare barrier (a fence here would
  // also wait for the GEMM2 weights in flight).
  wait_lgkm0();
  barrier_dma();

  // ---- GEMM2 (transposed): y^T = W_out^T h^T, + b_out, * gate ---------------------------
  const T* bout = (g < p.E ? p.b_out : p.b_sh_out)
                      ? per_group<T>(p.b_out, p.b_sh_out, g, p.E, d) : nullptr;
  float wrow[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) wrow[i] = s_w[i * 16 + lc];
  T* Y = (T*)p.y + slot0 * d;
  f32x4 acc[MB][3];
  auto g2step = [&](int q, const WSet& w) __attribute__((always_inline)) {
    const int pass = q / nk2, kb = q - pass * nk2;
    if (kb == 0) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    constexpr int HG = MB > 4 ? MB / 2 : MB;
#pragma unroll
    for (int i0 = 0; i0 < MB; i0 += HG) {
      Frag hf[HG];
#pragma unroll
      for (int i = 0; i < HG; ++i)
        hf[i] = frag_at<DT>(s_h, HP_PITCH, (i0 + i) * 16, kb * G::ROWB);
#pragma unroll
      for (int i = 0; i < HG; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) M::run(acc[i0 + i][j], w.f[j], hf[i]);
    }
    if (kb == nk2 - 1) {
      if constexpr (STAGE_Y) {
        // + b_out, * gate, packed into the staging tile (the previous pass's reads are
        // done once every wave has passed this barrier).
        wait_lgkm0();
        barrier_dma();
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int c0 = (wave * 3 + j) * 16 + lg * 4;  // column inside the pass
          const int n0 = pass * NP2 + c0;
          if (n0 >= d) continue;
          float bo[4] = {0.f, 0.f, 0.f, 0.f};
          if (bout) {
            const uint2 b = *(const uint2*)(bout + n0);
            bo[0] = unpack2<DT>(b.x, 0);
            bo[1] = unpack2<DT>(b.x, 1);
            bo[2] = unpack2<DT>(b.y, 0);
            bo[3] = unpack2<DT>(b.y, 1);
          }
#pragma unroll
          for (int i = 0; i < MB; ++i) {
            const int m = i * 16 + lc;
            const float wt = wrow[i];
            const uint32_t lo =
                pack2<DT>((acc[i][j][0] + bo[0]) * wt, (acc[i][j][1] + bo[1]) * wt);
            const uint32_t hi =
                pack2<DT>((acc[i][j][2] + bo[2]) * wt, (acc[i][j][3] + bo[3]) * wt);
            *(uint2*)(s_y + m * Y_PITCH + c0 * G::ES) = make_uint2(lo, hi);
          }
        }
        wait_lgkm0();
        barrier_dma();
        // TM rows x 24 chunks of 16 bytes; a wave's store covers 2.67 whole 384-byte rows.
        const int ncols = min(NP2, d - pass * NP2);
        constexpr int CPR = NP2 / G::VE;  // chunks per staged row
#pragma unroll
        for (int u = 0; u < TM * CPR / NT; ++u) {
          const int c = tid + u * NT, m = c / CPR, cc = c % CPR;
          if (m < rows && cc * G::VE < ncols) {
            const u32x4 v = *(const u32x4*)(s_y + m * Y_PITCH + cc * 16);
            *(u32x4*)(Y + (int64_t)m * d + pass * NP2 + cc * G::VE) = v;
          }
        }
      } else {
        // + b_out, * gate, then the wave's 48 columns of this pass (blocks 0..2) leave as
        // whole row segments in the quad-major lane order (store_block48).
        const int cw = pass * NP2 + wave * 48;  // wave-uniform
        float bo[3][4];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const int n0 = cw + j * 16 + lg * 4;
#pragma unroll
          for (int r = 0; r < 4; ++r) bo[j][r] = 0.0f;
          if (bout && n0 < d) {
            const uint2 b = *(const uint2*)(bout + n0);
            bo[j][0] = unpack2<DT>(b.x, 0);
            bo[j][1] = unpack2<DT>(b.x, 1);
            bo[j][2] = unpack2<DT>(b.y, 0);
            bo[j][3] = unpack2<DT>(b.y, 1);
          }
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const float wt = wrow[i];
          uint32_t lo[3], hi[3];
#pragma unroll
          for (int j = 0; j < 3; ++j) {
            lo[j] = pack2<DT>((acc[i][j][0] + bo[j][0]) * wt, (acc[i][j][1] + bo[j][1]) * wt);
            hi[j] = pack2<DT>((acc[i][j][2] + bo[j][2]) * wt, (acc[i][j][3] + bo[j][3]) * wt);
          }
          // The lane id passes an empty asm first, so the store's lane arithmetic is
          // computed here rather than hoisted to the kernel's start, where it would stay
          // live through GEMM1 (the kernel is at its register cap).
          int sl = lane;
          asm volatile("" : "+v"(sl));
          store_block48<DT>(lo, hi, Y, d, i * 16, rows, cw, sl);
        }
      }
    }
  };
  int q = 0;
  for (; q + D < n2; q += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      g2step(q + j, wset[j]);
      wset[j] = load_w2(q + j + D);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) g2step(q + j, wset[j]);
  wait_vmcnt<0>();  // nothing may be in flight when the workgroup retires
}

// ============================ backward ===================================================
//
// expert_bwd_async: one workgroup = one 64-row tile of one group; per k-step of d:
//   a1^T = W_in^T x[tok]^T   (gate and up, recomputed in fp32)   A = packed W_in (ring)
//   G^T  = W_out dout[tok]^T                                     A = W_out rows (ring)
// both token tiles (x and dout rows) arrive through the ring as B operands.  The GLU
// backward is lane-local (gate, up and G of one (row, column) share lane and register):
//   h = act(g) u,  dtopk_w += G h,  d_gate = w G u act'(g),  d_up = w G act(g),
// and dA1 = [d_gate | d_up] and w h leave as 8-byte row stores (for dX and both dW).
// The gate gradient also takes <dout[tok], b_out[g]> when the expert has an output bias.
template <int DT, int NBW, int S>
__global__ void __launch_bounds__(NT, 2) expert_bwd_async_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  constexpr int HPMAX = 64 * NBW;
  constexpr int A_BYTES = BM * G::ROWB;  // one token tile (x or dout): 4 KiB
  constexpr int NBF = 3 * NBW;           // gate, up and G fragments per wave per step
  constexpr int WB = NBF * G::PKB;
  constexpr int STAGE = 2 * A_BYTES + 4 * WB;
  constexpr int LOADS = 2 + NBF;         // copies per lane per step
  __shared__ __attribute__((aligned(1024))) char s_ring[S][STAGE];
  __shared__ int s_tok[BM];
  __shared__ int s_pair[BM];
  __shared__ float s_w[BM];
  __shared__ float s_dtw[5][BM];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + BM - 1) / BM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * BM;
  const int rows = min(BM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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
  const int ar = tid >> 2, ac = (tid & 3) ^ swz<DT>(ar);
  const int atok = s_tok[ar];
  const T* xrow = atok >= 0 ? (const T*)p.x + (int64_t)atok * d + ac * G::VE : nullptr;
  const T* drow = atok >= 0 ? (const T*)p.dout + (int64_t)atok * d + ac * G::VE : nullptr;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB + lane * G::FRAGB;
  // W_out fragment rows: lane l reads row (jb * 16 + l % 16), k elements 8 * (l / 16) ..
  const T* Wout = per_group<T>(p.w_out, p.w_sh_out, g, p.E, (int64_t)H * d);
  const int wk = (lane >> 4) * 8;
  const int nk = p.in_kb;

  auto issue = [&](int s) {
    char* st = s_ring[s % S];
    char* bw = st + 2 * A_BYTES + wave * WB;
    const int k0 = s * G::KC;
    const bool av = k0 + ac * G::VE < d;
    async_copy16(xrow && av ? (const void*)(xrow + k0) : (const void*)zero, st + wave * 1024);
    async_copy16(drow && av ? (const void*)(drow + k0) : (const void*)zero,
                 st + A_BYTES + wave * 1024);
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int jb = wave * NBW + j;
      async_copy16(P1 + ((int64_t)jb * nk + s) * G::PKB, bw + j * G::PKB);
      async_copy16(P1 + ((int64_t)(HPMAX / 16 + jb) * nk + s) * G::PKB,
                   bw + (NBW + j) * G::PKB);
      const int n = jb * 16 + lc;
      const bool wv = n < H && k0 + wk < d;
      async_copy16(wv ? (const void*)(Wout + (int64_t)n * d + k0 + wk) : (const void*)zero,
                   bw + (2 * NBW + j) * G::PKB);
    }
  };
  auto wait_for = [&](int s) {
    if (s + S - 2 < nk) wait_vmcnt<(S - 2) * LOADS>();
    else wait_step<S>(s, nk, [&](int) { return LOADS; });
  };

  for (int s = 0; s < S - 1 && s < nk; ++s) issue(s);
  f32x4 accg[4][NBW], accu[4][NBW], accG[4][NBW];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
      accg[i][j] = accu[i][j] = accG[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < nk; ++s) {
    wait_for(s);
    barrier_lds();
    if (s + S - 1 < nk) issue(s + S - 1);
    const char* st = s_ring[s % S];
    const char* bw = st + 2 * A_BYTES + wave * WB + lane * G::FRAGB;
    Frag wg[NBW], wu[NBW], wo[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      wg[j] = M::load(bw + j * G::PKB);
      wu[j] = M::load(bw + (NBW + j) * G::PKB);
      wo[j] = M::load(bw + (2 * NBW + j) * G::PKB);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const Frag xf = frag_sw<DT>(st, i * 16);
      const Frag df = frag_sw<DT>(st + A_BYTES, i * 16);
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        M::run(accg[i][j], wg[j], xf);
        M::run(accu[i][j], wu[j], xf);
        M::run(accG[i][j], wo[j], df);
      }
    }
  }

  // ---- GLU backward, lane-local: lane (lc, lg) of block (i, j) holds row i*16 + lc,
  // hidden columns n0 .. n0 + 3 ----
  const T* bin = (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
  T* DA = (T*)p.da1 + slot0 * twoH;
  T* HB = (T*)p.hbuf + slot0 * H;
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wrow[i] = s_w[i * 16 + lc];
  float part[4] = {0.f, 0.f, 0.f, 0.f};
  with_act(p.act, [&]<int ACT>() {
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int n0 = (wave * NBW + j) * 16 + lg * 4;
      if (n0 >= H) continue;  // H % 4 == 0: a group of 4 columns is all in or all out
      float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
      if (bin) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          bg[r] = Elem<DT>::to_f(bin[n0 + r]);
          bu[r] = Elem<DT>::to_f(bin[H + n0 + r]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = i * 16 + lc;
        const float w = wrow[i];
        float dg[4], du[4], wh[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float gg = accg[i][j][r] + bg[r], uu = accu[i][j][r] + bu[r];
          const float Gv = accG[i][j][r];
          float a, da;
          act_both_t<ACT>(gg, a, da);
          const float hv = a * uu;
          part[i] += Gv * hv;
          const float dh = w * Gv;
          dg[r] = dh * uu * da;
          du[r] = dh * a;
          wh[r] = w * hv;
        }
        if (m < rows) {
          T* da_row = DA + (int64_t)m * twoH;
          *(uint2*)(da_row + n0) = make_uint2(pack2<DT>(dg[0], dg[1]), pack2<DT>(dg[2], dg[3]));
          *(uint2*)(da_row + H + n0) =
              make_uint2(pack2<DT>(du[0], du[1]), pack2<DT>(du[2], du[3]));
          *(uint2*)(HB + (int64_t)m * H + n0) =
              make_uint2(pack2<DT>(wh[0], wh[1]), pack2<DT>(wh[2], wh[3]));
        }
      }
    }
  });
  // dtopk_w: sum of G h over the row's hidden columns (4 lanes per wave, then 4 waves).
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = part[i];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lg == 0) s_dtw[wave][i * 16 + lc] = v;
  }
  // <dout[tok], b_out[g]>: four lanes per row, strided over d.
  if (g < p.E && p.b_out) {
    const T* bo = (const T*)p.b_out + (int64_t)g * d;
    const int m = tid >> 2, q = tid & 3;
    float v = 0.0f;
    if (m < rows) {
      const T* dr = (const T*)p.dout + (int64_t)s_tok[m] * d;
      for (int c = q; c < d; c += 4) v += Elem<DT>::to_f(dr[c]) * Elem<DT>::to_f(bo[c]);
    }
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    if (q == 0 && m < rows) s_dtw[4][m] = v;
  }
  __syncthreads();
  if (g < p.E && tid < rows) {
    const float v = s_dtw[0][tid] + s_dtw[1][tid] + s_dtw[2][tid] + s_dtw[3][tid] + s_dtw[4][tid];
    ((T*)p.dtw)[s_pair[tid]] = Elem<DT>::from_f(v);
  }
}

// expert_dx_async: dX rows = dA1 W_in^T, one workgroup per 64-row tile, computed
// transposed (dX^T = W_in dA1^T): A = W_in rows (contiguous along 2H, the contraction
// index), B = the tile's dA1 rows; both through the ring, in passes of NP2 output columns
// (48 per wave).  Rows are reduced per token by `combine`.
template <int DT, int S>
__global__ void __launch_bounds__(NT, 2) expert_dx_async_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  constexpr int A_BYTES = BM * G::ROWB;
  constexpr int NBF = 3;
  constexpr int WB = NBF * G::PKB;
  constexpr int STAGE = A_BYTES + 4 * WB;
  constexpr int LOADS = 1 + NBF;
  __shared__ __attribute__((aligned(1024))) char s_ring[S][STAGE];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + BM - 1) / BM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * BM;
  const int rows = min(BM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = p.d, twoH = 2 * p.H;
  const int ar = tid >> 2, ac = (tid & 3) ^ swz<DT>(ar);
  const T* arow = ar < rows ? (const T*)p.da1 + (slot0 + ar) * twoH + ac * G::VE : nullptr;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const T* Win = per_group<T>(p.w_in, p.w_sh_in, g, p.E, (int64_t)d * twoH);
  const int wk = (lane >> 4) * 8;
  const int nkk = (twoH + G::KC - 1) / G::KC;
  const int npass = (d + NP2 - 1) / NP2;
  const int nsteps = npass * nkk;

  auto issue = [&](int s) {
    char* st = s_ring[s % S];
    char* bw = st + A_BYTES + wave * WB;
    const int pass = s / nkk, k0 = (s - pass * nkk) * G::KC;
    async_copy16(arow && k0 + ac * G::VE < twoH ? (const void*)(arow + k0) : (const void*)zero,
                 st + wave * 1024);
#pragma unroll
    for (int j = 0; j < NBF; ++j) {
      const int c = (pass * (NP2 / 16) + wave * 3 + j) * 16 + lc;
      const bool v = c < d && k0 + wk < twoH;
      async_copy16(v ? (const void*)(Win + (int64_t)c * twoH + k0 + wk) : (const void*)zero,
                   bw + j * G::PKB);
    }
  };
  auto wait_for = [&](int s) {
    if (s + S - 2 < nsteps) wait_vmcnt<(S - 2) * LOADS>();
    else wait_step<S>(s, nsteps, [&](int) { return LOADS; });
  };

  for (int s = 0; s < S - 1 && s < nsteps; ++s) issue(s);
  T* DX = (T*)p.dxrow + slot0 * d;
  for (int pass = 0; pass < npass; ++pass) {
    f32x4 acc[4][3];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kk = 0; kk < nkk; ++kk) {
      const int s = pass * nkk + kk;
      wait_for(s);
      barrier_lds();
      if (s + S - 1 < nsteps) issue(s + S - 1);
      const char* st = s_ring[s % S];
      const char* bw = st + A_BYTES + wave * WB + lane * G::FRAGB;
      Frag wf[3];
#pragma unroll
      for (int j = 0; j < 3; ++j) wf[j] = M::load(bw + j * G::PKB);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const Frag af = frag_sw<DT>(st, i * 16);
#pragma unroll
        for (int j = 0; j < 3; ++j) M::run(acc[i][j], wf[j], af);
      }
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int c0 = (pass * (NP2 / 16) + wave * 3 + j) * 16 + lg * 4;
      if (c0 >= d) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = i * 16 + lc;
        if (m < rows)
          *(uint2*)(DX + (int64_t)m * d + c0) =
              make_uint2(pack2<DT>(acc[i][j][0], acc[i][j][1]),
                         pack2<DT>(acc[i][j][2], acc[i][j][3]));
      }
    }
  }
  wait_vmcnt<0>();
}

// expert_bwd_reg / expert_dx_reg: expert_bwd_async / expert_dx_async with the schedule of
// expert_fwd_reg -- the packed W_in fragments (when a1 is recomputed) and dX's W_in
// fragments loaded into registers D k-steps ahead, the token tiles (x and dout; dA1 rows)
// and the GLU backward's W_out fragments copied through LDS rings, and the GLU backward's
// row outputs assembled in LDS and written as whole row segments with 16-byte stores.  Step s waits until only what slot s - 1 issued is in flight; all loads
// of a steady step are unconditional (zero page for fragments past the edge).
// Shapes: an even number of k-steps.

template <int DT, int NBW, int D, int MB, bool SA>
__global__ void __launch_bounds__(NT, SA && MB != 5 ? 3 : 2) expert_bwd_reg_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  static_assert(D >= 2 && D <= 4, "prefetch distance");
  static_assert(MB >= 2 && MB <= 6, "tiles of 32 .. 96 rows");
  constexpr int S = D + 1;
  constexpr int TM = MB * 16;            // tile rows
  constexpr int HPMAX = 64 * NBW;
  constexpr int A_BYTES = TM * G::ROWB;  // one token tile (x or dout)
  // Token tiles per ring stage: x and dout, or dout alone when the forward saved a1.
  constexpr int NA = SA ? 1 : 2;
  constexpr int DOFF = SA ? 0 : A_BYTES;  // dout's tile inside a stage
  // Copies per token tile and step: TM * 4 slots of 16 bytes, up to 256 per copy; copy x
  // of wave w fills slots 256 x + CL w + lane for the lanes below CL = min(64, TM - 64 x).
  constexpr int XC = (TM + 63) / 64;
  constexpr int GI = SA ? 0 : 2 * NBW;   // first G fragment of a step's set
  constexpr int NBF = GI + NBW;          // (gate, up and) G fragments per wave per step
  constexpr int SLOT = NBF + NA * XC;    // VM operations a steady slot issues
  constexpr int DA_PITCH = 2 * HPMAX * G::ES + 16;  // staged dA1 rows
  constexpr int HB_PITCH = HPMAX * G::ES + 16;      // staged w h rows
  constexpr int RING = S * NA * A_BYTES;
  // W_out fragments of the 4 waves for one k-step (NBW 16-row x 32-k fragments a wave),
  // copied with the token tiles into an S-stage ring of their own after the token ring.
  constexpr int WB = 4 * NBW * 1024;
  constexpr int WRING = S * WB;
  // The epilogue stages its rows in two passes of MBH row blocks (half the LDS of one pass:
  // 96-row tiles then fit three workgroups per CU).
  constexpr int MBH = (MB + 1) / 2;
  constexpr int STAGE_BYTES = MBH * 16 * (DA_PITCH + HB_PITCH);
  constexpr int LDS_BYTES = RING + WRING > STAGE_BYTES ? RING + WRING : STAGE_BYTES;
  __shared__ __attribute__((aligned(1024))) char s_lds[LDS_BYTES];
  __shared__ int s_tok[TM];
  __shared__ int s_pair[TM];
  __shared__ float s_w[TM];
  __shared__ float s_dtw[5][TM];
  __shared__ int s_loc[3];
  char* s_da = s_lds;                   // epilogue staging, over the ring
  char* s_hb = s_lds + MBH * 16 * DA_PITCH;
  auto ring = [&](int s) __attribute__((always_inline)) { return s_lds + (s % S) * NA * A_BYTES; };
  auto wring = [&](int s) __attribute__((always_inline)) { return s_lds + RING + (s % S) * WB; };

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + TM - 1) / TM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * TM;
  const int rows = min(TM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const char* P1 = p.p_in + (int64_t)g * p.in_nb * p.in_kb * G::PKB + lane * G::FRAGB;
  // W_out fragments reach LDS by LDS-DMA copies in the token tiles' swizzled row layout:
  // copy slot l of fragment jb holds chunk (l % 4) ^ swz(l / 4) of W_out row jb * 16 + l / 4,
  // so each lane quad reads one row's 64 contiguous bytes (a register load in the MFMA lane
  // order makes every quad touch four rows, three times the address-unit cycles), and the
  // step reads the fragment back with frag_sw.
  const T* Wout = per_group<T>(p.w_out, p.w_sh_out, g, p.E, (int64_t)H * d);
  const int wo_row = lane >> 2, wo_chunk = (lane & 3) ^ swz<DT>(lane >> 2);
  const int nk = p.in_kb;

  struct WSet {
    Frag f[GI > 0 ? GI : 1];  // the packed W_in gate / up fragments (recomputing a1 only)
  };
  auto load_w = [&](int s) __attribute__((always_inline)) -> WSet {
    const int k0 = s * G::KC;
    WSet w;
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int jb = wave * NBW + j;
      if constexpr (!SA) {
        w.f[j] = M::load(P1 + ((int64_t)jb * nk + s) * G::PKB);
        w.f[NBW + j] = M::load(P1 + ((int64_t)(HPMAX / 16 + jb) * nk + s) * G::PKB);
      }
      const int n = jb * 16 + wo_row;
      async_copy16(n < H ? (const void*)(Wout + (int64_t)n * d + k0 + wo_chunk * G::VE)
                         : (const void*)zero,
                   wring(s) + (wave * NBW + j) * 1024);
    }
    return w;
  };
  WSet wset[D];
#pragma unroll
  for (int j = 0; j < D; ++j) wset[j] = load_w(j);

  const bool routed = g < p.E;
  if (tid < TM) {
    int tok = -1, pair = -1;
    if (tid < rows) {
      if (routed) {
        pair = p.sorted_ids[slot0 + tid];
        tok = pair / p.k;
      } else {
        tok = m0 + tid;
      }
    }
    s_tok[tid] = tok;
    s_pair[tid] = pair;
    s_dtw[4][tid] = 0.0f;
  }
  __syncthreads();

  // Copy slot q (16 bytes) holds chunk (q % 4) ^ swz(r) of row r = q / 4.
  const T* xrow[XC];
  const T* drow[XC];
#pragma unroll
  for (int x = 0; x < XC; ++x) {
    const int cl = min(64, TM - 64 * x);
    const int q = 256 * x + cl * wave + lane, ar = q >> 2, ac = (q & 3) ^ swz<DT>(ar);
    const int atok = lane < cl ? s_tok[ar] : -1;
    xrow[x] = atok >= 0 ? (const T*)p.x + (int64_t)atok * d + ac * G::VE : nullptr;
    drow[x] = atok >= 0 ? (const T*)p.dout + (int64_t)atok * d + ac * G::VE : nullptr;
  }
  auto issue_x = [&](int s) __attribute__((always_inline)) {
    char* st = ring(s);
    const int k0 = s * G::KC;
#pragma unroll
    for (int x = 0; x < XC; ++x) {
      const int cl = min(64, TM - 64 * x);
      char* dst = st + 4096 * x + wave * cl * 16;
      if (cl == 64 || lane < cl) {
        if constexpr (!SA)
          async_copy16(xrow[x] ? (const void*)(xrow[x] + k0) : (const void*)zero, dst);
        async_copy16(drow[x] ? (const void*)(drow[x] + k0) : (const void*)zero, dst + DOFF);
      }
    }
  };
  // With SA, the forward's pre-activations of this lane's rows and columns (8 bytes of
  // gate and 8 of up per 16 x 16 block, act_block's layout: one 512-byte block per wave
  // and load; zeros outside the tile), into registers for the epilogue.  They go out
  // before the copies, so the first step's wait covers them and the steady state counts
  // stay those of the copies and weights alone.
  uint2 a1g[MB][NBW], a1u[MB][NBW];
  if constexpr (SA) {
    const T* A1 = (const T*)p.a1_in + act_block(p, g, m0) * (twoH / 16) * 256 + lane * 4;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int jb = wave * NBW + j;
        const bool ok = i * 16 + lc < rows && jb * 16 < H;
        const T* blk = A1 + (int64_t)i * (twoH / 16) * 256;
        a1g[i][j] = *(const uint2*)(ok ? (const char*)(blk + jb * 256) : zero);
        a1u[i][j] = *(const uint2*)(ok ? (const char*)(blk + (H / 16 + jb) * 256) : zero);
      }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) issue_x(j);
  // The gate weight of row tid % TM, needed only by the epilogue: its load goes out after
  // the copies, so the copies do not wait for it.  Every lane issues it (a zero word for
  // rows without one), which keeps each wave's count of outstanding loads uniform.
  const int wr = tid % TM;
  const int wpair = routed && wr < rows ? s_pair[wr] : -1;
  const T wraw = *(wpair >= 0 ? (const T*)p.topk_w + wpair : (const T*)g_zero_kib);

  f32x4 accg[MB][NBW], accu[MB][NBW], accG[MB][NBW];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int j = 0; j < NBW; ++j)
      accg[i][j] = accu[i][j] = accG[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](int s, const WSet& w) __attribute__((always_inline)) {
    barrier_dma();
    const char* st = ring(s);
    Frag gw[NBW];
#pragma unroll
    for (int j = 0; j < NBW; ++j) gw[j] = frag_sw<DT>(wring(s) + (wave * NBW + j) * 1024, 0);
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const Frag df = frag_sw<DT>(st + DOFF, i * 16);
      if constexpr (!SA) {
        const Frag xf = frag_sw<DT>(st, i * 16);
#pragma unroll
        for (int j = 0; j < NBW; ++j) {
          M::run(accg[i][j], w.f[j], xf);
          M::run(accu[i][j], w.f[NBW + j], xf);
        }
      }
#pragma unroll
      for (int j = 0; j < NBW; ++j) M::run(accG[i][j], gw[j], df);
    }
  };
  // Prologue order: w(0) .. w(D - 1) [row lookups] x(0) d(0) .. x(D - 1) d(D - 1), gate.
  // Every prologue load but step D - 1's copies and the gate weight: the steady-state
  // count below assumes that step s's copies are followed only by the loads of steps
  // s + 1 .. s + D - 1, which holds for the prologue steps below D - 1 only once their
  // copies are complete (and the gate load, older than every steady slot, is covered by
  // the first steady wait).
  wait_vmcnt<NA * XC + 1>();
  int s = 0;
  for (; s + D < nk; s += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      wait_vmcnt<(D - 1) * SLOT>();  // step s + j's weights and copies have landed
      mma(s + j, wset[j]);
      wset[j] = load_w(s + j + D);
      issue_x(s + j + D);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wait_vmcnt_dyn((D - 1 - j) * SLOT);  // a constant once unrolled
    mma(s + j, wset[j]);
  }
  if (tid < TM) s_w[tid] = routed ? (wr < rows ? Elem<DT>::to_f(wraw) : 0.0f) : (tid < rows ? 1.0f : 0.0f);
  wait_lgkm0();
  barrier_dma();  // every wave is done with the ring: the staging may overwrite it

  // ---- GLU backward, lane-local: lane (lc, lg) of block (i, j) holds row i*16 + lc,
  // hidden columns n0 .. n0 + 3 ----
  // (The saved pre-activations already carry the bias.)
  const T* bin = !SA && (g < p.E ? p.b_in : p.b_sh_in)
                     ? per_group<T>(p.b_in, p.b_sh_in, g, p.E, twoH) : nullptr;
  float wrow[MB], part[MB];
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    wrow[i] = s_w[i * 16 + lc];
    part[i] = 0.0f;
  }
  T* DA = (T*)p.da1 + slot0 * twoH;
  T* HB = (T*)p.hbuf + slot0 * H;
  const int da_cpr = twoH / G::VE, hb_cpr = H / G::VE;
  with_act(p.act, [&]<int ACT>() {
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int ib = pass * MBH, ie = pass ? MB : MBH;  // row blocks [ib, ie) of this pass
      if (pass) {
        __syncthreads();  // the first pass's stores have read the staging
      }
#pragma unroll
      for (int j = 0; j < NBW; ++j) {
        const int n0 = (wave * NBW + j) * 16 + lg * 4;
        if (n0 >= H) continue;  // H % 4 == 0: a group of 4 columns is all in or all out
        float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
        if (bin) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            bg[r] = Elem<DT>::to_f(bin[n0 + r]);
            bu[r] = Elem<DT>::to_f(bin[H + n0 + r]);
          }
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          if (i < ib || i >= ie) continue;  // resolved at compile time once unrolled
          const int m = (i - ib) * 16 + lc;  // the row's place in the staging
          const float w = wrow[i];
          float dg[4], du[4], wh[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float gg, uu;
            if constexpr (SA) {
              gg = unpack2<DT>(r < 2 ? a1g[i][j].x : a1g[i][j].y, r & 1);
              uu = unpack2<DT>(r < 2 ? a1u[i][j].x : a1u[i][j].y, r & 1);
            } else {
              gg = accg[i][j][r] + bg[r];
              uu = accu[i][j][r] + bu[r];
            }
            const float Gv = accG[i][j][r];
            float a, da;
            act_both_t<ACT>(gg, a, da);
            const float hv = a * uu;
            part[i] += Gv * hv;
            const float dh = w * Gv;
            dg[r] = dh * uu * da;
            du[r] = dh * a;
            wh[r] = w * hv;
          }
          char* da_row = s_da + m * DA_PITCH;
          *(uint2*)(da_row + n0 * G::ES) =
              make_uint2(pack2<DT>(dg[0], dg[1]), pack2<DT>(dg[2], dg[3]));
          *(uint2*)(da_row + (H + n0) * G::ES) =
              make_uint2(pack2<DT>(du[0], du[1]), pack2<DT>(du[2], du[3]));
          *(uint2*)(s_hb + m * HB_PITCH + n0 * G::ES) =
              make_uint2(pack2<DT>(wh[0], wh[1]), pack2<DT>(wh[2], wh[3]));
        }
      }
      __syncthreads();
      // Whole rows out: dA1 rows of 2H elements, w h rows of H elements, 16-byte chunks.
      const int r0 = ib * 16, nr = (ie - ib) * 16;
      for (int c = tid; c < nr * da_cpr; c += NT) {
        const int ml = c / da_cpr, cc = c - ml * da_cpr;
        if (r0 + ml < rows) {
          const int col = cc * G::VE;  // the staged row has the final layout: [gate H | up H]
          *(u32x4*)(DA + (int64_t)(r0 + ml) * twoH + col) =
              *(const u32x4*)(s_da + ml * DA_PITCH + col * G::ES);
        }
      }
      for (int c = tid; c < nr * hb_cpr; c += NT) {
        const int ml = c / hb_cpr, cc = c - ml * hb_cpr;
        if (r0 + ml < rows)
          *(u32x4*)(HB + (int64_t)(r0 + ml) * H + cc * G::VE) =
              *(const u32x4*)(s_hb + ml * HB_PITCH + cc * 16);
      }
    }
  });
  // dtopk_w: sum of G h over the row's hidden columns (4 lanes per wave, then 4 waves).
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    float v = part[i];
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    if (lg == 0) s_dtw[wave][i * 16 + lc] = v;
  }
  // <dout[tok], b_out[g]>: four lanes per row, strided over d.
  if (g < p.E && p.b_out) {
    const T* bo = (const T*)p.b_out + (int64_t)g * d;
    for (int m0r = 0; m0r < TM; m0r += NT / 4) {  // the same trip count in every lane
      const int m = m0r + (tid >> 2), q = tid & 3;
      float v = 0.0f;
      if (m < rows) {
        const T* dr = (const T*)p.dout + (int64_t)s_tok[m] * d;
        for (int c = q; c < d; c += 4) v += Elem<DT>::to_f(dr[c]) * Elem<DT>::to_f(bo[c]);
      }
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      if (q == 0 && m < rows) s_dtw[4][m] = v;
    }
  }
  __syncthreads();
  if (g < p.E && tid < rows) {
    const float v = s_dtw[0][tid] + s_dtw[1][tid] + s_dtw[2][tid] + s_dtw[3][tid] + s_dtw[4][tid];
    ((T*)p.dtw)[s_pair[tid]] = Elem<DT>::from_f(v);
  }
}

// Rows of a wave's 48-column slice of one 192-column pass, straight from the MFMA
// accumulators (acc[i][j]: row block i, column block j; lane (lc, lg) holds columns
// 4 lg .. 4 lg + 3 of row lc in each), rounded to the element type (store_block48).
template <int DT, int MB>
__device__ __forceinline__ void store_rows_direct(const f32x4 (&acc)[MB][3],
                                                  typename Elem<DT>::T* Y, int d, int rows,
                                                  int cw, int lane) {
#pragma unroll
  for (int i = 0; i < MB; ++i) {
    uint32_t lo[3], hi[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      lo[j] = pack2<DT>(acc[i][j][0], acc[i][j][1]);
      hi[j] = pack2<DT>(acc[i][j][2], acc[i][j][3]);
    }
    store_block48<DT>(lo, hi, Y, d, i * 16, rows, cw, lane);
  }
}

// Launched with 64-row tiles (MB = 4); 96-row tiles take expert_dx_res_kernel.
template <int DT, int D, int MB>
__global__ void __launch_bounds__(NT, D > 2 || MB == 6 ? 3 : 2) expert_dx_reg_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  static_assert(D >= 2 && D <= 4, "prefetch distance");
  static_assert(MB == 4 || MB == 6, "64- or 96-row tiles");
  constexpr int TM = MB * 16;            // tile rows
  constexpr int XC = MB == 4 ? 1 : 2;    // dA1 copies per wave per step
  constexpr bool STAGE_Y = MB == 4;      // 64-row tiles stage each pass of dX rows in LDS
  constexpr int S = D + 1;
  constexpr int A_BYTES = TM * G::ROWB;
  constexpr int NBF = 3;
  constexpr int SLOT = NBF + XC;
  constexpr int Y_PITCH = NP2 * G::ES + 16;
  __shared__ __attribute__((aligned(1024))) char s_ring[S][A_BYTES];
  __shared__ __attribute__((aligned(16))) char s_y[STAGE_Y ? TM * Y_PITCH : 16];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + TM - 1) / TM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * TM;
  const int rows = min(TM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = p.d, twoH = 2 * p.H;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const T* Win = per_group<T>(p.w_in, p.w_sh_in, g, p.E, (int64_t)d * twoH);
  const int wq = (lane & 3) * 8;  // this lane's k offset in a quad-major fragment
  const int fq = bperm_from_quads(lane);
  const int nkk = twoH / G::KC;  // <= KMAX in the resident-tile kernel (the launcher checks)
  const int npass = (d + NP2 - 1) / NP2;
  const int nsteps = npass * nkk;

  struct WSet {
    Frag f[NBF];
  };
  // W_in fragments in the quad-major lane order (lane 4 r + q: row 16 block + r, 16-byte
  // chunk q of the k-step), moved to the MFMA order with ds_bpermute when the step runs.
  auto load_w = [&](int s) __attribute__((always_inline)) -> WSet {
    const int pass = s / nkk, k0 = (s - pass * nkk) * G::KC;
    WSet w;
#pragma unroll
    for (int j = 0; j < NBF; ++j) {
      const int c = (pass * (NP2 / 16) + wave * 3 + j) * 16 + (lane >> 2);
      w.f[j] = M::load(c < d ? (const char*)(Win + (int64_t)c * twoH + k0 + wq) : zero);
    }
    return w;
  };
  // dA1 copies: copy slot c (16 bytes) holds chunk (c % 4) ^ swz(r) of row r = c / 4.  The
  // first copy of wave w fills slots 256 w / 4 ... = tid; for 96 rows the second fills
  // slots 256 + 32 w + lane (lanes < 32), rows 64 + 8 w + lane / 4.
  const int ar = tid >> 2, ac = (tid & 3) ^ swz<DT>(ar);
  const T* arow = ar < rows ? (const T*)p.da1 + (slot0 + ar) * twoH + ac * G::VE : nullptr;
  const T* arow2 = nullptr;
  if constexpr (XC == 2) {
    const int r2 = 64 + wave * 8 + (lane >> 2);
    const int ac2 = (lane & 3) ^ swz<DT>(r2);
    if (lane < 32 && r2 < rows) arow2 = (const T*)p.da1 + (slot0 + r2) * twoH + ac2 * G::VE;
  }
  auto issue_x = [&](int s) __attribute__((always_inline)) {
    const int k0 = (s % nkk) * G::KC;
    async_copy16(arow ? (const void*)(arow + k0) : (const void*)zero, s_ring[s % S] + wave * 1024);
    if constexpr (XC == 2) {
      if (lane < 32)
        async_copy16(arow2 ? (const void*)(arow2 + k0) : (const void*)zero,
                     s_ring[s % S] + 4096 + wave * 512);
    }
  };
  // Step s's weights and copies are issued together, D steps ahead of its MFMAs.
  WSet wset[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wset[j] = load_w(j);
    issue_x(j);
  }

  T* DX = (T*)p.dxrow + slot0 * d;
  f32x4 acc[MB][3];
  auto step = [&](int s, const WSet& w) __attribute__((always_inline)) {
    const int pass = s / nkk, kk = s - pass * nkk;
    if (kk == 0) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    Frag wf[NBF];
#pragma unroll
    for (int j = 0; j < NBF; ++j) wf[j].v = bperm4(fq, w.f[j].v);
    barrier_dma();
    const char* st = s_ring[s % S];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const Frag af = frag_sw<DT>(st, i * 16);
#pragma unroll
      for (int j = 0; j < 3; ++j) M::run(acc[i][j], wf[j], af);
    }
    if constexpr (!STAGE_Y) {
      if (kk == nkk - 1) store_rows_direct<DT, MB>(acc, DX, d, rows, pass * NP2 + wave * 48,
                                                    lane);
    } else if (kk == nkk - 1) {  // the pass's 192 columns: staged, then whole row segments out
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int c0 = (wave * 3 + j) * 16 + lg * 4;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const int m = i * 16 + lc;
          *(uint2*)(s_y + m * Y_PITCH + c0 * G::ES) =
              make_uint2(pack2<DT>(acc[i][j][0], acc[i][j][1]),
                         pack2<DT>(acc[i][j][2], acc[i][j][3]));
        }
      }
      wait_lgkm0();
      barrier_dma();
      const int ncols = min(NP2, d - pass * NP2);
      constexpr int CPR = NP2 / G::VE;
#pragma unroll
      for (int u = 0; u < TM * CPR / NT; ++u) {
        const int c = tid + u * NT, m = c / CPR, cc = c % CPR;
        if (m < rows && cc * G::VE < ncols)
          *(u32x4*)(DX + (int64_t)m * d + pass * NP2 + cc * G::VE) =
              *(const u32x4*)(s_y + m * Y_PITCH + cc * 16);
      }
      wait_lgkm0();
      barrier_dma();  // the staging is read out before the next pass writes it
    }
  };
  int s = 0;
  for (; s + D < nsteps; s += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      wait_vmcnt<(D - 1) * SLOT>();  // only steps s + j + 1 .. s + j + D - 1 in flight
      step(s + j, wset[j]);
      wset[j] = load_w(s + j + D);
      issue_x(s + j + D);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wait_vmcnt_dyn((D - 1 - j) * SLOT);  // a constant once unrolled
    step(s + j, wset[j]);
  }
  wait_vmcnt<0>();
}

// expert_dx_res: the same dX rows for 96-row tiles, with the tile's dA1 rows (all 2H
// columns: at most 8 k-steps of 32, 48 KiB) copied into LDS once and kept there for the
// whole tile.  The ring kernel above copies each k-step again for every pass over the
// output columns (3 passes at d = 576), and at 3 workgroups per CU those re-reads miss the
// XCD's L2 (a tile's 48 KiB times 96 workgroups per XCD is past its 4 MiB): measured
// FETCH_SIZE 2.4x the kernel's algorithmic reads.  With the tile resident, dA1 is read
// once; the k-loop streams only the weight fragments, D steps ahead, and holds no
// barrier (nothing is written to LDS after the copies land).
template <int DT, int D>
__global__ void __launch_bounds__(NT, 3) expert_dx_res_kernel(ExpParams p) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  static_assert(G::ES == 2, "16-bit types only");
  static_assert(D >= 2 && D <= 4, "prefetch distance");
  constexpr int MB = 6, TM = MB * 16;
  constexpr int KMAX = 8;                 // resident k-steps: 2H <= 256
  constexpr int A_BYTES = TM * G::ROWB;   // one k-step of the tile
  constexpr int NBF = 3;                  // weight fragments per wave per step
  __shared__ __attribute__((aligned(1024))) char s_tile[KMAX][A_BYTES];
  __shared__ int s_loc[3];

  const int tile = tile_of_block(p);
  Located loc;
  if (!locate(tile, p.E + p.S, [&](int g) { return (rows_of(p, g) + TM - 1) / TM; },
              [](int) { return 0; }, s_loc, loc))
    return;
  const int g = loc.g, m0 = loc.local * TM;
  const int rows = min(TM, rows_of(p, g) - m0);
  const int64_t slot0 = row_start(p, g) + m0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int d = p.d, twoH = 2 * p.H;
  const char* zero = (const char*)g_zero_kib + lane * 16;
  const T* Win = per_group<T>(p.w_in, p.w_sh_in, g, p.E, (int64_t)d * twoH);
  const int wq = (lane & 3) * 8;  // this lane's k offset in a quad-major fragment
  const int fq = bperm_from_quads(lane);
  const int nkk = twoH / G::KC;  // <= KMAX in the resident-tile kernel (the launcher checks)
  const int npass = (d + NP2 - 1) / NP2;
  const int nsteps = npass * nkk;

  // The tile's dA1 rows, every k-step, in the ring kernel's swizzled stage layout: slot c
  // of stage kk holds chunk (c % 4) ^ swz(r) of row r = c / 4, k-step kk.  Copy one of
  // wave w fills slots 64 w .. 64 w + 63 (rows 16 w .. 16 w + 15); copy two (lanes < 32)
  // rows 64 + 8 w + lane / 4.  Rows past the tile read the zero page.
  {
    const int ar = tid >> 2, ac = (tid & 3) ^ swz<DT>(ar);
    const T* arow = ar < rows ? (const T*)p.da1 + (slot0 + ar) * twoH + ac * G::VE : nullptr;
    const int r2 = 64 + wave * 8 + (lane >> 2);
    const int ac2 = (lane & 3) ^ swz<DT>(r2);
    const T* arow2 =
        lane < 32 && r2 < rows ? (const T*)p.da1 + (slot0 + r2) * twoH + ac2 * G::VE : nullptr;
    for (int kk = 0; kk < nkk; ++kk) {  // uniform
      const int k0 = kk * G::KC;
      async_copy16(arow ? (const void*)(arow + k0) : (const void*)zero,
                   s_tile[kk] + wave * 1024);
      if (lane < 32)
        async_copy16(arow2 ? (const void*)(arow2 + k0) : (const void*)zero,
                     s_tile[kk] + 4096 + wave * 512);
    }
  }

  struct WSet {
    Frag f[NBF];
  };
  // W_in fragments in the quad-major lane order (lane 4 r + q: row 16 block + r, 16-byte
  // chunk q of the k-step), moved to the MFMA order with ds_bpermute when the step runs.
  auto load_w = [&](int s) __attribute__((always_inline)) -> WSet {
    const int pass = s / nkk, k0 = (s - pass * nkk) * G::KC;
    WSet w;
#pragma unroll
    for (int j = 0; j < NBF; ++j) {
      const int c = (pass * (NP2 / 16) + wave * 3 + j) * 16 + (lane >> 2);
      w.f[j] = M::load(c < d ? (const char*)(Win + (int64_t)c * twoH + k0 + wq) : zero);
    }
    return w;
  };
  WSet wset[D];
#pragma unroll
  for (int j = 0; j < D; ++j) wset[j] = load_w(j);
  // The copies were issued before the D weight sets: once at most D * NBF operations are
  // outstanding, every copy of this wave has landed; the barrier publishes all waves'.
  wait_vmcnt<D * NBF>();
  barrier_dma();

  T* DX = (T*)p.dxrow + slot0 * d;
  f32x4 acc[MB][3];
  auto step = [&](int s, const WSet& w) __attribute__((always_inline)) {
    const int pass = s / nkk, kk = s - pass * nkk;
    if (kk == 0) {
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    Frag wf[NBF];
#pragma unroll
    for (int j = 0; j < NBF; ++j) wf[j].v = bperm4(fq, w.f[j].v);
    const char* st = s_tile[kk];
#pragma unroll
    for (int i = 0; i < MB; ++i) {
      const Frag af = frag_sw<DT>(st, i * 16);
#pragma unroll
      for (int j = 0; j < 3; ++j) M::run(acc[i][j], wf[j], af);
    }
    if (kk == nkk - 1)
      store_rows_direct<DT, MB>(acc, DX, d, rows, pass * NP2 + wave * 48, lane);
  };
  int s = 0;
  for (; s + D < nsteps; s += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      wait_vmcnt<(D - 1) * NBF>();  // weight set s + j has landed
      step(s + j, wset[j]);
      wset[j] = load_w(s + j + D);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wait_vmcnt_dyn((D - 1 - j) * NBF);  // a constant once unrolled
    step(s + j, wset[j]);
  }
  wait_vmcnt<0>();
}

static int device_cus();
static int64_t tile_grid(const ExpParams& p, int bm);

template <int DT, int MB, bool SA>
static void bwd_reg_launch_mb(const ExpParams& p, int nbw, int dist, hipStream_t s) {
  const unsigned grid = (unsigned)tile_grid(p, 16 * MB);
  if constexpr (SA) {  // distance 4 only without the gate / up accumulators
    if (dist == 4) {
      if (nbw == 1) expert_bwd_reg_kernel<DT, 1, 4, MB, SA><<<grid, NT, 0, s>>>(p);
      else expert_bwd_reg_kernel<DT, 2, 4, MB, SA><<<grid, NT, 0, s>>>(p);
      return;
    }
  }
  if (dist == 3) {
    if (nbw == 1) expert_bwd_reg_kernel<DT, 1, 3, MB, SA><<<grid, NT, 0, s>>>(p);
    else expert_bwd_reg_kernel<DT, 2, 3, MB, SA><<<grid, NT, 0, s>>>(p);
  } else {
    if (nbw == 1) expert_bwd_reg_kernel<DT, 1, 2, MB, SA><<<grid, NT, 0, s>>>(p);
    else expert_bwd_reg_kernel<DT, 2, 2, MB, SA><<<grid, NT, 0, s>>>(p);
  }
}

template <int DT, bool SA>
static void bwd_reg_launch_sa(const ExpParams& p, int nbw, int dist, int mb, hipStream_t s) {
  if constexpr (SA) {  // 96-row tiles only without the gate / up accumulators
    if (mb == 6) return bwd_reg_launch_mb<DT, 6, SA>(p, nbw, dist, s);
  }
  if (mb == 3) bwd_reg_launch_mb<DT, 3, SA>(p, nbw, dist, s);
  else if (mb == 5) bwd_reg_launch_mb<DT, 5, SA>(p, nbw, dist, s);
  else bwd_reg_launch_mb<DT, 4, SA>(p, nbw, dist, s);
}

template <int DT>
static void bwd_reg_launch(const ExpParams& p, int nbw, int dist, int mb, hipStream_t s) {
  if (p.a1_in) bwd_reg_launch_sa<DT, true>(p, nbw, dist, mb, s);
  else bwd_reg_launch_sa<DT, false>(p, nbw, dist, mb, s);
}

template <int DT>
static void dx_reg_launch(const ExpParams& p, int mb, int dist, hipStream_t s) {
  const unsigned g4 = (unsigned)tile_grid(p, 64), g6 = (unsigned)tile_grid(p, 96);
  // The register-tiled path takes H <= 128, so a 96-row tile's dA1 rows (2H <= 256
  // columns) always fit the resident 48 KiB.
  if (mb == 6) {
    if (dist == 4) expert_dx_res_kernel<DT, 4><<<g6, NT, 0, s>>>(p);
    else if (dist == 3) expert_dx_res_kernel<DT, 3><<<g6, NT, 0, s>>>(p);
    else expert_dx_res_kernel<DT, 2><<<g6, NT, 0, s>>>(p);
  } else {
    if (dist == 4) expert_dx_reg_kernel<DT, 4, 4><<<g4, NT, 0, s>>>(p);
    else if (dist == 3) expert_dx_reg_kernel<DT, 3, 4><<<g4, NT, 0, s>>>(p);
    else expert_dx_reg_kernel<DT, 2, 4><<<g4, NT, 0, s>>>(p);
  }
}

int launch_bwd_async(int dtype, const ExpParams& p, int nbw, int64_t grid, int part,
                     hipStream_t s) {
  if (!p.fast || nbw > 2 || (dtype != DT_BF16 && dtype != DT_F16)) return -1;
  if (grid <= 0) return NSMOE_OK;
  const int nsteps_dx = ((p.d + NP2 - 1) / NP2) * (2 * p.H / 32);
  if (p.d % 64 == 0 && (2 * p.H) % 32 == 0 && nsteps_dx % 2 == 0 && p.in_kb >= 4) {
    if (part == 0) {
      // 64-row tiles at 2 workgroups per CU with weight prefetch distance 3 (where the step
      // count divides by 3, else 2); once those tiles overflow one round of the resident
      // slots, 48-row tiles at distance 2, whose 162 registers fit 3 workgroups per CU (at
      // T = 8192: 1406 tiles over 768 slots instead of 1064 over 512, the last third of a
      // round nearly empty).  The "bwd_rows" / "bwd_dist" options force a tile height and
      // a distance; 80-row tiles take distance 2, which is all their registers allow.
      // With the forward's pre-activations saved (p.a1_in) the kernel streams dout alone
      // and holds no gate / up accumulators: 96-row tiles are allowed as well, and
      // distance 4 where the step count divides by 4.
      // The tile heights and distances measured fastest at T = 8192 (nanoSpeaker's
      // shape): without the saved pre-activations 48-row tiles at distance 2 once 64-row
      // tiles overflow two workgroups per CU; with them 96-row tiles at distance 2 once
      // 64-row tiles overflow three workgroups per CU (the epilogue's two staging passes
      // let 96-row tiles keep three per CU: at T = 8192 ~760 tiles in one round of the
      // 768 slots instead of ~1060 over two), else 64-row tiles at distance 3.  96-row
      // tiles take distance 2 only (a third stage would cost the third workgroup).
      const int64_t slots3 = 3 * (int64_t)device_cus();
      int mb = p.a1_in ? (tile_grid(p, 64) > slots3 ? 6 : 4)
                       : (tile_grid(p, 64) > 2 * (int64_t)device_cus() ? 3 : 4);
      if (const int64_t v = option(OPT_BWD_ROWS)) mb = (int)(v / 16);
      if (mb < 3 || mb > (p.a1_in ? 6 : 5)) mb = 4;
      int dist = mb != 3 && p.in_kb % 3 == 0 ? 3 : 2;
      if (const int64_t v = option(OPT_BWD_DIST))
        if ((v == 2 || v == 3 || (v == 4 && p.a1_in)) && p.in_kb % v == 0) dist = (int)v;
      if (mb >= 5 && !p.a1_in) dist = 2;
      if (mb == 6) dist = 2;
      KernelTimer timer("expert_bwd", s);
      if (dtype == DT_BF16) bwd_reg_launch<DT_BF16>(p, nbw, dist, mb, s);
      else bwd_reg_launch<DT_F16>(p, nbw, dist, mb, s);
      timer.stop();
      return check_launch("expert_bwd_reg_kernel");
    }
    // 96-row tiles once 64-row tiles overflow the resident workgroup slots (3 per CU), as
    // in the forward; weight prefetch distance 2 steps.  The "dx_rows" / "dx_dist" options
    // force a tile height and a distance.
    int mb = tile_grid(p, 64) > 3 * (int64_t)device_cus() ? 6 : 4;
    if (const int64_t v = option(OPT_DX_ROWS)) mb = (int)(v / 16);
    int dist = 2;
    if (const int64_t v = option(OPT_DX_DIST))
      if (nsteps_dx % v == 0) dist = (int)v;
    KernelTimer timer("expert_dx", s);
    if (dtype == DT_BF16) dx_reg_launch<DT_BF16>(p, mb, dist, s);
    else dx_reg_launch<DT_F16>(p, mb, dist, s);
    timer.stop();
    return check_launch("expert_dx_reg_kernel");
  }
  if (part == 0) {
    constexpr int S = 2;
    KernelTimer timer("expert_bwd", s);
    if (dtype == DT_BF16) {
      if (nbw == 1) expert_bwd_async_kernel<DT_BF16, 1, S><<<(unsigned)grid, NT, 0, s>>>(p);
      else expert_bwd_async_kernel<DT_BF16, 2, S><<<(unsigned)grid, NT, 0, s>>>(p);
    } else {
      if (nbw == 1) expert_bwd_async_kernel<DT_F16, 1, S><<<(unsigned)grid, NT, 0, s>>>(p);
      else expert_bwd_async_kernel<DT_F16, 2, S><<<(unsigned)grid, NT, 0, s>>>(p);
    }
    timer.stop();
    return check_launch("expert_bwd_async_kernel");
  }
  constexpr int S = 3;
  KernelTimer timer("expert_dx", s);
  if (dtype == DT_BF16) expert_dx_async_kernel<DT_BF16, S><<<(unsigned)grid, NT, 0, s>>>(p);
  else expert_dx_async_kernel<DT_F16, S><<<(unsigned)grid, NT, 0, s>>>(p);
  timer.stop();
  return check_launch("expert_dx_async_kernel");
}

// ============================ backward: dW ===============================================
//
// dW of one (group, row chunk, output tile), computed transposed:
//   D[n][m] = sum_r P[r][n] Q[r][m]
// where P rows carry the output's column index n (contiguous in dW) and Q rows its row
// index m, so each lane ends with 4 consecutive n of one m (8-byte dW stores, or 16-byte
// fp32 partials for groups split over several chunks).
//   MODE 0: dW_in[g]  [d, 2H] = sum_r x[tok_r]^T dA1[slot_r]      Q = x[tok], P = dA1[slot]
//   MODE 1: dW_out[g] [H, d]  = sum_r (w h)[slot_r]^T dout[tok_r] Q = w h,   P = dout[tok]
// Both operand tiles are 32 rows x tile width, row-major in LDS, filled by lane-linear
// async copies (the chunk swizzle applied on the source side) and read as MFMA operands
// with ds_read_b64_tr_b16, which transposes on the way out: no register transposes.
//
// Chunk swizzle: a transpose read of one fragment touches 2 chunks (32 B) of each of 4
// rows per 16 lanes; the swizzle spreads the 8 rows a half-wave reads over all 64 banks.
template <int ROWB>
__device__ __forceinline__ int dw_swz(int r) {
  static_assert(ROWB % 128 == 0, "rows of whole 128-byte lines");
  if constexpr (ROWB % 256 == 0) return ((r & 3) | (((r >> 3) & 1) << 2)) << 1;
  else return (((r >> 1) ^ (r >> 2)) & 3) << 1;
}

template <int MODE> struct DwTile;
template <> struct DwTile<0> {  // dW_in [d, 2H]: 192 x 128 tiles
  static constexpr int BMT = 192, BNT = 128, WM = 2, WN = 2;
};
template <> struct DwTile<1> {  // dW_out [H, d]: 128 x 192 tiles
  static constexpr int BMT = 128, BNT = 192, WM = 2, WN = 2;
};

template <int DT, int S>
struct DwLds {
  static constexpr int STAGE = Geo<DT>::KC * (DwTile<0>::BMT + DwTile<0>::BNT) * 2;
  static_assert(STAGE == Geo<DT>::KC * (DwTile<1>::BMT + DwTile<1>::BNT) * 2,
                "both modes stage the same bytes per step");
  char ring[S][STAGE];
  int tok[DW_RC];
  int loc[3];
};

// One (group, row chunk, output tile) item of dW; `item` indexes the mode's item space.
template <int DT, int MODE, int S>
__device__ __forceinline__ void dw_item(const ExpParams& p, int item, DwLds<DT, S>& L) {
  using G = Geo<DT>;
  using T = typename G::T;
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  using Tl = DwTile<MODE>;
  static_assert(G::ES == 2, "16-bit types only");
  constexpr int BMT = Tl::BMT, BNT = Tl::BNT;
  constexpr int TMB = BMT / 16 / Tl::WM, TNB = BNT / 16 / Tl::WN;  // blocks per wave
  constexpr int QROWB = BMT * 2, PROWB = BNT * 2;                 // LDS row bytes
  constexpr int QCPR = BMT / 8, PCPR = BNT / 8;                   // 16-byte chunks per row
  constexpr int QBYTES = G::KC * QROWB, PBYTES = G::KC * PROWB;
  constexpr int QBLK = QBYTES / 1024, PBLK = PBYTES / 1024;       // 1 KiB copy blocks
  constexpr int STAGE = QBYTES + PBYTES;
  constexpr int NBLK = QBLK + PBLK;
  static_assert(NBLK % 4 == 0, "copy blocks split evenly over the 4 waves");
  constexpr int LOADS = NBLK / 4;
  static_assert(STAGE == DwLds<DT, S>::STAGE, "stage layout");
  auto& s_ring = L.ring;
  int* s_tok = L.tok;
  int* s_loc = L.loc;

  const int d = p.d, H = p.H, twoH = 2 * p.H;
  const int Md = MODE == 0 ? d : H;
  const int Nd = MODE == 0 ? twoH : d;
  const int tn = (Nd + BNT - 1) / BNT, ntiles = ((Md + BMT - 1) / BMT) * tn;
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
  const int m0 = (t / tn) * BMT, n0 = (t % tn) * BNT;
  const int r0 = chunk * DW_RC, nr = max(0, min(rows_g, r0 + DW_RC) - r0);
  const int64_t rs = row_start(p, g) + r0;
  const int tid = threadIdx.x, lane = tid & 63, lc = lane & 15, lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / Tl::WN, wn = wave % Tl::WN;

  // s_tok holds each row's token as an element offset, tok * d (int32: the launchers
  // require T * d < 2^31).
  for (int r = tid; r < nr; r += NT)
    s_tok[r] = (g < p.E ? p.sorted_ids[rs + r] / p.k : r0 + r) * d;
  __syncthreads();

  const T* X = (const T*)p.x;
  const T* DA = (const T*)p.da1;
  const T* HB = (const T*)p.hbuf;
  const T* DO = (const T*)p.dout;
  const T* zero = (const T*)((const char*)g_zero_kib + lane * 16);
  const int nsteps = (nr + G::KC - 1) / G::KC;

  // The copy plan, fixed for the item.  Copy u of this wave moves one 16-byte chunk of
  // the 1 KiB block b = 4u + wave: chunk column (swizzled on the source side) and row
  // crow[u] of the step.  Blocks [0, QBLK) are Q and the rest P; QBLK % 4 == 0 makes that a
  // compile-time property of u once the loops are unrolled.  The token operand (Q = x in
  // MODE 0, P = dout in MODE 1) is gathered through s_tok, whose entries for the next step
  // are read one issue ahead (ctok); the other operand's rows are consecutive slots, so
  // its source is csrc[u] + k0 * stride.  A chunk past the tile's columns gets a row no
  // step reaches, so it always reads the zero block.
  static_assert(QBLK % 4 == 0, "Q / P split known per copy");
  auto gathered = [](int u) { return (4 * u < QBLK) == (MODE == 0); };
  const int lstride = MODE == 0 ? twoH : H;
  int crow[LOADS], ctok[LOADS];
  const T* csrc[LOADS];
#pragma unroll
  for (int u = 0; u < LOADS; ++u) {
    const bool isq = 4 * u < QBLK;
    const int q = (isq ? 4 * u + wave : 4 * u + wave - QBLK) * 64 + lane;
    int row, col;
    bool ok;
    if (isq) {
      row = q / QCPR;
      col = m0 + ((q % QCPR) ^ dw_swz<QROWB>(row)) * 8;
      ok = col < Md;
    } else {
      row = q / PCPR;
      col = n0 + ((q % PCPR) ^ dw_swz<PROWB>(row)) * 8;
      ok = col < Nd;
    }
    crow[u] = ok ? row : (1 << 20);
    ctok[u] = 0;
    if (gathered(u)) csrc[u] = (MODE == 0 ? X : DO) + col;
    else csrc[u] = (MODE == 0 ? DA : HB) + (rs + row) * lstride + col;
  }
  const uint32_t ring = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)&L.ring[0][0];
  auto read_tok = [&](int s) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u)
      if (gathered(u)) ctok[u] = s_tok[s * G::KC + (crow[u] & 31)];
  };
  auto issue = [&](int s, int stage) {
    const int k0 = s * G::KC;
    const uint32_t dst = ring + stage * STAGE + wave * 1024;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
      const T* src = gathered(u) ? csrc[u] + ctok[u] : csrc[u] + (int64_t)k0 * lstride;
      async_copy16_to(k0 + crow[u] < nr ? src : zero, dst + 4 * u * 1024);
    }
    if (s + 1 < nsteps) read_tok(s + 1);
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
    const uint2 lo = lds_read_tr16(tile + ra * RB + ((c ^ dw_swz<RB>(ra)) << 4) + cb);
    const uint2 hi = lds_read_tr16(tile + rb * RB + ((c ^ dw_swz<RB>(rb)) << 4) + cb);
    Frag f;
    f.v = u32x4{lo.x, lo.y, hi.x, hi.y};
    return f;
  };

  f32x4 acc[TNB][TMB];
#pragma unroll
  for (int j = 0; j < TNB; ++j)
#pragma unroll
    for (int i = 0; i < TMB; ++i) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  // One k-step on ring stage ST (a compile-time constant, so every fragment read is a
  // per-lane offset plus an immediate).
  auto step = [&](int s, auto stage_tag) {
    constexpr int ST = decltype(stage_tag)::value;
    wait_for(s);
    barrier_lds();
    if (s + S - 1 < nsteps) issue(s + S - 1, (ST + S - 1) % S);
    const char* st = L.ring[ST];
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
  };
  if (nsteps > 0) read_tok(0);
  for (int s = 0; s < S - 1 && s < nsteps; ++s) issue(s, s);
  // Steps in groups of S, so step s + I sits on stage I.
  for (int s = 0; s < nsteps; s += S) {
    [&]<int... I>(std::integer_sequence<int, I...>) {
      (void)((s + I < nsteps ? (step(s + I, std::integral_constant<int, I>{}), true) : false) &&
             ...);
    }(std::make_integer_sequence<int, S>{});
  }
  wait_vmcnt<0>();

  const int64_t mn = (int64_t)Md * Nd;
  T* dst = nullptr;
  float* pdst = nullptr;
  if (nch == 1) dst = g < p.E ? (T*)p.dw_a + (int64_t)g * mn : (T*)p.dw_sh + (int64_t)(g - p.E) * mn;
  else pdst = p.partial + (int64_t)(loc.aux + chunk) * mn;
#pragma unroll
  for (int j = 0; j < TNB; ++j) {
    const int n = n0 + (wn * TNB + j) * 16 + lg * 4;
    if (n >= Nd) continue;  // Nd % 4 == 0
#pragma unroll
    for (int i = 0; i < TMB; ++i) {
      const int m = m0 + (wm * TMB + i) * 16 + lc;
      if (m >= Md) continue;
      const f32x4 v = acc[j][i];
      if (dst)
        *(uint2*)(dst + (int64_t)m * Nd + n) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
      else
        *(f32x4*)(pdst + (int64_t)m * Nd + n) = v;
    }
  }
}

// Output tiles per (group, row chunk) of a dW mode: the run of items that read the same
// token rows, dealt to one XCD together.
template <int MODE>
__device__ __forceinline__ int dw_run(const ExpParams& p) {
  using Tl = DwTile<MODE>;
  const int Md = MODE == 0 ? p.d : p.H, Nd = MODE == 0 ? 2 * p.H : p.d;
  return ((Md + Tl::BMT - 1) / Tl::BMT) * ((Nd + Tl::BNT - 1) / Tl::BNT);
}

// dW_in and dW_out items in one launch: blocks [0, grid_in) take dW_in items, the rest
// dW_out items (each part dealt over the XCDs on its own; grid_in is a multiple of 8 so
// that block b - grid_in sits on the same XCD as b).  One launch fills the machine's
// workgroup slots with both item sets instead of leaving a nearly empty round after each.
template <int DT, int S>
__global__ void __launch_bounds__(NT, 2) dw_pair_kernel(ExpParams p_in, ExpParams p_out,
                                                        int grid_in) {
  __shared__ __attribute__((aligned(1024))) DwLds<DT, S> lds;
  const int b = blockIdx.x;
  if (b < grid_in) dw_item<DT, 0, S>(p_in, xcd_deal(b, grid_in, dw_run<0>(p_in)), lds);
  else
    dw_item<DT, 1, S>(p_out, xcd_deal(b - grid_in, (int)gridDim.x - grid_in, dw_run<1>(p_out)),
                      lds);
}

int launch_dw_pair_async(int dtype, const ExpParams& q_in, const ExpParams& q_out,
                         int64_t groups_chunks, hipStream_t s) {
  if (!q_in.fast || (dtype != DT_BF16 && dtype != DT_F16)) return -1;
  if (q_in.T * q_in.d >= (int64_t(1) << 31)) return -1;  // token offsets are int32
  const int d = q_in.d, H = q_in.H;
  // Rounded up to whole XCD rounds (the extra items are past the last real one and exit).
  const int64_t g_in =
      cdiv(groups_chunks * cdiv(d, DwTile<0>::BMT) * cdiv(2 * H, DwTile<0>::BNT), 8) * 8;
  const int64_t g_out = groups_chunks * cdiv(H, DwTile<1>::BMT) * cdiv(d, DwTile<1>::BNT);
  if (g_in + g_out <= 0) return NSMOE_OK;
  // Ring stages: 2 (one step of copies in flight, two workgroups per CU), which
  // measured ~1% faster per training step than 3; the "dw_stages" option asks for 3 or 4.
  const int st = option(OPT_DW_STAGES) ? (int)option(OPT_DW_STAGES) : 2;
  KernelTimer timer("dw", s);
  const unsigned grid = (unsigned)(g_in + g_out);
  auto go = [&](auto dt_tag) {
    constexpr int DT = decltype(dt_tag)::value;
    if (st == 3) dw_pair_kernel<DT, 3><<<grid, NT, 0, s>>>(q_in, q_out, (int)g_in);
    else if (st == 4) dw_pair_kernel<DT, 4><<<grid, NT, 0, s>>>(q_in, q_out, (int)g_in);
    else dw_pair_kernel<DT, 2><<<grid, NT, 0, s>>>(q_in, q_out, (int)g_in);
  };
  if (dtype == DT_BF16) go(std::integral_constant<int, DT_BF16>{});
  else go(std::integral_constant<int, DT_F16>{});
  timer.stop();
  return check_launch("dw_pair_kernel");
}

// Compute units of the current device (cached per device).
static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Upper bound on the token tiles of `bm` rows over all groups (routed, then shared).
static int64_t tile_grid(const ExpParams& p, int bm) {
  const int64_t M = p.T * p.k;
  const int64_t nonempty = M < p.E ? M : p.E;
  return cdiv(M, bm) + nonempty + (int64_t)p.S * cdiv(p.T, bm);
}

template <int DT, int NBW>
static void fwd_reg_launch(const ExpParams& p, int mb, int dist, hipStream_t s) {
  if (mb == 2) {
    const unsigned g2 = (unsigned)tile_grid(p, 32);
    if (dist == 6) expert_fwd_reg_kernel<DT, NBW, 2, 6><<<g2, NT, 0, s>>>(p);
    else if (dist == 3) expert_fwd_reg_kernel<DT, NBW, 2, 3><<<g2, NT, 0, s>>>(p);
    else expert_fwd_reg_kernel<DT, NBW, 2, 2><<<g2, NT, 0, s>>>(p);
    return;
  }
  if (dist == 3) {
    if (mb == 6) expert_fwd_reg_kernel<DT, NBW, 6, 3><<<(unsigned)tile_grid(p, 96), NT, 0, s>>>(p);
    else expert_fwd_reg_kernel<DT, NBW, 4, 3><<<(unsigned)tile_grid(p, 64), NT, 0, s>>>(p);
  } else {
    if (mb == 6) expert_fwd_reg_kernel<DT, NBW, 6, 2><<<(unsigned)tile_grid(p, 96), NT, 0, s>>>(p);
    else expert_fwd_reg_kernel<DT, NBW, 4, 2><<<(unsigned)tile_grid(p, 64), NT, 0, s>>>(p);
  }
}

int launch_fwd_async(int dtype, const ExpParams& p, int nbw, int64_t grid, hipStream_t s) {
  if (!p.fast || nbw > 2 || (dtype != DT_BF16 && dtype != DT_F16)) return -1;
  if (grid <= 0) return NSMOE_OK;
  constexpr int S = 3;
  KernelTimer timer("expert_fwd", s);
  const int n2 = ((p.d + NP2 - 1) / NP2) * p.out_kb;
  if (p.d % 64 == 0 && n2 % 2 == 0) {
    // 96-row tiles once 64-row tiles overflow the resident workgroup slots (3 per CU);
    // 32-row tiles at prefetch distance 6 while 64-row tiles would fill under half the
    // CUs (decode-sized calls: a tile's time is its weight stream's latency, not its
    // rows).  The "fwd_rows" option forces a tile height.
    const int64_t g64 = tile_grid(p, 64);
    int mb = g64 > 3 * (int64_t)device_cus() ? 6 : 2 * g64 <= device_cus() ? 2 : 4;
    if (const int64_t v = option(OPT_FWD_ROWS)) mb = (int)(v / 16);
    // Prefetch distance 2 (6 for 32-row tiles); the "fwd_dist" option asks for another,
    // taken where both GEMMs' step counts are multiples of it (6: 32-row tiles only).
    const int nk1 = p.in_kb;
    auto divides = [&](int v) { return nk1 % v == 0 && n2 % v == 0; };
    int dist = mb == 2 && divides(6) ? 6 : 2;
    if (const int64_t v = option(OPT_FWD_DIST))
      if ((v == 2 || v == 3 || (v == 6 && mb == 2)) && divides((int)v)) dist = (int)v;
    if (dtype == DT_BF16) {
      if (nbw == 1) fwd_reg_launch<DT_BF16, 1>(p, mb, dist, s);
      else fwd_reg_launch<DT_BF16, 2>(p, mb, dist, s);
    } else {
      if (nbw == 1) fwd_reg_launch<DT_F16, 1>(p, mb, dist, s);
      else fwd_reg_launch<DT_F16, 2>(p, mb, dist, s);
    }
    timer.stop();
    return check_launch("expert_fwd_reg_kernel");
  }
  if (dtype == DT_BF16) {
    if (nbw == 1) expert_fwd_async_kernel<DT_BF16, 1, S><<<(unsigned)grid, NT, 0, s>>>(p);
    else expert_fwd_async_kernel<DT_BF16, 2, S><<<(unsigned)grid, NT, 0, s>>>(p);
  } else {
    if (nbw == 1) expert_fwd_async_kernel<DT_F16, 1, S><<<(unsigned)grid, NT, 0, s>>>(p);
    else expert_fwd_async_kernel<DT_F16, 2, S><<<(unsigned)grid, NT, 0, s>>>(p);
  }
  timer.stop();
  return check_launch("expert_fwd_async_kernel");
}

}  // namespace nsmoe

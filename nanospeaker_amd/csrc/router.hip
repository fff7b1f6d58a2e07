// The router on device, GEMM included: logits = x W_r, softmax, top-k with CPU torch.topk's
// tie order, gates, the per-chunk expert histogram the dispatch places from, and the
// balance loss's column sums -- MoEBlock.forward's routing (src/model/router.py:56-111)
// for 16-bit blocks, in one launch instead of a library GEMM, the router tail and the
// dispatch's histogram pass.
//
// router_fwd_kernel: one workgroup of 16 waves per 32 tokens (one workgroup per CU at
// T = 8192).  All 16 waves issue the W_r loads.
//   * GEMM, on 4 of the waves (16 tokens x half the experts each): v_mfma_f32_16x16x32 with
//     the token rows as the A operand and W_r as the B operand.  The workgroup's 32 token
//     rows (one contiguous 36 KiB block of x at d = 576) and W_r [d, E] (87.5 KiB at E = 76)
//     are both copied whole into LDS, untransposed, by 1 KiB LDS-DMA copies spread over
//     all 16 waves: one memory round trip and one barrier before the MFMAs, and every
//     lane quad reads 64 contiguous bytes (register loads in the MFMA lane order would
//     make each quad touch four rows).  W_r is stored
//     with the expert index contiguous, so its fragments are read with ds_read_b64_tr_b16,
//     which hands each lane 4 consecutive k of one expert column.  The fp32 sums are
//     rounded to the block's dtype -- the value router.py:69's GEMM produces -- stored as
//     the logits, and kept in LDS.
//   * Softmax and the selection, on 8 of the waves: one token per 16-lane DPP row, a lane
//     holding E / 16 of its experts.  The selection is k rounds of arg-max; a round whose
//     maximum is not unique among the values still in play (or a NaN in the row) leaves
//     the token to the exact pass, since only the restated library algorithm fixes the
//     order of equal keys.
//   * The exact pass, on all 16 waves: one undecided token per wave, the restatement of
//     CPU topk (topk_exact.h) on the keys as the selection saw them.  About 17 % of bf16
//     rows tie, 5.5 of a workgroup's 32 on average; with 16 waves no wave takes a second
//     row unless more than 16 of the 32 tie, so the pass costs one row's latency.
//   * With the RMSNorm in front (RouterArgs::norm_w), the GEMM waves normalise their rows
//     in registers between the load and the first MFMA (the row's sum of squares over its
//     4 lanes) and one of each row's two waves stores the normalised row; the norm's weight
//     arrives in LDS with W_r's copies.
//   * Per workgroup it leaves the expert histogram of its tokens (a chunk of 32 k pairs for
//     the dispatch's place pass) and, in training, the column sums of probs for the
//     balance loss.
#include "balance.h"
#include "gemm_core.h"
#include "nsmoe_capi_internal.h"
#include "router_fused.h"
#include "topk_exact.h"

namespace nsmoe {

constexpr int RT_SEL_WAVES = RT_TOK / 4;    // waves of the selection: 4 tokens per wave
constexpr int RT_PART_STEPS = 6;            // k-steps of W_r per part in the 8-wave form

// The two workgroup shapes (W waves, one workgroup of RT_TOK tokens either way):
//   W = 16: one workgroup per CU; W_r whole in LDS (87.5 KiB at d = 576, E = 76).
//   W = 8:  two workgroups per CU (under 80 KiB of LDS and 128 registers each), so that
//           one workgroup's selection and exact pass overlap the other's copies and
//           GEMM once the grid is more than one workgroup per CU.  W_r arrives in parts
//           of RT_PART_STEPS k-steps, double-buffered between the stage and the token
//           rows' area (free once the GEMM waves hold their rows in registers): part
//           p + 1 is copied while part p's MFMAs run.
template <int W>
struct RtShape {
  static_assert(W == 16 || W == 8, "workgroup shapes");
  static constexpr int THREADS = W * 64;
  static constexpr int SPLIT = W == 16 ? 5 : 4;  // GEMM waves per 16-token tile
  static constexpr int MMA_WAVES = RT_TOK / 16 * SPLIT;
  static constexpr int WR_STEPS = W == 16 ? RT_MAX_STEPS : RT_PART_STEPS;  // W_r in the stage
  static constexpr int PER_CU = W == 16 ? 1 : 2;
};

// 16-lane DPP butterflies: every lane of each row of 16 ends with the row's reduction.
template <class Op>
__device__ __forceinline__ float row16(float v, Op op) {
  v = op(v, dpp<0xB1>(v));   // quad_perm [1, 0, 3, 2]
  v = op(v, dpp<0x4E>(v));   // quad_perm [2, 3, 0, 1]
  v = op(v, dpp<0x141>(v));  // row_half_mirror
  v = op(v, dpp<0x140>(v));  // row_mirror
  return v;
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ int row16_sum_i(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  v += dpp_i<0x141>(v);
  v += dpp_i<0x140>(v);
  return v;
}

__device__ __forceinline__ int row16_min_i(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  return v;
}

__device__ __forceinline__ float fmax_(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float fadd_(float a, float b) { return a + b; }

template <int DT, int NB, int W>
__global__ void __launch_bounds__(W * 64, RtShape<W>::PER_CU) router_fwd_kernel(RouterArgs a) {
  using ET = typename Elem<DT>::T;
  using Sh = RtShape<W>;
  constexpr int RT_WAVES = W, RT_THREADS = Sh::THREADS;
  constexpr int NC = NB * 16;               // expert columns, padded to whole MFMA blocks
  // W_r in LDS (whole, or one part of it), row-major as in memory ([d, E], E * 2 bytes a
  // row), plus slack: the last row's padding columns [E, NC) read past its end (their
  // logits are dropped).
  constexpr int WR_BYTES = Sh::WR_STEPS * 32 * RT_MAX_E * 2 + 64;
  constexpr int LGP = NC + 1;               // logit-tile pitch (floats)
  constexpr int POS = RT_WAVES * TOPK_SWAP_SLOTS * (int)sizeof(int2);
  constexpr int STAGE = WR_BYTES > POS ? WR_BYTES : POS;
  // W_r during the GEMM; the exact pass's swap slots afterwards.
  __shared__ __align__(1024) char s_stage[STAGE];
  __shared__ __align__(1024) char s_nw[(RT_MAX_STEPS * 64 + 1023) / 1024 * 1024];  // norm w
  // The workgroup's RT_TOK token rows, d * 2 bytes each, one contiguous block of x, copied
  // whole by LDS-DMA (x_slot's chunk order inside each row).
  __shared__ __align__(1024) char s_x[RT_TOK * RT_MAX_STEPS * 64];
  static_assert(W == 16 || (int)sizeof(s_x) >= WR_BYTES, "a W_r part fits the rows' area");
  __shared__ float s_lg[RT_TOK * LGP];      // per token: the logits, then its keys
  __shared__ float s_bias[RT_MAX_E];
  __shared__ float s_m[RT_TOK], s_inv[RT_TOK];
  __shared__ int32_t s_hist[128];
  __shared__ int32_t s_tie[RT_TOK];
  __shared__ int32_t s_ntie;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, j = lane & 15;
  const int64_t T = a.T;
  const int d = a.d, E = a.E, k = a.k;
  const bool train = a.flags & 1, normalize = a.flags & 2;
  const int64_t tok0 = (int64_t)blockIdx.x * RT_TOK;
  const bool mma_wave = wave < Sh::MMA_WAVES;  // uniform
  const int nks = d >> 5;
  const char* zero = (const char*)g_zero_kib + lane * 16;

  // ---- operands ----------------------------------------------------------------------------
  // W_r (and the norm's weight) go global -> LDS by LDS-DMA copies, 1 KiB per wave
  // instruction spread over all 16 waves, with no registers in flight and no staging
  // pass; d E 2 is a multiple of 256 (d % 32 == 0, E % 4 == 0), so only the last copy of
  // each is partial, its surplus lanes reading the zero page.
  // The 8-wave form copies W_r's chunks [c0, c1) (part p: k-steps 6 p .. 6 p + 5) into a
  // region that holds them from its start.
  const int nw16 = (d * E * 2) >> 4;  // 16-byte chunks of W_r
  const int part16 = (RT_PART_STEPS * 32 * E * 2) >> 4;
  const int nparts = (nks + RT_PART_STEPS - 1) / RT_PART_STEPS;
  auto copy_w = [&](int c0, int c1, char* dst) {
    const char* wsrc = (const char*)a.w;
    for (int i = wave; i * 64 < c1 - c0; i += RT_WAVES) {  // uniform
      const int c = c0 + i * 64 + lane;
      async_copy16(c < c1 ? (const void*)(wsrc + c * 16) : (const void*)zero,
                   dst + i * 1024);
    }
  };
  {
    if constexpr (W == 16) copy_w(0, nw16, s_stage);
    else copy_w(0, min(part16, nw16), s_stage);
    if (a.norm_w) {
      const int nn16 = (d * 2) >> 4;
      const char* nsrc = (const char*)a.norm_w;
      for (int i = wave; i * 64 < nn16; i += RT_WAVES) {
        const int c = i * 64 + lane;
        async_copy16(c < nn16 ? (const void*)(nsrc + c * 16) : (const void*)zero,
                     s_nw + i * 1024);
      }
    }
  }
  // The token rows: x[tok0 .. tok0 + RT_TOK) is one contiguous d * 2 * RT_TOK-byte block,
  // copied by 1 KiB LDS-DMA copies over all 16 waves (whole 64-byte row segments per lane
  // quad).  LDS slot (r, p) of row r holds the row's 16-byte chunk x_slot(p, r) (an
  // involution: chunks of whole 8-chunk groups XORed with r % 8), so that the 16 rows a
  // fragment read touches at one chunk position fall on 8 different bank groups.  Rows
  // past T read the zero page.
  const int cpr = d >> 3;                 // 16-byte chunks per row
  const int cpr8 = cpr & ~7;
  auto x_slot = [&](int c, int r) { return c < cpr8 ? c ^ (r & 7) : c; };
  {
    const int nslot = RT_TOK * cpr;
    const char* xsrc = (const char*)a.x;
    for (int i = wave; i * 64 < nslot; i += RT_WAVES) {  // uniform
      const int s = i * 64 + lane;
      const int r = s / cpr, p = s - r * cpr;
      const bool ok = s < nslot && tok0 + r < T;
      async_copy16(ok ? (const void*)(xsrc + ((tok0 + r) * d + x_slot(p, r) * 8) * 2)
                      : (const void*)zero,
                   s_x + i * 1024);
    }
  }
  // A GEMM wave's 16 token rows, whole (d <= 32 RT_MAX_STEPS), read from LDS once the
  // copies have landed.  Lane (g, j) holds row tok + j, elements 32 ks + 8 g .. + 7 (the A
  // operand of k-step ks).
  // A GEMM wave's column blocks: wave % SPLIT + SPLIT nb, nb < NBH.
  constexpr int NBH = (NB + Sh::SPLIT - 1) / Sh::SPLIT;  // column blocks per GEMM wave
  const int tile = wave / Sh::SPLIT, cw = wave % Sh::SPLIT;
  auto cblk = [&](int nb) { return cw + Sh::SPLIT * nb; };
  u32x4 xr[RT_MAX_STEPS];
  f32x4 acc[NBH];
  for (int e = tid; e < 128; e += RT_THREADS) s_hist[e] = 0;
  if (tid == 0) s_ntie = 0;
  for (int e = tid; e < E; e += RT_THREADS) s_bias[e] = a.bias ? a.bias[e] : 0.0f;
  wait_vmcnt<0>();  // this wave's copies have landed
  __syncthreads();  // every wave's copies and the LDS fills are visible
  // The packing waves (the 16-wave form's last RT_PACK_WAVES, 12 .. 15, which the GEMM and
  // the selection leave idle and the exact pass needs only for its thirteenth tie row on)
  // take the weight pack's wave items, grid-strided: the first item's loads now, under the
  // GEMM, its transpose and stores during the selection, two items beside the exact pass
  // (after any tie rows of their own), the rest after it.  Each has 8 KiB of LDS:
  // half of them in the token rows' area (free since the GEMM waves hold their rows), half
  // in the stage past the exact pass's swap slots (free since the GEMM read W_r).  Eight
  // packing waves (8 .. 15, one item at each phase) measured slower: the router launch
  // 31 -> 34.5 us against the 12.6 us the place launch saves.
  constexpr int PW = RT_PACK_WAVES;
  constexpr int POSR = (POS + 1023) / 1024 * 1024;
  const bool packer = W == 16 && a.pack_on && wave >= RT_WAVES - PW;  // uniform
  const int pw = wave - (RT_WAVES - PW);
  int64_t pu = (int64_t)blockIdx.x * PW + pw;
  const int64_t pstride = (int64_t)gridDim.x * PW;
  bool pdone = !packer;
  char* pwl = pw >= PW / 2 ? s_x + (pw - PW / 2) * PACK_WAVE_LDS
                           : s_stage + POSR + pw * PACK_WAVE_LDS;
  auto pack_some = [&](int n) {
    for (int i = 0; i < n && !pdone; ++i, pu += pstride)  // uniform
      pdone = !pack_pair_item<DT>(a.pack, pu, lane, pwl);
  };
  u32x4 pv[8];
  bool pfirst = false;
  if constexpr (W == 16) {
    if (packer) {
      pfirst = pack_pair_load<DT>(a.pack, pu, lane, pv);
      pdone = !pfirst;
    }
  }
  if (mma_wave) {
    const int r = tile * 16 + j;
    const char* xl = s_x + r * cpr * 16;
#pragma unroll
    for (int ks = 0; ks < RT_MAX_STEPS; ++ks)
      if (ks < nks) xr[ks] = *(const u32x4*)(xl + x_slot(ks * 4 + g, r) * 16);
  }

  if (a.norm_w && mma_wave) {  // uniform: RMSNorm of the rows in place (RouterArgs)
    // The row's sum of squares: this lane's 8 nks elements, then its 4 lanes (g = 0..3).
    const int64_t trow = tok0 + tile * 16 + j;
    float ss = 0.0f;
#pragma unroll
    for (int ks = 0; ks < RT_MAX_STEPS; ++ks) {
      if (ks < nks) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = unpack2<DT>(xr[ks][e], 0), hi = unpack2<DT>(xr[ks][e], 1);
          ss += lo * lo + hi * hi;
        }
      }
    }
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    const float rstd = 1.0f / sqrtf(ss / (float)d + a.norm_eps);
    const char* wn = s_nw + 16 * g;
    ET* xo = (ET*)a.xn + trow * d + 8 * g;
    const bool writer = cw == 0 && trow < T;  // one of the row's GEMM waves
#pragma unroll
    for (int ks = 0; ks < RT_MAX_STEPS; ++ks) {
      if (ks < nks) {
        const u32x4 w = *(const u32x4*)(wn + ks * 64);
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = pack2<DT>(unpack2<DT>(xr[ks][e], 0) * rstd * unpack2<DT>(w[e], 0),
                           unpack2<DT>(xr[ks][e], 1) * rstd * unpack2<DT>(w[e], 1));
        xr[ks] = o;
        if (writer) *(u32x4*)(xo + ks * 32) = o;
      }
    }
    if (writer && g == 0) a.rstd[trow] = rstd;
  }

  // ---- GEMM: 18 k-steps from W_r in LDS ------------------------------------------------
  // B fragment of k-step ks, column block nb: lane (g, j) reads rows 32 ks + 8 g + 4 h +
  // j / 4 and columns 16 nb + 4 (j % 4) .. + 3, for h = 0, 1 (ks counted from the first
  // k-step the region holds).
#pragma unroll
  for (int nb = 0; nb < NBH; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int EP = E * 2;  // bytes per W_r row
  const int lofs = (8 * g + (j >> 2)) * EP + 8 * (j & 3);
  // k-steps [KS0, KS0 + NKS) of the GEMM from `region`, which holds k-step KS0 first.
  auto gemm_steps = [&](const char* region, auto ks0_tag, auto nks_tag) {
    constexpr int KS0 = decltype(ks0_tag)::value, NKS = decltype(nks_tag)::value;
    if (!mma_wave) return;
#pragma unroll
    for (int ks = KS0; ks < KS0 + NKS; ++ks) {
      if (ks < nks) {  // uniform
        const char* sb = region + lofs + (ks - KS0) * 32 * EP;
#pragma unroll
        for (int nb = 0; nb < NBH; ++nb) {
          if (cblk(nb) < NB) {  // uniform
            const uint2 lo = lds_read_tr16(sb + cblk(nb) * 32);
            const uint2 hi = lds_read_tr16(sb + 4 * EP + cblk(nb) * 32);
            const typename Mma<DT>::Frag b{u32x4{lo.x, lo.y, hi.x, hi.y}};
            Mma<DT>::run(acc[nb], typename Mma<DT>::Frag{xr[ks]}, b);
          }
        }
      }
    }
  };
  using IC0 = std::integral_constant<int, 0>;
  if constexpr (W == 16) {
    gemm_steps(s_stage, IC0{}, std::integral_constant<int, RT_MAX_STEPS>{});
  } else {
    static_assert(RT_MAX_STEPS == 3 * RT_PART_STEPS, "three parts");
    using ICP = std::integral_constant<int, RT_PART_STEPS>;
    // Part 0 sits in the stage; the token rows' area is free once every GEMM wave holds
    // its rows, so part 1 goes there under part 0's MFMAs, and part 2 into the stage under
    // part 1's.  Each wait + barrier: the next part has landed (every wave's copies) and
    // no wave still reads the region the part after it overwrites.
    __syncthreads();
    if (nparts > 1) copy_w(part16, min(2 * part16, nw16), s_x);
    gemm_steps(s_stage, IC0{}, ICP{});
    if (nparts > 1) {  // uniform
      wait_vmcnt<0>();
      __syncthreads();
      if (nparts > 2) copy_w(2 * part16, nw16, s_stage);
      gemm_steps(s_x, ICP{}, ICP{});
      if (nparts > 2) {
        wait_vmcnt<0>();
        __syncthreads();
        gemm_steps(s_stage, std::integral_constant<int, 2 * RT_PART_STEPS>{}, ICP{});
      }
    }
  }

  // ---- logits: rounded to the dtype, stored, and kept in LDS as fp32 -----------------
  // acc[nb][i] holds the logit of token 16 tile + 4 g + i, expert 16 cblk(nb) + j.
  if (mma_wave) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tl = tile * 16 + 4 * g + i;
      const int64_t t = tok0 + tl;
#pragma unroll
      for (int nb = 0; nb < NBH; ++nb) {
        if (cblk(nb) >= NB) continue;  // uniform
        const int e = 16 * cblk(nb) + j;
        float l = acc[nb][i];
        if (e < E) l += s_bias[e];
        const ET lv = Elem<DT>::from_f(l);
        if (t < T && e < E) ((ET*)a.logits)[t * E + e] = lv;
        s_lg[tl * LGP + e] = e < E ? Elem<DT>::to_f(lv) : -INFINITY;
      }
    }
  }
  __syncthreads();

  // ---- softmax and the fast selection: token 4 wave + g on lanes 16 g .. 16 g + 15 ------
  if (wave < RT_SEL_WAVES) {  // uniform
    const int tl = wave * 4 + g;
    const int64_t t = tok0 + tl;
    const bool live = t < T;
    float key[NB];
    bool nan_here = false;
    float m = -INFINITY;
  #pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      key[nb] = s_lg[tl * LGP + 16 * nb + j];
      nan_here |= __builtin_isnan(key[nb]);
      m = fmaxf(m, key[nb]);
    }
    const bool nan_row = row16_sum_i(nan_here ? 1 : 0) != 0;
    m = row16(m, fmax_);
    if (nan_row) m = __uint_as_float(0x7fc00000u);
    float inv = 0.0f;
    if (train || !normalize) {  // uniform
      float ex[NB], s = 0.0f;
  #pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        ex[nb] = 16 * nb + j < E ? expf(key[nb] - m) : 0.0f;
        s += ex[nb];
      }
      inv = 1.0f / row16(s, fadd_);
      if (train) {
  #pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const int e = 16 * nb + j;
          if (e < E) {
            const float p = ex[nb] * inv;
            if (live) a.probs[t * E + e] = p;
            key[nb] = p;
            s_lg[tl * LGP + e] = p;  // the exact pass's keys and the column sums
          }
        }
      }
    }
    if (j == 0) {
      s_m[tl] = m;
      s_inv[tl] = inv;
    }
    uint32_t avail = 0;
  #pragma unroll
    for (int nb = 0; nb < NB; ++nb) avail |= (16 * nb + j < E ? 1u : 0u) << nb;
    bool exact = nan_row;
    float s_sel = 0.0f;
    int d_sel = 0;
    for (int r = 0; r < k; ++r) {
      float c = -INFINITY;
  #pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (avail >> nb & 1u) c = fmaxf(c, key[nb]);
      const float mx = row16(c, fmax_);
      int cnt = 0, loc = 1 << 20;
  #pragma unroll
      for (int nb = NB - 1; nb >= 0; --nb)
        if ((avail >> nb & 1u) && key[nb] == mx) {
          ++cnt;
          loc = 16 * nb + j;
        }
      exact |= row16_sum_i(cnt) != 1;
      const int id = row16_min_i(loc);
      if ((id & 15) == j && id < (1 << 20)) avail &= ~(1u << (id >> 4));
      if (j == r) {
        s_sel = mx;
        d_sel = id;
      }
    }
    {
      const bool o = j < k;
      const float s = o ? s_sel : 0.0f;
      float wgt = s;
      if (train) {
        if (normalize && k > 1) wgt = s / row16(s, fadd_);
      } else if (normalize) {
        const float mk = row16(o ? s : -INFINITY, fmax_);
        const float e = o ? expf(s - mk) : 0.0f;
        wgt = e * (1.0f / row16(e, fadd_));
      } else {
        wgt = expf(s - m) * inv;
      }
      if (live && !exact && o) {
        a.topk_idx[t * k + j] = d_sel;
        ((ET*)a.topk_w)[t * k + j] = Elem<DT>::from_f(wgt);
        atomicAdd(&s_hist[d_sel], 1);
      }
      if (live && exact && j == 0) s_tie[atomicAdd(&s_ntie, 1)] = tl;
    }
  }  // the selection waves
  if constexpr (W == 16) {
    static_assert(RT_SEL_WAVES <= RT_WAVES - PW, "packing waves select nothing");
    static_assert(PW / 2 * PACK_WAVE_LDS <= (int)sizeof(s_x) &&
                      POSR + PW / 2 * PACK_WAVE_LDS <= STAGE,
                  "packing regions fit the rows' area and the stage");
    if (pfirst) {  // the item loaded under the GEMM
      pack_pair_store<DT>(a.pack, pu, lane, pv, pwl);
      pu += pstride;
    }
  }
  __syncthreads();

  // ---- the exact pass for the undecided tokens: one wave per token -------------------
  // The keys come from LDS as the selection saw them; the stage holds the partitions'
  // swap slots now.
  const int nt = s_ntie;
  int2* pos = (int2*)s_stage + wave * TOPK_SWAP_SLOTS;
  const bool has0 = lane < E, has1 = lane + 64 < E;
  for (int q = wave; q < nt; q += RT_WAVES) {  // uniform
    const int rt = s_tie[q];
    const float* row = s_lg + rt * LGP;
    const float k0 = has0 ? row[lane] : -INFINITY, k1 = has1 ? row[lane + 64] : -INFINITY;
    RegRow rr{(int)ord_key(k0), (int)ord_key(k1), lane, lane + 64, lane};
    topk_select(rr, E, k, pos);
    const int a0 = (rr.i0 & 63) * 4, a1 = (rr.i1 & 63) * 4;
    const float lo0 = __int_as_float(__builtin_amdgcn_ds_bpermute(a0, __float_as_int(k0)));
    const float hi0 = __int_as_float(__builtin_amdgcn_ds_bpermute(a0, __float_as_int(k1)));
    const float lo1 = __int_as_float(__builtin_amdgcn_ds_bpermute(a1, __float_as_int(k0)));
    const float hi1 = __int_as_float(__builtin_amdgcn_ds_bpermute(a1, __float_as_int(k1)));
    write_route_row<DT>(tok0 + rt, k, lane, train, normalize, rr.i0 < 64 ? lo0 : hi0,
                        rr.i1 < 64 ? lo1 : hi1, rr.i0, rr.i1, s_m[rt], s_inv[rt],
                        (ET*)a.topk_w, a.topk_idx);
    if (lane < k) atomicAdd(&s_hist[rr.i0], 1);
    if (lane + 64 < k) atomicAdd(&s_hist[rr.i1], 1);
  }
  if constexpr (W == 16) pack_some(2);
  __syncthreads();

  // ---- this chunk's histogram and, in training, its column sums of probs -------------
  const int64_t wg = blockIdx.x;
  const int nlive = (int)min((int64_t)RT_TOK, T - tok0);
  for (int e = tid; e < E; e += RT_THREADS) {
    a.hist[wg * E + e] = s_hist[e];
    if (train && a.colsum) {
      float s = 0.0f;
      for (int q = 0; q < nlive; ++q) s += s_lg[q * LGP + e];
      a.colsum[wg * E + e] = s;
    }
  }
  if constexpr (W == 16) pack_some(1 << 30);
}

bool router_fused_supported(int dtype, int d, int E, int k) {
  return (dtype == DT_BF16 || dtype == DT_F16) && d >= 32 && d % 32 == 0 &&
         d <= 32 * RT_MAX_STEPS && E >= 1 && E <= RT_MAX_E && E % 4 == 0 && k >= 1 &&
         k <= RT_MAXK && k <= E;
}

size_t router_fused_ws_bytes(int64_t T, int E) {
  const int64_t nwg = router_fused_chunks(T);
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  return 2 * al(nwg * E * 4);
}

RouterArgs router_fused_args(void* ws, int64_t T, int E) {
  const int64_t nwg = router_fused_chunks(T);
  auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
  RouterArgs a{};
  a.hist = (int32_t*)ws;
  a.colsum = (float*)((char*)ws + al(nwg * E * 4));
  return a;
}

template <int DT, int NB>
static void launch_nb(const RouterArgs& a, unsigned grid, int waves, hipStream_t s) {
  if (waves == 8) router_fwd_kernel<DT, NB, 8><<<grid, 8 * 64, 0, s>>>(a);
  else router_fwd_kernel<DT, NB, 16><<<grid, 16 * 64, 0, s>>>(a);
}

template <int DT>
static void launch_fwd(const RouterArgs& a, unsigned grid, int waves, hipStream_t s) {
  switch ((a.E + 15) / 16) {
    case 1: launch_nb<DT, 1>(a, grid, waves, s); break;
    case 2: launch_nb<DT, 2>(a, grid, waves, s); break;
    case 3: launch_nb<DT, 3>(a, grid, waves, s); break;
    case 4: launch_nb<DT, 4>(a, grid, waves, s); break;
    default: launch_nb<DT, 5>(a, grid, waves, s); break;
  }
}

static int router_device_cus();

// 8-wave workgroups (two per CU) once the grid has more workgroups than CUs, else 16
// (one per CU, W_r copied whole); the "router_waves" option forces either.
static int router_waves_for(int64_t grid) {
  if (const int64_t v = option(OPT_ROUTER_WAVES)) return (int)v;
  return grid > router_device_cus() ? 8 : 16;
}

// At most 8 pack items per packing wave: about the length of the selection and the exact
// pass (an item is one 8 KiB load, a transpose and 8 KiB of stores).
bool router_fused_can_pack(int64_t T, int64_t items) {
  const int64_t grid = router_fused_chunks(T);
  return T > 0 && router_waves_for(grid) == 16 && items <= grid * RT_PACK_WAVES * 8 &&
         !option(OPT_PACK_IN_PLACE);
}

// Compute units of the current device (cached per device).
static int router_device_cus() {
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

int router_fused_launch(const RouterArgs& a, int dtype, hipStream_t s) {
  NSMOE_REQUIRE(((uintptr_t)a.w & 15) == 0 && ((uintptr_t)a.norm_w & 15) == 0,
                "router: the router weight and the norm weight must be 16-byte aligned");
  NSMOE_REQUIRE(router_fused_supported(dtype, a.d, a.E, a.k),
                "router: the fused router takes bf16/fp16, d %% 32 == 0, d <= %d, "
                "E %% 4 == 0, E <= %d, top_k <= %d (d %d, E %d, k %d)", 32 * RT_MAX_STEPS,
                RT_MAX_E, RT_MAXK, a.d, a.E, a.k);
  NSMOE_REQUIRE(a.x && a.w && a.logits && a.topk_w && a.topk_idx && a.hist &&
                    (!(a.flags & 1) || a.probs) && (!a.norm_w || (a.xn && a.rstd)),
                "router: NULL pointer");
  if (a.T == 0) return NSMOE_OK;
  const unsigned grid = (unsigned)router_fused_chunks(a.T);
  const int waves = router_waves_for(grid);
  NSMOE_REQUIRE(!a.pack_on || router_fused_can_pack(a.T, a.pack.items_in + a.pack.items_out),
                "router: the weight pack needs the 16-wave form and enough workgroups");
  KernelTimer timer("route_fwd", s);
  if (dtype == DT_BF16) launch_fwd<DT_BF16>(a, grid, waves, s);
  else launch_fwd<DT_F16>(a, grid, waves, s);
  timer.stop();
  return check_launch("router_fwd_kernel");
}

}  // namespace nsmoe

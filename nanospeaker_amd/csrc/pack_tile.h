// The 16-bit weight pack's block routine (pack.hip), shared with the dispatch's place
// launch (dispatch.hip), which packs beside its placement workgroups.
#pragma once

#include "gemm_core.h"

namespace nsmoe {

// The pack in wave items: a wave packs two k blocks of one 64-column tile -- eight 1 KiB
// fragments (f = 4 (k block % 2) + column block) -- and nothing is shared between waves,
// so there is no workgroup barrier.  Lane l of the wave loads and transposes one 8 x 8
// block in its registers: k block 2 kp + l / 32, rows kbl * 8 + r (r < 8) with
// kbl = (l % 32) / 8, columns 8 nbl .. 8 nbl + 7 of the tile with nbl = l % 8 (eight lanes
// read one row's 128 contiguous bytes).  Column c of the block is exactly one lane's
// 16-byte share of fragment (l / 32, nbl / 2): share 16 kbl + 8 (nbl % 2) + c, whose
// elements are the block's rows in order.  The shares go to the wave's 8 KiB of LDS in
// fragment order, and each fragment leaves as one 1 KiB store (lane l, share l): stores of
// 16 scattered bytes per lane would cost the L2 one request per lane.  Out-of-range rows
// and columns pack as zeros.
//
// LDS: share i of the region (16 bytes, i = 64 f + s) sits at
// i ^ 2 ((i / 64) % 4) ^ ((i / 16) % 2): any 16 consecutive lanes of one transposed write,
// and of one fragment read, then cover all 64 banks once.
constexpr int PACK_WAVE_LDS = 8 * 1024;

__device__ __forceinline__ int pack_share_off(int i) {
  return (i ^ (((i >> 6) & 3) << 1) ^ ((i >> 4) & 1)) << 4;
}

__host__ __device__ inline int64_t pack_items(int groups, int n_kb, int n_nb) {
  return (int64_t)groups * (n_nb / 4) * ((n_kb + 1) / 2);
}

// Items run tiles fastest, so consecutive waves read the same rows' neighbouring 128-byte
// segments, then k-block pairs, then groups.
struct PackItem {
  int g, kp, nt;
};
__device__ __forceinline__ PackItem pack_item_of(int64_t item, int n_kb, int n_nb) {
  const int nts = n_nb / 4, kps = (n_kb + 1) / 2;
  const int per_g = nts * kps;
  const int g = (int)(item / per_g), r0 = (int)(item - (int64_t)g * per_g);
  const int kp = r0 / nts;
  return PackItem{g, kp, r0 - kp * nts};
}

// The item's loads: lane l's 8 x 8 block, row r in v[r] (zeros out of range).  A caller
// may issue them early and finish the item later (pack_wave_store).
template <int DT, int MODE>
__device__ __forceinline__ void pack_wave_load(const typename Elem<DT>::T* __restrict__ routed,
                                               const typename Elem<DT>::T* __restrict__ shared,
                                               int E, int d, int H, int HP, int n_kb, int n_nb,
                                               int fast, int64_t item, int lane,
                                               u32x4 (&v)[8]) {
  using G = Geo<DT>;
  using T = typename G::T;
  static_assert(G::ES == 2 && G::VE == 8 && G::KC == 32 && G::PKB == 1024, "16-bit types");
  const PackItem it = pack_item_of(item, n_kb, n_nb);
  const int g = it.g, kp = it.kp, nt = it.nt;
  const int K = MODE == 0 ? d : H;
  const int ld = MODE == 0 ? 2 * H : d;
  const int64_t gstride = MODE == 0 ? (int64_t)d * 2 * H : (int64_t)H * d;
  const T* W = g < E ? routed + (int64_t)g * gstride : shared + (int64_t)(g - E) * gstride;
  int n0, nlim;
  if (MODE == 0) {
    const int c0 = nt * 64;  // packed column of the tile
    if (c0 < HP) {
      n0 = c0;
      nlim = H;
    } else {
      n0 = H + (c0 - HP);
      nlim = 2 * H;
    }
  } else {
    n0 = nt * 64;
    nlim = d;
  }
  const int half = lane >> 5, kbl = (lane >> 3) & 3, nbl = lane & 7;
  const int kb = 2 * kp + half;
  const int col = n0 + nbl * G::VE;
#pragma unroll
  for (int r = 0; r < G::VE; ++r) {
    v[r] = u32x4{0u, 0u, 0u, 0u};
    const int k = kb * G::KC + kbl * G::VE + r;
    if (k >= K) continue;  // also every row of a k block past n_kb
    const T* src = W + (int64_t)k * ld;
    if (fast) {
      if (col < nlim) v[r] = *(const u32x4*)(src + col);
    } else {
      T tmp[G::VE];
#pragma unroll
      for (int e = 0; e < G::VE; ++e) tmp[e] = (col + e < nlim) ? src[col + e] : T(0);
      __builtin_memcpy(&v[r], tmp, 16);
    }
  }
}

// The item's transpose and stores from its loaded blocks (pack_wave_load).
template <int DT>
__device__ __forceinline__ void pack_wave_store(int n_kb, int n_nb, char* __restrict__ out,
                                                int64_t item, int lane, const u32x4 (&v)[8],
                                                char* __restrict__ wl) {
  using G = Geo<DT>;
  const PackItem it = pack_item_of(item, n_kb, n_nb);
  const int g = it.g, kp = it.kp, nt = it.nt;
  const int half = lane >> 5, kbl = (lane >> 3) & 3, nbl = lane & 7;
  const int share0 = 64 * (4 * half + (nbl >> 1)) + 16 * kbl + 8 * (nbl & 1);
  constexpr uint32_t kLow = 0x05040100u, kHigh = 0x07060302u;  // low / high halves
#pragma unroll
  for (int c = 0; c < G::VE; ++c) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = __builtin_amdgcn_perm(v[2 * q + 1][c >> 1], v[2 * q][c >> 1],
                                   (c & 1) ? kHigh : kLow);
    *(u32x4*)(wl + pack_share_off(share0 + c)) = o;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  char* dst = out + (((int64_t)g * n_nb + nt * 4) * n_kb + 2 * kp) * G::PKB + lane * G::FRAGB;
#pragma unroll
  for (int f = 0; f < 8; ++f) {
    if (2 * kp + (f >> 2) >= n_kb) break;  // uniform: the odd k block past the last
    const u32x4 o = *(const u32x4*)(wl + pack_share_off(64 * f + lane));
    *(u32x4*)(dst + ((int64_t)(f & 3) * n_kb + (f >> 2)) * G::PKB) = o;
  }
  // the wave's next item must not overwrite the region before these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DT, int MODE>
__device__ __forceinline__ void pack_wave_item(const typename Elem<DT>::T* __restrict__ routed,
                                               const typename Elem<DT>::T* __restrict__ shared,
                                               int E, int d, int H, int HP, int n_kb, int n_nb,
                                               char* __restrict__ out, int fast, int64_t item,
                                               int lane, char* __restrict__ wl) {
  u32x4 v[8];
  pack_wave_load<DT, MODE>(routed, shared, E, d, H, HP, n_kb, n_nb, fast, item, lane, v);
  pack_wave_store<DT>(n_kb, n_nb, out, item, lane, v, wl);
}

// Both packs' operands and geometry (pack_pair_kernel, and the place launch's pack waves).
struct PackPairArgs {
  const void *w_in, *w_sh_in, *w_out, *w_sh_out;
  int E, G, d, H, HP, in_kb, in_nb, out_kb, out_nb, fast;
  char *p_in, *p_out;
  int64_t items_in, items_out;  // wave items of each stack (items_out 0: W_in alone)
};

// Wave item u of the pair: W_in's items first, then W_out's; false past the last.  wl is
// the wave's PACK_WAVE_LDS bytes of LDS (16-byte aligned).
template <int DT>
__device__ __forceinline__ bool pack_pair_item(const PackPairArgs& a, int64_t u, int lane,
                                               char* __restrict__ wl) {
  using T = typename Elem<DT>::T;
  if (u < a.items_in) {
    pack_wave_item<DT, 0>((const T*)a.w_in, (const T*)a.w_sh_in, a.E, a.d, a.H, a.HP,
                          a.in_kb, a.in_nb, a.p_in, a.fast, u, lane, wl);
    return true;
  }
  u -= a.items_in;
  if (u >= a.items_out) return false;
  pack_wave_item<DT, 1>((const T*)a.w_out, (const T*)a.w_sh_out, a.E, a.d, a.H, a.HP,
                        a.out_kb, a.out_nb, a.p_out, a.fast, u, lane, wl);
  return true;
}

// Wave item u of the pair in two halves: its loads (false past the last item, nothing
// loaded), then, later, its transpose and stores from those registers.
template <int DT>
__device__ __forceinline__ bool pack_pair_load(const PackPairArgs& a, int64_t u, int lane,
                                               u32x4 (&v)[8]) {
  using T = typename Elem<DT>::T;
  if (u < a.items_in) {
    pack_wave_load<DT, 0>((const T*)a.w_in, (const T*)a.w_sh_in, a.E, a.d, a.H, a.HP, a.in_kb,
                          a.in_nb, a.fast, u, lane, v);
    return true;
  }
  u -= a.items_in;
  if (u >= a.items_out) return false;
  pack_wave_load<DT, 1>((const T*)a.w_out, (const T*)a.w_sh_out, a.E, a.d, a.H, a.HP,
                        a.out_kb, a.out_nb, a.fast, u, lane, v);
  return true;
}
template <int DT>
__device__ __forceinline__ void pack_pair_store(const PackPairArgs& a, int64_t u, int lane,
                                                const u32x4 (&v)[8], char* __restrict__ wl) {
  if (u < a.items_in) pack_wave_store<DT>(a.in_kb, a.in_nb, a.p_in, u, lane, v, wl);
  else pack_wave_store<DT>(a.out_kb, a.out_nb, a.p_out, u - a.items_in, lane, v, wl);
}

// The arguments of the 16-bit pack pair for these weights (pack_pair_kernel's geometry);
// false where the pair path does not apply (fp32).
bool pack_pair_args(int dtype, const void* w_in, const void* w_out, const void* w_sh_in,
                    const void* w_sh_out, int E, int S, int d, int H, void* p_in, void* p_out,
                    PackPairArgs* out);

}  // namespace nsmoe

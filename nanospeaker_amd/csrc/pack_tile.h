// The 16-bit weight pack's tile routine (pack.hip), shared with the dispatch's place launch
// (dispatch.hip), which packs beside its placement workgroups.
#pragma once

#include "gemm_core.h"

namespace nsmoe {

// 16-bit types: 256 threads (tid 0 .. 255, four whole waves) pack KS k blocks of one
// 64-column tile; the caller's workgroup barrier (__syncthreads) separates the LDS writes
// from the reads, so every group of a workgroup must call this the same number of times
// (a call with kb0 >= n_kb moves nothing and only takes the barrier).  Thread t < 32 KS
// loads the 8 x 8 block (t % 32) of k block t / 32 (every load of the workgroup in flight
// at once) and transposes it into that k block's LDS tile; after a barrier wave w writes
// fragment (4 nt + w, kb) of each k block.  A workgroup per k block keeps only 32 threads
// and 4 KB of loads in flight, which leaves the pass at about half of HBM's rate.
// The tile is (g, nt, k blocks kb0 .. kb0 + KS - 1); `tile` is KS LDS tiles.
template <int DT, int MODE, int KS>
__device__ __forceinline__ void pack_ks_tile(const typename Elem<DT>::T* __restrict__ routed,
                                             const typename Elem<DT>::T* __restrict__ shared,
                                             int E, int d, int H, int HP, int n_kb, int n_nb,
                                             char* __restrict__ out, int fast, int g, int nt,
                                             int kb0, char (*tile)[64 * Geo<DT>::ROWB],
                                             int tid) {
  using G = Geo<DT>;
  using T = typename G::T;
  static_assert(G::ES == 2 && KS * 32 <= 256, "16-bit types, at most 8 k blocks");
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
  // This thread's 8 x 8 block: rows kb * 32 + kbl * 8 + r, columns n0 + nbl * 8 .. + 7.  The
  // column block is the fastest index, so each lane quad loads 64 contiguous bytes of one
  // row (a quad over four rows costs the L1's address unit about three times as much).
  const int step = tid >> 5, blk = tid & 31;
  const int kbl = blk >> 3, nbl = blk & 7;
  const int kb = kb0 + step;
  const bool on = step < KS && kb < n_kb;
  const int col = n0 + nbl * G::VE;
  u32x4 v[G::VE];
#pragma unroll
  for (int r = 0; r < G::VE; ++r) {
    v[r] = u32x4{0u, 0u, 0u, 0u};
    const int k = kb * G::KC + kbl * G::VE + r;
    if (!on || k >= K) continue;
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
  if (on) store_trans8<DT>(v, tile[step], nbl, kbl);
  __syncthreads();
  const int wave = tid >> 6;
  const int nb = nt * 4 + wave;
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    if (kb0 + st >= n_kb) break;
    const typename Mma<DT>::Frag f = frag_sw<DT>(tile[st], wave * 16);
    char* dst = out + (((int64_t)g * n_nb + nb) * n_kb + kb0 + st) * G::PKB + lane_id() * G::FRAGB;
    __builtin_memcpy(dst, &f, sizeof(f));
  }
}

constexpr int PACK_KS_IN = 6, PACK_KS_OUT = 4;

// Both packs' operands and geometry (pack_pair_kernel, and the place launch's pack groups).
struct PackPairArgs {
  const void *w_in, *w_sh_in, *w_out, *w_sh_out;
  int E, G, d, H, HP, in_kb, in_nb, out_kb, out_nb, fast;
  char *p_in, *p_out;
  int gx_in, gy_in, gx_out, gy_out;  // k block groups and column tiles of each part
};

// The arguments of the 16-bit pack pair for these weights (pack_pair_kernel's geometry);
// false where the pair path does not apply (fp32).
bool pack_pair_args(int dtype, const void* w_in, const void* w_out, const void* w_sh_in,
                    const void* w_sh_out, int E, int S, int d, int H, void* p_in, void* p_out,
                    PackPairArgs* out);

}  // namespace nsmoe

// Weight repacking into MFMA fragment order.
//
// GEMM1 (x @ W_in) and GEMM2 (h @ W_out) contract over the rows of W_in [d, 2H] and
// W_out [H, d], whose elements are contiguous along the *other* index.  Once per forward
// the two weight stacks are rewritten so that the 16 x 32 B-fragment (16 output
// columns, 32 contraction elements) of every (column block nb, k block kb) is one
// contiguous block laid out exactly as the 64 lanes consume it:
//   packed[g][nb][kb][lane][8]   lane = (k % 32) / 8 * 16 + n % 16,  element = k % 8
// so the expert kernels load each weight fragment with one coalesced 16-byte-per-lane
// load straight from L2, and never stage weights through LDS.
//
// W_in is packed with its gate and up halves at a fixed split: packed columns
// [0, HP) are gate columns [0, H), [HP, 2 HP) are up columns [H, 2H) (HP = the kernel's
// gate-tile width, a multiple of 64 >= H); padding columns and rows are zero.
#include "gemm_core.h"
#include "nsmoe_capi_internal.h"
#include "pack.h"
#include "pack_tile.h"

namespace nsmoe {

// fp32: one workgroup per group g, 64 packed columns [nt * 64, +64), k block kb.  The
// columns are staged transposed into a swizzled LDS tile (k-major rows), then each wave writes
// one 16-column fragment.
template <int DT, int MODE>
__global__ void __launch_bounds__(256)
pack_kernel(const typename Elem<DT>::T* __restrict__ routed,
            const typename Elem<DT>::T* __restrict__ shared, int E, int d, int H, int HP,
            int n_kb, int n_nb, char* __restrict__ out, int fast) {
  using G = Geo<DT>;
  using T = typename G::T;
  __shared__ __attribute__((aligned(16))) char tile[64 * G::ROWB];
  const int g = blockIdx.z, nt = blockIdx.y, kb = blockIdx.x;
  // MODE 0: W_in [d][2H] (K = d); MODE 1: W_out [H][d] (K = H).
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
  auto row = [&](int k) -> const T* { return W + (int64_t)k * ld; };
  TransStage<DT, 64, 256> st;
  st.load(row, NoScale{}, kb * G::KC, K, n0, nlim, fast);
  st.store(tile);
  __syncthreads();
  const int wave = threadIdx.x >> 6;
  const typename Mma<DT>::Frag f = frag_sw<DT>(tile, wave * 16);
  const int nb = nt * 4 + wave;
  char* dst = out + (((int64_t)g * n_nb + nb) * n_kb + kb) * G::PKB + lane_id() * G::FRAGB;
  __builtin_memcpy(dst, &f, sizeof(f));
}

// Both 16-bit packs in one launch (W_in alone when items_out is 0): every wave packs
// two wave items (pack_tile.h; two k blocks of a 64-column tile each) grid-stride, W_in's
// items first, then W_out's.  Waves share nothing, so there is no workgroup barrier, and
// every thread's eight 16-byte loads are in flight at once.  Two items per wave let the
// second item's reads overlap the first one's writes instead of all reads preceding all
// writes (which leaves the L2s full of dirty lines for the end of the launch to write
// back).
template <int DT>
__global__ void __launch_bounds__(256) pack_pair_kernel(PackPairArgs a) {
  __shared__ __attribute__((aligned(16))) char s_w[4][PACK_WAVE_LDS];
  const int wave = threadIdx.x >> 6;
  const int64_t stride = (int64_t)gridDim.x * 4;
  for (int64_t u = (int64_t)blockIdx.x * 4 + wave;; u += stride)
    if (!pack_pair_item<DT>(a, u, threadIdx.x & 63, s_w[wave])) break;  // uniform per wave
}

PackGeom pack_geom(int dtype, int d, int H, int E, int S) {
  PackGeom pg;
  const int es = dtype == DT_F32 ? 4 : 2;
  const int hp16 = (H + 15) / 16 * 16;
  pg.hp = hp16 <= 64 ? 64 : hp16 <= 128 ? 128 : 256;
  pg.in_kb = (d + 31) / 32;
  pg.in_nb = 2 * pg.hp / 16;
  pg.out_kb = (H + 31) / 32;
  pg.out_nb = (d + 63) / 64 * 4;
  const size_t pkb = (size_t)64 * 8 * es;
  const size_t groups = (size_t)E + S;
  pg.in_bytes = groups * pg.in_nb * pg.in_kb * pkb;
  pg.out_bytes = groups * pg.out_nb * pg.out_kb * pkb;
  return pg;
}

template <int DT>
static int launch_pack(const PackGeom& pg, const void* w_in, const void* w_out,
                       const void* w_sh_in, const void* w_sh_out, int E, int S, int d, int H,
                       void* p_in, void* p_out, bool fast, hipStream_t s) {
  using T = typename Elem<DT>::T;
  const int G = E + S;
  if constexpr (DT != DT_F32) {
    PackPairArgs a{w_in, w_sh_in, w_out, w_sh_out, E, G, d, H, pg.hp, pg.in_kb, pg.in_nb,
                   pg.out_kb, pg.out_nb, fast ? 1 : 0, (char*)p_in, (char*)p_out,
                   pack_items(G, pg.in_kb, pg.in_nb),
                   p_out ? pack_items(G, pg.out_kb, pg.out_nb) : 0};
    const int64_t blocks = cdiv(a.items_in + a.items_out, 8);
    NSMOE_REQUIRE(blocks < (int64_t)INT32_MAX, "pack: %lld workgroups", (long long)blocks);
    KernelTimer timer("pack", s);
    pack_pair_kernel<DT><<<(unsigned)blocks, 256, 0, s>>>(a);
    timer.stop();
    return check_launch("pack_pair_kernel");
  } else {
    KernelTimer timer("pack", s);
    dim3 grid((unsigned)pg.in_kb, (unsigned)(pg.in_nb / 4), (unsigned)G);
    pack_kernel<DT, 0><<<grid, 256, 0, s>>>((const T*)w_in, (const T*)w_sh_in, E, d, H, pg.hp,
                                           pg.in_kb, pg.in_nb, (char*)p_in, fast ? 1 : 0);
    timer.stop();
    NSMOE_TRY(check_launch("pack_kernel<w_in>"));
  }
  if constexpr (DT == DT_F32) {
    if (p_out) {
      dim3 grid((unsigned)pg.out_kb, (unsigned)(pg.out_nb / 4), (unsigned)G);
      pack_kernel<DT, 1><<<grid, 256, 0, s>>>((const T*)w_out, (const T*)w_sh_out, E, d, H,
                                             pg.hp, pg.out_kb, pg.out_nb, (char*)p_out,
                                             fast ? 1 : 0);
      NSMOE_TRY(check_launch("pack_kernel<w_out>"));
    }
  }
  return NSMOE_OK;
}

bool pack_pair_args(int dtype, const void* w_in, const void* w_out, const void* w_sh_in,
                    const void* w_sh_out, int E, int S, int d, int H, void* p_in, void* p_out,
                    PackPairArgs* out) {
  if (dtype == DT_F32 || !p_in || !p_out) return false;
  const PackGeom pg = pack_geom(dtype, d, H, E, S);
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15u) == 0; };
  const bool fast = d % 8 == 0 && H % 8 == 0 && al(w_in) && al(w_out) && al(w_sh_in) &&
                    al(w_sh_out);
  *out = PackPairArgs{w_in, w_sh_in, w_out, w_sh_out, E, E + S, d, H, pg.hp, pg.in_kb,
                      pg.in_nb, pg.out_kb, pg.out_nb, fast ? 1 : 0, (char*)p_in, (char*)p_out,
                      pack_items(E + S, pg.in_kb, pg.in_nb),
                      pack_items(E + S, pg.out_kb, pg.out_nb)};
  return true;
}

int pack_weights(int dtype, const void* w_in, const void* w_out, const void* w_sh_in,
                 const void* w_sh_out, int E, int S, int d, int H, void* p_in, void* p_out,
                 hipStream_t s) {
  const PackGeom pg = pack_geom(dtype, d, H, E, S);
  const int ve = dtype == DT_F32 ? 4 : 8;
  auto al = [](const void* q) { return q == nullptr || ((uintptr_t)q & 15u) == 0; };
  const bool fast = d % ve == 0 && H % ve == 0 && al(w_in) && al(w_out) && al(w_sh_in) &&
                    al(w_sh_out);
  switch (dtype) {
    case DT_BF16:
      return launch_pack<DT_BF16>(pg, w_in, w_out, w_sh_in, w_sh_out, E, S, d, H, p_in, p_out,
                                  fast, s);
    case DT_F16:
      return launch_pack<DT_F16>(pg, w_in, w_out, w_sh_in, w_sh_out, E, S, d, H, p_in, p_out,
                                 fast, s);
    default:
      return launch_pack<DT_F32>(pg, w_in, w_out, w_sh_in, w_sh_out, E, S, d, H, p_in, p_out,
                                 fast, s);
  }
}

}  // namespace nsmoe

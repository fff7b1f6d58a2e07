// Dispatch: the stable counting sort of (token, expert) pairs into expert-major runs.
//
// Reference: MoEBlock._plan (src/model/moe.py:208-223) defines the permutation --
// `topk_idx.flatten().sort(stable=True)`, so inside each expert's run the pairs are in
// increasing pair id p = t * k + j -- and moe_dispatch (src/model/moe_kernel.py:180-218)
// defines the buffers handed to the grouped GEMMs: sorted pair ids with every run
// padded to ALIGN_M slots (pad slots hold the sentinel M), the aligned-block -> expert
// map, run offsets, counts, the padded total and the inverse pair -> slot.
//
// The reference scatters with an atomic cursor, so its order inside a run is arbitrary
// (moe_kernel.py:35-36).  Here the order is the stable sort's, bit for bit, with no
// global atomics deciding it:
//   1. hist:    one workgroup per chunk of pairs (1024, or 256 for E > 256) counts its
//               experts in LDS;
//   2. place:   one workgroup per chunk again.  Each derives its chunk's base in every
//               expert's run (column sums of the [chunks, E] counts over the chunks
//               before it), the experts' totals and the padded run offsets by itself, so
//               no single-workgroup scan sits between the two launches.  It ranks its
//               pairs inside each expert -- every lane sets its bit in a per-wave 64-bit
//               LDS mask for its expert (ds_or_b64, order-free); the rank is then
//               popcount(mask & lanes-below) plus the popcounts of the same expert's
//               masks of the waves before it -- and places them; the block -> expert map
//               and the sentinels are split over the workgroups.
//   With the block's balance loss folded in, the place launch has one more workgroup: it
//   forms the experts' totals the same way and reduces the router's column-sum partials
//   to the loss (balance.h) while the others place their chunks.
#include <atomic>
#include <mutex>

#include "balance.h"
#include "nsmoe_capi_internal.h"
#include "nsmoe_common.h"
#include "pack_tile.h"

namespace nsmoe {

constexpr int ALIGN_M = 16;                  // run alignment (slots)
constexpr int DISPATCH_MAX_EXPERTS = 1024;

// Pairs per chunk = threads per workgroup of the hist and scatter kernels.  The scatter
// keeps one 64-bit mask per (wave, expert) in LDS, so wide chunks need few experts.
static inline int dispatch_chunk(int E) { return E <= 256 ? 1024 : 256; }

__global__ void __launch_bounds__(1024)
dispatch_hist_kernel(const int64_t* __restrict__ topk_idx, int64_t M, int E,
                     int32_t* __restrict__ hist) {
  extern __shared__ int32_t s_cnt[];
  for (int e = threadIdx.x; e < E; e += blockDim.x) s_cnt[e] = 0;
  __syncthreads();
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (p < M) {
    int64_t e = topk_idx[p];
    if (e >= 0 && e < E) atomicAdd(&s_cnt[e], 1);
  }
  __syncthreads();
  int32_t* row = hist + (int64_t)blockIdx.x * E;
  for (int e = threadIdx.x; e < E; e += blockDim.x) row[e] = s_cnt[e];
}

// One workgroup per chunk (the hist kernel's chunks).  Every workgroup derives what it
// needs from the [chunks, E] counts itself -- its chunk's base in each expert's run (the
// column sum over the chunks before it), the experts' totals and the ALIGN_M-padded run
// offsets -- then ranks and places its pairs.  The block -> expert map and the sentinel
// fill are split over the workgroups; workgroup 0 also writes counts, offsets and the
// padded total.  Column sums: thread (e, seg) owns a segment of expert e's column and
// issues its loads together; the segment sums are added in LDS.
struct PlaceParams {
  const int64_t* topk_idx;
  int64_t M;
  int E;
  const int32_t* hist;
  int64_t n_chunks;
  int hist_group, chunk_pairs;
  int64_t l_cap;
  int32_t *sorted_ids, *expert_ids, *offs, *counts, *npp, *inv;
  const float* bal_partial;  // the folded balance loss (or NULL): one more workgroup
  int64_t bal_nblk, bal_T;
  float bal_coef;
  float* bal_aux;
  float* zero_out;  // or NULL: 4 bytes the launch sets to zero (the eval branch's loss)
};

struct PlaceLds {
  int32_t base[DISPATCH_MAX_EXPERTS];
  int32_t tot[DISPATCH_MAX_EXPERTS];
  int32_t off[DISPATCH_MAX_EXPERTS + 1];
  int32_t seg_b[1024], seg_t[1024];
  int32_t wave[16];
  BalanceLds bal;
};

// The place pass of workgroup `chunk` (1024 threads); s_mask holds waves x E 64-bit masks.
// UNR: histogram loads per thread in flight together.
template <int UNR>
__device__ __forceinline__ void place_body(const PlaceParams& P, int64_t chunk, PlaceLds& Ls,
                                           unsigned long long* __restrict__ s_mask) {
  const int64_t* __restrict__ topk_idx = P.topk_idx;
  const int64_t M = P.M;
  const int E = P.E;
  const int32_t* __restrict__ hist = P.hist;
  const int64_t n_chunks = P.n_chunks;
  const int hist_group = P.hist_group, chunk_pairs = P.chunk_pairs;
  const int64_t l_cap = P.l_cap;
  int32_t* __restrict__ sorted_ids = P.sorted_ids;
  int32_t* __restrict__ expert_ids = P.expert_ids;
  int32_t* __restrict__ offs = P.offs;
  int32_t* __restrict__ counts = P.counts;
  int32_t* __restrict__ npp = P.npp;
  int32_t* __restrict__ inv = P.inv;
  int32_t* s_base = Ls.base;
  int32_t* s_tot = Ls.tot;
  int32_t* s_off = Ls.off;
  int32_t* s_seg_b = Ls.seg_b;
  int32_t* s_seg_t = Ls.seg_t;
  int32_t* s_wave = Ls.wave;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int lane = tid & 63, wave = tid >> 6, waves = nt >> 6;
  if (chunk == 0 && tid == 0 && P.zero_out) *P.zero_out = 0.0f;

  // This workgroup's pairs (the loads go out first) and the rank masks.  A workgroup
  // places chunk_pairs <= blockDim.x pairs, one per thread from thread 0: hist_group
  // consecutive rows of hist (n_chunks rows in all) count them.
  const int64_t p = chunk * chunk_pairs + tid;
  const bool mine = tid < chunk_pairs && p < M;
  int e_mine = -1;
  if (mine) {
    const int64_t v = topk_idx[p];
    if (v >= 0 && v < E) e_mine = (int)v;
  }
  for (int i = tid; i < waves * E; i += nt) s_mask[i] = 0ull;

  // Column sums of hist: before this chunk, and over all chunks.  Thread tid owns expert
  // base_e + tid % span and segment tid / span of that expert's column (span = E when the
  // workgroup holds several segments per expert): a wave's lanes read consecutive experts
  // of one chunk row, so each load instruction touches two or three cache lines.  A
  // segment is requested in batches of UNR loads, one memory round trip for up to UNR
  // chunk rows (256 chunks over 13 segments at T = 8192, E = 76).  The loads take 32-bit
  // byte offsets from the uniform base (the launchers keep hist under 1 GiB), so each
  // costs one VGPR.
  const char* hb = (const char*)hist;
  const int nseg = E <= nt ? nt / E : 1;
  const int span = nseg > 1 ? E : nt;
  const int64_t L = (n_chunks + nseg - 1) / nseg;
  for (int base_e = 0; base_e < E; base_e += span) {
    const int e = base_e + tid % span, seg = tid / span;
    const bool own = seg < nseg && e < E;
    int32_t before = 0, total = 0;
    if (own) {
      const int64_t c0 = seg * L, c1 = c0 + L < n_chunks ? c0 + L : n_chunks;
      for (int64_t c = c0; c < c1; c += UNR) {
        int32_t v[UNR];
#pragma unroll
        for (int u = 0; u < UNR; ++u)
          v[u] = c + u < c1 ? *(const int32_t*)(hb + (uint32_t)(((int)(c + u) * E + e) * 4))
                            : 0;
#pragma unroll
        for (int u = 0; u < UNR; ++u) {
          total += v[u];
          if (c + u < chunk * hist_group) before += v[u];
        }
      }
    }
    s_seg_b[tid] = before;
    s_seg_t[tid] = total;
    __syncthreads();
    if (own && seg == 0) {  // segments added in order
      int32_t b = 0, t = 0;
      for (int q = 0; q < nseg; ++q) {
        b += s_seg_b[q * span + tid];
        t += s_seg_t[q * span + tid];
      }
      s_base[e] = b;
      s_tot[e] = t;
    }
    __syncthreads();
  }
  const int64_t G = (n_chunks + hist_group - 1) / hist_group;  // the placing workgroups
  if (chunk == G) {  // the balance-loss workgroup (uniform): totals -> loss
    balance_loss_block(P.bal_partial, P.bal_nblk, s_tot, P.bal_T, E, P.bal_coef, P.bal_aux,
                       Ls.bal);
    return;
  }

  // Exclusive scan of the padded totals (one run of `per` experts per thread).
  const int per = (E + nt - 1) / nt;
  int32_t local = 0;
  const int e0 = tid * per;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) local += (s_tot[e] + ALIGN_M - 1) / ALIGN_M * ALIGN_M;
  }
  const int32_t incl = wave_scan_incl(local);
  if (lane == 63) s_wave[wave] = incl;
  if (e_mine >= 0) atomicOr(&s_mask[wave * E + e_mine], 1ull << lane);
  __syncthreads();
  int32_t wave_base = 0;
  for (int w = 0; w < wave; ++w) wave_base += s_wave[w];
  int32_t run = wave_base + incl - local;
  for (int i = 0; i < per; ++i) {
    const int e = e0 + i;
    if (e < E) {
      s_off[e] = run;
      run += (s_tot[e] + ALIGN_M - 1) / ALIGN_M * ALIGN_M;
    }
  }
  if (tid == nt - 1) {
    int32_t total = 0;
    for (int w = 0; w < waves; ++w) total += s_wave[w];
    s_off[E] = total;
  }
  __syncthreads();

  // Place this chunk's pairs: rank inside the expert = set bits below this lane in the
  // wave's mask plus the same expert's bits in the waves before.
  if (mine) {
    if (e_mine < 0) {
      inv[p] = -1;
    } else {
      const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      int rank = __popcll(s_mask[wave * E + e_mine] & below);
      for (int w = 0; w < wave; ++w) rank += __popcll(s_mask[w * E + e_mine]);
      const int32_t slot = s_off[e_mine] + s_base[e_mine] + rank;
      sorted_ids[slot] = (int32_t)p;
      inv[p] = slot;
    }
  }

  const int32_t total = s_off[E];
  if (chunk == 0) {
    for (int e = tid; e <= E; e += nt) offs[e] = s_off[e];
    for (int e = tid; e < E; e += nt) counts[e] = s_tot[e];
    if (tid == 0) npp[0] = total;
  }
  // Aligned block -> owning expert (the last expert whose run starts at or before it),
  // workgroup-strided over the blocks.
  const int64_t n_blocks = l_cap / ALIGN_M;
  for (int64_t b = chunk * nt + tid; b < n_blocks; b += G * nt) {
    int32_t owner = 0;
    const int64_t pos = b * ALIGN_M;
    if (pos < total) {
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= pos) lo = mid;
        else hi = mid - 1;
      }
      owner = lo;
    }
    expert_ids[b] = owner;
  }
  // Sentinel M in every pad slot and in the unused tail [total, l_cap).
  for (int64_t e = chunk * nt + tid; e < E; e += G * nt)
    for (int32_t q = s_off[e] + s_tot[e]; q < s_off[e + 1]; ++q) sorted_ids[q] = (int32_t)M;
  for (int64_t q = total + chunk * nt + tid; q < l_cap; q += G * nt) sorted_ids[q] = (int32_t)M;
}


__global__ void __launch_bounds__(1024) dispatch_place_kernel(PlaceParams P) {
  extern __shared__ unsigned long long s_mask[];  // [waves][E]
  __shared__ PlaceLds L;
  place_body<24>(P, blockIdx.x, L, s_mask);
}

// The place pass with the 16-bit weight pack beside it, in one launch: workgroups
// [0, n_place) place (as dispatch_place_kernel, E <= 128), the rest pack.  The pack does
// not depend on the routing, and the place pass's few latency-bound workgroups leave most
// CUs idle, so the packing runs in that time instead of in a launch of its own.
// A packing workgroup's 16 waves take the pack's wave items (pack_tile.h) grid-stride,
// each on its own with its own 8 KiB of LDS (no workgroup barrier).  LDS: one area, either
// the place pass's arrays and masks or the 16 waves' regions.
constexpr int PLACE_LDS = ((int)sizeof(PlaceLds) + 7) / 8 * 8 + 16 * 128 * 8;
constexpr int PLACE_PACK_LDS = PLACE_LDS > 16 * PACK_WAVE_LDS ? PLACE_LDS : 16 * PACK_WAVE_LDS;

template <int DT>
__global__ void __launch_bounds__(1024)
dispatch_place_pack_kernel(PlaceParams P, PackPairArgs K, int n_place) {
  __shared__ __attribute__((aligned(16))) char s_raw[PLACE_PACK_LDS];
  if ((int)blockIdx.x < n_place) {  // uniform
    place_body<24>(P, blockIdx.x, *(PlaceLds*)s_raw,
                   (unsigned long long*)(s_raw + (sizeof(PlaceLds) + 7) / 8 * 8));
    return;
  }
  const int64_t waves = (int64_t)(gridDim.x - n_place) * 16;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  char* wl = s_raw + wave * PACK_WAVE_LDS;
  for (int64_t u = (int64_t)(blockIdx.x - n_place) * 16 + wave;; u += waves)
    if (!pack_pair_item<DT>(K, u, lane, wl)) break;  // uniform per wave
}
}  // namespace nsmoe

using namespace nsmoe;

extern "C" int64_t nsmoe_align_m(void) { return ALIGN_M; }

// Host worst case for the padded slot count: every non-empty run adds < ALIGN_M pads
// (same bound as the reference's _l_cap, moe_kernel.py:100-108).
extern "C" int64_t nsmoe_dispatch_l_cap(int64_t n_pairs, int32_t n_experts) {
  if (n_pairs <= 0) return 0;
  int64_t nonempty = n_pairs < n_experts ? n_pairs : n_experts;
  return cdiv(n_pairs + nonempty * (ALIGN_M - 1), ALIGN_M) * ALIGN_M;
}

extern "C" size_t nsmoe_dispatch_workspace_size(int64_t n_pairs, int32_t n_experts) {
  if (n_pairs <= 0 || n_experts <= 0) return 0;
  return (size_t)cdiv(n_pairs, dispatch_chunk(n_experts)) * (size_t)n_experts * sizeof(int32_t);
}

namespace nsmoe {

int dispatch_launch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                    int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                    int32_t* counts, int32_t* n_post_pad, int32_t* inv, void* workspace,
                    size_t workspace_bytes, const BalanceArgs* bal, void* stream,
                    float* zero_out) {
  NSMOE_REQUIRE(n_pairs >= 0 && n_pairs < (int64_t)INT32_MAX / 2,
                "dispatch: n_pairs %lld out of range", (long long)n_pairs);
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= DISPATCH_MAX_EXPERTS,
                "dispatch: n_experts %d outside [1, %d]", n_experts, DISPATCH_MAX_EXPERTS);
  hipStream_t s = (hipStream_t)stream;
  if (n_pairs == 0) {
    // Nothing routed: offsets, counts and the padded total are all zero.
    // Cleared with a fill kernel rather than hipMemsetAsync so the call stays safe to
    // capture in a HIP graph.
    NSMOE_REQUIRE(pad_offsets && counts && n_post_pad, "dispatch: NULL pointer");
    NSMOE_TRY(fill_i32(pad_offsets, n_experts + 1, 0, s));
    NSMOE_TRY(fill_i32(counts, n_experts, 0, s));
    NSMOE_TRY(fill_i32(n_post_pad, 1, 0, s));
    if (zero_out) NSMOE_TRY(fill_i32((int32_t*)zero_out, 1, 0, s));
    return bal ? balance_final_launch(bal->partial, bal->T, n_experts, counts, bal->coef,
                                      bal->aux, s)
               : NSMOE_OK;
  }
  NSMOE_REQUIRE(!bal || (n_experts <= 128 && bal->partial && bal->aux),
                "dispatch: the folded balance loss takes E <= 128 and its buffers");
  NSMOE_REQUIRE(topk_idx && sorted_ids && expert_ids && pad_offsets && counts && n_post_pad &&
                    inv && workspace, "dispatch: NULL pointer");
  const size_t need = nsmoe_dispatch_workspace_size(n_pairs, n_experts);
  if (workspace_bytes < need) {
    set_error("dispatch: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  const int chunk = dispatch_chunk(n_experts);
  const int64_t n_chunks = cdiv(n_pairs, chunk);
  NSMOE_REQUIRE(n_chunks * n_experts <= (int64_t)1 << 28,
                "dispatch: %lld pairs over %d experts exceed the histogram's 1 GiB",
                (long long)n_pairs, n_experts);
  const int64_t l_cap = nsmoe_dispatch_l_cap(n_pairs, n_experts);
  int32_t* hist = (int32_t*)workspace;

  KernelTimer timer("dispatch", s);
  dispatch_hist_kernel<<<(unsigned)n_chunks, chunk, n_experts * sizeof(int32_t), s>>>(
      topk_idx, n_pairs, n_experts, hist);
  NSMOE_TRY(check_launch("dispatch_hist_kernel"));
  const bool fold = bal != nullptr;
  const PlaceParams P{topk_idx, n_pairs, n_experts, hist, n_chunks, 1, chunk, l_cap,
                      sorted_ids, expert_ids, pad_offsets, counts, n_post_pad, inv,
                      fold ? bal->partial : nullptr, fold ? bal->nblk : 0, fold ? bal->T : 1,
                      fold ? bal->coef : 0.0f, fold ? bal->aux : nullptr, zero_out};
  dispatch_place_kernel<<<(unsigned)(n_chunks + (fold ? 1 : 0)), chunk,
                          (chunk / 64) * n_experts * sizeof(unsigned long long), s>>>(P);
  timer.stop();
  return check_launch("dispatch_place_kernel");
}

// The place pass alone, from per-chunk histograms made elsewhere (the fused router):
// chunk c holds pairs [c chunk_pairs, (c + 1) chunk_pairs), hist is [n_chunks, E].  Each
// workgroup places as many whole chunks as fit 1024 pairs.
int dispatch_place_launch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                          const int32_t* hist, int64_t n_chunks, int chunk_pairs,
                          int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                          int32_t* counts, int32_t* n_post_pad, int32_t* inv,
                          const BalanceArgs* bal, hipStream_t s, const PackPairArgs* pack,
                          int pack_dtype, float* zero_out) {
  NSMOE_REQUIRE(n_pairs > 0 && n_pairs < (int64_t)INT32_MAX / 2,
                "dispatch_place: n_pairs %lld out of range", (long long)n_pairs);
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= 128 && chunk_pairs >= 1 &&
                    chunk_pairs <= 1024 && n_chunks * chunk_pairs >= n_pairs,
                "dispatch_place: bad chunking (E %d, %d pairs per chunk)", n_experts,
                chunk_pairs);
  NSMOE_REQUIRE(!bal || (bal->partial && bal->aux), "dispatch_place: balance buffers");
  NSMOE_REQUIRE(n_chunks * n_experts <= (int64_t)1 << 28,
                "dispatch_place: %lld chunks over %d experts exceed the histogram's 1 GiB",
                (long long)n_chunks, n_experts);
  const int64_t l_cap = nsmoe_dispatch_l_cap(n_pairs, n_experts);
  const bool fold = bal != nullptr;
  const int group = 1024 / chunk_pairs;
  const int64_t n_place = (n_chunks + group - 1) / group;
  const PlaceParams P{topk_idx, n_pairs, n_experts, hist, n_chunks, group,
                      group * chunk_pairs, l_cap, sorted_ids, expert_ids, pad_offsets, counts,
                      n_post_pad, inv, fold ? bal->partial : nullptr, fold ? bal->nblk : 0,
                      fold ? bal->T : 1, fold ? bal->coef : 0.0f, fold ? bal->aux : nullptr,
                      zero_out};
  const int np = (int)(n_place + (fold ? 1 : 0));
  if (pack && (pack_dtype == DT_BF16 || pack_dtype == DT_F16)) {
    // Packing workgroups: as many as are resident beside the placing ones (the kernel's
    // occupancy per CU, from the runtime), and no more than two wave items per wave
    // need.  With one item per wave every read would come first and every write last,
    // leaving the L2s full of dirty lines that the end of the launch must write back
    // before the next kernel starts (measured: ~6 us more between the launches); two
    // items per wave interleave the second item's reads with the first one's writes.
    // Both runtime queries are made once per device and dtype: the occupancy query costs
    // tens of microseconds of host time, which an eager call would pay every step.
    const int64_t items = pack->items_in + pack->items_out;
    static std::atomic<int> s_cus[64], s_per_cu[64][2];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = -1;
    const int di = pack_dtype == DT_BF16 ? 0 : 1;
    int cus = dev >= 0 ? s_cus[dev].load(std::memory_order_relaxed) : 0;
    int per_cu = dev >= 0 ? s_per_cu[dev][di].load(std::memory_order_relaxed) : 0;
    if (cus <= 0 || per_cu <= 0) {
      if (dev < 0 ||
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
          cus <= 0)
        cus = 256;
      const void* kfn = pack_dtype == DT_BF16
                            ? (const void*)dispatch_place_pack_kernel<DT_BF16>
                            : (const void*)dispatch_place_pack_kernel<DT_F16>;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, 1024, 0) != hipSuccess ||
          per_cu <= 0)
        per_cu = 1;
      (void)hipGetLastError();
      if (dev >= 0) {
        s_cus[dev].store(cus, std::memory_order_relaxed);
        s_per_cu[dev][di].store(per_cu, std::memory_order_relaxed);
      }
    }
    int64_t npack = (int64_t)per_cu * cus - np;
    if (npack < 8) npack = 8;
    if (npack > cdiv(items, 32)) npack = cdiv(items, 32);
    if (npack < 1) npack = 1;
    NSMOE_REQUIRE(np + npack < (int64_t)INT32_MAX, "place+pack: grid");
    KernelTimer timer("place_pack", s);
    if (pack_dtype == DT_BF16)
      dispatch_place_pack_kernel<DT_BF16><<<(unsigned)(np + npack), 1024, 0, s>>>(P, *pack, np);
    else
      dispatch_place_pack_kernel<DT_F16><<<(unsigned)(np + npack), 1024, 0, s>>>(P, *pack, np);
    timer.stop();
    return check_launch("dispatch_place_pack_kernel");
  }
  KernelTimer timer("dispatch", s);
  dispatch_place_kernel<<<(unsigned)np, 1024, 16 * n_experts * sizeof(unsigned long long), s>>>(
      P);
  timer.stop();
  return check_launch("dispatch_place_kernel");
}

}  // namespace nsmoe

extern "C" int nsmoe_dispatch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                              int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                              int32_t* counts, int32_t* n_post_pad, int32_t* inv,
                              void* workspace, size_t workspace_bytes, void* stream) {
  return dispatch_launch(topk_idx, n_pairs, n_experts, sorted_ids, expert_ids, pad_offsets,
                         counts, n_post_pad, inv, workspace, workspace_bytes, nullptr, stream);
}

// ---- nsmoe_dispatch_noalloc: the same dispatch with library-owned scratch ---------------
//
// The [chunks, E] histogram lives in a file-scope device array instead of a caller
// workspace, for callers that cannot allocate.  Each device that loads the library holds
// its own copy for the life of the process; its address on the current device comes from
// hipGetSymbolAddress, once per device, on that device's first call (the array's name is
// only a host-side stand-in and is never handed to a kernel).  The histogram kernel writes
// every entry the place kernel reads, so nothing in the array has to start at zero; it
// keeps the last call's contents.  Calls that overlap on one device race on it.

namespace nsmoe {

constexpr size_t kDispatchScratchBytes = 4u << 20;
static __device__ __align__(256) unsigned char scratch[kDispatchScratchBytes];

constexpr int kScratchDevices = 64;
static void* g_scratch[kScratchDevices];
static std::mutex g_scratch_mu;

// The symbol lookup is not a stream operation and may load the code object, which a
// graph capture must not see: a device's first call under capture is refused (one call
// outside capture, of any size, resolves the address for every later one).
static int dispatch_scratch(void** out, hipStream_t stream) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("dispatch_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return NSMOE_EHIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cs);
    if (e != hipSuccess || cs != hipStreamCaptureStatusNone) {
      set_error("dispatch_noalloc: the first call on device %d is under graph capture; "
                "make one call outside capture first (it resolves the scratch address)",
                dev);
      return NSMOE_EINVAL;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("dispatch_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
      return NSMOE_EHIP;
    }
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return NSMOE_OK;
}

}  // namespace nsmoe

extern "C" int nsmoe_dispatch_noalloc(const int64_t* topk_idx, int64_t n_pairs,
                                      int32_t n_experts, int32_t* sorted_ids,
                                      int32_t* expert_ids, int32_t* pad_offsets, int32_t* counts,
                                      int32_t* n_post_pad, int32_t* inv, void* stream) {
  NSMOE_REQUIRE(n_pairs >= 0 && n_pairs < (int64_t)INT32_MAX / 2,
                "dispatch_noalloc: n_pairs %lld out of range", (long long)n_pairs);
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= DISPATCH_MAX_EXPERTS,
                "dispatch_noalloc: n_experts %d outside [1, %d]", n_experts,
                DISPATCH_MAX_EXPERTS);
  const size_t need = nsmoe_dispatch_workspace_size(n_pairs, n_experts);
  NSMOE_REQUIRE(need <= kDispatchScratchBytes,
                "dispatch_noalloc: %lld pairs over %d experts need %zu B of scratch, above "
                "its %zu B maximum (use nsmoe_dispatch with a workspace)",
                (long long)n_pairs, n_experts, need, kDispatchScratchBytes);
  void* ws = nullptr;
  if (need > 0) NSMOE_TRY(dispatch_scratch(&ws, (hipStream_t)stream));
  return dispatch_launch(topk_idx, n_pairs, n_experts, sorted_ids, expert_ids, pad_offsets,
                         counts, n_post_pad, inv, ws, kDispatchScratchBytes, nullptr, stream);
}

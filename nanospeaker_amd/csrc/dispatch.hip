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
//   2. scan:    one workgroup turns the [chunks, E] counts into per-chunk run bases (a
//               segmented scan down each expert's column: every thread owns one
//               segment, so the loads of a column are issued together, not one by
//               one), the padded run offsets, the block -> expert map and the sentinels;
//   3. scatter: each chunk ranks its pairs inside each expert.  Every lane sets its bit
//               in a per-wave 64-bit LDS mask for its expert (ds_or_b64, order-free);
//               the rank is then popcount(mask & lanes-below) plus the popcounts of the
//               same expert's masks of the waves before it.
#include "nsmoe_capi_internal.h"
#include "nsmoe_common.h"

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

// One workgroup.  hist is rewritten in place into exclusive per-chunk bases.
__global__ void __launch_bounds__(1024)
dispatch_scan_kernel(int32_t* __restrict__ hist, int64_t n_chunks, int E, int64_t M,
                     int64_t l_cap, int32_t* __restrict__ sorted_ids,
                     int32_t* __restrict__ expert_ids, int32_t* __restrict__ offs,
                     int32_t* __restrict__ counts, int32_t* __restrict__ npp) {
  __shared__ int32_t s_off[DISPATCH_MAX_EXPERTS + 1];
  __shared__ int32_t s_cnt[DISPATCH_MAX_EXPERTS];
  __shared__ int32_t s_wave[16];
  const int tid = threadIdx.x;

  // Per-expert exclusive sums down the chunk column.  Thread (e, seg) owns chunks
  // [seg * L, (seg + 1) * L) of expert e's column: it sums them (independent loads),
  // the segment totals are scanned in LDS, then it rewrites its chunks as bases.
  // Segments of up to SEG_REG chunks are held in registers between the two passes, so
  // the rewrite issues no load after a store (the loads would wait for each store:
  // hist is read and written through the same pointer).
  constexpr int SEG_REG = 16;
  __shared__ int32_t s_seg[1024];
  const int nseg = E <= (int)blockDim.x ? (int)blockDim.x / E : 1;
  const int64_t L = (n_chunks + nseg - 1) / nseg;
  for (int base_e = 0; base_e < E; base_e += (int)blockDim.x / nseg) {
    const int e = base_e + tid / nseg, seg = tid % nseg;
    const bool own = tid / nseg < (int)blockDim.x / nseg && e < E;
    const int64_t c0 = seg * L, c1 = c0 + L < n_chunks ? c0 + L : n_chunks;
    const bool in_reg = L <= SEG_REG;
    int32_t buf[SEG_REG];
    int32_t sum = 0;
    if (own) {
      if (in_reg) {
#pragma unroll
        for (int i = 0; i < SEG_REG; ++i) buf[i] = c0 + i < c1 ? hist[(c0 + i) * E + e] : 0;
#pragma unroll
        for (int i = 0; i < SEG_REG; ++i) sum += buf[i];
      } else {
        for (int64_t c = c0; c < c1; ++c) sum += hist[c * E + e];
      }
    }
    s_seg[tid] = own ? sum : 0;
    __syncthreads();
    if (own) {
      int32_t run = 0;
      for (int q = 0; q < seg; ++q) run += s_seg[tid - seg + q];
      if (in_reg) {
#pragma unroll
        for (int i = 0; i < SEG_REG; ++i)
          if (c0 + i < c1) {
            hist[(c0 + i) * E + e] = run;
            run += buf[i];
          }
      } else {
        for (int64_t c = c0; c < c1; ++c) {
          const int32_t v = hist[c * E + e];
          hist[c * E + e] = run;
          run += v;
        }
      }
      if (seg == nseg - 1) {
        s_cnt[e] = run;
        counts[e] = run;
      }
    }
    __syncthreads();
  }

  // Exclusive scan of the ALIGN_M-padded counts (E <= 1024: one pass per thread chunk).
  const int per = (E + blockDim.x - 1) / blockDim.x;
  int32_t local = 0;
  const int e0 = tid * per;
  for (int i = 0; i < per; ++i) {
    int e = e0 + i;
    if (e < E) local += (s_cnt[e] + ALIGN_M - 1) / ALIGN_M * ALIGN_M;
  }
  // block-wide exclusive scan of `local`
  const int lane = tid & 63, wave = tid >> 6;
  int32_t incl = local;
  for (int o = 1; o < 64; o <<= 1) {
    int32_t v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wave[wave] = incl;
  __syncthreads();
  int32_t wave_base = 0;
  for (int w = 0; w < wave; ++w) wave_base += s_wave[w];
  int32_t run = wave_base + incl - local;
  for (int i = 0; i < per; ++i) {
    int e = e0 + i;
    if (e < E) {
      s_off[e] = run;
      run += (s_cnt[e] + ALIGN_M - 1) / ALIGN_M * ALIGN_M;
    }
  }
  if (tid == blockDim.x - 1) {
    int32_t total = 0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) total += s_wave[w];
    s_off[E] = total;
  }
  __syncthreads();
  for (int e = tid; e <= E; e += blockDim.x) offs[e] = s_off[e];
  const int32_t total = s_off[E];
  if (tid == 0) npp[0] = total;

  // Aligned block -> owning expert: the last expert whose run starts at or before it.
  const int64_t n_blocks = l_cap / ALIGN_M;
  for (int64_t b = tid; b < n_blocks; b += blockDim.x) {
    int32_t owner = 0;
    const int64_t pos = b * ALIGN_M;
    if (pos < total) {
      int lo = 0, hi = E - 1;  // largest e with s_off[e] <= pos
      while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (s_off[mid] <= pos) lo = mid;
        else hi = mid - 1;
      }
      owner = lo;
    }
    expert_ids[b] = owner;
  }

  // Sentinel M in every pad slot and in the unused tail [total, l_cap).
  for (int e = tid; e < E; e += blockDim.x) {
    for (int32_t s = s_off[e] + s_cnt[e]; s < s_off[e + 1]; ++s) sorted_ids[s] = (int32_t)M;
  }
  for (int64_t s = total + tid; s < l_cap; s += blockDim.x) sorted_ids[s] = (int32_t)M;
}

__global__ void __launch_bounds__(1024)
dispatch_scatter_kernel(const int64_t* __restrict__ topk_idx, int64_t M, int E,
                        const int32_t* __restrict__ chunk_base,
                        const int32_t* __restrict__ offs, int32_t* __restrict__ sorted_ids,
                        int32_t* __restrict__ inv) {
  extern __shared__ unsigned long long s_mask[];  // [waves][E]
  const int waves = blockDim.x >> 6;
  for (int i = threadIdx.x; i < waves * E; i += blockDim.x) s_mask[i] = 0ull;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int e = -1;
  if (p < M) {
    int64_t v = topk_idx[p];
    if (v >= 0 && v < E) e = (int)v;
  }
  if (e >= 0) atomicOr(&s_mask[wave * E + e], 1ull << lane);
  __syncthreads();
  if (p < M) {
    if (e < 0) {
      inv[p] = -1;
      return;
    }
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rank = __popcll(s_mask[wave * E + e] & below);
    for (int w = 0; w < wave; ++w) rank += __popcll(s_mask[w * E + e]);
    const int32_t slot = offs[e] + chunk_base[(int64_t)blockIdx.x * E + e] + rank;
    sorted_ids[slot] = (int32_t)p;
    inv[p] = slot;
  }
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

extern "C" int nsmoe_dispatch(const int64_t* topk_idx, int64_t n_pairs, int32_t n_experts,
                              int32_t* sorted_ids, int32_t* expert_ids, int32_t* pad_offsets,
                              int32_t* counts, int32_t* n_post_pad, int32_t* inv,
                              void* workspace, size_t workspace_bytes, void* stream) {
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
    return fill_i32(n_post_pad, 1, 0, s);
  }
  NSMOE_REQUIRE(topk_idx && sorted_ids && expert_ids && pad_offsets && counts && n_post_pad &&
                    inv && workspace, "dispatch: NULL pointer");
  const size_t need = nsmoe_dispatch_workspace_size(n_pairs, n_experts);
  if (workspace_bytes < need) {
    set_error("dispatch: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  const int chunk = dispatch_chunk(n_experts);
  const int64_t n_chunks = cdiv(n_pairs, chunk);
  const int64_t l_cap = nsmoe_dispatch_l_cap(n_pairs, n_experts);
  int32_t* hist = (int32_t*)workspace;

  KernelTimer timer("dispatch", s);
  dispatch_hist_kernel<<<(unsigned)n_chunks, chunk, n_experts * sizeof(int32_t), s>>>(
      topk_idx, n_pairs, n_experts, hist);
  NSMOE_TRY(check_launch("dispatch_hist_kernel"));
  dispatch_scan_kernel<<<1, 1024, 0, s>>>(hist, n_chunks, n_experts, n_pairs, l_cap,
                                          sorted_ids, expert_ids, pad_offsets, counts,
                                          n_post_pad);
  NSMOE_TRY(check_launch("dispatch_scan_kernel"));
  dispatch_scatter_kernel<<<(unsigned)n_chunks, chunk,
                            (chunk / 64) * n_experts * sizeof(unsigned long long), s>>>(
      topk_idx, n_pairs, n_experts, hist, pad_offsets, sorted_ids, inv);
  timer.stop();
  return check_launch("dispatch_scatter_kernel");
}

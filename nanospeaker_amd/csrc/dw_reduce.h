// The dW split-K reduce (experts.hip's dw_reduce kernels; also run inside combine_dx's
// launch, router_grad.hip): the fp32 partials of the multi-chunk groups summed in chunk
// order into dW.  The workgroup's column of the pass (bx of nbx) is an argument, so the
// body runs in any launch whose workgroups have NT threads.
#pragma once

#include "experts_common.h"

namespace nsmoe {

// Workgroup bx of nbx sums group g's partials: each thread 4 consecutive elements (one
// 16-byte vector per chunk, every chunk's load in flight at once), so the pass streams
// the partials at full width; the order of the additions is the chunk order for every
// element, whatever the launch shape.
template <int DT, int MODE>
__device__ __forceinline__ void dw_reduce_group(const ExpParams& p, int g, int bx, int nbx) {
  using T = typename Elem<DT>::T;
  const int nch = dw_chunks(rows_of(p, g));
  if (nch <= 1) return;
  // First partial of group g: the chunk counts of the multi-chunk groups before it,
  // counted by all threads at once (integer sum: the order does not matter).  A caller
  // may run several groups in turn (dw_reduce_pair_row): the barrier before the reset
  // keeps thread 0 from clearing s_base while a slower wave still reads the previous
  // group's value.
  __shared__ int s_base;
  __syncthreads();
  if (threadIdx.x == 0) s_base = 0;
  __syncthreads();
  int part = 0;
  for (int q = threadIdx.x; q < g; q += NT) {
    const int c = dw_chunks(rows_of(p, q));
    if (c > 1) part += c;
  }
  if (part) atomicAdd(&s_base, part);
  __syncthreads();
  const int d = p.d, H = p.H;
  const int64_t mn = MODE == 0 ? (int64_t)d * 2 * H : (int64_t)H * d;
  T* dst = g < p.E ? (T*)p.dw_a + (int64_t)g * mn : (T*)p.dw_sh + (int64_t)(g - p.E) * mn;
  const float* src = p.partial + (int64_t)s_base * mn;
  const int64_t n4 = (mn % 4 == 0) ? mn / 4 : 0;  // 16-byte vectors (every partial is 16-B aligned)
  for (int64_t i = (int64_t)bx * NT + threadIdx.x; i < n4; i += (int64_t)nbx * NT) {
    // Up to DEPTH chunks' loads in flight at once, added in chunk order.
    constexpr int DEPTH = 16;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < nch; c0 += DEPTH) {
      f32x4 a[DEPTH];
#pragma unroll
      for (int u = 0; u < DEPTH; ++u)
        if (c0 + u < nch) a[u] = ((const f32x4*)(src + (int64_t)(c0 + u) * mn))[i];
#pragma unroll
      for (int u = 0; u < DEPTH; ++u)
        if (c0 + u < nch) acc += a[u];
    }
    if (DT != DT_F32 && ((uintptr_t)dst & 7) == 0) {  // one 8-byte store (mn % 4 == 0)
      *(uint2*)(dst + i * 4) = make_uint2(pack2<DT>(acc[0], acc[1]), pack2<DT>(acc[2], acc[3]));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[i * 4 + e] = Elem<DT>::from_f(acc[e]);
    }
  }
  for (int64_t i = n4 * 4 + (int64_t)bx * NT + threadIdx.x; i < mn; i += (int64_t)nbx * NT) {
    float acc = 0.0f;
    for (int c = 0; c < nch; ++c) acc += src[(int64_t)c * mn + i];
    dst[i] = Elem<DT>::from_f(acc);
  }
}

// Both modes over the groups that can have several chunks: row y in [0, 2 NY),
// NY = S + routed_rows: mode = y / NY, row j = y % NY.  Rows j < S take shared group
// E + j.  With routed_rows = E, row S + r takes routed group r; with routed_rows = 1 the
// one row S finds the routed groups of several chunks (usually none or a few: routed
// groups average fewer rows than a chunk) and takes them in turn.  A pass over all
// 2 (E + S) groups spends most of its time on workgroups that only find one chunk.
struct DwReduceArgs {
  ExpParams p_in, p_out;  // dW_in and dW_out: pointers and partials
  int routed_rows;
  int nbx;                // workgroups per row (0: no reduce to run)
  int rows;               // 2 (S + routed_rows)
};

template <int DT>
__device__ __forceinline__ void dw_reduce_pair_row(const DwReduceArgs& r, int bx, int y) {
  const ExpParams& p_in = r.p_in;
  const int E = p_in.E, S = p_in.S, ny = S + r.routed_rows;
  const int mode = y >= ny ? 1 : 0, j = y - mode * ny;
  auto run = [&](int g) {
    if (mode == 0) dw_reduce_group<DT, 0>(r.p_in, g, bx, r.nbx);
    else dw_reduce_group<DT, 1>(r.p_out, g, bx, r.nbx);
  };
  if (j < S) {
    run(E + j);
  } else if (r.routed_rows == E) {
    run(j - S);
  } else {
    __shared__ int s_list[NT];
    __shared__ int s_n;
    for (int g0 = 0; g0 < E; g0 += NT) {
      if (threadIdx.x == 0) s_n = 0;
      __syncthreads();
      const int g = g0 + (int)threadIdx.x;
      if (g < E && dw_chunks(rows_of(p_in, g)) > 1) s_list[atomicAdd(&s_n, 1)] = g;
      __syncthreads();
      const int n = s_n;
      for (int i = 0; i < n; ++i) run(s_list[i]);
      __syncthreads();  // the list is read before the next round rewrites it
    }
  }
}

}  // namespace nsmoe

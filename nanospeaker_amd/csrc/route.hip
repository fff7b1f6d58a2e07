// Router tail on device: softmax, top-k selection with torch-CPU tie order, gate
// renormalisation, and the matching backward to d(logits).
//
// Reference: TopKRouter.forward (src/model/router.py:69-98).  The logits GEMM
// `(x @ W).float()` (router.py:69) and the optional exploration noise (router.py:76-77)
// stay in torch; this file takes the fp32 logits from there.
//
// Layout: one token row per wavefront, four rows per workgroup.  The wave's lanes load
// the row (coalesced), reduce max / sum for the softmax and write probs; the row's
// (key, expert id) pairs are staged in LDS as 64-bit words (key bits << 32 | id) so a
// swap in the selection is one 64-bit move.  The selection itself is sequential (lane 0
// of the wave): with one row per wave no lane waits on another row's control flow, and
// T rows give T independent waves to hide the LDS latency of the sequential passes.
//
// Selection has to reproduce torch's CPU topk bit for bit, ties included: the order of
// equal keys is whatever libstdc++'s nth_element / sort / partial_sort leave (see
// ATen/native/TopKImpl.h:44-94).  The routines below restate those published
// algorithms (introselect with median-of-three, unguarded Hoare partition, heap select,
// insertion sort, introsort) on the row in LDS.
#include "nsmoe_capi_internal.h"
#include "nsmoe_common.h"

namespace nsmoe {

constexpr int ROUTE_WAVES = 4;  // rows (waves) per workgroup
constexpr int ROUTE_THREADS = 64 * ROUTE_WAVES;

struct LaneRow {
  uint64_t* base;  // the row's element i
  __device__ __forceinline__ uint64_t& operator[](int i) const { return base[i]; }
};

__device__ __forceinline__ float key_of(uint64_t e) { return __uint_as_float((uint32_t)(e >> 32)); }
__device__ __forceinline__ int id_of(uint64_t e) { return (int)(uint32_t)e; }
__device__ __forceinline__ uint64_t pack(float key, int id) {
  return ((uint64_t)__float_as_uint(key) << 32) | (uint32_t)id;
}

// "x ranks before y": x is NaN and y is not, or x > y (TopKImpl.h:68-69).
__device__ __forceinline__ bool gt(uint64_t x, uint64_t y) {
  float a = key_of(x), b = key_of(y);
  return (__builtin_isnan(a) && !__builtin_isnan(b)) || a > b;
}

__device__ __forceinline__ void swap_at(const LaneRow& a, int i, int j) {
  uint64_t t = a[i];
  a[i] = a[j];
  a[j] = t;
}

__device__ __forceinline__ int lg2i(int n) { return 31 - __builtin_clz(n); }

// ---- heap primitives on a[first, first + len) ------------------------------------------

__device__ void push_heap_d(const LaneRow& a, int f, int hole, int top, uint64_t value) {
  int parent = (hole - 1) / 2;
  while (hole > top && gt(a[f + parent], value)) {
    a[f + hole] = a[f + parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a[f + hole] = value;
}

__device__ void adjust_heap_d(const LaneRow& a, int f, int hole, int len, uint64_t value) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (gt(a[f + second], a[f + second - 1])) second--;
    a[f + hole] = a[f + second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    a[f + hole] = a[f + second - 1];
    hole = second - 1;
  }
  push_heap_d(a, f, hole, top, value);
}

__device__ void make_heap_d(const LaneRow& a, int f, int len) {
  if (len < 2) return;
  int parent = (len - 2) / 2;
  for (;;) {
    uint64_t value = a[f + parent];
    adjust_heap_d(a, f, parent, len, value);
    if (parent == 0) return;
    parent--;
  }
}

// heap is a[f, f + len); the displaced element is a[f + res]
__device__ void pop_heap_d(const LaneRow& a, int f, int len, int res) {
  uint64_t value = a[f + res];
  a[f + res] = a[f];
  adjust_heap_d(a, f, 0, len, value);
}

__device__ void heap_select_d(const LaneRow& a, int f, int middle, int last) {
  make_heap_d(a, f, middle);
  for (int i = middle; i < last; ++i)
    if (gt(a[f + i], a[f])) pop_heap_d(a, f, middle, i);
}

__device__ void sort_heap_d(const LaneRow& a, int f, int last) {
  while (last > 1) {
    --last;
    pop_heap_d(a, f, last, last);
  }
}

// ---- insertion sorts -----------------------------------------------------------------

__device__ void unguarded_linear_insert_d(const LaneRow& a, int last) {
  uint64_t val = a[last];
  int next = last - 1;
  while (gt(val, a[next])) {
    a[last] = a[next];
    last = next;
    --next;
  }
  a[last] = val;
}

__device__ void insertion_sort_d(const LaneRow& a, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    if (gt(a[i], a[first])) {
      uint64_t val = a[i];
      for (int j = i; j > first; --j) a[j] = a[j - 1];
      a[first] = val;
    } else {
      unguarded_linear_insert_d(a, i);
    }
  }
}

// ---- partitioning --------------------------------------------------------------------

__device__ void move_median_to_first_d(const LaneRow& a, int result, int x, int y, int z) {
  if (gt(a[x], a[y])) {
    if (gt(a[y], a[z])) swap_at(a, result, y);
    else if (gt(a[x], a[z])) swap_at(a, result, z);
    else swap_at(a, result, x);
  } else if (gt(a[x], a[z])) {
    swap_at(a, result, x);
  } else if (gt(a[y], a[z])) {
    swap_at(a, result, z);
  } else {
    swap_at(a, result, y);
  }
}

__device__ int unguarded_partition_pivot_d(const LaneRow& a, int first, int last) {
  int mid = first + (last - first) / 2;
  move_median_to_first_d(a, first, first + 1, mid, last - 1);
  const uint64_t pivot = a[first];  // the pivot slot is not touched by the partition
  int lo = first + 1, hi = last;
  for (;;) {
    while (gt(a[lo], pivot)) ++lo;
    --hi;
    while (gt(pivot, a[hi])) --hi;
    if (!(lo < hi)) return lo;
    swap_at(a, lo, hi);
    ++lo;
  }
}

__device__ void nth_element_d(const LaneRow& a, int nth, int n) {
  if (n == 0 || nth == n) return;
  int first = 0, last = n, depth = lg2i(n) * 2;
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_d(a, first, nth + 1 - first, last - first);
      swap_at(a, first, nth);
      return;
    }
    --depth;
    int cut = unguarded_partition_pivot_d(a, first, last);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  insertion_sort_d(a, first, last);
}

// std::sort on a[0, n).  introsort_loop recurses on the right part and loops on the
// left; the subranges it leaves are disjoint, so visiting them from an explicit stack
// in another order gives the same array.
__device__ void sort_d(const LaneRow& a, int n) {
  if (n == 0) return;
  if (n > 16) {
    int st_first[40], st_last[40], st_depth[40];
    int sp = 0;
    st_first[0] = 0; st_last[0] = n; st_depth[0] = lg2i(n) * 2; sp = 1;
    while (sp > 0) {
      --sp;
      int first = st_first[sp], last = st_last[sp], depth = st_depth[sp];
      while (last - first > 16) {
        if (depth == 0) {
          heap_select_d(a, first, last - first, last - first);
          sort_heap_d(a, first, last - first);
          break;
        }
        --depth;
        int cut = unguarded_partition_pivot_d(a, first, last);
        st_first[sp] = cut; st_last[sp] = last; st_depth[sp] = depth; ++sp;
        last = cut;
      }
    }
    insertion_sort_d(a, 0, 16);
    for (int i = 16; i != n; ++i) unguarded_linear_insert_d(a, i);
  } else {
    insertion_sort_d(a, 0, n);
  }
}

// torch CPU topk(largest=True, sorted=True) over the lane's row: afterwards a[0, k)
// holds the selected (key, id) pairs in output order.
__device__ void topk_select(const LaneRow& a, int n, int k) {
  if (k == 0) return;
  if (k * 64 <= n) {
    heap_select_d(a, 0, k, n);
    sort_heap_d(a, 0, k);
  } else {
    nth_element_d(a, k - 1, n);
    sort_d(a, k - 1);
  }
}

// ---- wave reductions ---------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// ---- forward ---------------------------------------------------------------------------
//
// flags bit 0 (want_probs): training branch, probs = softmax(logits) and the selection
//   runs on probs (router.py:79-81); probs [T, E] is written out.
// flags bit 1 (normalize):  normalize_weights.
// Without want_probs the selection runs on the logits and the gates are
// softmax(topk logits) (normalize) or softmax(logits)[idx] (router.py:83-92).
// With want_probs and normalize and k > 1 the gates are p / sum(p) (router.py:96-97).
// E <= 128: each lane holds row elements lane and lane + 64.
// flags bit 2 (logits16): the logits are stored in the gate dtype DT (the bf16 / fp16 GEMM
//   output that router.py:69 widens with .float()); they are widened here on load.
template <int DT>
__global__ void __launch_bounds__(ROUTE_THREADS)
route_fwd_kernel(const void* __restrict__ logits, int64_t T, int E, int k, int flags,
                 typename Elem<DT>::T* __restrict__ topk_w, int64_t* __restrict__ topk_idx,
                 float* __restrict__ probs) {
  extern __shared__ uint64_t lds_q[];  // [ROUTE_WAVES][E]
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROUTE_WAVES + wave;
  const bool active = row < T;
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;
  uint64_t* q = lds_q + wave * E;
  const bool has0 = lane < E, has1 = lane + 64 < E;

  float v0 = -INFINITY, v1 = -INFINITY;
  if (active) {
    if (flags & 4) {
      const typename Elem<DT>::T* lrow = (const typename Elem<DT>::T*)logits + row * E;
      if (has0) v0 = Elem<DT>::to_f(lrow[lane]);
      if (has1) v1 = Elem<DT>::to_f(lrow[lane + 64]);
    } else {
      const float* lrow = (const float*)logits + row * E;
      if (has0) v0 = lrow[lane];
      if (has1) v1 = lrow[lane + 64];
    }
  }
  // Row max (NaN-propagating, like torch's softmax) and sum of exp.
  const bool nan_here = (has0 && __builtin_isnan(v0)) || (has1 && __builtin_isnan(v1));
  const bool any_nan = __ballot(nan_here) != 0ull;
  float m = wave_max(fmaxf(v0, v1));
  if (any_nan) m = __uint_as_float(0x7fc00000u);
  float row_inv_sum = 0.0f;
  float k0 = v0, k1 = v1;
  if (want_probs || !normalize) {
    const float e0 = has0 ? expf(v0 - m) : 0.0f;
    const float e1 = has1 ? expf(v1 - m) : 0.0f;
    row_inv_sum = 1.0f / wave_sum(e0 + e1);
    if (want_probs) {
      k0 = e0 * row_inv_sum;
      k1 = e1 * row_inv_sum;
      if (active) {
        float* prow = probs + row * E;
        if (has0) prow[lane] = k0;
        if (has1) prow[lane + 64] = k1;
      }
    }
  }
  // Fast path: k rounds of a wave-wide arg-max.  If every round's maximum is unique among
  // the values still in play (no NaN, no tie inside the top k, none at its boundary),
  // the sorted top k is unique, so any selection returns CPU topk's answer.  A row with
  // a tie anywhere that matters takes the exact restatement below instead.
  bool exact = any_nan || !active;
  if (!exact) {
    bool av0 = has0, av1 = has1;
    for (int t = 0; t < k; ++t) {
      const float c = fmaxf(av0 ? k0 : -INFINITY, av1 ? k1 : -INFINITY);
      const float mx = wave_max(c);
      const unsigned long long b0 = __ballot(av0 && k0 == mx);
      const unsigned long long b1 = __ballot(av1 && k1 == mx);
      if (__popcll(b0) + __popcll(b1) != 1) {
        exact = true;
        break;
      }
      const int src = b0 ? __ffsll((long long)b0) - 1 : __ffsll((long long)b1) - 1 + 64;
      if (lane == (src & 63)) {
        if (src < 64) av0 = false;
        else av1 = false;
      }
      if (lane == 0) q[t] = pack(mx, src);
    }
  }
  if (exact && active) {
    if (has0) q[lane] = pack(k0, lane);
    if (has1) q[lane + 64] = pack(k1, lane + 64);
  }
  __syncthreads();
  if (exact && active && lane == 0) topk_select(LaneRow{q}, E, k);
  __syncthreads();
  if (!active) return;

  // Lane j < k handles output j (and j + 64 when k > 64).
  using OutT = typename Elem<DT>::T;
  int64_t* idx_out = topk_idx + row * k;
  OutT* w_out = topk_w + row * k;
  const bool o0 = lane < k, o1 = lane + 64 < k;
  const float s0 = o0 ? key_of(q[lane]) : 0.0f, s1 = o1 ? key_of(q[lane + 64]) : 0.0f;
  if (o0) idx_out[lane] = id_of(q[lane]);
  if (o1) idx_out[lane + 64] = id_of(q[lane + 64]);
  float w0 = s0, w1 = s1;
  if (want_probs) {
    if (normalize && k > 1) {
      const float S = wave_sum(s0 + s1);
      w0 = s0 / S;
      w1 = s1 / S;
    }
  } else if (normalize) {
    const float mk = wave_max(fmaxf(o0 ? s0 : -INFINITY, o1 ? s1 : -INFINITY));
    const float e0 = o0 ? expf(s0 - mk) : 0.0f, e1 = o1 ? expf(s1 - mk) : 0.0f;
    const float inv = 1.0f / wave_sum(e0 + e1);
    w0 = e0 * inv;
    w1 = e1 * inv;
  } else {
    w0 = expf(s0 - m) * row_inv_sum;
    w1 = expf(s1 - m) * row_inv_sum;
  }
  if (o0) w_out[lane] = Elem<DT>::from_f(w0);
  if (o1) w_out[lane + 64] = Elem<DT>::from_f(w1);
}

// ---- backward --------------------------------------------------------------------------
//
// d(logits) for the same three branches, in fp32, one row per wave:
//   train: w = p_sel / S (normalize, k > 1)  ->  dp_j = (dw_j - sum_i dw_i w_i) / S
//          dprobs = grad_probs (aux loss, may be absent) + scatter(dp)
//          dlogits = p * (dprobs - sum_e p_e dprobs_e)
//   eval normalize:   w = softmax(l_sel) -> dl_sel = w * (dw - sum w dw)
//   eval !normalize:  w = softmax(l)[idx] -> softmax backward of scatter(dw)
// `src` holds probs for the train branch and logits otherwise.  Ids outside [0, E)
// (not produced by route_fwd) give the row a zero gradient.
// The balance loss aux = coef E sum_e f_e mean_t p[t, e] (router.py:110-111, f constant)
// adds d aux / d p[t, e] = grad_aux coef E f_e / T to d(probs), computed here from the
// counts (aux_counts non-NULL) instead of being materialised as a [T, E] tensor.
// flags bit 2 (logits16): in the eval branches `src` is stored in DT, and grad_logits is
// written in DT (the gradient of router.py:69's .float()); otherwise both are fp32.
template <int DT>
__global__ void __launch_bounds__(ROUTE_THREADS)
route_bwd_kernel(const void* __restrict__ src, const int64_t* __restrict__ topk_idx,
                 const typename Elem<DT>::T* __restrict__ grad_w,
                 const float* __restrict__ grad_probs, const float* __restrict__ grad_aux,
                 const int32_t* __restrict__ aux_counts, float aux_coef, int64_t T, int E,
                 int k, int flags, void* __restrict__ grad_logits_v) {
  extern __shared__ float lds_f[];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * ROUTE_WAVES + wave;
  if (row >= T) return;  // no workgroup barriers below: each wave works alone
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;
  float* sv = lds_f + wave * 2 * E;  // the row's src values
  float* sg = sv + E;                // running d(probs) or d(logits) row
  const bool has0 = lane < E, has1 = lane + 64 < E;
  const bool w16 = (flags & 4) != 0;
  using ET = typename Elem<DT>::T;
  float x0 = 0.0f, x1 = 0.0f;
  if (w16 && !want_probs) {
    const ET* srow = (const ET*)src + row * E;
    if (has0) x0 = Elem<DT>::to_f(srow[lane]);
    if (has1) x1 = Elem<DT>::to_f(srow[lane + 64]);
  } else {
    const float* srow = (const float*)src + row * E;
    if (has0) x0 = srow[lane];
    if (has1) x1 = srow[lane + 64];
  }
  float g0 = 0.0f, g1 = 0.0f;
  if (grad_probs && want_probs) {
    const float* gp = grad_probs + row * E;
    if (has0) g0 = gp[lane];
    if (has1) g1 = gp[lane + 64];
  }
  if (aux_counts && grad_aux && want_probs) {
    const float c0 = has0 ? (float)aux_counts[lane] : 0.0f;
    const float c1 = has1 ? (float)aux_counts[lane + 64] : 0.0f;
    const float scale = grad_aux[0] * aux_coef * (float)E / fmaxf(wave_sum(c0 + c1), 1.0f) /
                        (float)T;
    g0 += c0 * scale;
    g1 += c1 * scale;
  }
  // d(logits) is stored through these (fp32, or DT under logits16 in the eval branches).
  auto put = [&](int e, float v) {
    if (w16) ((ET*)grad_logits_v)[row * E + e] = Elem<DT>::from_f(v);
    else ((float*)grad_logits_v)[row * E + e] = v;
  };
  if (has0) { sv[lane] = x0; sg[lane] = want_probs ? g0 : 0.0f; }
  if (has1) { sv[lane + 64] = x1; sg[lane + 64] = want_probs ? g1 : 0.0f; }
  const bool o0 = lane < k, o1 = lane + 64 < k;
  int64_t i0 = o0 ? topk_idx[row * k + lane] : 0, i1 = o1 ? topk_idx[row * k + lane + 64] : 0;
  const bool bad = (o0 && (i0 < 0 || i0 >= E)) || (o1 && (i1 < 0 || i1 >= E));
  if (__ballot(bad) != 0ull) {
    if (has0) put(lane, 0.0f);
    if (has1) put(lane + 64, 0.0f);
    return;
  }
  const float d0 = o0 ? Elem<DT>::to_f(grad_w[row * k + lane]) : 0.0f;
  const float d1 = o1 ? Elem<DT>::to_f(grad_w[row * k + lane + 64]) : 0.0f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float s_0 = o0 ? sv[i0] : 0.0f, s_1 = o1 ? sv[i1] : 0.0f;  // selected src values

  float p0, p1;  // softmax probabilities of this lane's row elements
  if (want_probs) {
    const bool renorm = normalize && k > 1;
    float a0 = d0, a1 = d1;
    if (renorm) {
      const float S = wave_sum(s_0 + s_1);
      const float dot = wave_sum(d0 * (s_0 / S) + d1 * (s_1 / S));
      a0 = (d0 - dot) / S;
      a1 = (d1 - dot) / S;
    }
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] += a0;  // ids in a row are distinct: no two lanes hit one slot
    if (o1) sg[i1] += a1;
    p0 = x0;
    p1 = x1;
  } else if (normalize) {
    const float mk = wave_max(fmaxf(o0 ? s_0 : -INFINITY, o1 ? s_1 : -INFINITY));
    const float e0 = o0 ? expf(s_0 - mk) : 0.0f, e1 = o1 ? expf(s_1 - mk) : 0.0f;
    const float inv = 1.0f / wave_sum(e0 + e1);
    const float w0 = e0 * inv, w1 = e1 * inv;
    const float dot = wave_sum(w0 * d0 + w1 * d1);
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] = w0 * (d0 - dot);
    if (o1) sg[i1] = w1 * (d1 - dot);
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (has0) put(lane, sg[lane]);
    if (has1) put(lane + 64, sg[lane + 64]);
    return;
  } else {
    const float m = wave_max(fmaxf(has0 ? x0 : -INFINITY, has1 ? x1 : -INFINITY));
    const float e0 = has0 ? expf(x0 - m) : 0.0f, e1 = has1 ? expf(x1 - m) : 0.0f;
    const float inv = 1.0f / wave_sum(e0 + e1);
    p0 = e0 * inv;
    p1 = e1 * inv;
    __builtin_amdgcn_wave_barrier();
    if (o0) sg[i0] += d0;
    if (o1) sg[i1] += d1;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  const float q0 = has0 ? sg[lane] : 0.0f, q1 = has1 ? sg[lane + 64] : 0.0f;
  const float pd = wave_sum((has0 ? p0 * q0 : 0.0f) + (has1 ? p1 * q1 : 0.0f));
  if (has0) put(lane, p0 * (q0 - pd));
  if (has1) put(lane + 64, p1 * (q1 - pd));
}

// ---- balance loss (router.py:100-111) ----------------------------------------------------
//
// aux = coef * E * sum_e f_e * mean_t probs[t, e],  f = counts / max(sum counts, 1).
// Pass 1: each block sums BL_ROWS rows of probs per expert (coalesced along the row, 8
// independent accumulators so the loads overlap); pass 2: one block adds the partials in a
// fixed order (8 interleaved partial sums per expert, then combined in order) and forms
// the scalar, so the result is deterministic.
constexpr int BL_ROWS = 64;
constexpr int BL_UNROLL = 8;

__global__ void __launch_bounds__(128)
balance_partial_kernel(const float* __restrict__ probs, int64_t T, int E,
                       float* __restrict__ partial) {
  const int e = threadIdx.x;
  if (e >= E) return;
  const int64_t r0 = (int64_t)blockIdx.x * BL_ROWS;
  const int nr = (int)(r0 + BL_ROWS < T ? BL_ROWS : T - r0);
  float acc[BL_UNROLL];
#pragma unroll
  for (int u = 0; u < BL_UNROLL; ++u) acc[u] = 0.0f;
  for (int r = 0; r < nr; r += BL_UNROLL) {
#pragma unroll
    for (int u = 0; u < BL_UNROLL; ++u)
      if (r + u < nr) acc[u] += probs[(r0 + r + u) * E + e];
  }
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < BL_UNROLL; ++u) s += acc[u];
  partial[(int64_t)blockIdx.x * E + e] = s;
}

// 1024 threads: thread (q, e) with q = tid / 128 sums partial blocks q, q + 8, q + 16, ...
// of expert e; the 8 slices are then added in q order.
__global__ void __launch_bounds__(1024)
balance_final_kernel(const float* __restrict__ partial, int64_t nblk, const int32_t* counts,
                     int64_t T, int E, float coef, float* __restrict__ aux) {
  __shared__ float s_q[8][128];
  __shared__ float s_part[2][2];
  const int tid = threadIdx.x, e = tid & 127, q = tid >> 7;
  if (e < E) {
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    int64_t b = q;
    for (; b + 24 < nblk; b += 32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) acc[u] += partial[(b + 8 * u) * E + e];
    }
    for (int u = 0; b < nblk; b += 8, ++u) acc[u & 3] += partial[b * E + e];
    s_q[q][e] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  }
  __syncthreads();
  if (tid < 128) {
    const int lane = tid & 63, wave = tid >> 6;
    float col = 0.0f, c = 0.0f;
    if (e < E) {
#pragma unroll
      for (int qq = 0; qq < 8; ++qq) col += s_q[qq][e];
      c = (float)counts[e];
    }
    const float num = wave_sum(c * col), den = wave_sum(c);
    if (lane == 0) {
      s_part[wave][0] = num;
      s_part[wave][1] = den;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const float n = s_part[0][0] + s_part[1][0];
    const float dsum = fmaxf(s_part[0][1] + s_part[1][1], 1.0f);
    aux[0] = coef * (float)E * (n / dsum / (float)T);
  }
}

constexpr int ROUTE_MAX_EXPERTS = 128;  // two row elements per lane

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_route_fwd(const void* logits, int64_t n_tokens, int32_t n_experts,
                               int32_t top_k, int32_t flags, int32_t w_dtype, void* topk_w,
                               int64_t* topk_idx, float* probs, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_fwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_fwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_fwd: top_k %d outside [1, %d]",
                top_k, n_experts);
  NSMOE_REQUIRE(!(flags & 1) || probs, "route_fwd: probs requested but NULL");
  NSMOE_REQUIRE(!(flags & 4) || w_dtype != DT_F32, "route_fwd: 16-bit logits need a 16-bit dtype");
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(logits && topk_w && topk_idx, "route_fwd: NULL pointer");
  dim3 grid((unsigned)cdiv(n_tokens, ROUTE_WAVES)), block(ROUTE_THREADS);
  size_t lds = (size_t)n_experts * ROUTE_WAVES * sizeof(uint64_t);
  hipStream_t s = (hipStream_t)stream;
  KernelTimer timer("route_fwd", s);
  switch (w_dtype) {
    case DT_BF16:
      route_fwd_kernel<DT_BF16><<<grid, block, lds, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (uint16_t*)topk_w, topk_idx, probs);
      break;
    case DT_F16:
      route_fwd_kernel<DT_F16><<<grid, block, lds, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (uint16_t*)topk_w, topk_idx, probs);
      break;
    case DT_F32:
      route_fwd_kernel<DT_F32><<<grid, block, lds, s>>>(logits, n_tokens, n_experts, top_k,
          flags, (float*)topk_w, topk_idx, probs);
      break;
    default:
      NSMOE_REQUIRE(false, "route_fwd: unknown dtype %d", w_dtype);
  }
  timer.stop();
  return check_launch("route_fwd_kernel");
}

extern "C" int nsmoe_route_bwd(const void* src, const int64_t* topk_idx, const void* grad_w,
                               int32_t w_dtype, const float* grad_probs, const float* grad_aux,
                               const int32_t* aux_counts, float aux_coef, int64_t n_tokens,
                               int32_t n_experts, int32_t top_k, int32_t flags,
                               void* grad_logits, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_bwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_bwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_bwd: bad top_k %d", top_k);
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(src && topk_idx && grad_w && grad_logits, "route_bwd: NULL pointer");
  NSMOE_REQUIRE(!(flags & 4) || w_dtype != DT_F32, "route_bwd: 16-bit logits need a 16-bit dtype");
  dim3 grid((unsigned)cdiv(n_tokens, ROUTE_WAVES)), block(ROUTE_THREADS);
  size_t lds = (size_t)n_experts * ROUTE_WAVES * sizeof(float) * 2;
  hipStream_t s = (hipStream_t)stream;
  switch (w_dtype) {
    case DT_BF16:
      route_bwd_kernel<DT_BF16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits);
      break;
    case DT_F16:
      route_bwd_kernel<DT_F16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits);
      break;
    case DT_F32:
      route_bwd_kernel<DT_F32><<<grid, block, lds, s>>>(src, topk_idx, (const float*)grad_w,
          grad_probs, grad_aux, aux_counts, aux_coef, n_tokens, n_experts, top_k, flags,
          grad_logits);
      break;
    default:
      NSMOE_REQUIRE(false, "route_bwd: unknown dtype %d", w_dtype);
  }
  return check_launch("route_bwd_kernel");
}

extern "C" size_t nsmoe_balance_loss_workspace_size(int64_t n_tokens, int32_t n_experts) {
  if (n_tokens <= 0 || n_experts <= 0) return 0;
  return (size_t)cdiv(n_tokens, BL_ROWS) * (size_t)n_experts * sizeof(float);
}

extern "C" int nsmoe_balance_loss(const float* probs, const int32_t* counts, int64_t n_tokens,
                                  int32_t n_experts, float coef, float* aux, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "balance_loss: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "balance_loss: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(aux && counts, "balance_loss: NULL pointer");
  hipStream_t s = (hipStream_t)stream;
  if (n_tokens == 0) {
    // mean over no rows is NaN in torch (router.py:111 on an empty batch); the block never
    // calls this with T = 0, but keep the definition total.
    balance_final_kernel<<<1, 1024, 0, s>>>(nullptr, 0, counts, 0, n_experts, coef, aux);
    return check_launch("balance_final_kernel");
  }
  NSMOE_REQUIRE(probs && workspace, "balance_loss: NULL pointer");
  const size_t need = nsmoe_balance_loss_workspace_size(n_tokens, n_experts);
  if (workspace_bytes < need) {
    set_error("balance_loss: workspace %zu B < %zu B", workspace_bytes, need);
    return NSMOE_EWORKSPACE;
  }
  const int64_t nblk = cdiv(n_tokens, BL_ROWS);
  balance_partial_kernel<<<(unsigned)nblk, 128, 0, s>>>(probs, n_tokens, n_experts,
                                                        (float*)workspace);
  NSMOE_TRY(check_launch("balance_partial_kernel"));
  balance_final_kernel<<<1, 1024, 0, s>>>((const float*)workspace, nblk, counts, n_tokens,
                                          n_experts, coef, aux);
  return check_launch("balance_final_kernel");
}

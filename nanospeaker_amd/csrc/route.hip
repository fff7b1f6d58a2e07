// Router tail on device: softmax, top-k selection with torch-CPU tie order, gate
// renormalisation, and the matching backward to d(logits).
//
// Reference: TopKRouter.forward (src/model/router.py:69-98).  The logits GEMM
// `(x @ W).float()` (router.py:69) and the optional exploration noise (router.py:76-77)
// stay in torch; this file takes the fp32 logits from there.
//
// Layout: one token row per lane, 64 rows per workgroup.  The workgroup's [64, E]
// logit slab is read with coalesced loads into LDS, lane-interleaved (element e of
// lane l at [e * 64 + l]) so the per-lane passes over a row are bank-conflict free.
// Each LDS element is a 64-bit (key bits << 32 | expert id) pair, so a swap in the
// selection is one 64-bit move.
//
// Selection has to reproduce torch's CPU topk bit for bit, ties included: the order of
// equal keys is whatever libstdc++'s nth_element / sort / partial_sort leave (see
// ATen/native/TopKImpl.h:44-94).  The per-lane routines below restate those published
// algorithms (introselect with median-of-three, unguarded Hoare partition, heap select,
// insertion sort, introsort) on the lane's LDS row.
#include "nsmoe_capi_internal.h"
#include "nsmoe_common.h"

namespace nsmoe {

constexpr int ROUTE_ROWS = 64;  // rows per workgroup = lanes per wave

struct LaneRow {
  uint64_t* base;  // element i at base[i * ROUTE_ROWS]
  __device__ __forceinline__ uint64_t& operator[](int i) const { return base[i * ROUTE_ROWS]; }
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

// ---- forward ---------------------------------------------------------------------------
//
// flags bit 0 (want_probs): training branch, probs = softmax(logits) and the selection
//   runs on probs (router.py:79-81); probs [T, E] is written out.
// flags bit 1 (normalize):  normalize_weights.
// Without want_probs the selection runs on the logits and the gates are
// softmax(topk logits) (normalize) or softmax(logits)[idx] (router.py:83-92).
// With want_probs and normalize and k > 1 the gates are p / sum(p) (router.py:96-97).
template <int DT>
__global__ void __launch_bounds__(ROUTE_ROWS)
route_fwd_kernel(const float* __restrict__ logits, int64_t T, int E, int k, int flags,
                 typename Elem<DT>::T* __restrict__ topk_w, int64_t* __restrict__ topk_idx,
                 float* __restrict__ probs) {
  extern __shared__ uint64_t lds_q[];
  const int lane = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * ROUTE_ROWS;
  const int rows = (int)min((int64_t)ROUTE_ROWS, T - row0);
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;

  // Coalesced slab load: element (r, e) of the slab lands at [e * 64 + r].
  const float* slab = logits + row0 * E;
  for (int i = lane; i < rows * E; i += ROUTE_ROWS) {
    int r = i / E, e = i - r * E;
    lds_q[e * ROUTE_ROWS + r] = pack(slab[i], e);
  }
  __syncthreads();

  LaneRow a{lds_q + lane};
  const bool active = lane < rows;
  float row_max = 0.0f, row_inv_sum = 0.0f;
  if (active) {
    // max / sum over the full row: needed for probs (train) and for the eval
    // normalize=False branch.
    if (want_probs || !normalize) {
      float m = -INFINITY;
      bool any_nan = false;
      for (int e = 0; e < E; ++e) {
        float v = key_of(a[e]);
        any_nan |= __builtin_isnan(v);
        m = fmaxf(m, v);
      }
      if (any_nan) m = __uint_as_float(0x7fc00000u);
      float s = 0.0f;
      for (int e = 0; e < E; ++e) s += expf(key_of(a[e]) - m);
      row_max = m;
      row_inv_sum = 1.0f / s;
      if (want_probs) {
        for (int e = 0; e < E; ++e) a[e] = pack(expf(key_of(a[e]) - m) * row_inv_sum, e);
      }
    }
  }
  if (want_probs) {
    __syncthreads();
    float* prow = probs + row0 * E;
    for (int i = lane; i < rows * E; i += ROUTE_ROWS) {
      int r = i / E, e = i - r * E;
      prow[i] = key_of(lds_q[e * ROUTE_ROWS + r]);
    }
    __syncthreads();
  }
  if (!active) return;

  topk_select(a, E, k);

  using OutT = typename Elem<DT>::T;
  const int64_t row = row0 + lane;
  int64_t* idx_out = topk_idx + row * k;
  OutT* w_out = topk_w + row * k;
  for (int j = 0; j < k; ++j) idx_out[j] = id_of(a[j]);

  if (want_probs) {
    if (normalize && k > 1) {
      float s = 0.0f;
      for (int j = 0; j < k; ++j) s += key_of(a[j]);
      for (int j = 0; j < k; ++j) w_out[j] = Elem<DT>::from_f(key_of(a[j]) / s);
    } else {
      for (int j = 0; j < k; ++j) w_out[j] = Elem<DT>::from_f(key_of(a[j]));
    }
  } else if (normalize) {
    float m = -INFINITY;
    for (int j = 0; j < k; ++j) m = fmaxf(m, key_of(a[j]));
    float s = 0.0f;
    for (int j = 0; j < k; ++j) s += expf(key_of(a[j]) - m);
    float inv = 1.0f / s;
    for (int j = 0; j < k; ++j) w_out[j] = Elem<DT>::from_f(expf(key_of(a[j]) - m) * inv);
  } else {
    for (int j = 0; j < k; ++j)
      w_out[j] = Elem<DT>::from_f(expf(key_of(a[j]) - row_max) * row_inv_sum);
  }
}

// ---- backward --------------------------------------------------------------------------
//
// d(logits) for the same three branches, in fp32:
//   train: w = p_sel / S (normalize, k > 1)  ->  dp_j = (dw_j - sum_i dw_i w_i) / S
//          dprobs = grad_probs (aux loss, may be absent) + scatter(dp)
//          dlogits = p * (dprobs - sum_e p_e dprobs_e)
//   eval normalize:   w = softmax(l_sel) -> dl_sel = w * (dw - sum w dw)
//   eval !normalize:  w = softmax(l)[idx] -> softmax backward of scatter(dw)
// `src` holds probs for the train branch and logits otherwise.
template <int DT>
__global__ void __launch_bounds__(ROUTE_ROWS)
route_bwd_kernel(const float* __restrict__ src, const int64_t* __restrict__ topk_idx,
                 const typename Elem<DT>::T* __restrict__ grad_w,
                 const float* __restrict__ grad_probs, int64_t T, int E, int k, int flags,
                 float* __restrict__ grad_logits) {
  extern __shared__ float lds_f[];
  float* s_src = lds_f;                       // [E][64]
  float* s_g = lds_f + E * ROUTE_ROWS;        // [E][64] running d(probs) / d(logits)
  const int lane = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * ROUTE_ROWS;
  const int rows = (int)min((int64_t)ROUTE_ROWS, T - row0);
  const bool want_probs = flags & 1;
  const bool normalize = flags & 2;

  for (int i = lane; i < rows * E; i += ROUTE_ROWS) {
    int r = i / E, e = i - r * E;
    s_src[e * ROUTE_ROWS + r] = src[row0 * E + i];
    s_g[e * ROUTE_ROWS + r] = grad_probs ? grad_probs[row0 * E + i] : 0.0f;
  }
  __syncthreads();

  bool ids_ok = true;
  if (lane < rows) {
    const int64_t* idx = topk_idx + (row0 + lane) * k;
    for (int j = 0; j < k; ++j) ids_ok &= idx[j] >= 0 && idx[j] < E;
  }
  if (lane < rows && !ids_ok) {  // ids not from route_fwd: no gradient, no stray access
    float* sg = s_g + lane;
    for (int e = 0; e < E; ++e) sg[e * ROUTE_ROWS] = 0.0f;
  }
  if (lane < rows && ids_ok) {
    const int64_t row = row0 + lane;
    const int64_t* idx = topk_idx + row * k;
    const typename Elem<DT>::T* dw = grad_w + row * k;
    float* sv = s_src + lane;
    float* sg = s_g + lane;
    if (want_probs) {
      float S = 0.0f, dot = 0.0f;
      const bool renorm = normalize && k > 1;
      if (renorm) {
        for (int j = 0; j < k; ++j) S += sv[idx[j] * ROUTE_ROWS];
        for (int j = 0; j < k; ++j)
          dot += Elem<DT>::to_f(dw[j]) * (sv[idx[j] * ROUTE_ROWS] / S);
      }
      for (int j = 0; j < k; ++j) {
        float d = Elem<DT>::to_f(dw[j]);
        sg[idx[j] * ROUTE_ROWS] += renorm ? (d - dot) / S : d;
      }
      float pd = 0.0f;
      for (int e = 0; e < E; ++e) pd += sv[e * ROUTE_ROWS] * sg[e * ROUTE_ROWS];
      for (int e = 0; e < E; ++e)
        sg[e * ROUTE_ROWS] = sv[e * ROUTE_ROWS] * (sg[e * ROUTE_ROWS] - pd);
    } else if (normalize) {
      float m = -INFINITY;
      for (int j = 0; j < k; ++j) m = fmaxf(m, sv[idx[j] * ROUTE_ROWS]);
      float s = 0.0f;
      for (int j = 0; j < k; ++j) s += expf(sv[idx[j] * ROUTE_ROWS] - m);
      float dot = 0.0f;
      for (int j = 0; j < k; ++j)
        dot += expf(sv[idx[j] * ROUTE_ROWS] - m) / s * Elem<DT>::to_f(dw[j]);
      for (int e = 0; e < E; ++e) sg[e * ROUTE_ROWS] = 0.0f;
      for (int j = 0; j < k; ++j) {
        float w = expf(sv[idx[j] * ROUTE_ROWS] - m) / s;
        sg[idx[j] * ROUTE_ROWS] += w * (Elem<DT>::to_f(dw[j]) - dot);
      }
    } else {
      float m = -INFINITY;
      for (int e = 0; e < E; ++e) m = fmaxf(m, sv[e * ROUTE_ROWS]);
      float s = 0.0f;
      for (int e = 0; e < E; ++e) s += expf(sv[e * ROUTE_ROWS] - m);
      float inv = 1.0f / s;
      for (int e = 0; e < E; ++e) sg[e * ROUTE_ROWS] = 0.0f;
      for (int j = 0; j < k; ++j) sg[idx[j] * ROUTE_ROWS] += Elem<DT>::to_f(dw[j]);
      float pd = 0.0f;
      for (int e = 0; e < E; ++e) pd += expf(sv[e * ROUTE_ROWS] - m) * inv * sg[e * ROUTE_ROWS];
      for (int e = 0; e < E; ++e) {
        float p = expf(sv[e * ROUTE_ROWS] - m) * inv;
        sg[e * ROUTE_ROWS] = p * (sg[e * ROUTE_ROWS] - pd);
      }
    }
  }
  __syncthreads();
  for (int i = lane; i < rows * E; i += ROUTE_ROWS) {
    int r = i / E, e = i - r * E;
    grad_logits[row0 * E + i] = s_g[e * ROUTE_ROWS + r];
  }
}

constexpr int ROUTE_MAX_EXPERTS = 128;  // 64 rows x 128 x 8 B = 64 KiB of LDS

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_route_fwd(const float* logits, int64_t n_tokens, int32_t n_experts,
                               int32_t top_k, int32_t flags, int32_t w_dtype, void* topk_w,
                               int64_t* topk_idx, float* probs, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_fwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_fwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_fwd: top_k %d outside [1, %d]",
                top_k, n_experts);
  NSMOE_REQUIRE(!(flags & 1) || probs, "route_fwd: probs requested but NULL");
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(logits && topk_w && topk_idx, "route_fwd: NULL pointer");
  dim3 grid((unsigned)cdiv(n_tokens, ROUTE_ROWS)), block(ROUTE_ROWS);
  size_t lds = (size_t)n_experts * ROUTE_ROWS * sizeof(uint64_t);
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

extern "C" int nsmoe_route_bwd(const float* src, const int64_t* topk_idx, const void* grad_w,
                               int32_t w_dtype, const float* grad_probs, int64_t n_tokens,
                               int32_t n_experts, int32_t top_k, int32_t flags,
                               float* grad_logits, void* stream) {
  NSMOE_REQUIRE(n_tokens >= 0, "route_bwd: n_tokens < 0");
  NSMOE_REQUIRE(n_experts >= 1 && n_experts <= ROUTE_MAX_EXPERTS,
                "route_bwd: n_experts %d outside [1, %d]", n_experts, ROUTE_MAX_EXPERTS);
  NSMOE_REQUIRE(top_k >= 1 && top_k <= n_experts, "route_bwd: bad top_k %d", top_k);
  if (n_tokens == 0) return NSMOE_OK;
  NSMOE_REQUIRE(src && topk_idx && grad_w && grad_logits, "route_bwd: NULL pointer");
  dim3 grid((unsigned)cdiv(n_tokens, ROUTE_ROWS)), block(ROUTE_ROWS);
  size_t lds = (size_t)n_experts * ROUTE_ROWS * sizeof(float) * 2;
  hipStream_t s = (hipStream_t)stream;
  switch (w_dtype) {
    case DT_BF16:
      route_bwd_kernel<DT_BF16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, n_tokens, n_experts, top_k, flags, grad_logits);
      break;
    case DT_F16:
      route_bwd_kernel<DT_F16><<<grid, block, lds, s>>>(src, topk_idx, (const uint16_t*)grad_w,
          grad_probs, n_tokens, n_experts, top_k, flags, grad_logits);
      break;
    case DT_F32:
      route_bwd_kernel<DT_F32><<<grid, block, lds, s>>>(src, topk_idx, (const float*)grad_w,
          grad_probs, n_tokens, n_experts, top_k, flags, grad_logits);
      break;
    default:
      NSMOE_REQUIRE(false, "route_bwd: unknown dtype %d", w_dtype);
  }
  return check_launch("route_bwd_kernel");
}

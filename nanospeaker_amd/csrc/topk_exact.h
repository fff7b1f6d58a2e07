// CPU torch.topk's selection, restated for one row held by one wavefront (gfx950).
//
// torch's CPU topk (ATen/native/TopKImpl.h:44-94) orders equal keys the way libstdc++'s
// nth_element / sort / partial_sort leave them; routing must reproduce that order bit
// for bit, ties included.  The routines below restate those published algorithms
// (introselect with median-of-three, unguarded Hoare partition, heap select, insertion
// sort, introsort) on the row as the wave holds it in registers: element i is lane i % 64
// of register pair i / 64 (rows of up to 128 elements).  Every access takes a
// wave-uniform index (a v_readlane, or a lane compare-and-select for a store), so the
// sequential algorithm runs in uniform control flow with register latency; the
// partitions and the final small sort run wave-parallel (ballots and ranks).
//
// Used by the router tail (route.hip) and by the fused router's tie pass (router.hip).
#pragma once

#include "balance.h"
#include "nsmoe_common.h"

namespace nsmoe {

// (key, id) swap slots a wave's partitions need in LDS (partition_parallel).
constexpr int TOPK_SWAP_SLOTS = 128;

// ---- the row in registers --------------------------------------------------------------

// The exact path compares keys as order-preserving unsigned integers: x ranks before y
// ("x is NaN and y is not, or x > y", TopKImpl.h:68-69) iff ord_key(x) > ord_key(y).
// Every NaN maps to the top and -0 to +0's image, so equal keys stay equal.  Integer keys
// let the sequential steps compare in scalar registers (gfx950's scalar unit has no float
// compare); the output values are read back from the untouched row by id.
__device__ __forceinline__ uint32_t ord_key(float f) {
  if (__builtin_isnan(f)) return 0xFFFFFFFFu;
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

struct KV {
  uint32_t key;  // ord_key of the value
  int id;
};

__device__ __forceinline__ bool gt(uint32_t a, uint32_t b) { return a > b; }
__device__ __forceinline__ bool gt(KV x, KV y) { return x.key > y.key; }

// Lane `l` of v replaced by x (l wave-uniform): a compare and a select, the VALU
// equivalent of v_writelane.
__device__ __forceinline__ int put_lane(int v, int x, int l, int lane) { return lane == l ? x : v; }

// Element i of the row: lane i % 64 of register pair i / 64.  Indices are wave-uniform.
struct RegRow {
  int k0, k1;  // key bits of elements lane, lane + 64
  int i0, i1;  // their ids
  int lane;
  // Value selects only: `c ? k0 : k1` on the members would be an lvalue (a select of
  // member addresses), which keeps the struct in memory -- the compiler then places it
  // in LDS, and every access becomes an LDS round trip.
  // i is wave-uniform: both halves are read at lane i % 64 and a scalar select keeps the
  // one i lies in (no branch between the dependent scalar steps).
  __device__ __forceinline__ KV get(int i) const {
    const int l = i & 63;
    const uint32_t ka = (uint32_t)rl(k0, l), kb = (uint32_t)rl(k1, l);
    const int ia = rl(i0, l), ib = rl(i1, l);
    return i < 64 ? KV{ka, ia} : KV{kb, ib};
  }
  __device__ __forceinline__ uint32_t key(int i) const {
    const int l = i & 63;
    const uint32_t ka = (uint32_t)rl(k0, l), kb = (uint32_t)rl(k1, l);
    return i < 64 ? ka : kb;
  }
  // Both halves are written through selects (lane -1 matches no lane), so the compiler
  // keeps the four registers as registers instead of an indexed private array.
  __device__ __forceinline__ void set(int i, KV v) {
    const bool lo = i < 64;
    const int l0 = lo ? i : -1, l1 = lo ? -1 : i - 64;
    const int kb = (int)v.key;
    k0 = put_lane(k0, kb, l0, lane);
    i0 = put_lane(i0, v.id, l0, lane);
    k1 = put_lane(k1, kb, l1, lane);
    i1 = put_lane(i1, v.id, l1, lane);
  }
  __device__ __forceinline__ void swap(int i, int j) {
    const KV t = get(i);
    set(i, get(j));
    set(j, t);
  }
};

__device__ __forceinline__ int lg2i(int n) { return 31 - __builtin_clz(n); }

// ---- heap primitives on a[first, first + len) ------------------------------------------

__device__ __forceinline__ void push_heap_d(RegRow& a, int f, int hole, int top, KV value) {
  int parent = (hole - 1) / 2;
  while (hole > top) {
    const KV p = a.get(f + parent);
    if (!gt(p, value)) break;
    a.set(f + hole, p);
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a.set(f + hole, value);
}

__device__ __forceinline__ void adjust_heap_d(RegRow& a, int f, int hole, int len, KV value) {
  const int top = hole;
  int second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (gt(a.get(f + second), a.get(f + second - 1))) second--;
    a.set(f + hole, a.get(f + second));
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    a.set(f + hole, a.get(f + second - 1));
    hole = second - 1;
  }
  push_heap_d(a, f, hole, top, value);
}

__device__ __forceinline__ void make_heap_d(RegRow& a, int f, int len) {
  if (len < 2) return;
  int parent = (len - 2) / 2;
  for (;;) {
    adjust_heap_d(a, f, parent, len, a.get(f + parent));
    if (parent == 0) return;
    parent--;
  }
}

// heap is a[f, f + len); the displaced element is a[f + res]
__device__ __forceinline__ void pop_heap_d(RegRow& a, int f, int len, int res) {
  const KV value = a.get(f + res);
  a.set(f + res, a.get(f));
  adjust_heap_d(a, f, 0, len, value);
}

__device__ __forceinline__ void heap_select_d(RegRow& a, int f, int middle, int last) {
  make_heap_d(a, f, middle);
  for (int i = middle; i < last; ++i)
    if (gt(a.get(f + i), a.get(f))) pop_heap_d(a, f, middle, i);
}

__device__ __forceinline__ void sort_heap_d(RegRow& a, int f, int last) {
  while (last > 1) {
    --last;
    pop_heap_d(a, f, last, last);
  }
}

// ---- insertion sorts -----------------------------------------------------------------

// The scans below are "unguarded" in libstdc++: a sentinel stops them.  They also stop at
// the row's ends here, which changes nothing while the sentinels hold and keeps every
// loop bounded regardless.
__device__ __forceinline__ void unguarded_linear_insert_d(RegRow& a, int last) {
  const KV val = a.get(last);
  int next = last - 1;
  while (next >= 0) {
    const KV n = a.get(next);
    if (!gt(val, n)) break;
    a.set(last, n);
    last = next;
    --next;
  }
  a.set(last, val);
}

__device__ __forceinline__ void insertion_sort_d(RegRow& a, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    const KV v = a.get(i);
    if (gt(v, a.get(first))) {
      for (int j = i; j > first; --j) a.set(j, a.get(j - 1));
      a.set(first, v);
    } else {
      unguarded_linear_insert_d(a, i);
    }
  }
}

// ---- partitioning --------------------------------------------------------------------

__device__ __forceinline__ void move_median_to_first_d(RegRow& a, int result, int x, int y,
                                                       int z) {
  const uint32_t ax = a.key(x), ay = a.key(y), az = a.key(z);
  if (gt(ax, ay)) {
    if (gt(ay, az)) a.swap(result, y);
    else if (gt(ax, az)) a.swap(result, z);
    else a.swap(result, x);
  } else if (gt(ax, az)) {
    a.swap(result, x);
  } else if (gt(ay, az)) {
    a.swap(result, z);
  } else {
    a.swap(result, y);
  }
}

__device__ __forceinline__ int unguarded_partition_pivot_d(RegRow& a, int first, int last) {
  const int mid = first + (last - first) / 2;
  move_median_to_first_d(a, first, first + 1, mid, last - 1);
  const KV pivot = a.get(first);  // the pivot slot is not touched by the partition
  int lo = first + 1, hi = last;
  for (;;) {
    while (lo < last - 1 && gt(a.get(lo), pivot)) ++lo;
    --hi;
    while (hi > first && gt(pivot, a.get(hi))) --hi;
    if (!(lo < hi)) return lo;
    a.swap(lo, hi);
    ++lo;
  }
}

// std::sort on a[0, n).  introsort_loop recurses on the right part and loops on the
// left; the subranges it leaves are disjoint, so visiting them from an explicit stack
// in another order gives the same array.  The stack lives in lanes of three registers
// (entry sp in lane sp; at most 2 log2(n) + 1 <= 15 entries for n <= 128).
__device__ __forceinline__ void sort_d(RegRow& a, int n) {
  if (n == 0) return;
  if (n > 16) {
    int st_first = 0, st_last = 0, st_depth = 0;
    st_first = put_lane(st_first, 0, 0, a.lane);
    st_last = put_lane(st_last, n, 0, a.lane);
    st_depth = put_lane(st_depth, lg2i(n) * 2, 0, a.lane);
    int sp = 1;
    while (sp > 0) {
      --sp;
      int first = rl(st_first, sp), last = rl(st_last, sp), depth = rl(st_depth, sp);
      while (last - first > 16) {
        if (depth == 0) {
          heap_select_d(a, first, last - first, last - first);
          sort_heap_d(a, first, last - first);
          break;
        }
        --depth;
        const int cut = unguarded_partition_pivot_d(a, first, last);
        st_first = put_lane(st_first, cut, sp, a.lane);
        st_last = put_lane(st_last, last, sp, a.lane);
        st_depth = put_lane(st_depth, depth, sp, a.lane);
        ++sp;
        last = cut;
      }
    }
    insertion_sort_d(a, 0, 16);
    for (int i = 16; i != n; ++i) unguarded_linear_insert_d(a, i);
  } else {
    insertion_sort_d(a, 0, n);
  }
}

// ---- the same steps, wave-parallel ---------------------------------------------------

// Bits [a, b) of one 64-position half (a and b clamped to [0, 64]).
__device__ __forceinline__ uint64_t span_mask(int a, int b) {
  a = a < 0 ? 0 : (a > 64 ? 64 : a);
  b = b < a ? a : (b > 64 ? 64 : b);
  const uint64_t below_b = b >= 64 ? ~0ull : ((1ull << b) - 1ull);
  const uint64_t below_a = a >= 64 ? ~0ull : ((1ull << a) - 1ull);
  return below_b & ~below_a;
}

// Set bits of the wave-uniform mask m in the lanes below this one.
__device__ __forceinline__ int mbcnt64(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

__device__ __forceinline__ int ff1_64(uint64_t m) { return __builtin_ctzll(m); }

// Unguarded Hoare partition of [first, last) around pivot a[first] (key pk, which the
// caller already holds), computed from ranks.
// On the array as move_median_to_first left it, let L be the ascending positions in
// (first, last) where the left scan stops (!gt(a[p], pivot)) and R the descending
// positions in [first, last) where the right scan stops (!gt(pivot, a[p])).  Iteration i
// of the sequential loop meets lo = L[i], hi = R[i] and swaps them exactly while
// L[i] < R[i] (positions between the last swapped pair are untouched originals, and a
// swapped slot stops the opposite scan).  So the loop makes i* = #{i : L[i] < R[i]}
// swaps, all disjoint, and returns min(L[i*], R[i*-1]) (L[0] when i* = 0).
// L[i] < R[i] <=> more than i right stoppers lie above L[i]: each lane tests its own
// positions with ballots.  The swaps go through LDS: the element at L[i] (i < i*) is
// written to slot i and the one at R[i] to slot 64 + i; then L[i] reads slot 64 + i and
// R[i] reads slot i.  The 2 i* swapped positions are distinct, so i* <= n / 2 <= 64 and
// `kv`, the wave's LDS scratch of (key, id) pairs, needs TOPK_SWAP_SLOTS = 128 of them.
// The stopper sets are wave masks (one compare per half, the position range a scalar
// mask) and the ranks their bit counts below each lane (v_mbcnt).
__device__ __forceinline__ int partition_parallel(RegRow& a, int first, int last, int2* kv,
                                                  uint32_t pk) {
  const int lane = a.lane;
  const uint32_t x0 = (uint32_t)a.k0, x1 = (uint32_t)a.k1;
  // Stopper sets as wave masks: one compare per half, the position ranges as scalar masks.
  const uint64_t bl0 = __builtin_amdgcn_ballot_w64(x0 <= pk) & span_mask(first + 1, last);
  const uint64_t bl1 = __builtin_amdgcn_ballot_w64(x1 <= pk) & span_mask(first - 63, last - 64);
  const uint64_t br0 = __builtin_amdgcn_ballot_w64(x0 >= pk) & span_mask(first, last);
  const uint64_t br1 = __builtin_amdgcn_ballot_w64(x1 >= pk) & span_mask(first - 64, last - 64);
  const int nl0 = __builtin_popcountll(bl0);
  const int nr0 = __builtin_popcountll(br0), nr1 = __builtin_popcountll(br1);
  const bool isL0 = (bl0 >> lane) & 1ull, isL1 = (bl1 >> lane) & 1ull;
  const bool isR0 = (br0 >> lane) & 1ull, isR1 = (br1 >> lane) & 1ull;
  // rl: an L stopper's rank from the left; ar: the right stoppers strictly above the
  // position (an R stopper's rank from the right).
  const int rl0 = mbcnt64(bl0), rl1 = nl0 + mbcnt64(bl1);
  const int ar1 = nr1 - mbcnt64(br1) - (isR1 ? 1 : 0);
  const int ar0 = nr0 - mbcnt64(br0) - (isR0 ? 1 : 0) + nr1;
  const int istar = __builtin_popcountll(bl0 & __builtin_amdgcn_ballot_w64(ar0 > rl0)) +
                    __builtin_popcountll(bl1 & __builtin_amdgcn_ballot_w64(ar1 > rl1));
  const bool sl0 = isL0 && rl0 < istar, sl1 = isL1 && rl1 < istar;
  const bool sr0 = isR0 && ar0 < istar, sr1 = isR1 && ar1 < istar;
  if (sl0) kv[rl0] = make_int2(a.k0, a.i0);
  if (sl1) kv[rl1] = make_int2(a.k1, a.i1);
  if (sr0) kv[64 + ar0] = make_int2(a.k0, a.i0);
  if (sr1) kv[64 + ar1] = make_int2(a.k1, a.i1);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (sl0 || sr0) {
    const int2 v = kv[sl0 ? 64 + rl0 : ar0];
    a.k0 = v.x;
    a.i0 = v.y;
  }
  if (sl1 || sr1) {
    const int2 v = kv[sl1 ? 64 + rl1 : ar1];
    a.k1 = v.x;
    a.i1 = v.y;
  }
  // the next round's writes to kv must not overtake these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (istar == 0) return bl0 ? ff1_64(bl0) : (bl1 ? 64 + ff1_64(bl1) : 63);
  const uint64_t n0 = bl0 & __builtin_amdgcn_ballot_w64(rl0 == istar);
  const uint64_t n1 = bl1 & __builtin_amdgcn_ballot_w64(rl1 == istar);
  const uint64_t m0 = br0 & __builtin_amdgcn_ballot_w64(ar0 == istar - 1);
  const uint64_t m1 = br1 & __builtin_amdgcn_ballot_w64(ar1 == istar - 1);
  const int lnext = n0 ? ff1_64(n0) : n1 ? 64 + ff1_64(n1) : 1 << 20;
  const int rprev = m0 ? ff1_64(m0) : (m1 ? 64 + ff1_64(m1) : 63);
  return lnext < rprev ? lnext : rprev;
}

// libstdc++'s insertion sort with a strict comparator moves an element left only past
// elements it ranks strictly before, so it is the stable sort: the element at p lands at
// first + #{q : a[q] before a[p]} + #{q < p : a[q] equivalent to a[p]}.  For ranges
// inside the first 64 slots the ranks are counted in parallel and applied with one
// ds_permute; other ranges take the sequential routine.
__device__ __forceinline__ void stable_sort_d(RegRow& a, int first, int last) {
  if (last - first < 2) return;
  if (last > 64) {
    insertion_sort_d(a, first, last);
    return;
  }
  const int p = a.lane;
  const bool in = p >= first && p < last;
  const uint32_t kp = (uint32_t)a.k0;
  int rank = first;
  for (int q = first; q < last; ++q) {
    const uint32_t kq = (uint32_t)rl(a.k0, q);
    rank += (in && (gt(kq, kp) || (q < p && !gt(kp, kq)))) ? 1 : 0;
  }
  const int dst = (in ? rank : p) * 4;
  a.k0 = __builtin_amdgcn_ds_permute(dst, a.k0);
  a.i0 = __builtin_amdgcn_ds_permute(dst, a.i0);
}

// nth_element (introselect) with the partitions and the final insertion sort done
// wave-parallel; the heap-select fallback at depth 0 stays sequential.
__device__ __forceinline__ void nth_element_par(RegRow& a, int nth, int n, int2* pos) {
  if (n == 0 || nth == n) return;
  int first = 0, last = n, depth = lg2i(n) * 2;
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_d(a, first, nth + 1 - first, last - first);
      a.swap(first, nth);
      return;
    }
    --depth;
    // move_median_to_first(first, first + 1, mid, last - 1) from one read of the four
    // positions: the swap's values are then known scalars, and so is the pivot's key.
    const int x = first + 1, y = first + (last - first) / 2, z = last - 1;
    const KV ef = a.get(first), ex = a.get(x), ey = a.get(y), ez = a.get(z);
    int m;
    KV em;
    if (gt(ex, ey)) {
      if (gt(ey, ez)) m = y, em = ey;
      else if (gt(ex, ez)) m = z, em = ez;
      else m = x, em = ex;
    } else if (gt(ex, ez)) {
      m = x, em = ex;
    } else if (gt(ey, ez)) {
      m = z, em = ez;
    } else {
      m = y, em = ey;
    }
    a.set(first, em);
    a.set(m, ef);
    const int cut = partition_parallel(a, first, last, pos, em.key);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  stable_sort_d(a, first, last);
}

// torch CPU topk(largest=True, sorted=True) over the row: afterwards a[0, k) holds the
// selected (key, id) pairs in output order.
__device__ __forceinline__ void topk_select(RegRow& a, int n, int k, int2* pos) {
  if (k * 64 <= n) {
    heap_select_d(a, 0, k, n);
    sort_heap_d(a, 0, k);
  } else {
    nth_element_par(a, k - 1, n, pos);
    if (k - 1 <= 16) stable_sort_d(a, 0, k - 1);  // std::sort's insertion-sort branch
    else sort_d(a, k - 1);
  }
}

// Stores one routed row (router.py:79-98 after the selection): lane j < k holds output j
// (and lane j holds output j + 64 in the second register): its key s (prob or logit) and
// expert id d.  Gates: train branch p / sum(p) over the k (normalize, k > 1) or p itself;
// eval branch softmax over the k selected logits (normalize) or softmax over the row,
// exp(s - m) * row_inv_sum, at the selected ids.
template <int DT>
__device__ __forceinline__ void write_route_row(int64_t row, int k, int lane, bool want_probs,
                                                bool normalize, float s0, float s1, int d0,
                                                int d1, float m, float row_inv_sum,
                                                typename Elem<DT>::T* __restrict__ topk_w,
                                                int64_t* __restrict__ topk_idx) {
  int64_t* idx_out = topk_idx + row * k;
  typename Elem<DT>::T* w_out = topk_w + row * k;
  const bool o0 = lane < k, o1 = lane + 64 < k;
  if (!o0) s0 = 0.0f;
  if (!o1) s1 = 0.0f;
  if (o0) idx_out[lane] = d0;
  if (o1) idx_out[lane + 64] = d1;
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

}  // namespace nsmoe

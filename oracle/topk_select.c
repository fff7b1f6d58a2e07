/*
 * ORACLE -- test infrastructure only.  Nothing in nanospeaker_amd/ links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may use it, and only as the checker.
 *
 * CPU restatement of the selection step behind `probs.topk(k)` / `logits.topk(k)` in
 * the reference router (src/model/router.py:81 and :87).  The reference calls torch's
 * CPU topk, whose per-row loop is ATen/native/TopKImpl.h:44-94 (torch 2.10, built with
 * GCC 11.2's libstdc++):
 *
 *   use_partial_sort = k * 64 <= n
 *   partial_sort(q, q + k, q + n)                   if use_partial_sort
 *   nth_element(q, q + k - 1, q + n); sort(q, q + k - 1)   otherwise
 *
 * over pairs (value, index) with the comparator "x is NaN and y is not, or x > y".
 * The comparator looks at values only, so the order of tied values is whatever the
 * libstdc++ algorithms leave behind.  Bit-exact routing indices therefore need those
 * algorithms step for step: introselect (Musser 1997) with median-of-three pivots and
 * an unguarded Hoare partition, heap select, insertion sort and introsort.  They are
 * restated here from the published libstdc++ algorithm descriptions (stl_algo.h,
 * stl_heap.h); the steps have to be alike because the tie order is their output.
 *
 * Pinned by tests/test_oracle_topk.py against torch.topk itself on tie-heavy rows.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

typedef struct {
  double v;      /* TopKImpl.h uses acc_type<float> = double for the queue */
  int64_t i;
} elem_t;

static inline int cmp_gt(const elem_t* x, const elem_t* y) {
  return (isnan(x->v) && !isnan(y->v)) || (x->v > y->v);
}

static inline void swap_e(elem_t* a, elem_t* b) {
  elem_t t = *a;
  *a = *b;
  *b = t;
}

static inline int lg2(int64_t n) { return 63 - __builtin_clzll((unsigned long long)n); }

/* ---- heap primitives (stl_heap.h) ---- */
static void push_heap_(elem_t* a, int64_t hole, int64_t top, elem_t value) {
  int64_t parent = (hole - 1) / 2;
  while (hole > top && cmp_gt(&a[parent], &value)) {
    a[hole] = a[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a[hole] = value;
}

static void adjust_heap_(elem_t* a, int64_t hole, int64_t len, elem_t value) {
  const int64_t top = hole;
  int64_t second = hole;
  while (second < (len - 1) / 2) {
    second = 2 * (second + 1);
    if (cmp_gt(&a[second], &a[second - 1])) second--;
    a[hole] = a[second];
    hole = second;
  }
  if ((len & 1) == 0 && second == (len - 2) / 2) {
    second = 2 * (second + 1);
    a[hole] = a[second - 1];
    hole = second - 1;
  }
  push_heap_(a, hole, top, value);
}

static void make_heap_(elem_t* a, int64_t len) {
  if (len < 2) return;
  int64_t parent = (len - 2) / 2;
  for (;;) {
    elem_t value = a[parent];
    adjust_heap_(a, parent, len, value);
    if (parent == 0) return;
    parent--;
  }
}

/* pop_heap(first, last, result): the heap is a[0, len), result is a[res] */
static void pop_heap_(elem_t* a, int64_t len, int64_t res) {
  elem_t value = a[res];
  a[res] = a[0];
  adjust_heap_(a, 0, len, value);
}

static void heap_select_(elem_t* a, int64_t middle, int64_t last) {
  make_heap_(a, middle);
  for (int64_t i = middle; i < last; ++i)
    if (cmp_gt(&a[i], &a[0])) pop_heap_(a, middle, i);
}

static void sort_heap_(elem_t* a, int64_t last) {
  while (last > 1) {
    --last;
    pop_heap_(a, last, last);
  }
}

static void partial_sort_(elem_t* a, int64_t middle, int64_t last) {
  heap_select_(a, middle, last);
  sort_heap_(a, middle);
}

/* ---- insertion sorts (stl_algo.h) ---- */
static void unguarded_linear_insert_(elem_t* a, int64_t last) {
  elem_t val = a[last];
  int64_t next = last - 1;
  while (cmp_gt(&val, &a[next])) {
    a[last] = a[next];
    last = next;
    --next;
  }
  a[last] = val;
}

static void insertion_sort_(elem_t* a, int64_t first, int64_t last) {
  if (first == last) return;
  for (int64_t i = first + 1; i != last; ++i) {
    if (cmp_gt(&a[i], &a[first])) {
      elem_t val = a[i];
      memmove(&a[first + 1], &a[first], (size_t)(i - first) * sizeof(elem_t));
      a[first] = val;
    } else {
      unguarded_linear_insert_(a, i);
    }
  }
}

static void unguarded_insertion_sort_(elem_t* a, int64_t first, int64_t last) {
  for (int64_t i = first; i != last; ++i) unguarded_linear_insert_(a, i);
}

/* ---- partitioning ---- */
static void move_median_to_first_(elem_t* a, int64_t result, int64_t x, int64_t y, int64_t z) {
  if (cmp_gt(&a[x], &a[y])) {
    if (cmp_gt(&a[y], &a[z])) swap_e(&a[result], &a[y]);
    else if (cmp_gt(&a[x], &a[z])) swap_e(&a[result], &a[z]);
    else swap_e(&a[result], &a[x]);
  } else if (cmp_gt(&a[x], &a[z])) {
    swap_e(&a[result], &a[x]);
  } else if (cmp_gt(&a[y], &a[z])) {
    swap_e(&a[result], &a[z]);
  } else {
    swap_e(&a[result], &a[y]);
  }
}

static int64_t unguarded_partition_(elem_t* a, int64_t first, int64_t last, int64_t pivot) {
  for (;;) {
    while (cmp_gt(&a[first], &a[pivot])) ++first;
    --last;
    while (cmp_gt(&a[pivot], &a[last])) --last;
    if (!(first < last)) return first;
    swap_e(&a[first], &a[last]);
    ++first;
  }
}

static int64_t unguarded_partition_pivot_(elem_t* a, int64_t first, int64_t last) {
  int64_t mid = first + (last - first) / 2;
  move_median_to_first_(a, first, first + 1, mid, last - 1);
  return unguarded_partition_(a, first + 1, last, first);
}

static void introselect_(elem_t* a, int64_t first, int64_t nth, int64_t last, int depth) {
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_(a + first, nth + 1 - first, last - first);
      swap_e(&a[first], &a[nth]);
      return;
    }
    --depth;
    int64_t cut = unguarded_partition_pivot_(a, first, last);
    if (cut <= nth) first = cut;
    else last = cut;
  }
  insertion_sort_(a, first, last);
}

static void nth_element_(elem_t* a, int64_t nth, int64_t last) {
  if (last == 0 || nth == last) return;
  introselect_(a, 0, nth, last, lg2(last) * 2);
}

static void introsort_loop_(elem_t* a, int64_t first, int64_t last, int depth) {
  while (last - first > 16) {
    if (depth == 0) {
      partial_sort_(a + first, last - first, last - first);
      return;
    }
    --depth;
    int64_t cut = unguarded_partition_pivot_(a, first, last);
    introsort_loop_(a, cut, last, depth);
    last = cut;
  }
}

static void sort_(elem_t* a, int64_t last) {
  if (last == 0) return;
  introsort_loop_(a, 0, last, lg2(last) * 2);
  if (last > 16) {
    insertion_sort_(a, 0, 16);
    unguarded_insertion_sort_(a, 16, last);
  } else {
    insertion_sort_(a, 0, last);
  }
}

/* torch.topk(largest=True, sorted=True) over each row of a [rows, n] float matrix. */
int oracle_topk_rows(const float* vals, int64_t rows, int64_t n, int64_t k,
                     int64_t* out_idx, float* out_val, elem_t* scratch) {
  if (k < 0 || k > n) return 1;
  if (k == 0) return 0;
  for (int64_t r = 0; r < rows; ++r) {
    const float* v = vals + r * n;
    for (int64_t j = 0; j < n; ++j) {
      scratch[j].v = (double)v[j];
      scratch[j].i = j;
    }
    if (k * 64 <= n) {
      partial_sort_(scratch, k, n);
    } else {
      nth_element_(scratch, k - 1, n);
      sort_(scratch, k - 1);
    }
    for (int64_t j = 0; j < k; ++j) {
      out_idx[r * k + j] = scratch[j].i;
      if (out_val) out_val[r * k + j] = (float)scratch[j].v;
    }
  }
  return 0;
}

int64_t oracle_topk_scratch_elems(int64_t n) { return n; }

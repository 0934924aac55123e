/*
 * CPU oracle (test infrastructure only): C restatements of the integer/selection parts of
 * FERRY's per-GPU MoE path.  Nothing in the product links this file; only tests, the smoke
 * check and the CPU-baseline leg of the benchmark load it, to check results.
 *
 *  1. oracle_topk   -- torch's CPU top-k (ATen/native/TopKImpl.h, topk_impl_loop), which the
 *                      reference router calls at ferry/model.py:143.  torch selects with
 *                      std::partial_sort when k*64 <= n and otherwise with std::nth_element
 *                      followed by std::sort of the first k-1 entries; both are libstdc++
 *                      algorithms (bits/stl_algo.h __introselect/__introsort_loop/
 *                      __insertion_sort, bits/stl_heap.h __adjust_heap/__push_heap).  The
 *                      steps below follow those published algorithms so that the order of
 *                      tied values comes out exactly as torch produces it.  The comparator
 *                      orders by value only ("x.first > y.first", NaN first).
 *  2. oracle_plan_layer -- ferry/policy.py:130-194 (plan_layer) at world = 1 with
 *                      _choose_slot (policy.py:109-127) and the quota assert (quota.py:63).
 *  3. oracle_layer_slots -- ferry/policy.py:197-205.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>

typedef struct {
  float v;
  int64_t i;
} pair_t;

/* comparator of TopKImpl.h for largest=true / largest=false */
static int g_largest = 1;
static inline int before(const pair_t* x, const pair_t* y) {
  if (g_largest) return (isnan(x->v) && !isnan(y->v)) || (x->v > y->v);
  return (!isnan(x->v) && isnan(y->v)) || (x->v < y->v);
}
static inline void swap_p(pair_t* a, pair_t* b) {
  pair_t t = *a;
  *a = *b;
  *b = t;
}
static inline int64_t lg2(int64_t n) {
  int64_t r = 0;
  while (n > 1) {
    n >>= 1;
    ++r;
  }
  return r;
}

/* ---- heap primitives (stl_heap.h) ---- */
static void push_heap_(pair_t* first, int64_t hole, int64_t top, pair_t value) {
  int64_t parent = (hole - 1) / 2;
  while (hole > top && before(first + parent, &value)) {
    first[hole] = first[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  first[hole] = value;
}
static void adjust_heap_(pair_t* first, int64_t hole, int64_t len, pair_t value) {
  const int64_t top = hole;
  int64_t child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (before(first + child, first + (child - 1))) child--;
    first[hole] = first[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    first[hole] = first[child - 1];
    hole = child - 1;
  }
  push_heap_(first, hole, top, value);
}
static void make_heap_(pair_t* first, pair_t* last) {
  int64_t len = last - first;
  if (len < 2) return;
  int64_t parent = (len - 2) / 2;
  for (;;) {
    pair_t value = first[parent];
    adjust_heap_(first, parent, len, value);
    if (parent == 0) return;
    parent--;
  }
}
static void pop_heap_(pair_t* first, pair_t* last, pair_t* result) {
  pair_t value = *result;
  *result = *first;
  adjust_heap_(first, 0, last - first, value);
}
static void heap_select_(pair_t* first, pair_t* middle, pair_t* last) {
  make_heap_(first, middle);
  for (pair_t* i = middle; i < last; ++i)
    if (before(i, first)) pop_heap_(first, middle, i);
}
static void sort_heap_(pair_t* first, pair_t* last) {
  while (last - first > 1) {
    --last;
    pop_heap_(first, last, last);
  }
}

/* ---- sorting primitives (stl_algo.h) ---- */
static void unguarded_linear_insert_(pair_t* last) {
  pair_t val = *last;
  pair_t* next = last - 1;
  while (before(&val, next)) {
    *last = *next;
    last = next;
    --next;
  }
  *last = val;
}
static void insertion_sort_(pair_t* first, pair_t* last) {
  if (first == last) return;
  for (pair_t* i = first + 1; i != last; ++i) {
    if (before(i, first)) {
      pair_t val = *i;
      memmove(first + 1, first, (size_t)(i - first) * sizeof(pair_t));
      *first = val;
    } else {
      unguarded_linear_insert_(i);
    }
  }
}
static void move_median_to_first_(pair_t* result, pair_t* a, pair_t* b, pair_t* c) {
  if (before(a, b)) {
    if (before(b, c))
      swap_p(result, b);
    else if (before(a, c))
      swap_p(result, c);
    else
      swap_p(result, a);
  } else if (before(a, c)) {
    swap_p(result, a);
  } else if (before(b, c)) {
    swap_p(result, c);
  } else {
    swap_p(result, b);
  }
}
static pair_t* unguarded_partition_(pair_t* first, pair_t* last, pair_t* pivot) {
  for (;;) {
    while (before(first, pivot)) ++first;
    --last;
    while (before(pivot, last)) --last;
    if (!(first < last)) return first;
    swap_p(first, last);
    ++first;
  }
}
static pair_t* unguarded_partition_pivot_(pair_t* first, pair_t* last) {
  pair_t* mid = first + (last - first) / 2;
  move_median_to_first_(first, first + 1, mid, last - 1);
  return unguarded_partition_(first + 1, last, first);
}
static void introsort_loop_(pair_t* first, pair_t* last, int64_t depth) {
  while (last - first > 16) {
    if (depth == 0) {
      heap_select_(first, last, last);
      sort_heap_(first, last);
      return;
    }
    --depth;
    pair_t* cut = unguarded_partition_pivot_(first, last);
    introsort_loop_(cut, last, depth);
    last = cut;
  }
}
static void final_insertion_sort_(pair_t* first, pair_t* last) {
  if (last - first > 16) {
    insertion_sort_(first, first + 16);
    for (pair_t* i = first + 16; i != last; ++i) unguarded_linear_insert_(i);
  } else {
    insertion_sort_(first, last);
  }
}
static void sort_(pair_t* first, pair_t* last) {
  if (first != last) {
    introsort_loop_(first, last, lg2(last - first) * 2);
    final_insertion_sort_(first, last);
  }
}
static void introselect_(pair_t* first, pair_t* nth, pair_t* last, int64_t depth) {
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_(first, nth + 1, last);
      swap_p(first, nth);
      return;
    }
    --depth;
    pair_t* cut = unguarded_partition_pivot_(first, last);
    if (cut <= nth)
      first = cut;
    else
      last = cut;
  }
  insertion_sort_(first, last);
}
static void nth_element_(pair_t* first, pair_t* nth, pair_t* last) {
  if (first == last || nth == last) return;
  introselect_(first, nth, last, lg2(last - first) * 2);
}

/* Top-k of each of `rows` rows of length n (row-major), as torch.topk on CPU. */
int oracle_topk(const float* vals, int64_t rows, int64_t n, int64_t k, int largest, int sorted,
                float* out_v, int64_t* out_i) {
  if (k < 0 || k > n) return 1;
  if (k == 0) return 0;
  pair_t* q = (pair_t*)malloc((size_t)n * sizeof(pair_t));
  if (!q) return 2;
  g_largest = largest;
  const int partial = k * 64 <= n;
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = vals + r * n;
    for (int64_t j = 0; j < n; ++j) {
      q[j].v = row[j];
      q[j].i = j;
    }
    if (partial) {
      heap_select_(q, q + k, q + n);
      sort_heap_(q, q + k);
    } else {
      nth_element_(q, q + k - 1, q + n);
      if (sorted) sort_(q, q + k - 1);
    }
    for (int64_t j = 0; j < k; ++j) {
      out_v[r * k + j] = q[j].v;
      out_i[r * k + j] = q[j].i;
    }
  }
  free(q);
  return 0;
}

/* ------------------------------------------------------------------------------------------ */
/* Placement planner at world = 1 (ferry/policy.py).                                           */

/* ferry/policy.py:109-127 (_choose_slot) for rank 0. */
int64_t oracle_choose_slot(int64_t layer, const uint8_t* active, const int64_t* slots, int64_t cap,
                           const int64_t* last, const float* scores, int64_t experts) {
  int64_t best = -1;
  float best_score = INFINITY;
  int64_t best_used = (int64_t)1 << 60, best_key = (int64_t)1 << 60;
  for (int64_t i = 0; i < cap; ++i) {
    int64_t key = slots[i];
    if (key < 0) return i;
    if (key / experts == layer && active[key % experts]) continue;
    float score = scores[key];  /* scores is [layers, experts] row-major: index == key */
    int64_t used = last[key];
    if (score < best_score ||
        (score == best_score && (used < best_used || (used == best_used && key < best_key)))) {
      best = i;
      best_score = score;
      best_used = used;
      best_key = key;
    }
  }
  return best;
}

/*
 * ferry/policy.py:130-194 (plan_layer) at world = 1.  Updates slots/owner/last/scores in
 * place.  fetches_out receives m rows of (rank=0, key, slot).  Returns m >= 0, or -1 when the
 * misses exceed the admission capacity (quota.py:63 asserts) or no slot is found
 * (policy.py:177 asserts); the state is left as the reference leaves it when the assert
 * fires (no change before the capacity check, partial installs before a failed slot search).
 */
int64_t oracle_plan_layer(int64_t event, int64_t layer, const int64_t* selected, int64_t tokens,
                          int64_t topk, const float* gate_scores, int64_t* slots, int64_t cap,
                          int64_t* owner, int64_t* last, float* scores, int64_t experts,
                          int64_t* fetches_out, int64_t* destinations_out) {
  const int64_t tick = event + 1, base = layer * experts;
  memcpy(scores + base, gate_scores, (size_t)experts * sizeof(float));
  uint8_t* active = (uint8_t*)calloc((size_t)experts, 1);
  int64_t* misses = (int64_t*)malloc((size_t)experts * sizeof(int64_t));
  for (int64_t t = 0; t < tokens; ++t)
    for (int64_t j = 0; j < topk; ++j) active[selected[t * topk + j]] = 1;
  int64_t m = 0;
  for (int64_t e = 0; e < experts; ++e)
    if (active[e] && owner[base + e] < 0) misses[m++] = e;
  /* admission capacity u_0 (policy.py:37-46) and the quota check (quota.py:63) */
  int64_t u = 0;
  for (int64_t i = 0; i < cap; ++i) {
    int64_t key = slots[i];
    if (key < 0 || !(key / experts == layer && active[key % experts])) ++u;
  }
  if (m > u) {
    free(active);
    free(misses);
    return -1;
  }
  for (int64_t i = 0; i < m; ++i) {
    const int64_t key = base + misses[i];
    int64_t slot = oracle_choose_slot(layer, active, slots, cap, last, scores, experts);
    if (slot < 0) {
      free(active);
      free(misses);
      return -1;
    }
    int64_t victim = slots[slot];
    if (victim >= 0) owner[victim] = -1;
    slots[slot] = key;
    owner[key] = 0;
    fetches_out[i * 3 + 0] = 0;
    fetches_out[i * 3 + 1] = key;
    fetches_out[i * 3 + 2] = slot;
  }
  for (int64_t e = 0; e < experts; ++e)
    if (active[e]) last[base + e] = tick;
  if (destinations_out)
    for (int64_t t = 0; t < tokens * topk; ++t) destinations_out[t] = owner[base + selected[t]];
  free(active);
  free(misses);
  return m;
}

/* ferry/policy.py:197-205 */
void oracle_layer_slots(const int64_t* slots, int64_t cap, int64_t layer, int64_t experts,
                        int64_t* lookup) {
  for (int64_t e = 0; e < experts; ++e) lookup[e] = -1;
  for (int64_t i = 0; i < cap; ++i) {
    int64_t key = slots[i];
    if (key >= 0 && key / experts == layer) lookup[key % experts] = i;
  }
}

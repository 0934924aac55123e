// Router: fp32 softmax + top-k (+ renormalisation, scale, bf16 cast), one wavefront per row.
//
// Reference: ferry/model.py:141-146 (Qwen3 hook) and the greedy DeepSeek-V2 gate feeding
// ferry/model.py:151-157.  torch.topk there selects on the fp32 probabilities with torch's
// CPU algorithm (std::nth_element + std::sort of the first k-1 entries when k*64 > E, else
// std::partial_sort; comparator on values only, NaN first).  Two distinct logits can round to
// the same probability, which torch then treats as a tie, so the selection must run on the
// probabilities themselves, bit for bit.  The kernel therefore computes them exactly as
// torch's CPU softmax does (ATen/native/cpu/SoftMaxKernel.cpp, vectorized last-dim path):
//   m = max of the row; e_i = exp(x_i - m) with SLEEF's expf_u10 (the exp of
//   Vectorized<float>, ATen/cpu/vec/vec512/vec512_float.h:307-309), restated in sleef_expf;
//   s = their sum in vec::reduce_all's order for 16-lane vectors (ATen/cpu/vec/
//   functional_base.h:185-203 and the AVX-512 VecReduceAllSIMD at :78-98); p_i = e_i * (1/s).
// The renormalising sum of the Qwen3 hook, w.sum(-1), follows torch's CPU sum kernel for a
// short contiguous last dimension (see topk_weight_sum).  Both orders were identified on
// torch 2.10's CPU build and are checked against it bit for bit by the tests.  A row holding
// a NaN or +inf logit has all-NaN probabilities, i.e. all elements compare equal.
// Selection runs on order-preserving uint32 keys of the probabilities.
//
// Fast path (sorted output, nth_element regime, all top-k keys distinct and the k-th above
// the (k+1)-th): the selection is unique and comes out in descending order; k wavefront
// arg-max rounds find it.  Every other row replays the CPU algorithm exactly:
//  * wavefront-parallel introselect: the row is held 4 keys per lane (position
//    p = 64 * slot + lane); each median-of-3 / Hoare partition step is evaluated in one pass
//    -- the j-th left stop (ascending position holding a key <= pivot) is exchanged with the
//    j-th right stop (descending position holding a key >= pivot) while left < right, and
//    the stops are ranked with ballots -- so a partition costs a few LDS round trips
//    instead of a serial scan;
//  * the final std::sort of the first k-1 entries (k - 1 <= 16) is an insertion sort, i.e.
//    a stable descending sort, computed by ranking;
//  * the rare remainder (introselect depth limit reached -> heap select; partial_sort regime
//    k*64 <= n; k - 1 > 16) runs the sequential algorithm on lane 0 over the row in LDS.
#include "common.h"

// every rounding step below is the reference's: no contraction of a*b+c into one FMA
#pragma clang fp contract(off)

namespace ferry {
namespace {

constexpr int kMaxE = 256;  // 4 keys per lane
constexpr int kMaxK = 32;
constexpr int kWaves = 4;

struct Pair {
  uint32_t v;  // ordered key: larger key = "before" in the torch comparator
  int32_t i;
};

__device__ __forceinline__ bool before(const Pair& x, const Pair& y) { return x.v > y.v; }

// order-preserving key of a float: -0 == +0, NaN above +inf (all NaNs equal)
__device__ __forceinline__ uint32_t ordered_key(float f) {
  if (f != f) return 0xffffffffu;
  if (f == 0.f) f = 0.f;
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---------------------------------------------------------------------------------------------
// Sequential restatement (lane 0, row in LDS): libstdc++ introselect / introsort / heap select
// ---------------------------------------------------------------------------------------------
__device__ void push_heap_(Pair* a, int hole, int top, Pair value) {
  int parent = (hole - 1) / 2;
  while (hole > top && before(a[parent], value)) {
    a[hole] = a[parent];
    hole = parent;
    parent = (hole - 1) / 2;
  }
  a[hole] = value;
}
__device__ void adjust_heap_(Pair* a, int hole, int len, Pair value) {
  const int top = hole;
  int child = hole;
  while (child < (len - 1) / 2) {
    child = 2 * (child + 1);
    if (before(a[child], a[child - 1])) child--;
    a[hole] = a[child];
    hole = child;
  }
  if ((len & 1) == 0 && child == (len - 2) / 2) {
    child = 2 * (child + 1);
    a[hole] = a[child - 1];
    hole = child - 1;
  }
  push_heap_(a, hole, top, value);
}
__device__ void make_heap_(Pair* a, int len) {
  if (len < 2) return;
  int parent = (len - 2) / 2;
  for (;;) {
    Pair value = a[parent];
    adjust_heap_(a, parent, len, value);
    if (parent == 0) return;
    parent--;
  }
}
__device__ void pop_heap_(Pair* a, int len, int result) {
  Pair value = a[result];
  a[result] = a[0];
  adjust_heap_(a, 0, len, value);
}
__device__ void heap_select_(Pair* a, int middle, int last) {
  make_heap_(a, middle);
  for (int i = middle; i < last; ++i)
    if (before(a[i], a[0])) pop_heap_(a, middle, i);
}
__device__ void sort_heap_(Pair* a, int len) {
  while (len > 1) {
    --len;
    pop_heap_(a, len, len);
  }
}
__device__ void unguarded_linear_insert_(Pair* a, int last) {
  Pair val = a[last];
  int next = last - 1;
  while (before(val, a[next])) {
    a[last] = a[next];
    last = next;
    --next;
  }
  a[last] = val;
}
__device__ void insertion_sort_(Pair* a, int first, int last) {
  if (first == last) return;
  for (int i = first + 1; i != last; ++i) {
    if (before(a[i], a[first])) {
      Pair val = a[i];
      for (int j = i; j > first; --j) a[j] = a[j - 1];
      a[first] = val;
    } else {
      unguarded_linear_insert_(a, i);
    }
  }
}
__device__ __forceinline__ void swap_(Pair* a, int x, int y) {
  Pair t = a[x];
  a[x] = a[y];
  a[y] = t;
}
__device__ void move_median_to_first_(Pair* a, int result, int x, int y, int z) {
  if (before(a[x], a[y])) {
    if (before(a[y], a[z]))
      swap_(a, result, y);
    else if (before(a[x], a[z]))
      swap_(a, result, z);
    else
      swap_(a, result, x);
  } else if (before(a[x], a[z])) {
    swap_(a, result, x);
  } else if (before(a[y], a[z])) {
    swap_(a, result, z);
  } else {
    swap_(a, result, y);
  }
}
__device__ int unguarded_partition_(Pair* a, int first, int last, int pivot) {
  const Pair p = a[pivot];
  for (;;) {
    while (before(a[first], p)) ++first;
    --last;
    while (before(p, a[last])) --last;
    if (!(first < last)) return first;
    swap_(a, first, last);
    ++first;
  }
}
__device__ int partition_pivot_(Pair* a, int first, int last) {
  const int mid = first + (last - first) / 2;
  move_median_to_first_(a, first, first + 1, mid, last - 1);
  return unguarded_partition_(a, first + 1, last, first);
}
__device__ __forceinline__ int lg2_(int n) { return 31 - __clz(n); }

// std::sort of a[first, last): introsort loop down to ranges of 16, then insertion sort.
// stk holds 3 * kStack ints of LDS for the pending right-hand ranges.
constexpr int kStack = 16;
__device__ void sort_(Pair* a, int first, int last, int* stk) {
  if (last - first <= 1) return;
  int sp = 0;
  stk[0] = first;
  stk[1] = last;
  stk[2] = lg2_(last - first) * 2;
  ++sp;
  while (sp > 0) {
    --sp;
    int f = stk[3 * sp], l = stk[3 * sp + 1], depth = stk[3 * sp + 2];
    while (l - f > 16) {
      if (depth == 0) {
        heap_select_(a + f, l - f, l - f);
        sort_heap_(a + f, l - f);
        break;
      }
      --depth;
      const int cut = partition_pivot_(a, f, l);
      // the reference recurses on [cut, l) and loops on [f, cut): disjoint ranges, so the
      // processing order does not change the result.  Ranges here hold at most kMaxK - 1
      // elements, so the pending stack stays far below kStack entries.
      if (sp < kStack) {
        stk[3 * sp] = cut;
        stk[3 * sp + 1] = l;
        stk[3 * sp + 2] = depth;
        ++sp;
      }
      l = cut;
    }
  }
  if (last - first > 16) {
    insertion_sort_(a, first, first + 16);
    for (int i = first + 16; i != last; ++i) unguarded_linear_insert_(a, i);
  } else {
    insertion_sort_(a, first, last);
  }
}

// ---------------------------------------------------------------------------------------------
// Wavefront-parallel restatement
// ---------------------------------------------------------------------------------------------
struct WaveScratch {
  Pair stage[kMaxE];
  int16_t lstop[kMaxE];
  int16_t rstop[kMaxE];
  float prob[kMaxE];
  int32_t sel[kMaxK];
  int32_t stack[3 * kStack];
};

__device__ __forceinline__ void wave_sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// value at uniform position p = 64 * slot + lane: read lane (p & 63) of each of the four
// registers and select by slot (selecting between register values, not array elements, keeps
// the arrays out of scratch memory)
template <int NS>
__device__ __forceinline__ uint32_t key_at(const uint32_t (&k)[NS], int p) {
  const int l = p & 63, s = p >> 6;
  uint32_t r = (uint32_t)__builtin_amdgcn_readlane((int)k[0], l);
#pragma unroll
  for (int q = 1; q < NS; ++q) {
    const uint32_t rq = (uint32_t)__builtin_amdgcn_readlane((int)k[q], l);
    r = s == q ? rq : r;
  }
  return r;
}
template <int NS>
__device__ __forceinline__ int32_t idx_at(const int32_t (&ix)[NS], int p) {
  const int l = p & 63, s = p >> 6;
  int32_t r = __builtin_amdgcn_readlane(ix[0], l);
#pragma unroll
  for (int q = 1; q < NS; ++q) {
    const int32_t rq = __builtin_amdgcn_readlane(ix[q], l);
    r = s == q ? rq : r;
  }
  return r;
}
template <int NS>
__device__ __forceinline__ void set_at(uint32_t (&k)[NS], int32_t (&ix)[NS], int p, uint32_t kv,
                                       int32_t iv, int lane) {
  const bool mine = lane == (p & 63);
  const int s = p >> 6;
  // per-element selects (no indexed store, which would move the arrays to scratch)
#pragma unroll
  for (int q = 0; q < NS; ++q) {
    const bool hit = mine && q == s;
    k[q] = hit ? kv : k[q];
    ix[q] = hit ? iv : ix[q];
  }
}
template <int NS>
__device__ __forceinline__ void swap_at(uint32_t (&k)[NS], int32_t (&ix)[NS], int a, int b,
                                        int lane) {
  const uint32_t ka = key_at(k, a), kb = key_at(k, b);
  const int32_t ia = idx_at(ix, a), ib = idx_at(ix, b);
  set_at(k, ix, a, kb, ib, lane);
  set_at(k, ix, b, ka, ia, lane);
}

// One std::__unguarded_partition_pivot step on [first, last); returns the cut.
template <int NS>
__device__ __forceinline__ int wave_partition_pivot(uint32_t (&k)[NS], int32_t (&ix)[NS], int first, int last,
                                    int lane, WaveScratch& ws) {
  const int mid = first + (last - first) / 2;
  {
    // __move_median_to_first(first, first + 1, mid, last - 1)
    const int a = first + 1, b = mid, c = last - 1;
    const uint32_t ka = key_at(k, a), kb = key_at(k, b), kc = key_at(k, c);
    int m;
    if (ka > kb) {
      m = (kb > kc) ? b : (ka > kc) ? c : a;
    } else {
      m = (ka > kc) ? a : (kb > kc) ? c : b;
    }
    swap_at(k, ix, first, m, lane);
  }
  const uint32_t piv = key_at(k, first);
  // left stops: [first+1, last) with key <= pivot; right stops: [first, last) with key >= pivot
  uint64_t bl[NS], bg[NS];
  bool le[NS], ge[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    le[s] = pos > first && pos < last && k[s] <= piv;
    ge[s] = pos >= first && pos < last && k[s] >= piv;
    bl[s] = __ballot(le[s]);
    bg[s] = __ballot(ge[s]);
  }
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const uint64_t gt_mask = (lane == 63) ? 0ull : (~0ull << (lane + 1));
  int nl = 0, ng = 0;
  int rl[NS], rg[NS];
  int below_l = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    rl[s] = below_l + __popcll(bl[s] & lt_mask);
    below_l += __popcll(bl[s]);
  }
  nl = below_l;
  int above_g = 0;
#pragma unroll
  for (int s = NS - 1; s >= 0; --s) {
    rg[s] = above_g + __popcll(bg[s] & gt_mask);
    above_g += __popcll(bg[s]);
  }
  ng = above_g;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    if (le[s]) ws.lstop[rl[s]] = (int16_t)pos;
    if (ge[s]) ws.rstop[rg[s]] = (int16_t)pos;
    if (pos < last) ws.stage[pos] = Pair{k[s], ix[s]};
  }
  wave_sync_lds();
  // number of exchanges: prefix of m with lstop[m] < rstop[m]
  const int mm = nl < ng ? nl : ng;
  int nswap = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int m = s * 64 + lane;
    const bool f = m < mm && ws.lstop[m] < ws.rstop[m];
    nswap += __popcll(__ballot(f));
  }
  int cut;
  if (nswap == 0) {
    cut = nl > 0 ? ws.lstop[0] : last - 1;
  } else {
    const int lnext = nswap < nl ? ws.lstop[nswap] : 0x7fffffff;
    const int rprev = ws.rstop[nswap - 1];
    cut = lnext < rprev ? lnext : rprev;
  }
  // the median-of-3 pivot guarantees a left stop inside the range, so cut lies in
  // [first + 1, last - 1]; the clamp only keeps indices in range should that ever fail
  cut = cut < first + 1 ? first + 1 : (cut > last - 1 ? last - 1 : cut);
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    int src = -1;
    if (le[s] && rl[s] < nswap) src = ws.rstop[rl[s]];
    else if (ge[s] && rg[s] < nswap) src = ws.lstop[rg[s]];
    if (src >= 0) {
      const Pair p = ws.stage[src];
      k[s] = p.v;
      ix[s] = p.i;
    }
  }
  wave_sync_lds();
  return cut;
}

// stable descending sort of the uniform positions [first, last) (last - first <= 16):
// the result of std::__insertion_sort on that range
template <int NS>
__device__ __forceinline__ void wave_insertion_sort(uint32_t (&k)[NS], int32_t (&ix)[NS], int first, int last,
                                    int lane, WaveScratch& ws) {
  const int len = last - first;
  if (len <= 1) return;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    if (pos >= first && pos < last) ws.stage[pos] = Pair{k[s], ix[s]};
  }
  wave_sync_lds();
  int dest[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    dest[s] = -1;
    if (pos >= first && pos < last) {
      int d = first;
      for (int q = first; q < last; ++q) {
        const uint32_t kq = ws.stage[q].v;
        d += (kq > k[s]) || (kq == k[s] && q < pos);
      }
      dest[s] = d;
    }
  }
  wave_sync_lds();
#pragma unroll
  for (int s = 0; s < NS; ++s)
    if (dest[s] >= 0) ws.stage[dest[s]] = Pair{k[s], ix[s]};
  wave_sync_lds();
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    if (pos >= first && pos < last) {
      k[s] = ws.stage[pos].v;
      ix[s] = ws.stage[pos].i;
    }
  }
  wave_sync_lds();
}

// The partition step and the insertion sort on slot 0 alone when [first, last) lies within
// positions 0..63 (the keys of the other slots are outside the range and stay as they are): the
// same steps, with half (or a quarter) of the per-slot work.  introselect narrows the range
// around position k - 1 < 64 within a step or two.
template <int NS>
__device__ __forceinline__ int partition_step(uint32_t (&k)[NS], int32_t (&ix)[NS], int first, int last,
                                              int lane, WaveScratch& ws) {
  if constexpr (NS > 1) {
    if (last <= 64) {
      uint32_t k0[1] = {k[0]};
      int32_t i0[1] = {ix[0]};
      const int cut = wave_partition_pivot(k0, i0, first, last, lane, ws);
      k[0] = k0[0];
      ix[0] = i0[0];
      return cut;
    }
  }
  return wave_partition_pivot(k, ix, first, last, lane, ws);
}
template <int NS>
__device__ __forceinline__ void insertion_step(uint32_t (&k)[NS], int32_t (&ix)[NS], int first, int last,
                                               int lane, WaveScratch& ws) {
  if constexpr (NS > 1) {
    if (last <= 64) {
      uint32_t k0[1] = {k[0]};
      int32_t i0[1] = {ix[0]};
      wave_insertion_sort(k0, i0, first, last, lane, ws);
      k[0] = k0[0];
      ix[0] = i0[0];
      return;
    }
  }
  wave_insertion_sort(k, ix, first, last, lane, ws);
}

// Exact CPU top-k selection of the row (n keys, position p = 64*s + lane); the chosen indices
// are written to ws.sel[0..k).
template <int NS>
__device__ __forceinline__ void exact_select(uint32_t (&k)[NS], int32_t (&ix)[NS], int n, int kk, bool sorted,
                             int lane, WaveScratch& ws) {
  bool serial = kk * 64 <= n || (sorted && kk - 1 > 16);
  if (!serial) {
    // std::nth_element(first, first + kk - 1, last)
    const int nth = kk - 1;
    int first = 0, last = n;
    int depth = lg2_(n) * 2;
    if (nth != n) {
      while (last - first > 3) {
        if (depth == 0) {
          serial = true;  // heap select from this state on lane 0
          break;
        }
        --depth;
        const int cut = partition_step(k, ix, first, last, lane, ws);
        if (cut <= nth)
          first = cut;
        else
          last = cut;
      }
      if (!serial) insertion_step(k, ix, first, last, lane, ws);
    }
    if (serial) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int pos = s * 64 + lane;
        if (pos < n) ws.stage[pos] = Pair{k[s], ix[s]};
      }
      wave_sync_lds();
      if (lane == 0) {
        heap_select_(ws.stage + first, nth + 1 - first, last - first);
        swap_(ws.stage, first, nth);
        if (sorted) sort_(ws.stage, 0, kk - 1, ws.stack);
        for (int j = 0; j < kk; ++j) ws.sel[j] = ws.stage[j].i;
      }
      wave_sync_lds();
      return;
    }
    if (sorted) insertion_step(k, ix, 0, kk - 1, lane, ws);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int pos = s * 64 + lane;
      if (pos < kk) ws.sel[pos] = ix[s];
    }
    wave_sync_lds();
    return;
  }
  // partial_sort regime, or a final sort longer than 16: sequential on lane 0
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int pos = s * 64 + lane;
    if (pos < n) ws.stage[pos] = Pair{k[s], ix[s]};
  }
  wave_sync_lds();
  if (lane == 0) {
    Pair* a = ws.stage;
    if (kk * 64 <= n) {
      heap_select_(a, kk, n);
      sort_heap_(a, kk);
    } else {
      int first = 0, last = n, depth = lg2_(n) * 2;
      const int nth = kk - 1;
      bool done = false;
      if (nth != n) {
        while (last - first > 3) {
          if (depth == 0) {
            heap_select_(a + first, nth + 1 - first, last - first);
            swap_(a, first, nth);
            done = true;
            break;
          }
          --depth;
          const int cut = partition_pivot_(a, first, last);
          if (cut <= nth)
            first = cut;
          else
            last = cut;
        }
        if (!done) insertion_sort_(a, first, last);
      }
      if (sorted) sort_(a, 0, kk - 1, ws.stack);
    }
    for (int j = 0; j < kk; ++j) ws.sel[j] = a[j].i;
  }
  wave_sync_lds();
}

// Wavefront reductions through DPP lane moves (a few cycles each, against an LDS round trip
// per step for __shfl_xor): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror and row_mirror
// combine each row of 16 lanes in every lane; row_bcast:15 and row_bcast:31 then carry rows 0-2
// into the last row, and lane 63 holds the result, which readlane makes wave-uniform.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ float dpp_asf(uint32_t v) { return __uint_as_float(v); }
__device__ __forceinline__ float wave_max(float v) {
  uint32_t u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0xB1>(u, u)));
  u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0x4E>(u, u)));
  u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0x141>(u, u)));
  u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0x140>(u, u)));
  u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0x142, 0xa>(u, u)));
  u = __float_as_uint(v);
  v = fmaxf(v, dpp_asf(dpp_u<0x143, 0xc>(u, u)));
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), 63));
}
__device__ __forceinline__ uint32_t umax_(uint32_t a, uint32_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
  v = umax_(v, dpp_u<0xB1>(v, v));
  v = umax_(v, dpp_u<0x4E>(v, v));
  v = umax_(v, dpp_u<0x141>(v, v));
  v = umax_(v, dpp_u<0x140>(v, v));
  v = umax_(v, dpp_u<0x142, 0xa>(v, v));
  v = umax_(v, dpp_u<0x143, 0xc>(v, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// SLEEF's single-precision exp with 1.0-ulp bound (xexpf of SLEEF 3, sleefsimdsp.c; the
// published Cody-Waite reduction by ln 2 in two parts, a degree-6 polynomial for e^s - 1 - s in
// Horner form with fused multiply-adds, and a two-step scaling by 2^q).  Restated from that
// method; checked against the SLEEF routine torch calls on all 2^32 fp32 inputs.
__device__ __forceinline__ float pow2i_(int q) { return __uint_as_float((uint32_t)(q + 0x7f) << 23); }
__device__ __forceinline__ float sleef_expf(float d) {
  if (d != d) return d;
  if (d < -104.f) return 0.f;
  if (d > 100.f) return INFINITY;
  const float kRln2 = 1.442695040888963407359924681001892137f;
  const float kL2U = 0.693145751953125f, kL2L = 1.428606765330187045e-06f;
  const int q = (int)__builtin_rintf(d * kRln2);
  float s = __builtin_fmaf((float)q, -kL2U, d);
  s = __builtin_fmaf((float)q, -kL2L, s);
  float u = 0.000198527617612853646278381f;
  u = __builtin_fmaf(u, s, 0.00139304355252534151077271f);
  u = __builtin_fmaf(u, s, 0.00833336077630519866943359f);
  u = __builtin_fmaf(u, s, 0.0416664853692054748535156f);
  u = __builtin_fmaf(u, s, 0.166666671633720397949219f);
  u = __builtin_fmaf(u, s, 0.5f);
  u = 1.0f + __builtin_fmaf(s * s, u, s);
  return u * pow2i_(q >> 1) * pow2i_(q - (q >> 1));
}

// Sum of e[0..n) (in LDS) in the order of torch's vec::reduce_all(+) for 16-lane vectors:
// n < 16: left to right; otherwise lane l of an accumulator vector adds e[16c + l] over the
// full chunks c in order, the tail chunk adds into its first n % 16 lanes, and the 16 lanes are
// combined by the halving butterfly (l + 8, then l + 4, l + 2, l + 1).  The chunks are read
// into registers at once; the butterfly moves lanes with DPP row shifts (row_shl:h, lane l
// reads lane l + h of its row of 16), and lane 0 holds the sum.  Wave-uniform result.
template <int NS>
__device__ __forceinline__ float torch_softmax_sum(const float* e, int n, int lane) {
  float acc = 0.f;
  if (n < 16) {
    if (lane == 0) {
      acc = e[0];
      for (int i = 1; i < n; ++i) acc += e[i];
    }
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(acc), 0));
  }
  const int full = n - n % 16;
  const int l16 = lane & 15;
  float v[4 * NS];
#pragma unroll
  for (int c = 0; c < 4 * NS; ++c) v[c] = 16 * c < full ? e[16 * c + l16] : 0.f;
  const float tail = l16 < n - full ? e[full + l16] : 0.f;
  acc = v[0];
#pragma unroll
  for (int c = 1; c < 4 * NS; ++c)
    if (16 * c < full) acc += v[c];
  if (l16 < n - full) acc += tail;
  uint32_t u = __float_as_uint(acc);
  acc += dpp_asf(dpp_u<0x108>(u, u));
  u = __float_as_uint(acc);
  acc += dpp_asf(dpp_u<0x104>(u, u));
  u = __float_as_uint(acc);
  acc += dpp_asf(dpp_u<0x102>(u, u));
  u = __float_as_uint(acc);
  acc += dpp_asf(dpp_u<0x101>(u, u));
  return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(acc), 0));
}

// torch's CPU sum over a contiguous last dimension of k <= 32 fp32 values (the renormalising
// w.sum(-1) of the Qwen3 hook), w_j held by lane j.  torch runs its 8-lane (AVX2) reduction
// kernel here: for k < 8 a scalar sum with four interleaved partial sums (partial j takes
// w[4i + j], the tail w[4 * (k / 4)..] goes into partial 0, then partial 0 + 1 + 2 + 3); for
// k >= 8, lane l of an 8-lane vector sums w[8i + l] over the k / 8 full vectors, and the result
// is the sum, left to right, of the scalar tail w[8 * (k / 8)..] followed by the 8 lanes.
// Identified by testing against torch's CPU sum for every k <= 32; wave-uniform result.
__device__ __forceinline__ float topk_weight_sum(float wv, int kk) {
  auto at = [&](int j) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(wv), j));
  };
  if (kk < 8) {
    float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
    int i = 0;
    if (kk >= 4) {
      p0 = at(0);
      p1 = at(1);
      p2 = at(2);
      p3 = at(3);
      i = 4;
    }
    for (; i < kk; ++i) p0 += at(i);
    return ((p0 + p1) + p2) + p3;
  }
  const int nv = kk / 8;
  float acc = 0.f;
  for (int i = 8 * nv; i < kk; ++i) acc += at(i);
  for (int l = 0; l < 8; ++l) {
    float lane_sum = at(l);
    for (int v = 1; v < nv; ++v) lane_sum += at(8 * v + l);
    acc += lane_sum;
  }
  return acc;
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p);
template <>
__device__ __forceinline__ float load_logit<float>(const float* p) {
  return *p;
}
template <>
__device__ __forceinline__ float load_logit<bf16_t>(const bf16_t* p) {
  return bf16_to_f32(*p);
}

template <typename T, int NS>
__global__ __launch_bounds__(64 * kWaves) void router_kernel(
    const T* __restrict__ logits, int64_t tokens, int n, int kk, int renorm, float scale,
    int sorted, int64_t* __restrict__ idx_out, bf16_t* __restrict__ w_out,
    float* __restrict__ probs_out, int32_t* __restrict__ tie_rows) {
  __shared__ WaveScratch scratch[kWaves];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  WaveScratch& ws = scratch[wave];
  for (int64_t row = (int64_t)blockIdx.x * kWaves + wave; row < tokens;
       row += (int64_t)gridDim.x * kWaves) {
    const T* src = logits + row * n;
    float x[NS];
    bool bad = false;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int e = s * 64 + lane;
      x[s] = e < n ? load_logit<T>(src + e) : -INFINITY;
      bad |= (e < n) && (x[s] != x[s] || x[s] == INFINITY);
    }
    const bool row_bad = __any(bad);  // softmax of this row is all NaN
    // softmax in fp32, rounding step for rounding step as torch's CPU kernel
    float m = x[0];
#pragma unroll
    for (int s = 1; s < NS; ++s) m = fmaxf(m, x[s]);
    m = wave_max(m);
    float ex[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int e = s * 64 + lane;
      ex[s] = e < n ? sleef_expf(x[s] - m) : 0.f;
      if (e < n) ws.prob[e] = ex[s];
    }
    wave_sync_lds();
    const float sum = torch_softmax_sum<NS>(ws.prob, n, lane);
    wave_sync_lds();
    const float inv = 1.0f / sum;
    uint32_t key[NS];
    int32_t ix[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int e = s * 64 + lane;
      const float p = row_bad ? __builtin_nanf("") : ex[s] * inv;
      if (e < n) {
        ws.prob[e] = p;
        if (probs_out) probs_out[row * n + e] = p;
      }
      key[s] = e < n ? (row_bad ? 0xffffffffu : ordered_key(p)) : 0u;
      ix[s] = e;
    }
    // fast path: kk arg-max rounds on distinct keys (nth_element regime, sorted output)
    bool exact = !sorted || row_bad || kk * 64 <= n;
    if (!exact) {
      uint32_t cur[NS];
#pragma unroll
      for (int s = 0; s < NS; ++s) cur[s] = (s * 64 + lane < n) ? key[s] : 0u;
      for (int r = 0; r < kk; ++r) {
        uint32_t lm = cur[0];
#pragma unroll
        for (int s = 1; s < NS; ++s) lm = cur[s] > lm ? cur[s] : lm;
        const uint32_t best = wave_max_u(lm);
        int eq = 0, where = 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const bool hit = (s * 64 + lane < n) && cur[s] == best;
          eq += hit;
          if (hit) where = s * 64 + lane;
        }
        const uint64_t hits = __ballot(eq > 0);
        const int total = __popcll(hits) == 1 ? __builtin_amdgcn_readlane(eq, __ffsll((long long)hits) - 1) : 2;
        if (total != 1 || best == 0u) {
          exact = true;  // a tie decides membership or order
          break;
        }
        const int owner = __ffsll((long long)hits) - 1;
        const int pos = __builtin_amdgcn_readlane(where, owner);
        if (lane == 0) ws.sel[r] = pos;
#pragma unroll
        for (int s = 0; s < NS; ++s) cur[s] = (lane == owner && s == (pos >> 6)) ? 0u : cur[s];
      }
      wave_sync_lds();
    }
    if (exact) {
      exact_select(key, ix, n, kk, sorted != 0, lane, ws);
      if (lane == 0 && tie_rows) atomicAdd(tie_rows, 1);
    }
    wave_sync_lds();
    // weights: lanes 0..kk-1 each own one selected expert
    float wv = 0.f;
    int e = 0;
    if (lane < kk) {
      e = ws.sel[lane];
      wv = ws.prob[e];
    }
    const float tot = renorm ? topk_weight_sum(wv, kk) : 0.f;
    if (lane < kk) {
      float w = renorm ? wv / tot : wv;
      w = w * scale;
      idx_out[row * kk + lane] = e;
      w_out[row * kk + lane] = f32_to_bf16(w);
    }
    wave_sync_lds();
  }
}

}  // namespace
}  // namespace ferry

using namespace ferry;

extern "C" int ferry_router_topk(const void* logits, int32_t logits_dtype, int64_t tokens,
                                 int64_t experts, int64_t topk, int32_t renorm, float scale,
                                 int32_t sorted, int64_t* idx_out, void* w_out_bf16,
                                 float* probs_out, int32_t* tie_rows, void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0, "tokens must be >= 0 (got %lld)", (long long)tokens);
  FERRY_CHECK_ARG(experts >= 1 && experts <= kMaxE, "experts must be in [1, %d] (got %lld)",
                  kMaxE, (long long)experts);
  FERRY_CHECK_ARG(topk >= 1 && topk <= experts && topk <= kMaxK,
                  "topk must be in [1, min(experts, %d)] (got %lld)", kMaxK, (long long)topk);
  FERRY_CHECK_ARG(logits_dtype == FERRY_BF16 || logits_dtype == FERRY_F32,
                  "logits dtype must be bf16 or fp32");
  FERRY_CHECK_ARG(tokens == 0 || (logits && idx_out && w_out_bf16), "null pointer argument");
  if (tokens == 0) return 0;
  const int64_t want = ceil_div(tokens, kWaves);
  const int grid = (int)(want < 65535 ? want : 65535);
  hipStream_t s = (hipStream_t)stream;
  // NS = 64-key slots per lane: the exact path's wave-parallel steps scale with it
  auto go = [&](auto kernel, const auto* lg) {
    launch("router_kernel", kernel, dim3(grid), dim3(64 * kWaves), 0, s, lg, tokens, (int)experts,
           (int)topk, renorm, scale, sorted, idx_out, (bf16_t*)w_out_bf16, probs_out, tie_rows);
  };
  if (logits_dtype == FERRY_BF16) {
    const bf16_t* lg = (const bf16_t*)logits;
    if (experts <= 64) go(router_kernel<bf16_t, 1>, lg);
    else if (experts <= 128) go(router_kernel<bf16_t, 2>, lg);
    else go(router_kernel<bf16_t, 4>, lg);
  } else {
    const float* lg = (const float*)logits;
    if (experts <= 64) go(router_kernel<float, 1>, lg);
    else if (experts <= 128) go(router_kernel<float, 2>, lg);
    else go(router_kernel<float, 4>, lg);
  }
  FERRY_LAUNCHED("router_kernel");
  return 0;
}

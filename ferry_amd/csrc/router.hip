// Router: fp32 softmax + top-k (+ renormalisation, scale, bf16 cast), one wavefront per row.
//
// Reference: ferry/model.py:141-146 (Qwen3 hook) and the greedy DeepSeek-V2 gate feeding
// ferry/model.py:151-157.  torch.topk there selects on the fp32 probabilities with torch's
// CPU algorithm (std::nth_element + std::sort of the first k-1 entries when k*64 > E, else
// std::partial_sort; comparator on values only).  Softmax is strictly increasing in the
// logit, so the order relation -- ties included -- is that of the logits whenever the
// probabilities compared are normal fp32 numbers; this kernel therefore selects on the
// logits themselves, which makes the tie pattern independent of the exp implementation.
//
// Fast path (sorted output, all top-k values distinct, k-th > (k+1)-th): the selection is
// unique and comes out in descending order; it is found with k wavefront arg-max
// reductions.  Every other row (ties, NaN, or unsorted output, whose order depends on the
// partition steps) is resolved by lane 0 running the same selection algorithm as the CPU
// (median-of-3 introselect with insertion sort below 4 elements, heap select after the
// depth limit, introsort for the final sort) on the row staged in LDS.
#include "common.h"

namespace ferry {
namespace {

constexpr int kMaxE = 256;  // 4 values per lane
constexpr int kMaxK = 32;
constexpr int kWaves = 4;

struct Pair {
  float v;
  int32_t i;
};

__device__ __forceinline__ bool before(const Pair& x, const Pair& y) {
  const bool xn = x.v != x.v, yn = y.v != y.v;
  return (xn && !yn) || (x.v > y.v);
}

// ---- heap primitives ----
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

// ---- sorting primitives ----
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

// introsort of a[first, last): partition until ranges of <= 16, then one insertion sort.
__device__ void sort_(Pair* a, int first, int last) {
  if (first == last) return;
  // explicit stack replaces the recursion on the right part
  int st_first[32], st_last[32], st_depth[32];
  int sp = 0;
  st_first[sp] = first;
  st_last[sp] = last;
  st_depth[sp] = lg2_(last - first) * 2;
  ++sp;
  while (sp > 0) {
    --sp;
    int f = st_first[sp], l = st_last[sp], depth = st_depth[sp];
    while (l - f > 16) {
      if (depth == 0) {
        heap_select_(a + f, l - f, l - f);
        sort_heap_(a + f, l - f);
        break;
      }
      --depth;
      const int cut = partition_pivot_(a, f, l);
      // the reference recurses on [cut, l) first, then loops on [f, cut); processing
      // order does not change the result because the ranges are disjoint.
      st_first[sp] = cut;
      st_last[sp] = l;
      st_depth[sp] = depth;
      ++sp;
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

__device__ void nth_element_(Pair* a, int nth, int n) {
  if (n == 0 || nth == n) return;
  int first = 0, last = n;
  int depth = lg2_(n) * 2;
  while (last - first > 3) {
    if (depth == 0) {
      heap_select_(a + first, nth + 1 - first, last - first);
      swap_(a, first, nth);
      return;
    }
    --depth;
    const int cut = partition_pivot_(a, first, last);
    if (cut <= nth)
      first = cut;
    else
      last = cut;
  }
  insertion_sort_(a, first, last);
}

// The full CPU selection on a row staged in LDS; result in a[0..k).
__device__ void exact_topk_(Pair* a, int n, int k, bool sorted) {
  if (k * 64 <= n) {
    heap_select_(a, k, n);
    sort_heap_(a, k);
  } else {
    nth_element_(a, k - 1, n);
    if (sorted) sort_(a, 0, k - 1);
  }
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
// arg-max with the torch comparator on values; equal values -> lower index
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float ov = __shfl_xor(v, off, 64);
    int oi = __shfl_xor(i, off, 64);
    if (ov > v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
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

template <typename T>
__global__ __launch_bounds__(64 * kWaves) void router_kernel(
    const T* __restrict__ logits, int64_t tokens, int n, int k, int renorm, float scale,
    int sorted, int64_t* __restrict__ idx_out, bf16_t* __restrict__ w_out,
    float* __restrict__ probs_out, int32_t* __restrict__ tie_rows) {
  __shared__ Pair stage[kWaves][kMaxE];
  __shared__ float prob_lds[kWaves][kMaxE];
  __shared__ int sel[kWaves][kMaxK];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float NEG = -INFINITY;
  for (int64_t row = (int64_t)blockIdx.x * kWaves + wave; row < tokens;
       row += (int64_t)gridDim.x * kWaves) {
    const T* src = logits + row * n;
    float x[4];
    bool has_nan = false;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int e = lane + 64 * s;
      x[s] = e < n ? load_logit<T>(src + e) : NEG;
      has_nan |= (e < n) && (x[s] != x[s]);
    }
    // softmax in fp32
    float m = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    m = wave_max(m);
    float ex[4], part = 0.f;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int e = lane + 64 * s;
      ex[s] = e < n ? expf(x[s] - m) : 0.f;
      part += ex[s];
    }
    const float inv = 1.0f / wave_sum(part);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int e = lane + 64 * s;
      if (e < n) {
        const float p = ex[s] * inv;
        prob_lds[wave][e] = p;
        if (probs_out) probs_out[row * n + e] = p;
      }
    }
    // fast path: k arg-max rounds; any repeated value among the top k (or at the k-th /
    // (k+1)-th boundary) sends the row to the exact path.
    bool exact = !sorted || __any(has_nan);
    if (!exact && k * 64 > n) {
      float cur[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) cur[s] = x[s];
      for (int r = 0; r < k && !exact; ++r) {
        float bv = NEG;
        int bi = 1 << 30;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int e = lane + 64 * s;
          if (e < n && (cur[s] > bv || (cur[s] == bv && e < bi)) && cur[s] != NEG) {
            bv = cur[s];
            bi = e;
          }
        }
        wave_argmax(bv, bi);
        int eq = 0;
#pragma unroll
        for (int s = 0; s < 4; ++s) eq += (lane + 64 * s < n) && (cur[s] == bv);
        eq = wave_sum_i(eq);
        if (eq != 1 || bv == NEG) {
          exact = true;  // a tie (or -inf values) decides membership or order
        } else {
          if (lane == (bi & 63)) cur[bi >> 6] = NEG;
          if (lane == 0) sel[wave][r] = bi;
        }
      }
    } else if (!exact) {
      exact = true;  // partial-sort regime (k*64 <= n): run the CPU algorithm
    }
    if (exact) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int e = lane + 64 * s;
        if (e < n) stage[wave][e] = Pair{x[s], e};
      }
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (lane == 0) {
        exact_topk_(stage[wave], n, k, sorted != 0);
        for (int j = 0; j < k; ++j) sel[wave][j] = stage[wave][j].i;
        if (tie_rows) atomicAdd(tie_rows, 1);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (lane == 0) {
      float sum = 0.f;
      for (int j = 0; j < k; ++j) sum += prob_lds[wave][sel[wave][j]];
      for (int j = 0; j < k; ++j) {
        const int e = sel[wave][j];
        float w = prob_lds[wave][e];
        if (renorm) w = w / sum;
        w = w * scale;
        idx_out[row * k + j] = e;
        w_out[row * k + j] = f32_to_bf16(w);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
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
  if (logits_dtype == FERRY_BF16) {
    hipLaunchKernelGGL(router_kernel<bf16_t>, dim3(grid), dim3(64 * kWaves), 0, s,
                       (const bf16_t*)logits, tokens, (int)experts, (int)topk, renorm, scale,
                       sorted, idx_out, (bf16_t*)w_out_bf16, probs_out, tie_rows);
  } else {
    hipLaunchKernelGGL(router_kernel<float>, dim3(grid), dim3(64 * kWaves), 0, s,
                       (const float*)logits, tokens, (int)experts, (int)topk, renorm, scale,
                       sorted, idx_out, (bf16_t*)w_out_bf16, probs_out, tie_rows);
  }
  FERRY_LAUNCHED("router_kernel");
  return 0;
}

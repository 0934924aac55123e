// Selection-frequency history (window W) on the device, plus the uint8 ID payload that the
// host planner copies back.
//
// Reference: ferry/metadata.py:15-38 (GateHistory) fed by RouteGather.collect at world = 1
// (ferry/metadata.py:67-83): the history rows of a layer call are the one-hot selection
// indicators of its last min(T, ceil(W / world)) tokens; a batch of >= W rows replaces the
// window, a shorter one is appended ring-wise; scores = float32(sum(rows) / max(1, count)).
// Because rows are 0/1, the window sum is the integer count c_e of the last n = min(W, seen)
// tokens that selected e, so the device keeps per-layer integer counters and a ring of the
// IDs of the tokens in the window; score = float32(double(c_e) / double(n)) reproduces the
// reference's float64 mean followed by the float32 cast exactly.
#include "common.h"

namespace ferry {
int ffn_timeouts_address(int32_t** timeouts);
namespace {

constexpr int kMaxE = 512;
constexpr int kThreads = 256;
constexpr int kIdsPerBlock = kThreads * 16;

// Block 0 updates the window of `layer`; blocks >= 1 write the uint8 copy of selected, with
// 0xFF for an ID outside [0, E) (E <= 255 then, so the host planner rejects it).  With ready_out,
// each block then writes ready_value to ready_out[block] with a system-scope release, after its
// other writes are visible to the host.
__device__ void history_block0(const int64_t* __restrict__ selected, int64_t tokens, int k, int E,
                               int W, int64_t layer, int32_t* __restrict__ ring,
                               int32_t* __restrict__ counts, int32_t* __restrict__ meta,
                               float* __restrict__ scores_out,
                               const int32_t* __restrict__ timeouts_src,
                               int32_t* __restrict__ timeouts_out);

__global__ __launch_bounds__(kThreads) void history_kernel(
    const int64_t* __restrict__ selected, int64_t tokens, int k, int E, int W, int64_t layer,
    int32_t* __restrict__ ring, int32_t* __restrict__ counts, int32_t* __restrict__ meta,
    float* __restrict__ scores_out, uint8_t* __restrict__ ids_out,
    const int32_t* __restrict__ timeouts_src, int32_t* __restrict__ timeouts_out,
    int32_t* __restrict__ ready_out, int32_t ready_value) {
  if (blockIdx.x > 0) {
    const int64_t n = tokens * k;
    const int64_t i0 = (int64_t)(blockIdx.x - 1) * kIdsPerBlock;
    for (int64_t i = i0 + threadIdx.x; i < n && i < i0 + kIdsPerBlock; i += kThreads) {
      const int64_t e = selected[i];
      ids_out[i] = (e >= 0 && e < E) ? (uint8_t)e : (uint8_t)0xFF;
    }
  } else {
    history_block0(selected, tokens, k, E, W, layer, ring, counts, meta, scores_out, timeouts_src,
                   timeouts_out);
  }
  if (ready_out) {
    // every wavefront's writes reach the system scope before the block's ready word does
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0)
      __hip_atomic_store(&ready_out[blockIdx.x], ready_value, __ATOMIC_RELEASE,
                         __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

__device__ void history_block0(const int64_t* __restrict__ selected, int64_t tokens, int k, int E,
                               int W, int64_t layer, int32_t* __restrict__ ring,
                               int32_t* __restrict__ counts, int32_t* __restrict__ meta,
                               float* __restrict__ scores_out,
                               const int32_t* __restrict__ timeouts_src,
                               int32_t* __restrict__ timeouts_out) {
  __shared__ int32_t c[kMaxE];
  int32_t* lring = ring + layer * (int64_t)W * k;
  int32_t* lcount = counts + layer * (int64_t)E;
  const int count = meta[layer * 2 + 0];
  const int head = meta[layer * 2 + 1];
  const int tail = (int)(tokens < W ? tokens : W);
  const bool replace = tail >= W;
  for (int e = threadIdx.x; e < E; e += kThreads) c[e] = replace ? 0 : lcount[e];
  __syncthreads();
  if (replace) {
    // window := the last W tokens, ring position r = token T - W + r
    for (int idx = threadIdx.x; idx < W * k; idx += kThreads) {
      const int r = idx / k, j = idx % k;
      const int64_t e = selected[(tokens - W + r) * k + j];
      lring[idx] = (int32_t)e;
      if (e >= 0 && e < E) atomicAdd(&c[e], 1);
    }
  } else {
    // append ring-wise; position (head + r) % W holds an old row iff r >= W - count
    for (int idx = threadIdx.x; idx < tail * k; idx += kThreads) {
      const int r = idx / k, j = idx % k;
      const int pos = (head + r) % W;
      if (r >= W - count) {
        const int32_t old = lring[pos * k + j];
        if (old >= 0 && old < E) atomicSub(&c[old], 1);
      }
      const int64_t e = selected[(tokens - tail + r) * k + j];
      lring[pos * k + j] = (int32_t)e;
      if (e >= 0 && e < E) atomicAdd(&c[e], 1);
    }
  }
  __syncthreads();
  const int new_count = replace ? W : (count + tail < W ? count + tail : W);
  const int n = new_count > 1 ? new_count : 1;
  for (int e = threadIdx.x; e < E; e += kThreads) {
    lcount[e] = c[e];
    scores_out[e] = (float)((double)c[e] / (double)n);
  }
  if (threadIdx.x == 0) {
    meta[layer * 2 + 0] = new_count;
    meta[layer * 2 + 1] = replace ? 0 : (head + tail) % W;
    if (timeouts_out)
      *timeouts_out = __hip_atomic_load(timeouts_src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace
}  // namespace ferry

using namespace ferry;

extern "C" int64_t ferry_history_ready_words(int64_t tokens, int64_t topk) {
  return tokens < 0 || topk < 1 ? -1 : 1 + ceil_div(tokens * topk, kIdsPerBlock);
}

extern "C" int ferry_history_update(const int64_t* selected, int64_t tokens, int64_t topk,
                                    int64_t experts, int64_t window, int64_t layer,
                                    int32_t* ring, int32_t* counts, int32_t* meta,
                                    float* scores_out, uint8_t* ids_out,
                                    int32_t* ffn_timeouts_out, int32_t* ready_out,
                                    int32_t ready_value, void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0 && topk >= 1 && layer >= 0, "bad sizes");
  FERRY_CHECK_ARG(experts >= 1 && experts <= kMaxE, "experts must be in [1, %d]", kMaxE);
  FERRY_CHECK_ARG(experts <= 255 || ids_out == nullptr, "uint8 IDs need experts <= 255");
  FERRY_CHECK_ARG(window >= 1 && window <= (1 << 20), "window must be in [1, 2^20]");
  FERRY_CHECK_ARG(ring && counts && meta && scores_out, "null pointer argument");
  FERRY_CHECK_ARG(tokens == 0 || selected, "null pointer argument");
  FERRY_CHECK_ARG(ready_out == nullptr || ids_out != nullptr, "ready_out needs ids_out");
  const int64_t nids = ids_out ? tokens * topk : 0;
  const int64_t grid = 1 + ceil_div(nids, kIdsPerBlock);
  FERRY_CHECK_ARG(grid < (1 << 30), "too many tokens");
  int32_t* timeouts_src = nullptr;
  if (ffn_timeouts_out) {
    const int rc = ffn_timeouts_address(&timeouts_src);
    if (rc != 0) return rc;
  }
  launch("history_kernel", history_kernel, dim3((unsigned)grid), dim3(kThreads), 0, (hipStream_t)stream,
                     selected, tokens, (int)topk, (int)experts, (int)window, layer, ring, counts,
                     meta, scores_out, ids_out, timeouts_src, ffn_timeouts_out, ready_out,
                     ready_value);
  FERRY_LAUNCHED("history_kernel");
  return 0;
}

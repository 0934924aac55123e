// Dispatch layout at world = 1: per-token ID sort, per-expert histogram, exclusive scan and a
// stable token permutation.
//
// Reference: ferry/layout.py:12-94.  At world = 1 every route is local, so build_layout
// reduces to: send_idx = arange(T); send_ids[t] = sorted(selected[t]) (insertion sort,
// :28-33); counts = histogram of send_ids; starts = exclusive prefix (:61-63); (rows, cols)
// = a stable counting sort of all (token, position) pairs by expert, tokens ascending within
// an expert (:64-74).  The packet weights of pack_dispatch (ferry/csrc/expert_ops.cpp:57-60)
// are the routing weights reordered into send_ids order.
//
// Design: tokens are processed in blocks of 1024 (16 wavefronts x 64 lanes, one token per
// lane).  Within a wavefront the rank of a token among the earlier tokens that chose the
// same expert is a popcount of a 64-bit per-expert lane mask built with LDS atomic ORs; the
// wavefront and block offsets come from exclusive scans.  No global atomics are used, so the
// permutation is deterministic.  A single block (T <= 1024) does everything in one launch;
// larger T uses count -> scan -> scatter launches.
#include "common.h"

#include <mutex>

namespace ferry {
namespace {

constexpr int kMaxE = 512;
constexpr int kMaxK = 16;
constexpr int kWaves = 16;
constexpr int kBlockTokens = 64 * kWaves;

struct TokenIds {
  int32_t id[kMaxK];
  bf16_t w[kMaxK];
};

// Load one token's k IDs and weights and sort them by ID (IDs of a token are distinct, so any
// sort gives the insertion-sort result); out-of-range entries carry the key kMaxE, padding
// entries kMaxE + 1.  `bad` is set for a token with an out-of-range or a repeated ID: such a
// token breaks the layout's contract (its entries would share one permutation slot).
__device__ __forceinline__ void load_sorted(const int64_t* __restrict__ selected,
                                            const bf16_t* __restrict__ weights, int64_t t, int k,
                                            int E, TokenIds& s, bool& bad) {
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) {
    if (j < k) {
      int64_t e = selected[t * k + j];
      bad |= (e < 0 || e >= E);
      s.id[j] = (e < 0 || e >= E) ? kMaxE : (int32_t)e;
      s.w[j] = weights ? weights[t * k + j] : (bf16_t)0;
    } else {
      s.id[j] = kMaxE + 1;
      s.w[j] = 0;
    }
  }
  // odd-even transposition sort over kMaxK slots (static indices keep it in registers)
#pragma unroll
  for (int r = 0; r < kMaxK; ++r) {
#pragma unroll
    for (int j = r & 1; j + 1 < kMaxK; j += 2) {
      if (s.id[j] > s.id[j + 1]) {
        int32_t ti = s.id[j];
        s.id[j] = s.id[j + 1];
        s.id[j + 1] = ti;
        bf16_t tw = s.w[j];
        s.w[j] = s.w[j + 1];
        s.w[j + 1] = tw;
      }
    }
  }
#pragma unroll
  for (int j = 0; j + 1 < kMaxK; ++j) bad |= (j + 1 < k && s.id[j] < E && s.id[j] == s.id[j + 1]);
}

struct LayoutShared {
  unsigned long long mask[kWaves][kMaxE];  // lanes of the wavefront that chose expert e
  int32_t wave_base[kWaves][kMaxE];        // exclusive prefix over wavefronts, per expert
};

// Phase 1 of a block: build the lane masks of its tokens and the per-wavefront prefix.
// Returns (in block_count[e], when non-null) the number of the block's tokens per expert.
__device__ void block_masks(LayoutShared& sh, const int64_t* __restrict__ selected,
                            const bf16_t* __restrict__ weights, int64_t tokens, int k, int E,
                            int64_t t0, TokenIds& s, bool& valid, bool& bad,
                            int32_t* block_count) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < kWaves * E; i += blockDim.x) sh.mask[i / E][i % E] = 0ull;
  __syncthreads();
  const int64_t t = t0 + threadIdx.x;
  valid = t < tokens;
  if (valid) {
    load_sorted(selected, weights, t, k, E, s, bad);
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
      if (j < k && s.id[j] < E) atomicOr(&sh.mask[wave][s.id[j]], 1ull << lane);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int32_t run = 0;
    for (int w = 0; w < kWaves; ++w) {
      sh.wave_base[w][e] = run;
      run += __popcll(sh.mask[w][e]);
    }
    if (block_count) block_count[e] = run;
  }
  __syncthreads();
}

// Phase 2 of a block: write the sorted IDs, packet weights and the permutation entries.
// base[e] = grouped position of the block's first entry of expert e.
__device__ void block_scatter(const LayoutShared& sh, const int32_t* base, int64_t t, int k,
                              const TokenIds& s, int64_t* __restrict__ send_ids,
                              bf16_t* __restrict__ w_sorted, int64_t* __restrict__ rows,
                              int64_t* __restrict__ cols, int32_t* __restrict__ pair_pos,
                              int E) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int j = 0; j < kMaxK; ++j) {
    if (j < k) {
      const int32_t e = s.id[j];
      send_ids[t * k + j] = e < E ? e : -1;
      if (w_sorted) w_sorted[t * k + j] = s.w[j];
      if (e < E) {
        const int64_t pos =
            (int64_t)base[e] + sh.wave_base[wave][e] + __popcll(sh.mask[wave][e] & below);
        rows[pos] = t;
        cols[pos] = j;
        if (pair_pos) pair_pos[t * k + j] = (int32_t)pos;
      } else if (pair_pos) {
        pair_pos[t * k + j] = -1;
      }
    }
  }
}

__global__ __launch_bounds__(kBlockTokens) void layout_single(
    const int64_t* __restrict__ selected, const bf16_t* __restrict__ weights, int64_t tokens,
    int k, int E, int64_t* __restrict__ send_ids, bf16_t* __restrict__ w_sorted,
    int64_t* __restrict__ starts, int64_t* __restrict__ rows, int64_t* __restrict__ cols,
    int32_t* __restrict__ pair_pos, int32_t* __restrict__ err) {
  __shared__ LayoutShared sh;
  __shared__ int32_t count[kMaxE];
  __shared__ int32_t base[kMaxE];
  TokenIds s;
  bool valid, bad = false;
  if (threadIdx.x == 0) *err = 0;  // ordered before the atomics by the barriers below
  block_masks(sh, selected, weights, tokens, k, E, 0, s, valid, bad, count);
  if (threadIdx.x == 0) {
    int32_t run = 0;
    for (int e = 0; e < E; ++e) {
      base[e] = run;
      starts[e] = run;
      run += count[e];
    }
    starts[E] = run;
  }
  __syncthreads();
  if (valid) {
    block_scatter(sh, base, threadIdx.x, k, s, send_ids, w_sorted, rows, cols, pair_pos, E);
    if (bad) atomicAdd(err, 1);
  }
}

__global__ __launch_bounds__(kBlockTokens) void layout_count(
    const int64_t* __restrict__ selected, int64_t tokens, int k, int E,
    int32_t* __restrict__ block_hist) {
  __shared__ LayoutShared sh;
  TokenIds s;
  bool valid, bad = false;
  block_masks(sh, selected, nullptr, tokens, k, E, (int64_t)blockIdx.x * kBlockTokens, s, valid,
              bad, block_hist + (int64_t)blockIdx.x * E);
}

// One block: per expert, exclusive prefix over blocks; starts = exclusive prefix of totals.
__global__ __launch_bounds__(kMaxE) void layout_scan(int32_t* __restrict__ block_hist, int nblk,
                                                     int E, int64_t* __restrict__ starts,
                                                     int32_t* __restrict__ err) {
  __shared__ int32_t total[kMaxE];
  const int e = threadIdx.x;
  if (e == 0) *err = 0;
  if (e < E) {
    int32_t run = 0;
    for (int b = 0; b < nblk; ++b) {
      const int32_t c = block_hist[(int64_t)b * E + e];
      block_hist[(int64_t)b * E + e] = run;
      run += c;
    }
    total[e] = run;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t run = 0;
    for (int i = 0; i < E; ++i) {
      starts[i] = run;
      run += total[i];
    }
    starts[E] = run;
  }
}

__global__ __launch_bounds__(kBlockTokens) void layout_scatter(
    const int64_t* __restrict__ selected, const bf16_t* __restrict__ weights, int64_t tokens,
    int k, int E, const int32_t* __restrict__ block_hist, const int64_t* __restrict__ starts,
    int64_t* __restrict__ send_ids, bf16_t* __restrict__ w_sorted, int64_t* __restrict__ rows,
    int64_t* __restrict__ cols, int32_t* __restrict__ pair_pos, int32_t* __restrict__ err) {
  __shared__ LayoutShared sh;
  __shared__ int32_t base[kMaxE];
  TokenIds s;
  bool valid, bad = false;
  const int64_t t0 = (int64_t)blockIdx.x * kBlockTokens;
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    base[e] = (int32_t)(starts[e] + block_hist[(int64_t)blockIdx.x * E + e]);
  block_masks(sh, selected, weights, tokens, k, E, t0, s, valid, bad, nullptr);
  if (valid) {
    block_scatter(sh, base, t0 + threadIdx.x, k, s, send_ids, w_sorted, rows, cols, pair_pos, E);
    if (bad) atomicAdd(err, 1);
  }
}

// The workspace of ferry_layout_noalloc: a file-scope device array instead of caller memory.
// Each GPU holds its own copy for the life of the process; its device address is looked up
// once per device (hipGetSymbolAddress) and only that address is handed to kernels.  Nothing in
// it needs clearing between calls: the error counter is zeroed by the layout kernels themselves
// and the per-block histograms are fully rewritten by every multi-block call.
constexpr int64_t kScratchBytes = 256 + 128 * (int64_t)kMaxE * (int64_t)sizeof(int32_t);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];  // device address of `scratch` on each device, or null

// Device address of `scratch` on the current device (resolved on first use per device).
int scratch_address(void** out) {
  int dev = -1;
  FERRY_HIP(hipGetDevice(&dev));
  FERRY_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    FERRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}

}  // namespace
}  // namespace ferry

using namespace ferry;

extern "C" int64_t ferry_layout_workspace_bytes(int64_t tokens, int64_t topk, int64_t experts) {
  (void)topk;
  const int64_t nblk = ceil_div(tokens > 0 ? tokens : 1, kBlockTokens);
  // error counter (256 B aligned) + per-block histograms
  return 256 + nblk * experts * (int64_t)sizeof(int32_t);
}

extern "C" int ferry_layout(const int64_t* selected, const void* weights_bf16, int64_t tokens,
                            int64_t topk, int64_t experts, int64_t* send_ids,
                            void* w_sorted_bf16, int64_t* starts, int64_t* rows, int64_t* cols,
                            int32_t* pair_pos, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0, "tokens must be >= 0");
  FERRY_CHECK_ARG(experts >= 1 && experts <= kMaxE, "experts must be in [1, %d]", kMaxE);
  FERRY_CHECK_ARG(topk >= 1 && topk <= kMaxK && topk <= experts,
                  "topk must be in [1, min(experts, %d)]", kMaxK);
  FERRY_CHECK_ARG(tokens * topk < (int64_t)1 << 31, "tokens*topk must be < 2^31");
  FERRY_CHECK_ARG(starts && workspace, "null pointer argument");
  FERRY_CHECK_ARG(workspace_bytes >= ferry_layout_workspace_bytes(tokens, topk, experts),
                  "workspace too small (%lld < %lld bytes)", (long long)workspace_bytes,
                  (long long)ferry_layout_workspace_bytes(tokens, topk, experts));
  FERRY_CHECK_ARG(tokens == 0 || (selected && send_ids && rows && cols), "null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  int32_t* err = (int32_t*)workspace;
  int32_t* hist = (int32_t*)((char*)workspace + 256);
  const int k = (int)topk, E = (int)experts;
  const bf16_t* w = (const bf16_t*)weights_bf16;
  bf16_t* ws = (bf16_t*)w_sorted_bf16;
  if (tokens <= kBlockTokens) {
    launch("layout_single", layout_single, dim3(1), dim3(kBlockTokens), 0, s, selected, w, tokens, k,
                       E, send_ids, ws, starts, rows, cols, pair_pos, err);
    FERRY_LAUNCHED("layout_single");
    return 0;
  }
  const int nblk = (int)ceil_div(tokens, kBlockTokens);
  launch("layout_count", layout_count, dim3(nblk), dim3(kBlockTokens), 0, s, selected, tokens, k, E,
                     hist);
  FERRY_LAUNCHED("layout_count");
  launch("layout_scan", layout_scan, dim3(1), dim3(kMaxE), 0, s, hist, nblk, E, starts, err);
  FERRY_LAUNCHED("layout_scan");
  launch("layout_scatter", layout_scatter, dim3(nblk), dim3(kBlockTokens), 0, s, selected, w, tokens, k,
                     E, hist, starts, send_ids, ws, rows, cols, pair_pos, err);
  FERRY_LAUNCHED("layout_scatter");
  return 0;
}

extern "C" int ferry_layout_noalloc(const int64_t* selected, const void* weights_bf16,
                                    int64_t tokens, int64_t topk, int64_t experts,
                                    int64_t* send_ids, void* w_sorted_bf16, int64_t* starts,
                                    int64_t* rows, int64_t* cols, int32_t* pair_pos,
                                    void* stream) {
  clear_error();
  FERRY_CHECK_ARG(tokens >= 0, "tokens must be >= 0");
  FERRY_CHECK_ARG(experts >= 1 && experts <= kMaxE, "experts must be in [1, %d]", kMaxE);
  const int64_t need = ferry_layout_workspace_bytes(tokens, topk, experts);
  FERRY_CHECK_ARG(need <= kScratchBytes,
                  "layout_noalloc: %lld tokens x %lld experts need %lld scratch bytes, the static "
                  "buffer holds %lld (at most %lld tokens at this expert count)",
                  (long long)tokens, (long long)experts, (long long)need, (long long)kScratchBytes,
                  (long long)((kScratchBytes - 256) / (experts * (int64_t)sizeof(int32_t)) *
                              kBlockTokens));
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != 0) return rc;
  return ferry_layout(selected, weights_bf16, tokens, topk, experts, send_ids, w_sorted_bf16,
                      starts, rows, cols, pair_pos, ws, kScratchBytes, stream);
}

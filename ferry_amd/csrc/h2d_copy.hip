// Copy kernel of the H2D fetch engine: expert rows of the pinned host pool -> cache slots.
//
// A fetch of m rows as m hipMemcpyAsync calls leaves the host link idle between copies
// (measured on MI355X with decode-sized fetches of 6 rows of 9 MiB over two DMA streams:
// 54.6 GB/s, against 57.0 GB/s for one launch of this kernel).  The kernel reads the pool over
// PCIe through its device mapping and writes the slots in HBM; one launch moves a whole fetch
// call.  32 workgroups of 256 threads, each thread keeping four 16-byte loads in flight, carry
// about 512 KiB of reads in flight, which is enough to cover the link's latency; more
// workgroups measured no faster.  The kernel uses no LDS and few registers, so it shares CUs
// with the compute kernels that run while it copies.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "pack_format.h"

namespace ferry {

constexpr int kCopyRows = 128;     // rows per launch (kernel argument list)
constexpr int kCopyGroups = 32;    // workgroups per launch

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct CopyList {
  int32_t key[kCopyRows];   // pool row
  int32_t slot[kCopyRows];  // cache row
  int32_t n;
};

namespace {

__global__ __launch_bounds__(256) void h2d_copy_kernel(const u32x4* __restrict__ pool,
                                                       u32x4* __restrict__ cache, int64_t units,
                                                       CopyList list) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int r = 0; r < list.n; ++r) {
    const u32x4* src = pool + (int64_t)list.key[r] * units;
    u32x4* dst = cache + (int64_t)list.slot[r] * units;
    int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; u + 3 * stride < units; u += 4 * stride) {
      const u32x4 v0 = src[u], v1 = src[u + stride], v2 = src[u + 2 * stride],
                  v3 = src[u + 3 * stride];
      dst[u] = v0;
      dst[u + stride] = v1;
      dst[u + 2 * stride] = v2;
      dst[u + 3 * stride] = v3;
    }
    for (; u < units; u += stride) dst[u] = src[u];
  }
}

// Unpacks packed rows (pack_format.h) from the staging buffers into cache slots.  A workgroup
// of 256 threads decodes one block of 8192 values: a thread turns 32 values (32 bytes of the
// sign | mantissa plane, 4 bytes of each code plane) into 64 bytes of bf16.  The block's slice
// of the level-2 codes and of the third-level list is staged in LDS; a block-wide prefix sum of
// the threads' escape counts gives each escape its rank in that slice.
constexpr int kUnpackThreads = 256;
constexpr int kL3Lds = 256;   // third-level entries of a block staged in LDS (more: global search)

__device__ __forceinline__ uint32_t level3_global(const uint32_t* idx, const uint8_t* ex, int64_t lo,
                                                  int64_t hi, uint32_t i) {
  while (hi - lo > 1) {   // idx[lo] <= i < idx[hi], as the entry for i is in [lo, hi)
    const int64_t mid = (lo + hi) >> 1;
    if (idx[mid] <= i) lo = mid; else hi = mid;
  }
  return ex[lo];
}

struct UnpackLds {
  uint8_t c[kPackBlock / 2 + 16];
  uint16_t li[kL3Lds];
  uint8_t le[kL3Lds];
  uint32_t wave[kUnpackThreads / 64];
};

// block blk of row r of the list
__device__ __forceinline__ void unpack_block(const UnpackList& list, int64_t n, int r, int64_t blk,
                                             UnpackLds& lds) {
  uint8_t* lds_c = lds.c;
  uint16_t* lds_li = lds.li;
  uint8_t* lds_le = lds.le;
  uint32_t* lds_wave = lds.wave;
  const int t = threadIdx.x;
  const uint8_t* src = list.src[r];
  if (list.raw[r]) {   // a row kept raw: the workgroup copies its block's 16 KiB as they are
    const int64_t v = blk * kPackBlock + 32 * t;
    if (v < n) {
      const u32x4* s = reinterpret_cast<const u32x4*>(src + 2 * v);
      u32x4* d = reinterpret_cast<u32x4*>(list.dst[r] + v);
      const u32x4 x0 = s[0], x1 = s[1], x2 = s[2], x3 = s[3];
      d[0] = x0;
      d[1] = x1;
      d[2] = x2;
      d[3] = x3;
    }
    return;
  }
  const PackHeader* hd = reinterpret_cast<const PackHeader*>(src);
  const uint32_t base1 = hd->base1, base2 = hd->base2;
  const PackOffsets o = pack_offsets(n, (int64_t)hd->esc1, (int64_t)hd->esc2);
  const uint32_t* pre = reinterpret_cast<const uint32_t*>(src + o.p);
  const uint32_t e_lo = pre[2 * blk], e_hi = pre[2 * blk + 2];
  const uint32_t l_lo = pre[2 * blk + 1], l_hi = pre[2 * blk + 3];
  const uint32_t* lidx = reinterpret_cast<const uint32_t*>(src + o.l_idx);
  const uint8_t* lexp = src + o.l_exp;
  // the block's level-2 nibbles [e_lo, e_hi) lie in bytes [e_lo / 2, (e_hi + 1) / 2)
  const int c_bytes = (int)(((e_hi + 1) >> 1) - (e_lo >> 1));
  for (int i = t; i < c_bytes; i += kUnpackThreads) lds_c[i] = src[o.c + (e_lo >> 1) + i];
  const int l_cnt = (int)(l_hi - l_lo);
  if (l_cnt <= kL3Lds)
    for (int i = t; i < l_cnt; i += kUnpackThreads) {
      lds_li[i] = (uint16_t)(lidx[l_lo + i] - (uint32_t)(blk * kPackBlock));
      lds_le[i] = lexp[l_lo + i];
    }
  const int64_t v0 = blk * kPackBlock + 32 * t;
  const bool active = v0 < n;   // n is a multiple of 32: a thread has 32 values or none
  u32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
  uint32_t p0 = 0, p1 = 0, p2 = 0;
  if (active) {
    const u32x4* pa = reinterpret_cast<const u32x4*>(src + o.a + v0);
    a0 = pa[0];
    a1 = pa[1];
    p0 = *reinterpret_cast<const uint32_t*>(src + o.b0 + v0 / 8);
    p1 = *reinterpret_cast<const uint32_t*>(src + o.b1 + v0 / 8);
    p2 = *reinterpret_cast<const uint32_t*>(src + o.b2 + v0 / 8);
  }
  const uint32_t esc = p0 & p1 & p2;   // code 7
  // block-wide exclusive prefix sum of the escape counts
  const uint32_t cnt = (uint32_t)__popc(esc);
  const int lane = t & 63, wave = t >> 6;
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) lds_wave[wave] = incl;
  __syncthreads();   // also publishes the staged nibbles and third-level entries
  uint32_t rank = incl - cnt;
  for (int w = 0; w < wave; ++w) rank += lds_wave[w];
  if (!active) return;
  const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  uint32_t w[16];
#pragma unroll
  for (int h = 0; h < 16; ++h) {
    uint32_t pair = 0;
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int q = 2 * h + q2;
      const uint32_t b = (a[q >> 2] >> (8 * (q & 3))) & 0xFFu;
      const uint32_t c = ((p0 >> q) & 1u) | (((p1 >> q) & 1u) << 1) | (((p2 >> q) & 1u) << 2);
      const uint32_t e = c == (uint32_t)kPackWindow1 ? 0u : base1 + c;   // escapes: filled below
      pair |= (((b & 0x80u) << 8) | (e << 7) | (b & 0x7Fu)) << (16 * q2);
    }
    w[h] = pair;
  }
  // escapes, in value order: level-2 code from LDS, or the third-level list
  const uint32_t nib0 = (e_lo & 1u) + rank;
  for (uint32_t m = esc, k = 0; m != 0; m &= m - 1, ++k) {
    const int q = __builtin_ctz(m);
    const uint32_t nib = nib0 + k;
    const uint32_t c2 = (lds_c[nib >> 1] >> (4 * (nib & 1u))) & 0xFu;
    uint32_t e;
    if (c2 < (uint32_t)kPackWindow2) {
      e = base2 + c2;
    } else {
      const uint32_t li = (uint32_t)(32 * t + q);   // index within the block
      if (l_cnt <= kL3Lds) {
        int j = 0;
        while (j + 1 < l_cnt && lds_li[j] != li) ++j;
        e = lds_le[j];
      } else {
        e = level3_global(lidx, lexp, l_lo, l_hi, (uint32_t)(blk * kPackBlock) + li);
      }
    }
    const uint32_t bits = e << (7 + 16 * (q & 1));
#pragma unroll
    for (int h = 0; h < 16; ++h) w[h] |= (h == (q >> 1)) ? bits : 0u;
  }
  u32x4* dst = reinterpret_cast<u32x4*>(list.dst[r] + v0);
#pragma unroll
  for (int h = 0; h < 4; ++h) dst[h] = u32x4{w[4 * h], w[4 * h + 1], w[4 * h + 2], w[4 * h + 3]};
}

// Workgroup g takes blocks g, g + G, g + 2G, ... (G = gridDim.x) of the list's rows in row
// order.  With one workgroup per block (staging buffers in HBM) every block is dispatched at
// once; a packed pool read over the link is served by a few hundred workgroups that loop,
// which leaves the CUs' other slots to kernels running beside the fetch.
__global__ __launch_bounds__(kUnpackThreads) void unpack_kernel(UnpackList list, int64_t n) {
  __shared__ UnpackLds lds;
  const int64_t blocks = (n + kPackBlock - 1) / kPackBlock;
  const int64_t items = blocks * list.n_rows;
  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int r = (int)(it / blocks);
    unpack_block(list, n, r, it - r * blocks, lds);
    __syncthreads();   // the next block rewrites the LDS slices
  }
}

}  // namespace

// Unpacks list.n_rows packed rows of n values each (n a multiple of 32), on `stream`, with at
// most max_groups workgroups (0: one per block).
hipError_t h2d_unpack_launch(const UnpackList& list, int64_t n, hipStream_t stream,
                             int64_t max_groups) {
  if (list.n_rows <= 0) return hipSuccess;
  const int64_t items = (n + kPackBlock - 1) / kPackBlock * list.n_rows;
  const int64_t groups = max_groups > 0 && max_groups < items ? max_groups : items;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)groups), dim3(kUnpackThreads), 0, stream, list,
                     n);
  return hipGetLastError();
}

// Copies rows keys[i] of `pool` (device address of the mapped host pool) into rows slots[i] of
// `cache`, rows of row_bytes (a multiple of 16, both bases 16-byte aligned), on `stream`.  The
// caller has checked the indices.  Returns the launch status.
hipError_t h2d_copy_launch(const void* pool, void* cache, int64_t row_bytes, const int64_t* keys,
                           const int64_t* slots, int64_t n, hipStream_t stream) {
  for (int64_t b = 0; b < n; b += kCopyRows) {
    CopyList list;
    list.n = (int32_t)(n - b < kCopyRows ? n - b : kCopyRows);
    for (int i = 0; i < list.n; ++i) {
      list.key[i] = (int32_t)keys[b + i];
      list.slot[i] = (int32_t)slots[b + i];
    }
    hipLaunchKernelGGL(h2d_copy_kernel, dim3(kCopyGroups), dim3(256), 0, stream,
                       (const u32x4*)pool, (u32x4*)cache, row_bytes / 16, list);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace ferry

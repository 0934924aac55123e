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

// Unpacks packed rows (pack_format.h) into cache slots.  A workgroup of 256 threads decodes one
// block of 8192 values: a thread turns 32 values (32 bytes of the sign | mantissa plane, 4 bytes
// of each code plane) into 64 bytes of bf16.  The block's slices of the level-2 and level-3 code
// streams and of the list are staged in LDS; a block-wide prefix sum of the threads' level-1
// escapes gives each its position in the level-2 slice, and a second one, of the level-2 escapes
// the threads then find there, their positions in the level-3 slice.
constexpr int kUnpackThreads = 256;
constexpr int kListLds = 256;   // list entries of a block staged in LDS (more: global search)

__device__ __forceinline__ uint32_t list_global(const uint32_t* idx, const uint8_t* ex, int64_t lo,
                                                int64_t hi, uint32_t i) {
  while (hi - lo > 1) {   // idx[lo] <= i < idx[hi], as the entry for i is in [lo, hi)
    const int64_t mid = (lo + hi) >> 1;
    if (idx[mid] <= i) lo = mid; else hi = mid;
  }
  return ex[lo];
}

constexpr int kEscStride = 9;   // words per thread in UnpackLds::esc (8 + 1 against bank conflicts)

struct UnpackLds {
  uint32_t c2[kPackBlock / 16 + 4];   // level-2 code words of the block (16 codes a word)
  uint32_t c3[kPackBlock / 8 + 8];    // level-3 code words (8 codes a word)
  uint16_t li[kListLds];
  uint8_t le[kListLds];
  uint32_t wave[2][kUnpackThreads / 64];
  uint32_t esc[kUnpackThreads * kEscStride];   // per thread: its escapes' exponents, byte q = value q
};

// exclusive block-wide prefix sum of cnt over the workgroup's threads (all of them call it);
// its barrier also publishes the LDS writes made before it
__device__ __forceinline__ uint32_t block_rank(uint32_t cnt, uint32_t* wave_total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t incl = cnt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t y = __shfl_up(incl, d, 64);
    if (lane >= d) incl += y;
  }
  if (lane == 63) wave_total[wave] = incl;
  __syncthreads();
  uint32_t rank = incl - cnt;
  for (int w = 0; w < wave; ++w) rank += wave_total[w];
  return rank;
}

__device__ __forceinline__ uint32_t pick3(uint32_t c, uint32_t x0, uint32_t x1, uint32_t x2) {
  return c == 0 ? x0 : (c == 1 ? x1 : x2);
}

// block blk of row r of the list
__device__ __forceinline__ void unpack_block(const UnpackList& list, int64_t n, int r, int64_t blk,
                                             UnpackLds& lds) {
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
  // the planes of this thread's 32 values (their offsets do not depend on the header)
  const int64_t v0 = blk * kPackBlock + 32 * t;
  const bool active = v0 < n;   // n is a multiple of 32: a thread has 32 values or none
  u32x4 a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
  uint32_t p0 = 0, p1 = 0;
  if (active) {
    const u32x4* pa = reinterpret_cast<const u32x4*>(src + kPackHeaderBytes + v0);
    a0 = pa[0];
    a1 = pa[1];
    p0 = *reinterpret_cast<const uint32_t*>(src + kPackHeaderBytes + n + v0 / 8);
    p1 = *reinterpret_cast<const uint32_t*>(src + kPackHeaderBytes + n + n / 8 + v0 / 8);
  }
  const PackHeader* hd = reinterpret_cast<const PackHeader*>(src);
  const uint32_t t10 = hd->t1[0], t11 = hd->t1[1], t12 = hd->t1[2];
  const uint32_t t20 = hd->t2[0], t21 = hd->t2[1], t22 = hd->t2[2];
  const uint32_t base3 = hd->base3;
  const PackOffsets o =
      pack_offsets(n, (int64_t)hd->esc1, (int64_t)hd->esc2, (int64_t)hd->esc3);
  const uint32_t* pre = reinterpret_cast<const uint32_t*>(src + o.p) + 3 * blk;
  const uint32_t e1_lo = pre[0], e2_lo = pre[1], e3_lo = pre[2];
  const uint32_t e1_hi = pre[3], e2_hi = pre[4], e3_hi = pre[5];
  // the block's code words and list entries
  const uint32_t* c2g = reinterpret_cast<const uint32_t*>(src + o.c2);
  const uint32_t* c3g = reinterpret_cast<const uint32_t*>(src + o.c3);
  const int w2 = (int)(((e1_hi + 15) >> 4) - (e1_lo >> 4));
  for (int i = t; i < w2; i += kUnpackThreads) lds.c2[i] = c2g[(e1_lo >> 4) + i];
  const int w3 = (int)(((e2_hi + 7) >> 3) - (e2_lo >> 3));
  for (int i = t; i < w3; i += kUnpackThreads) lds.c3[i] = c3g[(e2_lo >> 3) + i];
  const uint32_t* lidx = reinterpret_cast<const uint32_t*>(src + o.l_idx);
  const uint8_t* lexp = src + o.l_exp;
  const int l_cnt = (int)(e3_hi - e3_lo);
  if (l_cnt <= kListLds)
    for (int i = t; i < l_cnt; i += kUnpackThreads) {
      lds.li[i] = (uint16_t)(lidx[e3_lo + i] - (uint32_t)(blk * kPackBlock));
      lds.le[i] = lexp[e3_lo + i];
    }
  const uint32_t m1 = p0 & p1;   // level-1 code 3
  const uint32_t cnt1 = (uint32_t)__popc(m1);
  const uint32_t rank1 = block_rank(cnt1, lds.wave[0]);   // also publishes the staged slices
  // the level-2 codes of this thread's escapes: 2-bit codes (e1_lo % 16) + rank1 ... of the slice
  uint64_t codes2 = 0;
  if (cnt1) {
    const uint32_t bit0 = 2 * ((e1_lo & 15) + rank1);
    const uint32_t w = bit0 >> 5, sh = bit0 & 31;
    codes2 = ((uint64_t)lds.c2[w] | ((uint64_t)lds.c2[w + 1] << 32)) >> sh;
    if (sh) codes2 |= (uint64_t)lds.c2[w + 2] << (64 - sh);
    if (cnt1 < 32) codes2 &= (1ull << (2 * cnt1)) - 1;
  }
  const uint32_t cnt2 = (uint32_t)__popcll(codes2 & (codes2 >> 1) & 0x5555555555555555ull);
  const uint32_t rank2 = block_rank(cnt2, lds.wave[1]);
  if (!active) return;
  // escapes, in value order (level-2 table, else the level-3 window, else the list): their
  // exponents go to this thread's bytes of lds.esc, which start cleared
  uint32_t* esc = lds.esc + t * kEscStride;
  if (m1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) esc[i] = 0;
    uint8_t* escb = reinterpret_cast<uint8_t*>(esc);
    uint32_t pos3 = (e2_lo & 7) + rank2;   // this thread's next level-3 code in the slice
    for (uint32_t m = m1, k = 0; m != 0; m &= m - 1, ++k) {
      const int q = __builtin_ctz(m);
      const uint32_t c2 = (uint32_t)(codes2 >> (2 * k)) & 3u;
      uint32_t e;
      if (c2 < (uint32_t)kPackTable) {
        e = pick3(c2, t20, t21, t22);
      } else {
        const uint32_t c3 = (lds.c3[pos3 >> 3] >> (4 * (pos3 & 7))) & 0xFu;
        ++pos3;
        if (c3 < (uint32_t)kPackWindow3) {
          e = base3 + c3;
        } else {
          const uint32_t li = (uint32_t)(32 * t + q);   // index within the block
          if (l_cnt <= kListLds) {
            int j = 0;
            while (j + 1 < l_cnt && lds.li[j] != li) ++j;
            e = lds.le[j];
          } else {
            e = list_global(lidx, lexp, e3_lo, e3_hi, (uint32_t)(blk * kPackBlock) + li);
          }
        }
      }
      escb[q] = (uint8_t)e;
    }
  }
  const uint32_t a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
  // code 3 reads 0 from the table word, and the escape bytes are 0 for the other values
  const uint32_t lut1 = t10 | (t11 << 8) | (t12 << 16);
  uint32_t ew[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (m1) {
#pragma unroll
    for (int i = 0; i < 8; ++i) ew[i] = esc[i];
  }
  uint32_t w[16];
#pragma unroll
  for (int h = 0; h < 16; ++h) {
    uint32_t pair = 0;
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
      const int q = 2 * h + q2;
      const uint32_t b = (a[q >> 2] >> (8 * (q & 3))) & 0xFFu;
      const uint32_t c = ((p0 >> q) & 1u) | (((p1 >> q) & 1u) << 1);
      const uint32_t e = __builtin_amdgcn_ubfe(lut1, 8 * c, 8) | ((ew[q >> 2] >> (8 * (q & 3))) & 0xFFu);
      pair |= (((b & 0x80u) << 8) | (e << 7) | (b & 0x7Fu)) << (16 * q2);
    }
    w[h] = pair;
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

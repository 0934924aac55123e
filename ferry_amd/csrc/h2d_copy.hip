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

// Unpacks packed rows (pack_format.h) from the staging buffers into cache slots: a thread turns
// 8 values (8 bytes of plane A, 4 of plane B) into 16 bytes of bf16; an escape code looks its
// exponent up by binary search in the row's escape list.
__device__ __forceinline__ uint32_t escape_exponent(const uint32_t* idx, const uint8_t* ex,
                                                    int64_t count, uint32_t i) {
  int64_t lo = 0, hi = count;  // idx[lo .. hi) may hold i
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (idx[mid] <= i) lo = mid; else hi = mid;
  }
  return (count > 0 && idx[lo] == i) ? ex[lo] : 0u;
}

__global__ __launch_bounds__(256) void unpack_kernel(UnpackList list, int64_t n) {
  const int r = blockIdx.y;
  const uint8_t* src = list.src[r];
  const PackHeader* hd = reinterpret_cast<const PackHeader*>(src);
  const uint32_t base = hd->base;
  const int64_t esc = (int64_t)hd->escapes;
  const uint64_t* pa = reinterpret_cast<const uint64_t*>(src + kPackHeaderBytes);
  const uint32_t* pb = reinterpret_cast<const uint32_t*>(src + kPackHeaderBytes + n);
  const uint32_t* eidx = reinterpret_cast<const uint32_t*>(src + kPackHeaderBytes + n + n / 2);
  const uint8_t* eexp = reinterpret_cast<const uint8_t*>(eidx + esc);
  u32x4* dst = reinterpret_cast<u32x4*>(list.dst[r]);
  const int64_t groups = n / 8;
  for (int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x; g < groups;
       g += (int64_t)gridDim.x * 256) {
    const uint64_t A = pa[g];
    const uint32_t B = pb[g];
    uint32_t w[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      uint32_t pair = 0;
#pragma unroll
      for (int q2 = 0; q2 < 2; ++q2) {
        const int q = 2 * h + q2;
        const uint32_t a = (uint32_t)(A >> (8 * q)) & 0xFFu;
        const uint32_t c = (B >> (4 * q)) & 0xFu;
        uint32_t e = base + c;
        if (c == (uint32_t)kPackWindow) e = escape_exponent(eidx, eexp, esc, (uint32_t)(8 * g + q));
        const uint32_t v = ((a & 0x80u) << 8) | (e << 7) | (a & 0x7Fu);
        pair |= v << (16 * q2);
      }
      w[h] = pair;
    }
    dst[g] = u32x4{w[0], w[1], w[2], w[3]};
  }
}

}  // namespace

// Unpacks list.n_rows packed rows of n values each, on `stream`.
hipError_t h2d_unpack_launch(const UnpackList& list, int64_t n, hipStream_t stream) {
  if (list.n_rows <= 0) return hipSuccess;
  const int64_t blocks = (n / 8 + 255) / 256;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)(blocks < 2048 ? blocks : 2048),
                                         (unsigned)list.n_rows),
                     dim3(256), 0, stream, list, n);
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

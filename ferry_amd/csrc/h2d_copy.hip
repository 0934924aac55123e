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

}  // namespace

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

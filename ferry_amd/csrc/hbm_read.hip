// A plain read of device memory at the rate this device's HBM allows: the measured ceiling that
// the memory-bound kernels' rooflines are read against (a measurement aid; it has no reference
// counterpart).  Workgroups of 256 threads each read one 32 KiB span once: every wavefront issues
// its eight 1 KiB loads (64 lanes x 16 B, contiguous) before the first wait, folds them with XOR,
// reduces the wavefront with lane shuffles and stores the result, 16 bytes per wavefront, so that
// the loads cannot be dropped and the caller can check what was read (one atomic word for all
// wavefronts serialises them: 0.18 TB/s).  Of the decompositions measured (one-shot workgroups
// of 32-256 KiB, grid-stride loops over 936-2048 workgroups), this one read cold data fastest.
#include "common.h"

namespace ferry {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadLoads = 8;                        // per lane, all in flight
constexpr int64_t kReadSpan = 256 * kReadLoads;      // 16-byte units per workgroup (32 KiB)

__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                       u32x4* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t base = (int64_t)blockIdx.x * kReadSpan + (threadIdx.x >> 6) * (64 * kReadLoads) + lane;
  u32x4 v[kReadLoads];
#pragma unroll
  for (int i = 0; i < kReadLoads; ++i) {
    const int64_t at = base + 64 * i;
    v[i] = at < n16 ? p[at] : u32x4{0, 0, 0, 0};
  }
  u32x4 acc = v[0];
#pragma unroll
  for (int i = 1; i < kReadLoads; ++i) acc ^= v[i];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    acc.x ^= __shfl_xor(acc.x, off, 64);
    acc.y ^= __shfl_xor(acc.y, off, 64);
    acc.z ^= __shfl_xor(acc.z, off, 64);
    acc.w ^= __shfl_xor(acc.w, off, 64);
  }
  if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = acc;
}

}  // namespace
}  // namespace ferry

using namespace ferry;

extern "C" int64_t ferry_hbm_read_sink_bytes(int64_t bytes) {
  return bytes > 0 ? 16 * 4 * ceil_div(ceil_div(bytes, 16), kReadSpan) : 0;
}

extern "C" int ferry_hbm_read(const void* data, int64_t bytes, void* sink, int64_t sink_bytes,
                              void* stream) {
  clear_error();
  FERRY_CHECK_ARG(bytes >= 0 && bytes % 16 == 0, "bytes must be a non-negative multiple of 16");
  FERRY_CHECK_ARG(bytes == 0 || (data && sink), "null pointer argument");
  FERRY_CHECK_ARG((uintptr_t)data % 16 == 0 && (uintptr_t)sink % 16 == 0,
                  "data and sink must be 16-byte aligned");
  FERRY_CHECK_ARG(sink_bytes >= ferry_hbm_read_sink_bytes(bytes),
                  "sink holds %lld bytes, %lld needed", (long long)sink_bytes,
                  (long long)ferry_hbm_read_sink_bytes(bytes));
  if (bytes == 0) return 0;
  const int64_t n16 = bytes / 16;
  const int64_t grid = ceil_div(n16, kReadSpan);
  FERRY_CHECK_ARG(grid < ((int64_t)1 << 31), "too many bytes");
  launch("hbm_read_kernel", hbm_read_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
         (const u32x4*)data, n16, (u32x4*)sink);
  FERRY_LAUNCHED("hbm_read_kernel");
  return 0;
}

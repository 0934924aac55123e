// Shared helpers of the ferry_amd HIP library (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/ferry_amd.h"

namespace ferry {

// Thread-local last-error message, returned by ferry_last_error().
void set_error(const char* fmt, ...);
void clear_error();

#define FERRY_CHECK_ARG(cond, ...)        \
  do {                                    \
    if (!(cond)) {                        \
      ::ferry::set_error(__VA_ARGS__);    \
      return 2;                           \
    }                                     \
  } while (0)

#define FERRY_HIP(expr)                                                                   \
  do {                                                                                    \
    hipError_t _e = (expr);                                                               \
    if (_e != hipSuccess) {                                                               \
      ::ferry::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e), __FILE__, \
                         __LINE__);                                                       \
      return 3;                                                                           \
    }                                                                                     \
  } while (0)

// Launch-error check after a <<<>>> launch.
#define FERRY_LAUNCHED(name)                                                               \
  do {                                                                                     \
    hipError_t _e = hipGetLastError();                                                     \
    if (_e != hipSuccess) {                                                                \
      ::ferry::set_error("launch of %s failed: %s", name, hipGetErrorString(_e));          \
      return 3;                                                                            \
    }                                                                                      \
  } while (0)

typedef uint16_t bf16_t;  // raw bf16 bits

__host__ __device__ inline float bf16_to_f32(bf16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet), as torch's c10::BFloat16(float).
// On the device this is the hardware conversion (v_cvt_pk_bf16_f32), which rounds the same way.
__host__ __device__ inline bf16_t f32_to_bf16(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(bf16_t, (__bf16)f);
#else
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
#endif
}

// the float value of v rounded to bf16
__host__ __device__ inline float bf16r(float v) { return bf16_to_f32(f32_to_bf16(v)); }

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Per-launch kernel timing (ferry_timing_enable): when on, kernels are launched with
// hipExtLaunchKernel and a start/stop event pair that brackets exactly that dispatch.
bool timing_enabled();
void timing_events(const char* name, hipEvent_t* start, hipEvent_t* stop);

template <typename K, typename... Args>
inline void launch(const char* name, K kernel, dim3 grid, dim3 block, uint32_t shmem,
                   hipStream_t stream, Args... args) {
  if (timing_enabled()) {
    hipEvent_t a = nullptr, b = nullptr;
    timing_events(name, &a, &b);
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, stream, a, b, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
  }
}

}  // namespace ferry

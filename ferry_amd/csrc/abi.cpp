// Error reporting and version of the ferry_amd C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ferry_amd.h"

namespace ferry {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

namespace {
struct TimedLaunch {
  const char* name;
  hipEvent_t start, stop;
};
std::mutex g_timing_mu;
bool g_timing = false;
std::vector<TimedLaunch> g_launches;

void release_launches() {
  for (auto& l : g_launches) {
    (void)hipEventDestroy(l.start);
    (void)hipEventDestroy(l.stop);
  }
  g_launches.clear();
}
}  // namespace

bool timing_enabled() { return g_timing; }

void timing_events(const char* name, hipEvent_t* start, hipEvent_t* stop) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (hipEventCreate(start) != hipSuccess || hipEventCreate(stop) != hipSuccess) {
    *start = *stop = nullptr;  // launch untimed
    return;
  }
  g_launches.push_back(TimedLaunch{name, *start, *stop});
}

}  // namespace ferry

// Turn per-launch kernel timing on (clearing earlier records) or off.
extern "C" int ferry_timing_enable(int32_t enable) {
  std::lock_guard<std::mutex> lock(ferry::g_timing_mu);
  ferry::release_launches();
  ferry::g_timing = enable != 0;
  return 0;
}

// Number of timed launches of `kernel` and their summed duration in ms (waits for them).
extern "C" int ferry_timing_summary(const char* kernel, int64_t* launches, double* total_ms) {
  std::lock_guard<std::mutex> lock(ferry::g_timing_mu);
  int64_t n = 0;
  double ms = 0.0;
  for (auto& l : ferry::g_launches) {
    if (std::strcmp(l.name, kernel) != 0) continue;
    if (hipEventSynchronize(l.stop) != hipSuccess) return 3;
    float t = 0.f;
    if (hipEventElapsedTime(&t, l.start, l.stop) != hipSuccess) return 3;
    ms += t;
    ++n;
  }
  *launches = n;
  *total_ms = ms;
  return 0;
}

// Number of launches recorded so far: a position in the timing log.
extern "C" int64_t ferry_timing_mark(void) {
  std::lock_guard<std::mutex> lock(ferry::g_timing_mu);
  return (int64_t)ferry::g_launches.size();
}

// Summed duration in ms of the timed launches at log positions [begin, end) (waits for them).
extern "C" int ferry_timing_range(int64_t begin, int64_t end, double* total_ms) {
  std::lock_guard<std::mutex> lock(ferry::g_timing_mu);
  const int64_t n = (int64_t)ferry::g_launches.size();
  double ms = 0.0;
  for (int64_t i = begin < 0 ? 0 : begin; i < end && i < n; ++i) {
    const auto& l = ferry::g_launches[(size_t)i];
    if (hipEventSynchronize(l.stop) != hipSuccess) return 3;
    float t = 0.f;
    if (hipEventElapsedTime(&t, l.start, l.stop) != hipSuccess) return 3;
    ms += t;
  }
  *total_ms = ms;
  return 0;
}

// Summed overlap in ms of the timed launches at log positions [begin, end) with the window
// between two caller events t0 and t1 (timing-enabled hipEvent_t, on any stream): for each
// launch, the length of [start, stop] inside [t0, t1].  Launches of one stream do not overlap
// each other, so for one stream this is the time the window was covered by its kernels.
extern "C" int ferry_timing_overlap(int64_t begin, int64_t end, void* t0, void* t1,
                                    double* total_ms) {
  std::lock_guard<std::mutex> lock(ferry::g_timing_mu);
  hipEvent_t a = (hipEvent_t)t0, b = (hipEvent_t)t1;
  if (hipEventSynchronize(b) != hipSuccess) return 3;
  float win = 0.f;
  if (hipEventElapsedTime(&win, a, b) != hipSuccess) return 3;
  const int64_t n = (int64_t)ferry::g_launches.size();
  double ms = 0.0;
  for (int64_t i = begin < 0 ? 0 : begin; i < end && i < n; ++i) {
    const auto& l = ferry::g_launches[(size_t)i];
    if (hipEventSynchronize(l.stop) != hipSuccess) return 3;
    float s = 0.f, e = 0.f;
    if (hipEventElapsedTime(&s, a, l.start) != hipSuccess) return 3;   // negative if before t0
    if (hipEventElapsedTime(&e, a, l.stop) != hipSuccess) return 3;
    const float lo = s > 0.f ? s : 0.f, hi = e < win ? e : win;
    if (hi > lo) ms += hi - lo;
  }
  *total_ms = ms;
  return 0;
}

extern "C" const char* ferry_last_error(void) { return ferry::g_last_error.c_str(); }

extern "C" int32_t ferry_abi_version(void) { return 6; }

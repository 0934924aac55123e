// Error reporting and version of the ferry_amd C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

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

}  // namespace ferry

extern "C" const char* ferry_last_error(void) { return ferry::g_last_error.c_str(); }

extern "C" int32_t ferry_abi_version(void) { return 1; }

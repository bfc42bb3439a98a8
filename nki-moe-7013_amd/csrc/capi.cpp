// Error plumbing, the version query of the C ABI and device facts shared by
// the launchers.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "common.hpp"

namespace qmoe {

static thread_local char g_last_error[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

constexpr int CU_MAX_DEVICES = 64;
static std::atomic<int> g_cus[CU_MAX_DEVICES];

int current_device_cus() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= CU_MAX_DEVICES) return 0;
  int n = g_cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace qmoe

extern "C" int qmoe_version(void) { return QMOE_VERSION; }

extern "C" const char* qmoe_last_error(void) { return qmoe::g_last_error; }

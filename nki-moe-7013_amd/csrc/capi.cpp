// Error plumbing and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

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

}  // namespace qmoe

extern "C" int qmoe_version(void) { return QMOE_VERSION; }

extern "C" const char* qmoe_last_error(void) { return qmoe::g_last_error; }

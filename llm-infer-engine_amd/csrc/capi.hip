// C-ABI support: version and per-thread last-error string.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace mi {
namespace {
thread_local char g_last_error[512] = {0};
}

void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace mi

extern "C" int32_t mi_version(void) { return 100; }

extern "C" const char* mi_last_error(void) { return mi::g_last_error; }

// Library-wide C ABI helpers: version and per-thread error message.
#include <cstdarg>
#include <cstdio>

#include "mpx_common.h"

namespace mpx {

namespace {
thread_local char g_last_error[512] = {0};
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace mpx

extern "C" int mpx_version(void) { return (0 << 16) | 1; }

extern "C" const char* mpx_last_error(void) { return mpx::g_last_error; }

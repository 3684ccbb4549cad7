// Error reporting and version of the bsx C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/bsx.h"

namespace bsx {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace bsx

extern "C" const char* bsx_last_error(void) { return bsx::g_last_error; }

extern "C" int bsx_version(void) { return 1; }

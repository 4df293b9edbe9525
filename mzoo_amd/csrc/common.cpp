// Host-side plumbing of the C ABI: version and per-thread last-error text.
#include <stdarg.h>
#include <stdio.h>

#include "../../include/mzk.h"

namespace mzk {

static thread_local char g_last_error[512] = "";

void set_last_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace mzk

extern "C" int mzk_version(void) { return 100; }

extern "C" const char* mzk_last_error(void) { return mzk::g_last_error; }

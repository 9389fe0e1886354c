// Error reporting and version for the mi355q C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mi355q {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace mi355q

extern "C" const char* mi355q_last_error(void) { return mi355q::g_last_error; }

extern "C" int mi355q_version(void) { return 1; }

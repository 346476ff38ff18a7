// Library-wide C ABI pieces: error message storage and version.
#include "common.h"

#include <string.h>

namespace yh {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

}  // namespace yh

extern "C" const char* yh_last_error(void) { return yh::g_error; }

extern "C" int yh_abi_version(void) { return 106; }

// Error state and version of the C ABI.
#include "capi.hpp"

#include <string.h>

namespace logo {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

}  // namespace logo

extern "C" const char* logo_last_error(void) { return logo::g_last_error; }

extern "C" int logo_abi_version(void) { return 7; }

// Error slot and version query of the C ABI (include/dexter_gfx950.h).
#include "dx_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace dx {

namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

}  // namespace dx

extern "C" const char* dx_last_error(void) { return dx::g_error; }

extern "C" int dx_abi_version(void) { return DX_ABI_VERSION; }

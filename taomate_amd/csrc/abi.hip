// Library identity and per-thread error text for the C ABI.
#include <stdarg.h>

#include "ltx_common.h"

namespace ltx {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace ltx

extern "C" int ltx_abi_version(void) { return LTX_ABI_VERSION; }

extern "C" const char* ltx_last_error(void) { return ltx::g_err; }

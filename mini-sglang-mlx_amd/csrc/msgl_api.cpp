// Host-side C ABI glue: ABI version and the per-thread error message.
#include <cstdarg>
#include <cstdio>

#include "msgl_common.h"

namespace msgl {

static thread_local char g_last_error[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

}  // namespace msgl

extern "C" int msgl_abi_version(void) { return MSGL_ABI_VERSION; }

extern "C" const char* msgl_last_error(void) { return msgl::g_last_error; }

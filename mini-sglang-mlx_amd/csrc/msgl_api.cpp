// Host-side C ABI glue: ABI version, the per-thread error message and the
// per-thread launch-timing events.
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

// Events the calling thread's next main-kernel launch records (one use).
static thread_local hipEvent_t g_prof_start = nullptr;
static thread_local hipEvent_t g_prof_stop = nullptr;

bool take_profile_events(hipEvent_t& start, hipEvent_t& stop) {
  if (g_prof_start == nullptr) return false;
  start = g_prof_start;
  stop = g_prof_stop;
  g_prof_start = g_prof_stop = nullptr;
  return true;
}

}  // namespace msgl

extern "C" int msgl_abi_version(void) { return MSGL_ABI_VERSION; }

extern "C" const char* msgl_last_error(void) { return msgl::g_last_error; }

extern "C" int msgl_profile_next_launch(void* start_event, void* stop_event) {
  msgl::clear_error();
  if ((start_event == nullptr) != (stop_event == nullptr)) {
    msgl::set_error("msgl_profile_next_launch: give both events or neither");
    return MSGL_ERR_INVALID;
  }
  msgl::g_prof_start = reinterpret_cast<hipEvent_t>(start_event);
  msgl::g_prof_stop = reinterpret_cast<hipEvent_t>(stop_event);
  return MSGL_OK;
}

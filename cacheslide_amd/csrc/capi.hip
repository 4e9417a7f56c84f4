// Library-level entry points: version string and per-thread error messages.
#include "common.h"

namespace cs {
namespace {
thread_local char g_error[512] = "";
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}
}  // namespace cs

extern "C" const char* cs_version(void) { return "cacheslide_hip 0.1.0 gfx950"; }

extern "C" const char* cs_last_error(void) { return cs::g_error; }

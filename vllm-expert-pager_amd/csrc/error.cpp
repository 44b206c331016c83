// Per-thread error message of libxp (plain C++, no HIP): every entry point
// returns a status and leaves the reason here for xp_last_error().
#include <cstdarg>
#include <cstdio>

namespace xp {

static thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace xp

extern "C" const char* xp_last_error(void) { return xp::g_err; }

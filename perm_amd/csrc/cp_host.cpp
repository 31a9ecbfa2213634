// Thread-local error message behind cp_last_error().
#include "cp_host.h"

namespace cp {

static thread_local char g_err[512] = "";

int set_error(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_err[0] = '\0'; }

}  // namespace cp

extern "C" const char* cp_last_error(void) { return cp::g_err; }

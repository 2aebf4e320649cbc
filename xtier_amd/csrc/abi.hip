// Library-wide entry points of the C ABI: version and last-error text.
#include "xt_host.h"

#include <string.h>

namespace xt {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_last_error[0] = 0;
  return XT_OK;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(XT_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

}  // namespace xt

extern "C" int xt_version(void) { return 100; }

extern "C" const char* xt_last_error(void) { return xt::g_last_error; }

// Library-wide C-ABI plumbing: version, per-thread error text, HIP status translation.
#include <stdarg.h>
#include <stdio.h>

#include "hn_common.h"

namespace hn {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return HN_OK;
  set_error("%s: %s", what, hipGetErrorString(e));
  return HN_ERR_HIP;
}

}  // namespace hn

extern "C" int hn_version(void) { return 200; }

extern "C" const char* hn_last_error(void) { return hn::g_error; }

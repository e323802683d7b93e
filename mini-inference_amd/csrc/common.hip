// Error reporting for the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "miq_common.h"

namespace miq {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return MIQ_ERR_LAUNCH;
  }
  return MIQ_OK;
}

}  // namespace miq

extern "C" const char* miq_last_error(void) { return miq::g_error; }

extern "C" int miq_abi_version(void) { return 1; }

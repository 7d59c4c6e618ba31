// Error reporting and version of the C ABI (include/deltaattn.h).
#include <stdarg.h>
#include <stdio.h>

#include "da_common.hpp"

namespace da {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return DA_OK;
}

}  // namespace da

extern "C" const char* da_last_error(void) { return da::g_last_error; }

extern "C" int da_version(void) { return 1; }

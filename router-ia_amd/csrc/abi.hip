// Library-wide C ABI plumbing: version, thread-local last-error string.
#include <stdarg.h>
#include <stdio.h>

#include "ria_common.h"

namespace ria {

static thread_local char g_last_error[1024] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(RIA_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  }
  return RIA_OK;
}

}  // namespace ria

extern "C" int ria_abi_version(void) { return RIA_ABI_VERSION; }

extern "C" const char* ria_last_error(void) { return ria::g_last_error; }

// abi.hip -- version, thread-local error reporting and launch checks for the
// C ABI declared in include/fat_abi.h.
#include <stdarg.h>
#include <stdio.h>

#include "fat_common.h"

namespace {
thread_local char g_last_error[512] = {0};
}

namespace fat_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return FAT_E_LAUNCH;
  }
  return FAT_OK;
}

}  // namespace fat_host

extern "C" int fat_abi_version(void) { return FAT_ABI_VERSION; }

extern "C" const char* fat_last_error(void) { return g_last_error; }

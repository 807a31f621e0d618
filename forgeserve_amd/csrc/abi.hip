// Error reporting shared by every C-ABI entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_error[512] = "";
}

namespace fs {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int arg_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return FS_ERR_ARG;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

}  // namespace fs

extern "C" const char* fs_last_error(void) { return g_error; }
extern "C" int fs_abi_version(void) { return 3; }

// Library-level entry points: version, target and the thread-local error.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace mi {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return MI355X_ELAUNCH;
  }
  return MI355X_OK;
}

}  // namespace mi

extern "C" {

int mi355x_abi_version(void) { return 6; }

const char* mi355x_last_error(void) { return mi::g_error; }

const char* mi355x_target(void) { return "gfx950"; }

#ifndef MI355X_SOURCE_HASH
#define MI355X_SOURCE_HASH "unknown"
#endif
const char* mi355x_source_hash(void) { return MI355X_SOURCE_HASH; }

}  // extern "C"

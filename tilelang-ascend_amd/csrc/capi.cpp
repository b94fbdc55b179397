// Error channel and version query of the C ABI (include/dsa_mi355x.h).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "dsa_common.h"

namespace {
thread_local char g_last_error[1024] = "";
}

namespace dsa {

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
    return set_error(kHipError, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return kOk;
}

}  // namespace dsa

extern "C" {

const char* dsa_last_error(void) { return g_last_error; }

void dsa_clear_error(void) { g_last_error[0] = '\0'; }

int dsa_abi_version(void) { return 1; }

}  // extern "C"

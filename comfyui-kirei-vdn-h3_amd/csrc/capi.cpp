// Error channel and version of the libvdnh3 C ABI.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "common.h"

namespace {
thread_local std::string g_last_error;
}

namespace vdnh3 {

int set_error(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(VDNH3_ERR_RUNTIME, "%s: HIP launch failed: %s", what, hipGetErrorString(err));
  }
  return VDNH3_OK;
}

}  // namespace vdnh3

extern "C" const char *vdnh3_last_error(void) { return g_last_error.c_str(); }

extern "C" int vdnh3_abi_version(void) { return 102; }

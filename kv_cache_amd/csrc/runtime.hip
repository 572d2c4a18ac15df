// Error plumbing and version of the libqkv C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace qkv {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(QKV_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return QKV_OK;
}

}  // namespace qkv

QKV_EXPORT int qkv_abi_version(void) { return QKV_ABI_VERSION; }

QKV_EXPORT const char* qkv_last_error(void) { return g_last_error; }

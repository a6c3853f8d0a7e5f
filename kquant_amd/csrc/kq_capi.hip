// ABI version and error reporting for the kquant_amd C interface.
#include <stdarg.h>
#include <stdio.h>

#include "kq_internal.h"

static thread_local char g_last_error[512] = "";

int kq_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int kq_check_launch(hipError_t err, const char* where) {
  if (err == hipSuccess) return KQ_OK;
  return kq_fail(KQ_ERR_HIP, "%s: %s", where, hipGetErrorString(err));
}

extern "C" int kq_version(void) { return (1 << 16) | 0; }

extern "C" const char* kq_last_error(void) { return g_last_error; }

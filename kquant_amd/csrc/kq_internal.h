// Host-side helpers shared by the C-ABI entry points: status codes, the
// per-thread error message and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kquant_amd.h"

// Record a printf-style message as this thread's last error and return code.
int kq_fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// KQ_OK if err == hipSuccess, else KQ_ERR_HIP with the HIP error string.
int kq_check_launch(hipError_t err, const char* where);

static inline bool kq_misaligned(const void* p, uintptr_t align) {
  return (reinterpret_cast<uintptr_t>(p) & (align - 1)) != 0;
}

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

namespace kq {
// One X4T matrix kind over all experts, as the routed scale expansion reads
// it, and where it writes: fixed stream [experts][tiles][16 (1 + ceil(cols/8))],
// exceptions (matrix-local position | value << 24), tile_index [experts *
// tiles + 1] (first exception of each 16-row tile), and the output slots
// [slot][out_rgs][cols / 4][64] of which this plane fills row groups
// [out_rg0, out_rg0 + tiles).
struct X4TPlane {
  const uint8_t* fixed;
  const uint32_t* exceptions;
  const uint32_t* tile_index;
  uint8_t* out;
  int64_t tiles, out_rgs, out_rg0;
  int cols;
};
struct X4TExpandArgs {
  X4TPlane p[3];
  int n;  // planes used (2 or 3)
};
// Expand matrix routed[r] of every plane into slot r, r < max_routed
// (entries of -1 are skipped).
hipError_t x4t_expand_routed(const X4TExpandArgs& args, const int* routed, int max_routed, hipStream_t st);
}  // namespace kq

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

// The MXFP8 linear with fp32 output split over K and unit scales
// (kq_linear.hip): mx_linear_slices gives the slice count that fills this
// device's CUs for an [m, n] output and k_steps 64-deep steps (1 when the
// tiles fill them); mx_linear_planes_unit writes slice s of c = A W^T (A
// bf16 [m, k], k = a whole multiple of kb, the weight's K, which it wraps;
// W E4M3 [n, kb] with every block scale 1) to c + s plane, row stride ldc,
// for the caller to sum in plane order.  It takes the direct-load path
// only: mx_linear_planes_ok must hold.  split3_rows writes fp32 rows as
// their exact three-term bf16 split [a0 | a1 | a2] ([m, 3k]).
int mx_linear_slices(int64_t m, int64_t n, int64_t k_steps);
bool mx_linear_planes_ok(int64_t lda, int64_t kb);
hipError_t mx_linear_planes_unit(const uint16_t* a, int64_t lda, const uint8_t* wq, float* c, int64_t ldc,
                                 int64_t plane, int m, int n, int k, int kb, int slices, hipStream_t st);
hipError_t split3_rows(const float* a, int64_t lda, int64_t m, int64_t k, uint16_t* out, hipStream_t st);
}  // namespace kq

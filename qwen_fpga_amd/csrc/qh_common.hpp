// Host-side helpers shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qh_decode.h"

namespace qh {

// hipError_t -> status (0 ok, positive hipError_t otherwise)
inline int hip_status(hipError_t e) { return e == hipSuccess ? QH_OK : (int)e; }

// With QH_VERBOSE=1 in the environment, a failing HIP call is named on stderr.
int hip_report(hipError_t e, const char* what, const char* file, int line);
bool verbose();   // QH_VERBOSE is set (read once)

#define QH_TRY(expr)                         \
  do {                                       \
    const int st_ = (expr);                  \
    if (st_ != QH_OK) return st_;            \
  } while (0)
#define QH_HIP(expr) QH_TRY(::qh::hip_report((expr), #expr, __FILE__, __LINE__))

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// RoPE row for one position, exactly as the reference computes it
// (rope.hpp:17-27): inv_j = 1 / powf(theta, (2j)/64), f = pos * inv_j,
// out[j] = cosf(f), out[32 + j] = sinf(f) for j < 32.
void rope_row(int pos, float* out64);

}  // namespace qh

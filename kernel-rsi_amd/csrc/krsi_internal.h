// Host-side helpers shared by the C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "krsi.h"

namespace krsi {

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Round a byte count up to a 256-byte boundary (workspace sub-buffers).
inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Launch-status check: the HIP runtime reports a rejected launch through
// hipGetLastError(); map it to the ABI status.
inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KRSI_OK : KRSI_ERR_LAUNCH;
}

}  // namespace krsi

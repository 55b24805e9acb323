// Host-side plumbing shared by the C-ABI entry points: status codes, the
// per-thread error message and launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/popcorn_amd.h"

namespace pk {

// Records a printf-style message for pk_last_error() and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Converts the launch status of the kernels just enqueued into a C-ABI status.
int launched(const char* what);

// Compute units of the current device (cached per device; 256 on MI355X).
int cu_count();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int elem_size(int dtype) { return dtype == PK_F32 ? 4 : 2; }

inline bool known_dtype(int dtype) { return dtype == PK_F32 || dtype == PK_BF16 || dtype == PK_F16; }

}  // namespace pk

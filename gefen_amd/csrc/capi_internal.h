// Error reporting and argument checks shared by the C entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>

#include "gefen_hip.h"

namespace gefen {

void set_error(const char* fmt, ...);

// Record a message and return GEFEN_EINVAL.
int fail_inval(const char* fmt, ...);

// Return GEFEN_ERUNTIME with the HIP error text when e != hipSuccess.
int hip_status(hipError_t e, const char* what);

// Check the last launch of the calling thread.
inline int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

inline bool valid_dtype(int dt) { return dt == GEFEN_F32 || dt == GEFEN_F16 || dt == GEFEN_BF16; }
inline int dtype_size(int dt) { return dt == GEFEN_F32 ? 4 : 2; }
inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

}  // namespace gefen

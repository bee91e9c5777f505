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

// Every device allocation of the library (pools, workspaces, temporaries) goes
// through these, which count them for gefen_device_allocations().
hipError_t device_malloc(void** ptr, size_t bytes);
hipError_t device_malloc_async(void** ptr, size_t bytes, hipStream_t st);

// Check the last launch of the calling thread.
inline int launch_status(const char* what) { return hip_status(hipGetLastError(), what); }

inline bool valid_dtype(int dt) { return dt == GEFEN_F32 || dt == GEFEN_F16 || dt == GEFEN_BF16; }
inline int dtype_size(int dt) { return dt == GEFEN_F32 ? 4 : 2; }
inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// The per-tensor scalars of GefenMuon's update (gefen_muon.py:325-329) as the
// kernels use them: wdf = f32(1 - lr * wd); alpha = f32(-lr_adj), rounded to the
// parameter dtype for a reduced dtype (torch.tensor(-lr_adj).to(dtype)); the
// product rounded first for a reduced dtype and a transposed update.
struct MuonApplyScalars {
    float wdf, alpha;
    int do_wd, round_prod;
};
inline MuonApplyScalars muon_apply_scalars(const gefen_muon_apply_task& in) {
    MuonApplyScalars s;
    s.wdf = (float)(1.0 - in.lr * in.weight_decay);
    s.do_wd = in.weight_decay > 0.0;
    const float a32 = (float)(-in.adjusted_lr);
    if (in.param_dtype == GEFEN_F32) {
        s.alpha = a32;
    } else if (in.param_dtype == GEFEN_BF16) {
        uint32_t u;
        __builtin_memcpy(&u, &a32, 4);
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
        __builtin_memcpy(&s.alpha, &u, 4);
    } else {
        s.alpha = (float)(_Float16)a32;
    }
    s.round_prod = (in.param_dtype != GEFEN_F32 && in.transposed) ? 1 : 0;
    return s;
}

}  // namespace gefen

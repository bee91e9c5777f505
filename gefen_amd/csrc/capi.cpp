// Thread-local error text of the C ABI.
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "capi_internal.h"

namespace {
thread_local char g_error[512] = "";
std::atomic<int64_t> g_allocations{0};
}

namespace gefen {

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

int fail_inval(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return GEFEN_EINVAL;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return GEFEN_OK;
    set_error("%s: %s", what, hipGetErrorString(e));
    return GEFEN_ERUNTIME;
}

hipError_t device_malloc(void** ptr, size_t bytes) {
    g_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipMalloc(ptr, bytes);
}

hipError_t device_malloc_async(void** ptr, size_t bytes, hipStream_t st) {
    g_allocations.fetch_add(1, std::memory_order_relaxed);
    return hipMallocAsync(ptr, bytes, st);
}

}  // namespace gefen

extern "C" int64_t gefen_device_allocations(void) { return g_allocations.load(std::memory_order_relaxed); }

extern "C" const char* gefen_last_error(void) { return g_error; }
extern "C" int gefen_abi_version(void) { return 1; }
extern "C" size_t gefen_struct_size(int which) {
    return which == 0   ? sizeof(gefen_step_task)
           : which == 1 ? sizeof(gefen_muon_task)
           : which == 2 ? sizeof(gefen_muon_apply_task)
                        : 0;
}

// Thread-local error text of the C ABI.
#include <stdio.h>
#include <string.h>

#include "capi_internal.h"

namespace {
thread_local char g_error[512] = "";
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

}  // namespace gefen

extern "C" const char* gefen_last_error(void) { return g_error; }
extern "C" int gefen_abi_version(void) { return 1; }
extern "C" size_t gefen_struct_size(int which) {
    return which == 0   ? sizeof(gefen_step_task)
           : which == 1 ? sizeof(gefen_muon_task)
           : which == 2 ? sizeof(gefen_muon_apply_task)
                        : 0;
}

// Test helper (not part of the library): checks, for every float h in
// [lo, hi) (bit patterns), that the reciprocal the period-one step kernel uses,
// fma(fma(-h, r, 1), r, r) with r = v_rcp_f32(h), equals the IEEE quotient
// 1.0f / h, and that the IEEE quotient equals the float64 quotient rounded to
// float.  Built by gefen_amd/build.py into tests/hip/libreciprocal_check.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

__global__ void k_reciprocal_check(uint32_t lo, uint32_t count, unsigned long long* bad, uint32_t* first) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= count) return;
    const float h = __uint_as_float(lo + i);
    const float ref = 1.0f / h;
    const float r = __builtin_amdgcn_rcpf(h);
    const float e = __builtin_fmaf(-h, r, 1.0f);
    const float r1 = __builtin_fmaf(e, r, r);
    if (__float_as_uint((float)(1.0 / (double)h)) != __float_as_uint(ref)) atomicAdd(bad + 1, 1ull);
    if (__float_as_uint(r1) != __float_as_uint(ref)) {
        const unsigned long long n = atomicAdd(bad, 1ull);
        if (n < 8) first[n] = lo + i;
    }
}

// out[0]: reciprocal mismatches, out[1]: IEEE vs float64 mismatches; first[0..7]:
// the first mismatching bit patterns.  Returns 0, or 1 on a HIP error.
extern "C" int gefen_test_reciprocal(uint32_t lo, uint32_t hi, unsigned long long* out, uint32_t* first) {
    unsigned long long* bad = nullptr;
    uint32_t* fd = nullptr;
    if (hipMalloc(&bad, 2 * sizeof(unsigned long long)) != hipSuccess) return 1;
    if (hipMalloc(&fd, 8 * sizeof(uint32_t)) != hipSuccess) return 1;
    if (hipMemset(bad, 0, 2 * sizeof(unsigned long long)) != hipSuccess) return 1;
    if (hipMemset(fd, 0, 8 * sizeof(uint32_t)) != hipSuccess) return 1;
    const uint32_t chunk = 1u << 28;
    for (uint32_t s = lo; s < hi; s += (hi - s < chunk ? hi - s : chunk)) {
        const uint32_t cnt = hi - s < chunk ? hi - s : chunk;
        hipLaunchKernelGGL(k_reciprocal_check, dim3((cnt + 255) / 256), dim3(256), 0, 0, s, cnt, bad, fd);
        if (hipGetLastError() != hipSuccess) return 1;
    }
    int rc = hipDeviceSynchronize() == hipSuccess ? 0 : 1;
    if (!rc && hipMemcpy(out, bad, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
    if (!rc && hipMemcpy(first, fd, 8 * sizeof(uint32_t), hipMemcpyDeviceToHost) != hipSuccess) rc = 1;
    (void)hipFree(bad);
    (void)hipFree(fd);
    return rc;
}

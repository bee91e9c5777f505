// Test helper (not part of the library): the wave butterflies of the step
// kernels (wave_group_max_u32 / wave_group_sum: DPP, ds_swizzle and
// ds_bpermute lane exchanges) beside the ds_bpermute loops they replace
// (group_max_u32 / group_sum), for every group width 1..64, on the same lanes.
// Built by gefen_amd/build.py into tests/hip/libbutterfly_check.so.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

using namespace gefen;

// in: n words (n a multiple of 256); out: [4][7][n] = max new, max old, sum new,
// sum old (float bits) for the widths 1, 2, 4, ..., 64.
__global__ __launch_bounds__(256) void k_butterfly_check(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                        int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t v = in[i];
    const float f = __uint_as_float(v);
#pragma unroll
    for (int l = 0; l < 7; ++l) {
        const int width = 1 << l;
        out[(0 * 7 + l) * n + i] = wave_group_max_u32(v, width);
        out[(1 * 7 + l) * n + i] = group_max_u32(v, width);
        out[(2 * 7 + l) * n + i] = __float_as_uint(wave_group_sum(f, width));
        out[(3 * 7 + l) * n + i] = __float_as_uint(group_sum(f, width));
    }
}

extern "C" int gefen_test_butterfly(const uint32_t* in, uint32_t* out, int n, hipStream_t stream) {
    if (n <= 0 || n % 256) return 1;
    hipLaunchKernelGGL(k_butterfly_check, dim3(n / 256), dim3(256), 0, stream, in, out, n);
    return hipGetLastError() == hipSuccess ? 0 : 1;
}

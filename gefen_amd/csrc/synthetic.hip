// Device twin of gefen_amd/synthetic.py: fills tensors with the same bytes the
// numpy generator produces (integer splitmix64 stream, Irwin-Hall normals,
// dyadic scales, IEEE-exact float64 arithmetic).  Used by the benchmark and the
// GPU tests to create large inputs in HBM without host transfers.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "capi_internal.h"
#include "common.h"

namespace gefen {
namespace synth {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kM1 = 0xBF58476D1CE4E5B9ull;
constexpr uint64_t kM2 = 0x94D049BB133111EBull;
constexpr uint64_t kKeyMul = 0xD1B54A32D192ED03ull;

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + kGamma;
    z = (z ^ (z >> 30)) * kM1;
    z = (z ^ (z >> 27)) * kM2;
    return z ^ (z >> 31);
}
__host__ __device__ __forceinline__ uint64_t make_key(uint64_t seed, uint64_t stream) {
    return splitmix64(seed * kKeyMul + stream);
}
__device__ __forceinline__ uint64_t word(uint64_t key, uint64_t c) { return splitmix64(key + c * kGamma); }

__device__ __forceinline__ double normal_at(uint64_t key, uint64_t i) {
    int64_t s = 0;
    for (int j = 0; j < 3; ++j) {
        const uint64_t w = word(key, 3 * i + j);
        for (int k = 0; k < 4; ++k) s += (int64_t)((w >> (16 * k)) & 0xFFFFull);
    }
    return (double)(2 * s - 12 * 65535) / 131072.0;
}
__device__ __forceinline__ double dyadic_scale_at(uint64_t key, uint64_t r, int e_lo, int e_hi) {
    const uint64_t w = word(key, r);
    const uint64_t span = (uint64_t)(e_hi - e_lo + 1);
    const int e = (int)(w % span) + e_lo;
    const double m = (double)((w >> 32) % 8ull);
    return ldexp((8.0 + m) / 8.0, e);
}

template <typename T>
__device__ __forceinline__ void store(T* out, int64_t i, double v) {
    out[i] = from_f32<T>((float)v);
}
template <>
__device__ __forceinline__ void store<f16_t>(f16_t* out, int64_t i, double v) {
    _Float16 h = (_Float16)v;
    __builtin_memcpy(&out[i].bits, &h, 2);
}

// kind 0: normal * per-row dyadic scale; kind 1: normal * mult; kind 2: student_t3 * mult
template <typename T>
__global__ void k_fill(T* __restrict__ out, int64_t n, int64_t cols, uint64_t key, uint64_t skey, int e_lo, int e_hi,
                       int kind, double mult) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        double v;
        if (kind == 0) {
            v = normal_at(key, (uint64_t)i) * dyadic_scale_at(skey, (uint64_t)(i / cols), e_lo, e_hi);
        } else if (kind == 1) {
            v = normal_at(key, (uint64_t)i) * mult;
        } else {
            const double z0 = normal_at(key, 4 * (uint64_t)i), z1 = normal_at(key, 4 * (uint64_t)i + 1);
            const double z2 = normal_at(key, 4 * (uint64_t)i + 2), z3 = normal_at(key, 4 * (uint64_t)i + 3);
            const double chi = (z1 * z1 + z2 * z2) + z3 * z3;
            v = (z0 / sqrt(chi / 3.0)) * mult;
        }
        store<T>(out, i, v);
    }
}

}  // namespace synth
namespace synth {
// Plain copy of 16-byte vectors: a kernel of known traffic (n bytes read, n
// written) for scaling the HBM byte counters of the profiler.
__global__ __launch_bounds__(256) void k_copy16(const uint4* __restrict__ src, uint4* __restrict__ dst, int64_t n16) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

}  // namespace synth
}  // namespace gefen

using namespace gefen;

extern "C" int gefen_synth_copy(const void* src, void* dst, int64_t nbytes, gefen_stream_t hstream) {
    if (nbytes < 0 || nbytes % 16 || (nbytes > 0 && (!src || !dst))) return fail_inval("bad copy size");
    if (!aligned(src, 16) || !aligned(dst, 16)) return fail_inval("copy buffers must be 16-byte aligned");
    const int64_t n16 = nbytes / 16;
    if (n16 == 0) return GEFEN_OK;
    const int64_t blocks = (n16 + 255) / 256;
    if (blocks > INT32_MAX) return fail_inval("copy too large");
    hipLaunchKernelGGL(synth::k_copy16, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(hstream),
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16);
    return launch_status("gefen_synth_copy");
}

extern "C" int gefen_synth_fill(void* out, int dtype, int64_t numel, int64_t cols, uint64_t seed, uint64_t stream,
                                int e_lo, int e_hi, int kind, double mult, gefen_stream_t hstream) {
    if (!valid_dtype(dtype)) return fail_inval("bad dtype");
    if (numel < 0 || cols <= 0 || (numel > 0 && !out)) return fail_inval("bad shape");
    if (numel == 0) return GEFEN_OK;
    const uint64_t key = synth::make_key(seed, stream);
    const uint64_t skey = synth::make_key(seed, stream ^ 0x5CA1Eull);
    int64_t blocks = (numel + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipStream_t st = reinterpret_cast<hipStream_t>(hstream);
    if (dtype == GEFEN_F32)
        hipLaunchKernelGGL(synth::k_fill<float>, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<float*>(out),
                           numel, cols, key, skey, e_lo, e_hi, kind, mult);
    else if (dtype == GEFEN_BF16)
        hipLaunchKernelGGL(synth::k_fill<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<bf16_t*>(out),
                           numel, cols, key, skey, e_lo, e_hi, kind, mult);
    else
        hipLaunchKernelGGL(synth::k_fill<f16_t>, dim3((unsigned)blocks), dim3(256), 0, st, static_cast<f16_t*>(out),
                           numel, cols, key, skey, e_lo, e_hi, kind, mult);
    return launch_status("gefen_synth_fill");
}

// Shared device helpers for the Gefen HIP kernels (gfx950 / CDNA4, wave64).
//
// Numerics follow the reference's CPU path (torch 2.10 CPU): every torch op
// result is rounded to its tensor dtype (round to nearest even), lerp and
// add(alpha=) are single fused multiply-adds, divisions are IEEE correctly
// rounded.  Build with -ffp-contract=off: only the __builtin_fmaf calls written
// here are fused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gefen_hip.h"

namespace gefen {

// ----------------------------------------------------------------- dtypes
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return __uint_as_float((uint32_t)v.bits << 16); }
__device__ __forceinline__ float to_f32(f16_t v) {
    _Float16 h;
    __builtin_memcpy(&h, &v.bits, 2);
    return (float)h;
}

template <typename T> struct Conv;
template <> struct Conv<float> {
    __device__ __forceinline__ static float from(float v) { return v; }
};
template <> struct Conv<bf16_t> {
    __device__ __forceinline__ static bf16_t from(float v) {
        __bf16 b = (__bf16)v;  // v_cvt_pk_bf16_f32: round to nearest even
        bf16_t r;
        __builtin_memcpy(&r.bits, &b, 2);
        return r;
    }
};
template <> struct Conv<f16_t> {
    __device__ __forceinline__ static f16_t from(float v) {
        // v is a float32 result that is rounded to half here.  The empty asm keeps
        // the backend from folding the operation that produced v into the
        // conversion (v_fma_mixlo_f16 rounds a * b + c to half once, which differs
        // from the float32 result rounded to half where that result is a half
        // midpoint: p * (1 - lr * wd) of a half p is one such case).
        __asm__("" : "+v"(v));
        f16_t r;
        const float a = fabsf(v);
        if (a < 6.103515625e-05f) {
            // half subnormal (or zero): v_cvt_f16_f32 does not round these to
            // nearest even in every case, so round in fp32: a + 0.5 has an ulp
            // of 2^-24, the half subnormal spacing, and its low bits are the result.
            const float t = a + 0.5f;
            r.bits = (uint16_t)((__float_as_uint(t) - 0x3f000000u) | ((__float_as_uint(v) >> 16) & 0x8000u));
            return r;
        }
        _Float16 h = (_Float16)v;  // v_cvt_f16_f32: round to nearest even
        __builtin_memcpy(&r.bits, &h, 2);
        return r;
    }
};
template <typename T>
__device__ __forceinline__ T from_f32(float v) { return Conv<T>::from(v); }
// value of v after a round trip through dtype T
template <typename T>
__device__ __forceinline__ float round_to(float v) { return to_f32(from_f32<T>(v)); }

// GefenMuon's update of one parameter element in dtype D (gefen_muon.py:325-329):
// p.mul_(1 - lr * wd), rounded to D, when decaying; then p.add_(u, alpha) as
// torch evaluates it: one fma for float32; for a reduced dtype (alpha already
// rounded to D) the product u * alpha is exact in float32, rounded to D first
// when the update is a transposed view (torch's element-wise path), and added.
template <typename D>
__device__ __forceinline__ float muon_apply_value(float pf, float uf, float wdf, float alpha, bool do_wd,
                                                  bool round_prod) {
    if (do_wd) pf = round_to<D>(pf * wdf);
    if constexpr (sizeof(D) == 4) return __builtin_fmaf(uf, alpha, pf);
    float prod = uf * alpha;
    if (round_prod) prod = round_to<D>(prod);
    return pf + prod;
}

// NaN-propagating maximum of non-negative values (torch amax semantics)
__device__ __forceinline__ float nanmax(float a, float b) { return (b > a || b != b) ? b : a; }
// Maximum that skips NaN: b replaces a only when b > a, a comparison NaN never
// passes (the running-maximum loops of lloyd_max_fused_kernel.cu:78-95).
__device__ __forceinline__ float max_skip_nan(float a, float b) { return b > a ? b : a; }

// ----------------------------------------------------------------- vector access
// W consecutive elements of type T moved with one load/store of W*sizeof(T) bytes.
template <typename T, int W>
struct alignas(sizeof(T) * W) Vec { T v[W]; };

template <typename T, int W>
__device__ __forceinline__ Vec<T, W> vload(const T* base, int64_t elem) {
    return *reinterpret_cast<const Vec<T, W>*>(base + elem);
}
template <typename T, int W>
__device__ __forceinline__ void vstore(T* base, int64_t elem, const Vec<T, W>& x) {
    *reinterpret_cast<Vec<T, W>*>(base + elem) = x;
}
// Same with a wave-uniform base and a 32-bit element offset: global memory
// instructions take the base from scalar registers and the byte offset from
// one vector register.
template <typename T, int W>
__device__ __forceinline__ Vec<T, W> vload32(const T* base, uint32_t elem) {
    const uint32_t off = elem * (uint32_t)sizeof(T);
    return *reinterpret_cast<const Vec<T, W>*>(reinterpret_cast<const char*>(base) + off);
}
template <typename T, int W>
__device__ __forceinline__ void vstore32(T* base, uint32_t elem, const Vec<T, W>& x) {
    const uint32_t off = elem * (uint32_t)sizeof(T);
    *reinterpret_cast<Vec<T, W>*>(reinterpret_cast<char*>(base) + off) = x;
}

// Non-temporal (streaming) variants: the data is touched once per step, so the
// loads and stores carry the nt hint and do not displace reused lines in L2.
template <int BYTES> struct RawVec;
template <> struct RawVec<32> { typedef uint32_t type __attribute__((ext_vector_type(8))); };
template <> struct RawVec<16> { typedef uint32_t type __attribute__((ext_vector_type(4))); };
template <> struct RawVec<8> { typedef uint32_t type __attribute__((ext_vector_type(2))); };
template <> struct RawVec<4> { typedef uint32_t type; };
template <> struct RawVec<2> { typedef uint16_t type; };
template <> struct RawVec<1> { typedef uint8_t type; };

template <typename T, int W>
__device__ __forceinline__ Vec<T, W> vload32_nt(const T* base, uint32_t elem) {
    using R = typename RawVec<sizeof(T) * W>::type;
    const uint32_t off = elem * (uint32_t)sizeof(T);
    const R r = __builtin_nontemporal_load(reinterpret_cast<const R*>(reinterpret_cast<const char*>(base) + off));
    Vec<T, W> x;
    __builtin_memcpy(&x, &r, sizeof(x));
    return x;
}
template <typename T, int W>
__device__ __forceinline__ void vstore32_nt(T* base, uint32_t elem, const Vec<T, W>& x) {
    using R = typename RawVec<sizeof(T) * W>::type;
    const uint32_t off = elem * (uint32_t)sizeof(T);
    R r;
    __builtin_memcpy(&r, &x, sizeof(r));
    __builtin_nontemporal_store(r, reinterpret_cast<R*>(reinterpret_cast<char*>(base) + off));
}

// ----------------------------------------------------------------- wave reductions
// Butterfly over groups of `width` lanes (width a power of two <= 64).
__device__ __forceinline__ float group_max(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v = nanmax(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float group_max_skip_nan(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v = max_skip_nan(v, __shfl_xor(v, off, 64));
    return v;
}
__device__ __forceinline__ float group_sum(float v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}

// ----------------------------------------------------------------- codebook tables
// Prepared once per codebook (gefen_prepare_codebook):
//   cb[k]    codebook (sorted ascending), K <= 256 entries
//   thr[k]   for k = 1..K-1 the largest float x in (cb[k-1], cb[k]] for which the
//            reference's tie rule |x - cb[k-1]| <= |x - cb[k]| (fp32 differences)
//            picks the left entry, or cb[k-1] if none; thr[K] = +inf sentinel.
//            The nearest index of a non-NaN x is #{k in 1..K-1 : thr[k] < x}.
//   bucket[e] for e = 0..4096: #{k : thr[k] < -1 + e/2048}.
//   max_probe: most thresholds a search started one bucket low can meet before
//            reaching x (1 << 20 if thresholds lie below -1); <= 2 lets the
//            kernels use the fixed two-probe search.
//   bucket8  the same counts as bytes (every count is <= 255), padded with zeros
//            to 4112 entries: the compact copy the step kernels keep in LDS.
//   bucket_fine, max_probe_fine: the same on a grid twice as fine,
//            bucket_fine[e] = #{k : thr[k] < -1 + e/4096} for e = 0..8192 as
//            bytes, padded with zeros to 8208 entries; max_probe_fine <= 1 lets
//            the 16-bit parameter step kernels search with a single probe.
constexpr int kBucket8Bytes = 4112;
constexpr int kFineCells = 8192;  // cells of width 2^-12 over [-1, 1]
constexpr int kFineBytes = 8208;
//   nb16[i]  the nearest index of the bf16 value with bits kNb16Lo + i (i < kNb16Side)
//            at entry kNb16Side + i, and of its negative at entry kNb16Side - 1 - i
//            (so the entry is kNb16Side + (i ^ s) with s = 0 or -1 from the sign
//            bit): every bf16 x with 2^-20 <= |x| <= 1.0078125, the range of the
//            GefenMuon quotients.
constexpr uint32_t kNb16Lo = 0x3580u;                 // 2^-20
constexpr uint32_t kNb16Side = 0x3F82u - kNb16Lo;     // up to 0x3F81 = 1.0078125
constexpr int kNb16Bytes = (2 * kNb16Side + 15) / 16 * 16;
struct CodebookTables {
    float cb[256];
    float thr[260];
    uint8_t bucket8[kBucket8Bytes];
    uint8_t bucket_fine[kFineBytes];
    uint16_t bucket[4100];
    int32_t K;
    int32_t max_probe;
    int32_t max_probe_fine;
    int32_t pad;
    alignas(16) uint8_t nb16[kNb16Bytes];
};

// Nearest codebook index (gefen.py:122-143) from LDS copies of thr and bucket.
__device__ __forceinline__ int nearest_index(float x, const float* thr, const uint16_t* bucket, int K) {
    if (x != x) return K - 1;  // searchsorted(NaN) = K -> right = left = K-1
    int k = 0;
    if (x >= -1.0f) {
        float y = fminf((x + 1.0f) * 2048.0f, 4096.0f);
        int b = (int)y;  // y >= 0: truncation == floor
        // x + 1 may round up across one bucket edge for x >= 0: step back if the
        // edge (exact: a multiple of 2^-11 in [-1, 1]) exceeds x
        if (-1.0f + (float)b * 0.00048828125f > x) b -= 1;
        k = bucket[b];
    }
    while (k < K - 1 && thr[k + 1] < x) ++k;
    return k;
}


// Exact float32 quotient a / b for a b shared by many a (a block magnitude):
// a * RN64(1/b) in float64, rounded once to float32.  The float64 product is
// within 2^-52 (relative) of a/b, while a quotient of two float32 numbers is
// never a float32 rounding midpoint and lies at least 2^-49 (relative) away
// from every midpoint (|a - m b| >= 2^e(m)+e(b) when nonzero, m b < 2^49 of
// that unit).  Hence rounding the float64 product gives RN32(a/b), the IEEE
// division.  rb = 1 / (double)b is computed once per block.
__device__ __forceinline__ float div_by_block(float a, double rb) { return (float)((double)a * rb); }

// |x| as an ordered integer: NaN (any payload, sign cleared) compares above inf,
// so an unsigned max over these keys is torch's NaN-propagating absmax.
__device__ __forceinline__ uint32_t abs_key(float x) { return __float_as_uint(x) & 0x7fffffffu; }
__device__ __forceinline__ uint32_t group_max_u32(uint32_t v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

// v of lane (this lane ^ OFF) in a wave whose 64 lanes are all active, without
// lane-address arithmetic on the vector ALU: DPP quad permutations for 1 and 2,
// DPP rotation by 8 inside each row of 16 lanes for 8 (i + 8 mod 16 == i ^ 8),
// ds_swizzle (bitmask mode: source lane = lane ^ OFF inside 32 lanes) for 4 and
// 16, ds_bpermute for 32.
template <int OFF>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    if constexpr (OFF == 1) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    } else if constexpr (OFF == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    } else if constexpr (OFF == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);  // row_ror:8
    } else if constexpr (OFF == 4 || OFF == 16) {
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (OFF << 10) | 0x1f);
    } else {
        static_assert(OFF == 32, "lane_xor: offsets 1, 2, 4, 8, 16, 32");
        return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(((threadIdx.x & 63u) ^ 32u) << 2), (int)v);
    }
}

// The butterflies of group_max_u32 / group_sum (the same lane pairs, offsets
// width/2 down to 1, the same operand order, so the same results) for a width
// that is uniform across the wave and a wave with every lane active.
__device__ __forceinline__ uint32_t wave_group_max_u32(uint32_t v, int width) {
    auto mx = [](uint32_t a, uint32_t b) { return b > a ? b : a; };
    if (width > 32) v = mx(v, lane_xor<32>(v));
    if (width > 16) v = mx(v, lane_xor<16>(v));
    if (width > 8) v = mx(v, lane_xor<8>(v));
    if (width > 4) v = mx(v, lane_xor<4>(v));
    if (width > 2) v = mx(v, lane_xor<2>(v));
    if (width > 1) v = mx(v, lane_xor<1>(v));
    return v;
}
__device__ __forceinline__ float wave_group_sum(float v, int width) {
    if (width > 32) v = v + __uint_as_float(lane_xor<32>(__float_as_uint(v)));
    if (width > 16) v = v + __uint_as_float(lane_xor<16>(__float_as_uint(v)));
    if (width > 8) v = v + __uint_as_float(lane_xor<8>(__float_as_uint(v)));
    if (width > 4) v = v + __uint_as_float(lane_xor<4>(__float_as_uint(v)));
    if (width > 2) v = v + __uint_as_float(lane_xor<2>(__float_as_uint(v)));
    if (width > 1) v = v + __uint_as_float(lane_xor<1>(__float_as_uint(v)));
    return v;
}

// Nearest codebook index of x with at most two threshold probes in the common
// case, from bucket8 (FINE: bucket_fine).  The bucket is taken one below
// floor((x + 1) * cells / 2) so that the fma's rounding can only move it down;
// its count of thresholds < edge is <= the answer, and the remaining thresholds
// in [edge, x) are counted by probing.
template <bool FINE>
__device__ __forceinline__ int nearest_fast(float x, const float* thr, const uint8_t* bucket, int K) {
    constexpr float kHalf = FINE ? 4096.0f : 2048.0f;
    float y = __builtin_fmaf(x, kHalf, kHalf);
    y = fminf(fmaxf(y, 1.0f), 2.0f * kHalf + 1.0f);
    const int b = (int)y - 1;
    int k = (x < -1.0f) ? 0 : (int)bucket[b];
    k += (thr[k + 1] < x) ? 1 : 0;  // thr[K] = +inf stops every probe at K - 1
    k += (thr[k + 1] < x) ? 1 : 0;
    while (thr[k + 1] < x) ++k;    // only when three or more thresholds share the window
    return (x != x) ? K - 1 : k;
}

}  // namespace gefen

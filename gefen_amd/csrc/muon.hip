// GefenMuon kernels around the Newton-Schulz products (gefen_muon.py:33-37,
// 325-329):
//
//   * gefen_ns_prepare: X /= max(||X||, eps) for a stack of bf16 matrices
//     (norm in fp32, rounded to bf16 like torch's bf16 norm; the division in
//     fp32 and rounded to bf16 like torch's bf16 div_), in place, and X^T
//     into a second buffer (64 x 64 tiles transposed through LDS).  The norm is
//     a two-level reduction in a fixed order, so it is deterministic.
//   * gefen_muon_apply_tasks: p <- p * (1 - lr * wd), then p <- p + (-lr_adj) *
//     update with the reference's CPU rounding, for many tensors per launch.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "capi_internal.h"
#include "common.h"

namespace gefen {
namespace muon {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kNormThreads = 256;
constexpr int64_t kNormChunk = (int64_t)kNormThreads * 8 * 16;  // elements per block: 16 vectors per thread

// partial[g * nblk + b] = sum of squares (fp32) of chunk b of matrix g
__global__ __launch_bounds__(kNormThreads) void k_sumsq(const uint16_t* __restrict__ x, int64_t per, int nblk,
                                                       float* __restrict__ partial) {
    __shared__ float red[kNormThreads / 64];
    const int g = blockIdx.y, b = blockIdx.x;
    const uint16_t* src = x + (int64_t)g * per;
    const int64_t e0 = (int64_t)b * kNormChunk;
    const int64_t e1 = min(e0 + kNormChunk, per);
    float s = 0.0f;
    for (int64_t e = e0 + (int64_t)threadIdx.x * 8; e < e1; e += (int64_t)kNormThreads * 8) {
        if (e + 8 <= e1) {
            const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + e));
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float lo = __uint_as_float(v[c] << 16), hi = __uint_as_float(v[c] & 0xffff0000u);
                s = __builtin_fmaf(lo, lo, s);
                s = __builtin_fmaf(hi, hi, s);
            }
        } else {
            for (int64_t i = e; i < e1; ++i) {
                const float f = __uint_as_float((uint32_t)src[i] << 16);
                s = __builtin_fmaf(f, f, s);
            }
        }
    }
    s = group_sum(s, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
        for (int w = 0; w < kNormThreads / 64; ++w) t = t + red[w];
        partial[(int64_t)g * nblk + b] = t;
    }
}

// div[g] = max(bf16(sqrt(sum)), bf16(eps)) as a float (clamp(min=eps) of a bf16 norm)
__global__ void k_norm(const float* __restrict__ partial, int nblk, int batch, float eps_bf16,
                       float* __restrict__ div) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= batch) return;
    double s = 0.0;
    for (int b = 0; b < nblk; ++b) s += (double)partial[(int64_t)g * nblk + b];
    const float nrm = round_to<bf16_t>((float)sqrt(s));
    div[g] = (nrm < eps_bf16) ? eps_bf16 : nrm;
}

// clamp(min=eps) of a bf16 tensor compares with eps rounded to bf16
inline float eps_to_bf16(double eps) {
    const float f = (float)eps;
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

// Divisor of matrix g from its float64 sum of squares (gefen_ns_prepare_sumsq):
// max(bf16(sqrt(sum)), bf16(eps)), as k_norm forms it.
__device__ __forceinline__ float divisor_from_sumsq(double s, float eps_bf16) {
    const float nrm = round_to<bf16_t>((float)sqrt(s));
    return (nrm < eps_bf16) ? eps_bf16 : nrm;
}

// x[g] = bf16(x[g] / d_g) in place, xt[g] = x[g]^T; one 64 x 64 tile per block.
// d_g = div[g], or from the sum of the GEFEN_SUMSQ_SLOTS partial sums of
// task index[g] (or g) when sumsq is given.  The
// quotient is the float64 product with 1 / d_g rounded to float (the IEEE
// quotient: see div_by_block), then rounded to bf16 as torch's bf16 div_ does.
constexpr int kTile = 64;
// TPW tiles of one row band per workgroup (the divisor is formed once): two
// when cols is a multiple of 128 (8% faster on the GefenMuon stacks), else one.
template <int TPW, bool WRITE_X>
__global__ __launch_bounds__(256) void k_scale_transpose(uint16_t* __restrict__ x, uint16_t* __restrict__ xt,
                                                         int rows, int cols, const float* __restrict__ div,
                                                         const double* __restrict__ sumsq,
                                                         const int32_t* __restrict__ index, float eps_bf16) {
    __shared__ uint16_t tile[kTile][kTile + 2];
    const int g = blockIdx.z;
    const int r0 = blockIdx.y * kTile;
    const int64_t per = (int64_t)rows * cols;
    uint16_t* src = x + (int64_t)g * per;
    uint16_t* dst = xt + (int64_t)g * per;
    float d;
    if (sumsq) {
        const double* slots = sumsq + (size_t)(index ? index[g] : g) * GEFEN_SUMSQ_STRIDE;
        double s = 0.0;
        for (int i = 0; i < GEFEN_SUMSQ_SLOTS; ++i) s += slots[16 * i];
        d = divisor_from_sumsq(s, eps_bf16);
    } else {
        d = div[g];
    }
    const double rd = 1.0 / (double)d;
    const int t = threadIdx.x;
    // every tile's loads first (6% faster than loading each tile after the
    // previous one is written)
    u32x4 vin[TPW][2];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const uint16_t* p = src + (int64_t)(r0 + (t >> 2)) * cols + (blockIdx.x * TPW + tt) * kTile + (t & 3) * 16;
#pragma unroll
        for (int h = 0; h < 2; ++h) vin[tt][h] = *reinterpret_cast<const u32x4*>(p + 8 * h);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int c0 = (blockIdx.x * TPW + tt) * kTile;
        {
            const int r = t >> 2, cc = (t & 3) * 16;  // 16 elements of row r
            uint16_t* p = src + (int64_t)(r0 + r) * cols + c0 + cc;
            u32x4* v = vin[tt];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const float lo = div_by_block(__uint_as_float(v[h][c] << 16), rd);
                    const float hi = div_by_block(__uint_as_float(v[h][c] & 0xffff0000u), rd);
                    const uint32_t blo = from_f32<bf16_t>(lo).bits, bhi = from_f32<bf16_t>(hi).bits;
                    v[h][c] = blo | (bhi << 16);
                    tile[r][cc + 8 * h + 2 * c] = (uint16_t)blo;
                    tile[r][cc + 8 * h + 2 * c + 1] = (uint16_t)bhi;
                }
                if (WRITE_X) *reinterpret_cast<u32x4*>(p + 8 * h) = v[h];
            }
        }
        __syncthreads();
        {
            const int c = t >> 2, rr = (t & 3) * 16;  // 16 elements of column c (row c of x^T)
            uint16_t* q = dst + (int64_t)(c0 + c) * rows + r0 + rr;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                u32x4 v;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    v[k] = (uint32_t)tile[rr + 8 * h + 2 * k][c] | ((uint32_t)tile[rr + 8 * h + 2 * k + 1][c] << 16);
                *reinterpret_cast<u32x4*>(q + 8 * h) = v;
            }
        }
        if (TPW > 1) __syncthreads();  // the tile is rewritten by the next column tile
    }
}

template <bool WRITE_X>
void launch_scale_transpose(uint16_t* x, uint16_t* xt, int batch, int rows, int cols, const float* div,
                            const double* sumsq, const int32_t* index, float eps_bf16, hipStream_t st) {
    if (cols % (2 * kTile) == 0)
        hipLaunchKernelGGL((k_scale_transpose<2, WRITE_X>), dim3(cols / (2 * kTile), rows / kTile, batch), dim3(256), 0,
                           st, x, xt, rows, cols, div, sumsq, index, eps_bf16);
    else
        hipLaunchKernelGGL((k_scale_transpose<1, WRITE_X>), dim3(cols / kTile, rows / kTile, batch), dim3(256), 0, st,
                           x, xt, rows, cols, div, sumsq, index, eps_bf16);
}

// x[g] = bf16(x[g] / d_g) in place (d_g from the sums of squares as above):
// 8 elements per thread, rows * cols a multiple of 2048.
constexpr int kScaleElems = 256 * 8;
__global__ __launch_bounds__(256) void k_scale(uint16_t* __restrict__ x, int64_t per, const double* __restrict__ sumsq,
                                                const int32_t* __restrict__ index, float eps_bf16) {
    const int g = blockIdx.y;
    const double* slots = sumsq + (size_t)(index ? index[g] : g) * GEFEN_SUMSQ_STRIDE;
    double s = 0.0;
    for (int i = 0; i < GEFEN_SUMSQ_SLOTS; ++i) s += slots[16 * i];
    const double rd = 1.0 / (double)divisor_from_sumsq(s, eps_bf16);
    uint16_t* p = x + (int64_t)g * per + (int64_t)blockIdx.x * kScaleElems + 8 * threadIdx.x;
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t lo = from_f32<bf16_t>(div_by_block(__uint_as_float(v[c] << 16), rd)).bits;
        const uint32_t hi = from_f32<bf16_t>(div_by_block(__uint_as_float(v[c] & 0xffff0000u), rd)).bits;
        v[c] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(p) = v;
}

// ---------------------------------------------------------------------------
// parameter update (gefen_muon.py:325-329)
constexpr int kMaxApply = 24;
constexpr int kApplyThreads = 256;
constexpr int kApplyPer = kApplyThreads * 8;  // elements per workgroup

struct ApplyTask {
    void* p;
    const uint16_t* u;  // bf16 update, numel elements in the parameter's layout
    int64_t numel;
    float wdf;          // f32(1 - lr * wd)
    float alpha;        // f32(-lr_adj), rounded to the parameter dtype for reduced dtypes
    int32_t do_wd;
    int32_t round_prod;  // reduced dtype, transposed update: the product is rounded first
    int32_t vec;         // p and u 16-byte aligned
    int32_t nwg;
};
struct ApplyBatch {
    ApplyTask t[kMaxApply];
    int32_t wg_begin[kMaxApply + 1];
    int32_t ntasks;
};

template <typename D>
__device__ __forceinline__ float apply_one(float pf, float uf, const ApplyTask& T) {
    return muon_apply_value<D>(pf, uf, T.wdf, T.alpha, T.do_wd, T.round_prod);
}

template <typename D>
__global__ __launch_bounds__(kApplyThreads) void k_apply(const ApplyBatch B) {
    int ti = 0;
    while (ti + 1 < B.ntasks && B.wg_begin[ti + 1] <= (int)blockIdx.x) ++ti;
    const ApplyTask& T = B.t[ti];
    D* p = static_cast<D*>(T.p);
    const int64_t e = (int64_t)(blockIdx.x - B.wg_begin[ti]) * kApplyPer + (int64_t)threadIdx.x * 8;
    if (e >= T.numel) return;
    if (T.vec && e + 8 <= T.numel) {
        const u32x4 uv = *reinterpret_cast<const u32x4*>(T.u + e);
        Vec<D, 8> pv = vload<D, 8>(p, e);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t w = uv[c >> 1];
            const float uf = __uint_as_float((c & 1) ? (w & 0xffff0000u) : (w << 16));
            pv.v[c] = from_f32<D>(apply_one<D>(to_f32(pv.v[c]), uf, T));
        }
        vstore<D, 8>(p, e, pv);
    } else {
        const int64_t n = min((int64_t)8, T.numel - e);
        for (int64_t i = 0; i < n; ++i) {
            const float uf = __uint_as_float((uint32_t)T.u[e + i] << 16);
            p[e + i] = from_f32<D>(apply_one<D>(to_f32(p[e + i]), uf, T));
        }
    }
}

}  // namespace muon
}  // namespace gefen

using namespace gefen;

extern "C" int gefen_ns_prepare(void* x, void* xt, int batch, int rows, int cols, double eps,
                                gefen_stream_t stream) {
    if (batch < 0 || rows < 0 || cols < 0) return fail_inval("negative size");
    if (batch == 0 || rows == 0 || cols == 0) return GEFEN_OK;
    if (!x || !xt) return fail_inval("null tensor pointer");
    if (rows % muon::kTile || cols % muon::kTile)
        return fail_inval("gefen_ns_prepare needs rows and cols that are multiples of 64 (got %d, %d)", rows, cols);
    if (!aligned(x, 16) || !aligned(xt, 16)) return fail_inval("gefen_ns_prepare needs 16-byte aligned buffers");
    if (batch > 65535) return fail_inval("batch too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t per = (int64_t)rows * cols;
    const int nblk = (int)((per + muon::kNormChunk - 1) / muon::kNormChunk);
    void* ws = nullptr;
    hipError_t e = device_malloc_async(&ws, ((size_t)batch * nblk + batch) * sizeof(float), st);
    if (e != hipSuccess) return hip_status(e, "hipMallocAsync(norm partials)");
    float* partial = static_cast<float*>(ws);
    float* div = partial + (size_t)batch * nblk;
    const float eps_bf16 = muon::eps_to_bf16(eps);
    auto* X = static_cast<uint16_t*>(x);
    hipLaunchKernelGGL(muon::k_sumsq, dim3(nblk, batch), dim3(muon::kNormThreads), 0, st, X, per, nblk, partial);
    int rc = launch_status("gefen_ns_prepare (norm)");
    if (rc == GEFEN_OK) {
        hipLaunchKernelGGL(muon::k_norm, dim3((batch + 63) / 64), dim3(64), 0, st, partial, nblk, batch, eps_bf16, div);
        rc = launch_status("gefen_ns_prepare (norm)");
    }
    if (rc == GEFEN_OK) {
        muon::launch_scale_transpose<true>(X, static_cast<uint16_t*>(xt), batch, rows, cols, div, nullptr, nullptr, 0.0f,
                                           st);
        rc = launch_status("gefen_ns_prepare (scale)");
    }
    (void)hipFreeAsync(ws, st);
    return rc;
}

extern "C" int gefen_ns_prepare_sumsq(void* x, void* xt, int batch, int rows, int cols, double eps,
                                     const double* sumsq, const int32_t* index, gefen_stream_t stream) {
    if (batch < 0 || rows < 0 || cols < 0) return fail_inval("negative size");
    if (batch == 0 || rows == 0 || cols == 0) return GEFEN_OK;
    if (!x || !xt || !sumsq) return fail_inval("null pointer");
    if (rows % muon::kTile || cols % muon::kTile)
        return fail_inval("gefen_ns_prepare needs rows and cols that are multiples of 64 (got %d, %d)", rows, cols);
    if (!aligned(x, 16) || !aligned(xt, 16)) return fail_inval("gefen_ns_prepare needs 16-byte aligned buffers");
    if (batch > 65535) return fail_inval("batch too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    muon::launch_scale_transpose<true>(static_cast<uint16_t*>(x), static_cast<uint16_t*>(xt), batch, rows, cols,
                                       nullptr, sumsq, index, muon::eps_to_bf16(eps), st);
    return launch_status("gefen_ns_prepare_sumsq");
}

extern "C" int gefen_ns_normalize_sumsq(void* x, void* out, int batch, int rows, int cols, double eps,
                                        const double* sumsq, const int32_t* index, int transpose,
                                        gefen_stream_t stream) {
    if (batch < 0 || rows < 0 || cols < 0) return fail_inval("negative size");
    if (batch == 0 || rows == 0 || cols == 0) return GEFEN_OK;
    if (!x || !sumsq || (transpose && !out)) return fail_inval("null pointer");
    if (rows % muon::kTile || cols % muon::kTile)
        return fail_inval("gefen_ns_normalize_sumsq needs rows and cols that are multiples of 64 (got %d, %d)", rows,
                          cols);
    if (!aligned(x, 16) || (out && !aligned(out, 16))) return fail_inval("gefen_ns_normalize_sumsq needs 16-byte aligned buffers");
    if (batch > 65535) return fail_inval("batch too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (transpose) {
        if (out == x) return fail_inval("the transposed output cannot overwrite its input");
        muon::launch_scale_transpose<false>(static_cast<uint16_t*>(x), static_cast<uint16_t*>(out), batch, rows, cols,
                                            nullptr, sumsq, index, muon::eps_to_bf16(eps), st);
    } else {
        if (out && out != x) return fail_inval("the normalisation without transpose is in place (out must be x or null)");
        const int64_t per = (int64_t)rows * cols;  // a multiple of 4096
        hipLaunchKernelGGL(muon::k_scale, dim3((unsigned)(per / muon::kScaleElems), batch), dim3(256), 0, st,
                           static_cast<uint16_t*>(x), per, sumsq, index, muon::eps_to_bf16(eps));
    }
    return launch_status("gefen_ns_normalize_sumsq");
}

extern "C" int gefen_muon_apply_tasks(const gefen_muon_apply_task* tasks, int ntasks, gefen_stream_t stream) {
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    for (int dt : {GEFEN_F32, GEFEN_BF16, GEFEN_F16}) {
        muon::ApplyBatch b;
        memset(&b, 0, sizeof(b));
        int n = 0;
        int64_t wg = 0;
        auto flush = [&]() -> int {
            if (n == 0) return GEFEN_OK;
            b.wg_begin[n] = (int32_t)wg;
            b.ntasks = n;
            if (dt == GEFEN_F32) hipLaunchKernelGGL(muon::k_apply<float>, dim3((unsigned)wg), dim3(muon::kApplyThreads), 0, st, b);
            else if (dt == GEFEN_BF16) hipLaunchKernelGGL(muon::k_apply<bf16_t>, dim3((unsigned)wg), dim3(muon::kApplyThreads), 0, st, b);
            else hipLaunchKernelGGL(muon::k_apply<f16_t>, dim3((unsigned)wg), dim3(muon::kApplyThreads), 0, st, b);
            int rc = launch_status("gefen_muon_apply_tasks");
            memset(&b, 0, sizeof(b));
            n = 0;
            wg = 0;
            return rc;
        };
        for (int i = 0; i < ntasks; ++i) {
            const gefen_muon_apply_task& in = tasks[i];
            if (!valid_dtype(in.param_dtype)) return fail_inval("unsupported parameter dtype %d", in.param_dtype);
            if (in.param_dtype != dt || in.numel == 0) continue;
            if (in.numel < 0) return fail_inval("numel must be non-negative");
            if (!in.p || !in.update) return fail_inval("null tensor pointer");
            const int64_t nwg = (in.numel + muon::kApplyPer - 1) / muon::kApplyPer;
            if (nwg > INT32_MAX / 2) return fail_inval("tensor too large");
            if (n == muon::kMaxApply || wg + nwg > INT32_MAX) {
                int rc = flush();
                if (rc) return rc;
            }
            muon::ApplyTask& t = b.t[n];
            t.p = in.p;
            t.u = static_cast<const uint16_t*>(in.update);
            t.numel = in.numel;
            const MuonApplyScalars sc = muon_apply_scalars(in);
            t.wdf = sc.wdf;
            t.alpha = sc.alpha;
            t.do_wd = sc.do_wd;
            t.round_prod = sc.round_prod;
            const int esz = dtype_size(dt);
            t.vec = aligned(in.p, 8 * esz) && aligned(in.update, 16) ? 1 : 0;
            t.nwg = (int32_t)nwg;
            b.wg_begin[n] = (int32_t)wg;
            wg += nwg;
            ++n;
        }
        int rc = flush();
        if (rc) return rc;
    }
    return GEFEN_OK;
}

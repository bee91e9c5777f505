// Partition-block statistics for the automatic period (partitioning.py).
//
// Score of a divisor p of n (partitioning.py:43-78): with L_i = log(x_i + eps),
// m_j the mean of L over block j of p elements, score = mean_j |m_{j+1} - m_j|.
// All divisors of one gradient are scored together: block sums of a divisor p
// are built from the block sums of its largest listed divisor q | p (or from
// the values when there is none), so the logarithms are evaluated once per
// base divisor instead of once per divisor, and no host synchronisation happens
// between divisors.  float64 throughout; block sums are formed in a fixed
// order, so the scores agree with numpy's pairwise sums to ~1e-15 relative.
#include <math.h>
#include <string.h>

#include <vector>

#include "capi_internal.h"
#include "common.h"

namespace gefen {

// x of one element: mode 0 = f64(f32(v)); 1 = f64(f32(v)*f32(v)); 2 = f64(f32(v))^2
template <typename T>
__device__ __forceinline__ double transform(T raw, int mode) {
    const float v = to_f32(raw);
    if (mode == 1) {
        const float sq = v * v;
        return (double)sq;
    }
    const double d = (double)v;
    if (mode == 2) return d * d;
    return d;
}

// out[j] = sum over block j (blen items) of f(src).  Lane groups of 2^lpr_log2
// lanes per block; each lane sums its strided items in order, then a butterfly.
template <typename T, bool LOG>
__global__ __launch_bounds__(256) void k_block_sums(const T* __restrict__ src, int64_t nblocks, int64_t blen,
                                                    int lpr_log2, int mode, double eps, double* __restrict__ out,
                                                    unsigned long long* __restrict__ invalid) {
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int lir = lane & (lpr - 1);
    const int64_t rpw = 64 >> lpr_log2;
    const int64_t units = (nblocks + rpw - 1) / rpw;
    for (int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); unit < units; unit += (int64_t)gridDim.x * 4) {
        const int64_t blk = unit * rpw + (lane >> lpr_log2);
        const bool active = blk < nblocks;
        double s = 0.0;
        unsigned bad = 0;
        if (active) {
            const int64_t base = blk * blen;
            for (int64_t j = lir; j < blen; j += lpr) {
                if constexpr (LOG) {
                    const double y = transform(src[base + j], mode) + eps;
                    if (y <= 0.0) ++bad;  // numpy / the reference: NaN does not count
                    s = s + log(y);
                } else {
                    s = s + (double)src[base + j];
                }
            }
        }
        for (int off = lpr >> 1; off > 0; off >>= 1) s = s + __shfl_xor(s, off, 64);
        if (invalid && bad) atomicAdd(invalid, (unsigned long long)bad);
        if (active && lir == 0) out[blk] = s;
    }
}

// partial[b] = sum over its slice of |S[j+1]/p - S[j]/p|, j < nblocks - 1, for
// every divisor of a batch: divisor t owns workgroups [wg_begin[t], wg_begin[t+1])
// (one per partial), so all divisors of a gradient take one launch.
constexpr int kAdjBatch = 80;
struct AdjBatch {
    int64_t s_off[kAdjBatch];    // element offset of the divisor's block sums in S
    int64_t nblocks[kAdjBatch];
    int64_t p_off[kAdjBatch];    // offset of the divisor's first partial
    double p[kAdjBatch];
    int32_t wg_begin[kAdjBatch + 1];
    int32_t count;
};
static_assert(sizeof(AdjBatch) <= 4000, "kernel arguments are limited to 4 KB");

__global__ __launch_bounds__(256) void k_adjacent_partials(const double* __restrict__ S0, const AdjBatch B,
                                                           double* __restrict__ partial0) {
    __shared__ double red[4];
    int t = 0;
    {
        int lo_t = 0, hi_t = B.count - 1;
        while (lo_t < hi_t) {
            const int mid = (lo_t + hi_t + 1) >> 1;
            if (B.wg_begin[mid] <= (int)blockIdx.x) lo_t = mid;
            else hi_t = mid - 1;
        }
        t = lo_t;
    }
    const double* __restrict__ S = S0 + B.s_off[t];
    double* __restrict__ partial = partial0 + B.p_off[t];
    const double p = B.p[t];
    const int nwg = B.wg_begin[t + 1] - B.wg_begin[t];
    const int wb = (int)blockIdx.x - B.wg_begin[t];
    const int64_t ndiff = B.nblocks[t] - 1;
    const int64_t per = (ndiff + nwg - 1) / nwg;
    const int64_t lo = (int64_t)wb * per;
    const int64_t hi = lo + per < ndiff ? lo + per : ndiff;
    double s = 0.0;
    for (int64_t j = lo + threadIdx.x; j < hi; j += 256) {
        const double a = S[j] / p, b = S[j + 1] / p;
        s = s + fabs(b - a);
    }
    for (int off = 32; off > 0; off >>= 1) s = s + __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) partial[wb] = (red[0] + red[1]) + (red[2] + red[3]);
}

// score[d] = (sum of partials of divisor d in order) / (nblocks_d - 1); score[ndiv] = invalid count
constexpr int kFinalBatch = 96;
struct FinalBatch {
    int64_t pbegin[kFinalBatch];
    int64_t nblk[kFinalBatch];
    int32_t pcount[kFinalBatch];
    int32_t first;  // index of the first divisor of this batch
    int32_t count;
};

__global__ void k_adjacent_final(const double* __restrict__ partial, const FinalBatch B, int ndiv,
                                 const unsigned long long* __restrict__ invalid, double* __restrict__ scores) {
    const int i = threadIdx.x;
    if (i < B.count) {
        double s = 0.0;
        for (int k = 0; k < B.pcount[i]; ++k) s = s + partial[B.pbegin[i] + k];
        scores[B.first + i] = s / (double)(B.nblk[i] - 1);
    }
    if (i == 0 && B.first == 0) scores[ndiv] = (double)(*invalid);
}

__global__ void k_zero_u64(unsigned long long* p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0ull;
}
__global__ void k_zero_f64(double* p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0.0;
}

// ------------------------------------------------------------------ variance / CoV
template <typename T>
__global__ __launch_bounds__(256) void k_block_var(const T* __restrict__ v, int64_t nblocks, int64_t period,
                                                   int squared, int cov, double* __restrict__ acc) {
    const int lane = threadIdx.x & 63;
    for (int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); blk < nblocks; blk += (int64_t)gridDim.x * 4) {
        const int64_t base = blk * period;
        float sx = 0.0f, sx2 = 0.0f;
        for (int64_t j = lane; j < period; j += 64) {
            const float a = to_f32(v[base + j]);
            const float x = squared ? a : a * a;
            const float x2 = x * x;
            sx = sx + x;
            sx2 = sx2 + x2;
        }
        sx = group_sum(sx, 64);
        sx2 = group_sum(sx2, 64);
        if (lane == 0) {
            const float mean = sx / (float)period;
            float var = sx2 / (float)period;
            const float m2 = mean * mean;
            var = var - m2;
            if (var < 0.0f) var = 0.0f;
            if (!cov) {
                atomicAdd(&acc[0], (double)var);
            } else if (mean < 0.0f) {
                atomicAdd(&acc[2], 1.0);
            } else if (mean > 0.0f) {
                atomicAdd(&acc[0], (double)(sqrtf(var) / mean));
                atomicAdd(&acc[1], 1.0);
            }
        }
    }
}

__global__ void k_var_final(double* acc, int64_t nblocks) { acc[0] = sqrt(acc[0] / (double)nblocks); }

namespace {
int lpr_log2_for_len(int64_t len) {
    int l = 0;
    while ((1LL << l) < len && l < 6) ++l;
    return l;
}
int grid_cap(int64_t units) {
    int64_t g = (units + 3) / 4;
    if (g < 1) g = 1;
    if (g > 4096) g = 4096;
    return (int)g;
}

struct Plan {
    std::vector<int64_t> off;     // byte offset of each divisor's block sums
    std::vector<int> parent;      // index of the parent divisor, -1 = from values
    std::vector<int64_t> pbegin;  // first partial of each divisor
    std::vector<int32_t> pcount;  // number of partials
    size_t sums_bytes = 0, partial_count = 0, total = 0;
    size_t off_partial = 0, off_invalid = 0;
};

constexpr int kPartials = 256;

int make_plan(int64_t n, const int64_t* divs, int ndiv, Plan& P) {
    P.off.resize(ndiv);
    P.parent.assign(ndiv, -1);
    P.pbegin.resize(ndiv);
    P.pcount.resize(ndiv);
    size_t o = 0, pc = 0;
    for (int d = 0; d < ndiv; ++d) {
        const int64_t p = divs[d];
        if (p <= 0 || n % p) return fail_inval("divisor %lld does not divide numel %lld", (long long)p, (long long)n);
        if (n / p < 2) return fail_inval("Expected at least two blocks to compare adjacent block means.");
        if (d > 0 && divs[d] <= divs[d - 1]) return fail_inval("divisors must be strictly ascending");
        int best = -1;
        for (int e = 0; e < d; ++e)
            if (p % divs[e] == 0 && (best < 0 || divs[e] > divs[best])) best = e;
        P.parent[d] = best;
        P.off[d] = (int64_t)o;
        o += sizeof(double) * (size_t)(n / p);
        o = (o + 255) & ~(size_t)255;
        const int64_t ndiff = n / p - 1;
        const int64_t np = ndiff < kPartials ? ndiff : kPartials;
        P.pbegin[d] = (int64_t)pc;
        P.pcount[d] = (int32_t)np;
        pc += (size_t)np;
    }
    P.sums_bytes = o;
    P.partial_count = pc;
    P.off_partial = o;
    o += sizeof(double) * pc;
    o = (o + 255) & ~(size_t)255;
    P.off_invalid = o;
    o += 256;
    P.total = o;
    return GEFEN_OK;
}

template <typename T>
void launch_block_sums_values(const T* v, int64_t nblocks, int64_t blen, int mode, double eps, double* out,
                              unsigned long long* invalid, hipStream_t st) {
    const int l2 = lpr_log2_for_len(blen);
    const int64_t units = (nblocks + (64 >> l2) - 1) / (64 >> l2);
    hipLaunchKernelGGL((k_block_sums<T, true>), dim3(grid_cap(units)), dim3(256), 0, st, v, nblocks, blen, l2,
                       mode, eps, out, invalid);
}

int run_scores(const void* values, int dtype, int64_t n, const int64_t* divs, int ndiv, int mode, double eps,
               double* scores, char* ws, const Plan& P, hipStream_t st) {
    unsigned long long* invalid = reinterpret_cast<unsigned long long*>(ws + P.off_invalid);
    hipLaunchKernelGGL(k_zero_u64, dim3(1), dim3(64), 0, st, invalid, 1);
    int rc = launch_status("gefen period zero");
    if (rc) return rc;
    bool counted = false;
    for (int d = 0; d < ndiv; ++d) {
        const int64_t p = divs[d];
        double* S = reinterpret_cast<double*>(ws + P.off[d]);
        const int64_t nb = n / p;
        if (P.parent[d] < 0) {
            // the first base divisor also counts the inputs with x + eps <= 0
            unsigned long long* inv = counted ? nullptr : invalid;
            counted = true;
            if (dtype == GEFEN_F32)
                launch_block_sums_values(static_cast<const float*>(values), nb, p, mode, eps, S, inv, st);
            else if (dtype == GEFEN_BF16)
                launch_block_sums_values(static_cast<const bf16_t*>(values), nb, p, mode, eps, S, inv, st);
            else
                launch_block_sums_values(static_cast<const f16_t*>(values), nb, p, mode, eps, S, inv, st);
        } else {
            const int q = P.parent[d];
            const int64_t r = p / divs[q];
            const int l2 = lpr_log2_for_len(r);
            const int64_t units = (nb + (64 >> l2) - 1) / (64 >> l2);
            hipLaunchKernelGGL((k_block_sums<double, false>), dim3(grid_cap(units)), dim3(256), 0, st,
                               reinterpret_cast<const double*>(ws + P.off[q]), nb, r, l2, 0, 0.0, S, nullptr);
        }
        rc = launch_status("gefen period block sums");
        if (rc) return rc;
    }
    // the adjacent-difference partials of every divisor, kAdjBatch divisors per launch
    for (int first = 0; first < ndiv; first += kAdjBatch) {
        AdjBatch B;
        memset(&B, 0, sizeof(B));
        B.count = ndiv - first < kAdjBatch ? ndiv - first : kAdjBatch;
        int32_t wg = 0;
        for (int i = 0; i < B.count; ++i) {
            const int d = first + i;
            B.s_off[i] = P.off[d] / (int64_t)sizeof(double);
            B.nblocks[i] = n / divs[d];
            B.p_off[i] = P.pbegin[d];
            B.p[i] = (double)divs[d];
            B.wg_begin[i] = wg;
            wg += P.pcount[d];
        }
        B.wg_begin[B.count] = wg;
        hipLaunchKernelGGL(k_adjacent_partials, dim3(wg), dim3(256), 0, st, reinterpret_cast<const double*>(ws), B,
                           reinterpret_cast<double*>(ws + P.off_partial));
        rc = launch_status("gefen period partials");
        if (rc) return rc;
    }
    for (int first = 0; first < ndiv; first += kFinalBatch) {
        FinalBatch B;
        memset(&B, 0, sizeof(B));
        B.first = first;
        B.count = ndiv - first < kFinalBatch ? ndiv - first : kFinalBatch;
        for (int i = 0; i < B.count; ++i) {
            B.pbegin[i] = P.pbegin[first + i];
            B.nblk[i] = n / divs[first + i];
            B.pcount[i] = P.pcount[first + i];
        }
        hipLaunchKernelGGL(k_adjacent_final, dim3(1), dim3(kFinalBatch), 0, st,
                           reinterpret_cast<const double*>(ws + P.off_partial), B, ndiv, invalid, scores);
        rc = launch_status("gefen period final");
        if (rc) return rc;
    }
    return GEFEN_OK;
}

int check_values(const void* v, int dt, int64_t n, int64_t period) {
    if (!valid_dtype(dt)) return fail_inval("Expected a floating-point tensor.");
    if (period <= 0) return fail_inval("Expected a positive period.");
    if (n <= 0) return fail_inval("Expected a non-empty tensor.");
    if (n % period) return fail_inval("Expected tensor length to be divisible by period.");
    if (!v) return fail_inval("null values pointer");
    return GEFEN_OK;
}
}  // namespace
}  // namespace gefen

using namespace gefen;

extern "C" size_t gefen_period_scores_workspace_size(int64_t numel, const int64_t* divs, int ndiv) {
    if (numel <= 0 || ndiv <= 0 || !divs) return 0;
    Plan P;
    if (make_plan(numel, divs, ndiv, P)) return 0;
    return P.total;
}

extern "C" int gefen_period_scores(const void* values, int dtype, int64_t numel, const int64_t* divs, int ndiv,
                                   int mode, double epsilon, double* scores, void* workspace,
                                   gefen_stream_t stream) {
    if (ndiv <= 0 || !divs) return fail_inval("no divisors");
    int rc = check_values(values, dtype, numel, 1);
    if (rc) return rc;
    if (mode < 0 || mode > 2) return fail_inval("invalid mode %d", mode);
    if (!scores || !workspace) return fail_inval("null pointer");
    Plan P;
    rc = make_plan(numel, divs, ndiv, P);
    if (rc) return rc;
    return run_scores(values, dtype, numel, divs, ndiv, mode, epsilon, scores, static_cast<char*>(workspace), P,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int gefen_average_adjacent_log_block_mean_difference(const void* values, int dtype, int64_t numel,
                                                                int64_t period, int input_is_squared,
                                                                double epsilon, double* out,
                                                                gefen_stream_t stream) {
    int rc = check_values(values, dtype, numel, period);
    if (rc) return rc;
    if (!(epsilon > 0.0)) return fail_inval("Expected a positive epsilon.");
    if (numel / period < 2) return fail_inval("Expected at least two blocks to compare adjacent block means.");
    if (!out) return fail_inval("null output pointer");
    const int64_t divs[1] = {period};
    Plan P;
    rc = make_plan(numel, divs, 1, P);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    void* ws = nullptr;
    hipError_t e = device_malloc_async(&ws, P.total, st);
    if (e != hipSuccess) return hip_status(e, "hipMallocAsync(period workspace)");
    rc = run_scores(values, dtype, numel, divs, 1, input_is_squared ? 0 : 2, epsilon, out, static_cast<char*>(ws),
                    P, st);
    (void)hipFreeAsync(ws, st);
    return rc;
}

static int block_var_common(const void* values, int dtype, int64_t numel, int64_t period, int squared, double* out,
                            int cov, gefen_stream_t stream) {
    int rc = check_values(values, dtype, numel, period);
    if (rc) return rc;
    if (!out) return fail_inval("null output pointer");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(k_zero_f64, dim3(1), dim3(64), 0, st, out, cov ? 3 : 1);
    rc = launch_status("gefen block variance zero");
    if (rc) return rc;
    const int64_t nb = numel / period;
    const int grid = grid_cap(nb);
    if (dtype == GEFEN_F32)
        hipLaunchKernelGGL(k_block_var<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(values), nb,
                           period, squared, cov, out);
    else if (dtype == GEFEN_BF16)
        hipLaunchKernelGGL(k_block_var<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(values), nb,
                           period, squared, cov, out);
    else
        hipLaunchKernelGGL(k_block_var<f16_t>, dim3(grid), dim3(256), 0, st, static_cast<const f16_t*>(values), nb,
                           period, squared, cov, out);
    rc = launch_status("gefen block variance");
    if (rc || cov) return rc;
    hipLaunchKernelGGL(k_var_final, dim3(1), dim3(1), 0, st, out, nb);
    return launch_status("gefen block variance final");
}

extern "C" int gefen_average_within_block_variance(const void* values, int dtype, int64_t numel, int64_t period,
                                                   int input_is_squared, double* out, gefen_stream_t stream) {
    return block_var_common(values, dtype, numel, period, input_is_squared, out, 0, stream);
}

extern "C" int gefen_average_within_block_coefficient_of_variation(const void* values, int dtype, int64_t numel,
                                                                   int64_t period, int input_is_squared,
                                                                   double* out, gefen_stream_t stream) {
    return block_var_common(values, dtype, numel, period, input_is_squared, out, 1, stream);
}

// Codebook learning on the device: lookup tables for the nearest-codeword
// search, the block-normalised 4096-bin histogram, the exact-DP quantiser and
// the Lloyd-Max accumulators.
//
// Histogram: gefen.py:350-366.  Exact DP: quantization.py:206-258 with the
// histogram statistics of gefen.py:373-399; the DP is evaluated level by level
// (one launch per cluster count), one wave per segment end, with the
// reference's strict "<" (first best start wins) reproduced by a lexicographic
// (cost, start) minimum.  All float64 arithmetic is written without
// contraction, so every cost and codeword equals the reference's.
#include <math.h>
#include <string.h>

#include "capi_internal.h"
#include "common.h"

namespace gefen {

// ---------------------------------------------------------------------------
// codebook tables (see CodebookTables in common.h)
__device__ __forceinline__ int32_t f_ord(float x) {
    const uint32_t b = __float_as_uint(x);
    return (b & 0x80000000u) ? -(int32_t)(b & 0x7fffffffu) : (int32_t)b;
}
__device__ __forceinline__ float f_dec(int32_t o) {
    return o >= 0 ? __uint_as_float((uint32_t)o) : __uint_as_float(0x80000000u | (uint32_t)(-o));
}

// byte offsets of the fields the GPU tests read from a prepared table
static_assert(offsetof(CodebookTables, bucket_fine) == 6176 && offsetof(CodebookTables, max_probe) == 22588 &&
                  offsetof(CodebookTables, max_probe_fine) == 22592 && offsetof(CodebookTables, nb16) == 22608,
              "codebook table layout");

__global__ __launch_bounds__(256) void k_prepare_codebook(const float* __restrict__ cb, int K,
                                                          CodebookTables* __restrict__ T) {
    __shared__ float thr[260];
    __shared__ uint16_t bk[kFineCells + 1];
    __shared__ int probe_max, probe_max_fine;
    const int t = threadIdx.x;
    T->cb[t] = t < K ? cb[t] : __builtin_inff();
    if (t == 0) T->K = K;
    // thr[k], k = 1..K-1: largest x in (cb[k-1], cb[k]] where the left entry wins
    for (int k = t; k < 260; k += 256) {
        float v = __builtin_inff();
        if (k >= 1 && k < K) {
            const float a = cb[k - 1], b = cb[k];
            if (!(b > a)) {
                v = a;
            } else {
                int32_t lo = f_ord(a), hi = f_ord(b);  // pred(lo) holds (or lo is a), pred(hi) fails
                while (hi - lo > 1) {
                    const int32_t mid = lo + (hi - lo) / 2;
                    const float x = f_dec(mid);
                    if (fabsf(x - a) <= fabsf(x - b)) lo = mid; else hi = mid;
                }
                v = f_dec(lo);
            }
        } else if (k == 0) {
            v = -__builtin_inff();
        }
        thr[k] = v;
        T->thr[k] = v;
    }
    __syncthreads();
    // bucket_fine[e] = #{k in 1..K-1 : thr[k] < -1 + e/4096}; bucket[e] = bucket8[e] = bucket_fine[2e]
    for (int e = t; e <= kFineCells; e += 256) {
        const float edge = -1.0f + (float)e * 0.000244140625f;  // exact: a multiple of 2^-12
        int lo = 1, hi = K;  // first k in [1, K) with thr[k] >= edge
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (thr[mid] < edge) lo = mid + 1; else hi = mid;
        }
        const uint16_t c = (uint16_t)(lo - 1);
        T->bucket_fine[e] = (uint8_t)c;  // c <= K - 1 <= 255
        if (!(e & 1)) {
            T->bucket[e >> 1] = c;
            T->bucket8[e >> 1] = (uint8_t)c;
        }
        bk[e] = c;
    }
    for (int e = kFineCells + 1 + t; e < kFineBytes; e += 256) T->bucket_fine[e] = 0;
    if (t < kBucket8Bytes - 4097) T->bucket8[4097 + t] = 0;
    if (t < 3) T->bucket[4097 + t] = 0;
    if (t == 0) probe_max = probe_max_fine = 0;
    __syncthreads();
    // a search from bucket b (one below x's bucket) meets the thresholds in
    // [edge_b, edge_b+2); past the last edges it meets every finite one left
    int worst = 0, worst_fine = 0;
    for (int b = t; b <= kFineCells; b += 256) {
        const int hi = (b + 2 <= kFineCells) ? (int)bk[b + 2] : (K - 1);
        const int n = hi - (int)bk[b];
        worst_fine = n > worst_fine ? n : worst_fine;
        if (!(b & 1)) {
            const int hc = (b + 4 <= kFineCells) ? (int)bk[b + 4] : (K - 1);
            const int nc = hc - (int)bk[b];
            worst = nc > worst ? nc : worst;
        }
    }
    atomicMax(&probe_max, worst);
    atomicMax(&probe_max_fine, worst_fine);
    __syncthreads();
    if (t == 0) {
        T->max_probe = (bk[0] != 0) ? 1 << 20 : probe_max;
        T->max_probe_fine = (bk[0] != 0) ? 1 << 20 : probe_max_fine;
    }
    // nb16: #{k in 1..K-1 : thr[k] < x} for the bf16 values x of the table
    for (int i = t; i < kNb16Bytes; i += 256) {
        uint8_t c = 0;
        if (i < 2 * (int)kNb16Side) {
            const uint32_t bits = i >= (int)kNb16Side ? kNb16Lo + (uint32_t)(i - (int)kNb16Side)
                                                      : 0x8000u | (kNb16Lo + kNb16Side - 1u - (uint32_t)i);
            const float x = __uint_as_float(bits << 16);
            int lo = 1, hi = K;  // first k in [1, K) with thr[k] >= x
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (thr[mid] < x) lo = mid + 1; else hi = mid;
            }
            c = (uint8_t)(lo - 1);
        }
        T->nb16[i] = c;
    }
}

// ---------------------------------------------------------------------------
// histogram: one lane group per block row, LDS-privatised counts per workgroup
template <typename G>
__global__ __launch_bounds__(256) void k_histogram(const G* __restrict__ g, int64_t nrows, int64_t period,
                                                   int lpr_log2, int bins, float bw,
                                                   unsigned long long* __restrict__ counts) {
    __shared__ uint32_t h[4096];
    for (int i = threadIdx.x; i < bins; i += 256) h[i] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int lir = lane & (lpr - 1);
    const int64_t rpw = 64 >> lpr_log2;
    const int64_t units = (nrows + rpw - 1) / rpw;
    for (int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); unit < units;
         unit += (int64_t)gridDim.x * 4) {
        const int64_t row = unit * rpw + (lane >> lpr_log2);
        const bool active = row < nrows;
        const int64_t base = row * period;
        float amax = 0.0f;
        if (active)
            for (int64_t j = lir; j < period; j += lpr) amax = nanmax(amax, fabsf(to_f32(g[base + j])));
        amax = group_max(amax, lpr);
        if (!active) continue;
        for (int64_t j = lir; j < period; j += lpr) {
            const float v = to_f32(g[base + j]);
            const float x = (amax > 0.0f) ? v / amax : 0.0f;
            const float y = floorf((x + 1.0f) / bw);
            int b;
            if (!(y >= 0.0f)) b = 0;  // negative, or NaN (-> INT64_MIN) clamps to 0
            else if (y >= (float)(bins - 1)) b = bins - 1;
            else b = (int)y;
            atomicAdd(&h[b], 1u);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < bins; i += 256)
        if (h[i]) atomicAdd(&counts[i], (unsigned long long)h[i]);
}

__global__ void k_accumulate_counts(float* __restrict__ acc, const int64_t* __restrict__ counts, int bins) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < bins) acc[i] = acc[i] + (float)counts[i];
}

// ---------------------------------------------------------------------------
// exact DP workspace:
//   header  int32[64]      : [0] N active bins, [1] status (0 ok, 1 padded done, 2 empty)
//   pw, pwx, pwx2          : double[bins + 1] each (prefix sums, sequential order)
//   dp                     : double[(K + 1) * (bins + 1)], level-major
//   bt                     : int32[(K + 1) * (bins + 1)]
//   cw                     : float[bins] active centres
struct DpLayout {
    size_t pw, pwx, pwx2, dp, bt, cw, total;
    DpLayout(int bins, int K) {
        size_t o = 256;
        pw = o;  o += sizeof(double) * (bins + 1);
        pwx = o; o += sizeof(double) * (bins + 1);
        pwx2 = o; o += sizeof(double) * (bins + 1);
        dp = o;  o += sizeof(double) * (size_t)(K + 1) * (bins + 1);
        bt = o;  o += sizeof(int32_t) * (size_t)(K + 1) * (bins + 1);
        cw = o;  o += sizeof(float) * bins;
        total = o;
    }
};

constexpr int kDpMaxBins = 4096;
constexpr int kDpInitThreads = 256;

// Active bins (count > 0) in bin order, their centres -1 + (2b+1)/bins (exact
// for power-of-two bins), and the float64 prefix sums of w, w x, w x^2
// (torch.cumsum on the CPU, quantization.py:226-231: the element products in
// parallel, then the sums in sequential order).  The workgroup compacts the
// active bins into LDS (a scan of per-thread counts); one thread then runs the
// three running sums in registers.
__global__ __launch_bounds__(kDpInitThreads) void k_dp_init(const float* __restrict__ counts, int bins, int K,
                                                            int force, char* __restrict__ ws, DpLayout L,
                                                            float* __restrict__ out) {
    constexpr int kPer = kDpMaxBins / kDpInitThreads;  // bins per thread
    __shared__ double sw_[kDpMaxBins], swx_[kDpMaxBins], swx2_[kDpMaxBins];
    __shared__ int offs[kDpInitThreads + 1];
    int32_t* hdr = reinterpret_cast<int32_t*>(ws);
    double* pw = reinterpret_cast<double*>(ws + L.pw);
    double* pwx = reinterpret_cast<double*>(ws + L.pwx);
    double* pwx2 = reinterpret_cast<double*>(ws + L.pwx2);
    double* dp = reinterpret_cast<double*>(ws + L.dp);
    float* cw = reinterpret_cast<float*>(ws + L.cw);
    const int t = threadIdx.x;
    const int b0 = t * kPer;  // this thread's bins b0 .. b0 + kPer - 1 (in order)
    int mine = 0;
    for (int k = 0; k < kPer; ++k) mine += (b0 + k < bins && counts[b0 + k] > 0.0f) ? 1 : 0;
    offs[t + 1] = mine;
    if (t == 0) offs[0] = 0;
    __syncthreads();
    if (t == 0)
        for (int i = 1; i <= kDpInitThreads; ++i) offs[i] += offs[i - 1];
    __syncthreads();
    const double inv_bins = 1.0 / (double)bins;  // exact: bins is a power of two
    int n = offs[t];
    for (int k = 0; k < kPer; ++k) {
        const int b = b0 + k;
        if (b >= bins) break;
        const float c = counts[b];
        if (c > 0.0f) {
            const float center = (float)(-1.0 + (2.0 * b + 1.0) * inv_bins);
            const double w = (double)c, x = (double)center;
            sw_[n] = w;
            swx_[n] = w * x;
            swx2_[n] = w * (x * x);
            cw[n] = center;
            ++n;
        }
    }
    __syncthreads();
    const int N = offs[kDpInitThreads];
    if (t == 0) {  // the running sums in bin order, in place in LDS (16 elements read ahead)
        constexpr int kB = 16;
        double a0 = 0.0, a1 = 0.0, a2 = 0.0;
        int i = 0;
        for (; i + kB <= N; i += kB) {
            double v0[kB], v1[kB], v2[kB];
#pragma unroll
            for (int u = 0; u < kB; ++u) { v0[u] = sw_[i + u]; v1[u] = swx_[i + u]; v2[u] = swx2_[i + u]; }
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                a0 = a0 + v0[u];
                a1 = a1 + v1[u];
                a2 = a2 + v2[u];
                v0[u] = a0;
                v1[u] = a1;
                v2[u] = a2;
            }
#pragma unroll
            for (int u = 0; u < kB; ++u) { sw_[i + u] = v0[u]; swx_[i + u] = v1[u]; swx2_[i + u] = v2[u]; }
        }
        for (; i < N; ++i) {
            a0 = a0 + sw_[i];
            a1 = a1 + swx_[i];
            a2 = a2 + swx2_[i];
            sw_[i] = a0;
            swx_[i] = a1;
            swx2_[i] = a2;
        }
    }
    __syncthreads();
    for (int i = t; i <= N; i += kDpInitThreads) {
        pw[i] = i ? sw_[i - 1] : 0.0;
        pwx[i] = i ? swx_[i - 1] : 0.0;
        pwx2[i] = i ? swx2_[i - 1] : 0.0;
    }
    if (N > 0 && K <= N)  // dp[0][e]: no segmentation of e > 0 points into zero clusters
        for (int e = t; e <= N; e += kDpInitThreads) dp[e] = e ? __builtin_inf() : 0.0;
    if (t != 0) return;
    hdr[0] = N;
    if (N == 0) { hdr[1] = 2; return; }
    if (K > N) {  // quantization.py:68-81 padded codebook
        for (int k = 0; k < K; ++k) out[k] = cw[k < N ? k : N - 1];
        if (force) { out[0] = -1.0f; out[K - 1] = 1.0f; }
        for (int i = 1; i < K; ++i) {  // insertion sort (ascending)
            const float v = out[i];
            int j = i - 1;
            while (j >= 0 && out[j] > v) { out[j + 1] = out[j]; --j; }
            out[j + 1] = v;
        }
        hdr[1] = 1;
        return;
    }
    hdr[1] = 0;
}
static_assert(kDpMaxBins % kDpInitThreads == 0, "whole bins per thread");

// One DP level (quantization.py:158-186): for every segment end e in [c, N],
// the first start s in [c, e] minimising dp[c-1][s-1] + cost(s, e), in
// float64 with the reference's expression order; strict < keeps the first
// minimum, and the cross-lane reduction takes the lexicographic (cost, start)
// minimum.  The prefix sums and the previous level are staged in LDS (4 x
// (N + 1) doubles, 131 KB at N = 4096) and every candidate reads them from
// there.  Wave p of the grid takes the ends c + p and N - p, whose candidate
// counts add up to N - c + 2, so the waves carry equal work.
constexpr int kDpThreads = 512;
constexpr int kDpWaves = kDpThreads / 64;
static_assert(4 * (kDpMaxBins + 1) * sizeof(double) <= 160 * 1024, "the staged arrays fit in the LDS of one CU");

// Segment cost of starts s (prefix index s - 1) for end e: MODE 0 the
// free-centre cost sum_wx2 - sum_wx^2 / sum_w, MODE -1 / +1 the cost about
// the fixed centre -1 / +1 (force_endpoints, first / last cluster).
template <int MODE>
__device__ __forceinline__ double dp_cost(double Pe, double PXe, double PX2e, const double* spw, const double* spwx,
                                          const double* spwx2, int i) {
    const double sw = Pe - spw[i];
    const double swx = PXe - spwx[i];
    const double swx2 = PX2e - spwx2[i];
    if (MODE == 0) {
        const double sq = swx * swx;
        return swx2 - sq / sw;
    }
    const double fc = (double)MODE;
    const double t1 = (2.0 * fc) * swx;
    const double t2 = (fc * fc) * sw;
    return (swx2 - t1) + t2;
}

// Best start for end e over this lane's starts s = c + lane + 64 j, in
// ascending order (strict < keeps the first minimum); kDpUnroll independent
// candidates per iteration.
#ifndef GEFEN_DP_UNROLL
#define GEFEN_DP_UNROLL 4
#endif
constexpr int kDpUnroll = GEFEN_DP_UNROLL;
template <int MODE>
__device__ __forceinline__ void dp_scan(int e, int c, int lane, const double* spw, const double* spwx,
                                        const double* spwx2, const double* sprev, double& best, int& bs) {
    const double Pe = spw[e], PXe = spwx[e], PX2e = spwx2[e];
    int s = c + lane;
    for (; s + 64 * (kDpUnroll - 1) <= e; s += 64 * kDpUnroll) {
        double cand[kDpUnroll];
#pragma unroll
        for (int u = 0; u < kDpUnroll; ++u) {
            const int i = s + 64 * u - 1;
            cand[u] = sprev[i] + dp_cost<MODE>(Pe, PXe, PX2e, spw, spwx, spwx2, i);
        }
#pragma unroll
        for (int u = 0; u < kDpUnroll; ++u)
            if (cand[u] < best) { best = cand[u]; bs = s + 64 * u; }
    }
    for (; s <= e; s += 64) {
        const double cand = sprev[s - 1] + dp_cost<MODE>(Pe, PXe, PX2e, spw, spwx, spwx2, s - 1);
        if (cand < best) { best = cand; bs = s; }
    }
}

__device__ __forceinline__ void dp_end(int e, int c, int K, int force, int lane, const double* spw, const double* spwx,
                                       const double* spwx2, const double* sprev, double* dpc, int32_t* btc) {
    double best = __builtin_inf();
    int bs = -1;
    if (force && c == 1) dp_scan<-1>(e, c, lane, spw, spwx, spwx2, sprev, best, bs);
    else if (force && c == K) dp_scan<1>(e, c, lane, spw, spwx, spwx2, sprev, best, bs);
    else dp_scan<0>(e, c, lane, spw, spwx, spwx2, sprev, best, bs);
    for (int off = 32; off > 0; off >>= 1) {
        const double ob = __shfl_xor(best, off, 64);
        const int os = __shfl_xor(bs, off, 64);
        if (os >= 0 && (bs < 0 || ob < best || (ob == best && os < bs))) { best = ob; bs = os; }
    }
    if (lane == 0) {
        dpc[e] = bs >= 0 ? best : __builtin_inf();
        btc[e] = bs;
    }
}

__global__ __launch_bounds__(kDpThreads) void k_dp_level(int c, int K, int force, int bins, char* __restrict__ ws,
                                                         DpLayout L) {
    __shared__ double spw[kDpMaxBins + 1], spwx[kDpMaxBins + 1], spwx2[kDpMaxBins + 1], sprev[kDpMaxBins + 1];
    const int32_t* hdr = reinterpret_cast<const int32_t*>(ws);
    if (hdr[1] != 0) return;
    const int N = hdr[0];
    const size_t stride = (size_t)bins + 1;
    const double* pw = reinterpret_cast<const double*>(ws + L.pw);
    const double* pwx = reinterpret_cast<const double*>(ws + L.pwx);
    const double* pwx2 = reinterpret_cast<const double*>(ws + L.pwx2);
    double* dp = reinterpret_cast<double*>(ws + L.dp);
    int32_t* bt = reinterpret_cast<int32_t*>(ws + L.bt);
    const double* prev = dp + (size_t)(c - 1) * stride;
    double* dpc = dp + (size_t)c * stride;
    int32_t* btc = bt + (size_t)c * stride;
    if (blockIdx.x == 0) {  // ends below c have no segmentation into c clusters
        for (int e = threadIdx.x; e < c && e <= N; e += kDpThreads) {
            dpc[e] = __builtin_inf();
            btc[e] = -1;
        }
    }
    const int cnt = N - c + 1;  // ends c .. N
    if (blockIdx.x > 0 && 2 * (int)blockIdx.x * kDpWaves >= cnt) return;  // no pair of ends here (uniform)
    // indices c - 1 .. N of the four arrays (s - 1 >= c - 1, e <= N); every load of
    // a thread is issued before its first LDS store, so the staging waits for one
    // round trip to L2 instead of one per pass
    constexpr int kStage = (kDpMaxBins + 1 + kDpThreads - 1) / kDpThreads;
    double st[4][kStage];
#pragma unroll
    for (int r = 0; r < kStage; ++r) {
        const int i = c - 1 + (int)threadIdx.x + r * kDpThreads;
        if (i <= N) {
            st[0][r] = pw[i];
            st[1][r] = pwx[i];
            st[2][r] = pwx2[i];
            st[3][r] = prev[i];
        }
    }
#pragma unroll
    for (int r = 0; r < kStage; ++r) {
        const int i = c - 1 + (int)threadIdx.x + r * kDpThreads;
        if (i <= N) {
            spw[i] = st[0][r];
            spwx[i] = st[1][r];
            spwx2[i] = st[2][r];
            sprev[i] = st[3][r];
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    for (int p = blockIdx.x * kDpWaves + (int)(threadIdx.x >> 6); 2 * p < cnt; p += gridDim.x * kDpWaves) {
        dp_end(c + p, c, K, force, lane, spw, spwx, spwx2, sprev, dpc, btc);
        if (N - p != c + p) dp_end(N - p, c, K, force, lane, spw, spwx, spwx2, sprev, dpc, btc);
    }
}

__global__ void k_dp_backtrack(int K, int force, int bins, char* __restrict__ ws, DpLayout L,
                               float* __restrict__ out) {
    int32_t* hdr = reinterpret_cast<int32_t*>(ws);
    if (threadIdx.x != 0 || hdr[1] != 0) return;
    const int N = hdr[0];
    const size_t stride = (size_t)bins + 1;
    const double* pw = reinterpret_cast<const double*>(ws + L.pw);
    const double* pwx = reinterpret_cast<const double*>(ws + L.pwx);
    const int32_t* bt = reinterpret_cast<const int32_t*>(ws + L.bt);
    int e = N;
    for (int c = K; c >= 1; --c) {
        const int s = bt[(size_t)c * stride + e];
        if (s < 1) { hdr[1] = 3; return; }
        if (force && c == 1) out[c - 1] = -1.0f;
        else if (force && c == K) out[c - 1] = 1.0f;
        else out[c - 1] = (float)((pwx[e] - pwx[s - 1]) / (pw[e] - pw[s - 1]));
        e = s - 1;
    }
    for (int i = 1; i < K; ++i) {
        const float v = out[i];
        int j = i - 1;
        while (j >= 0 && out[j] > v) { out[j + 1] = out[j]; --j; }
        out[j + 1] = v;
    }
}

// ---------------------------------------------------------------------------
// Lloyd-Max accumulators (reference CUDA semantics; fp32 sums are order dependent).
// The block absmax skips NaN elements as the reference's running maximum does
// (lloyd_max_fused_kernel.cu:78-95, 141-158).
struct LloydLds {
    float thr[260];
    uint16_t bucket[4100];
};

// Codeword of a normalised value in the Lloyd kernels, as the reference's
// binary search picks it (lloyd_max_fused_kernel.cu:17-48): the lower bound k
// and its left neighbour k-1, ties to the left.  For x inside the codebook this
// is nearest_index.  It differs in two places: NaN (no codeword compares below
// it, and NaN distances fail the <= test) takes index 0, and x above the last
// codeword compares the last two entries instead of taking the last one.
__device__ __forceinline__ int lloyd_index(float x, const float* thr, const uint16_t* bucket, int K, float cb_prev,
                                           float cb_last) {
    if (x != x) return 0;
    if (K >= 2 && x > cb_last) return fabsf(x - cb_prev) <= fabsf(x - cb_last) ? K - 2 : K - 1;
    return nearest_index(x, thr, bucket, K);
}

template <typename G>
__global__ __launch_bounds__(256) void k_lloyd_accumulate(const G* __restrict__ g, int64_t nrows, int64_t period,
                                                          const CodebookTables* __restrict__ T,
                                                          float* __restrict__ sums,
                                                          unsigned long long* __restrict__ counts) {
    __shared__ LloydLds L;
    __shared__ float s_sum[256];
    __shared__ uint32_t s_cnt[256];
    const int K = T->K;
    const float cb_last = T->cb[K - 1], cb_prev = T->cb[K >= 2 ? K - 2 : 0];
    for (int i = threadIdx.x; i < 260; i += 256) L.thr[i] = T->thr[i];
    for (int i = threadIdx.x; i < 4100; i += 256) L.bucket[i] = T->bucket[i];
    s_sum[threadIdx.x] = 0.0f;
    s_cnt[threadIdx.x] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < nrows; row += (int64_t)gridDim.x * 4) {
        const int64_t base = row * period;
        float amax = 0.0f;
        for (int64_t j = lane; j < period; j += 64) amax = max_skip_nan(amax, fabsf(to_f32(g[base + j])));
        amax = group_max_skip_nan(amax, 64);
        for (int64_t j = lane; j < period; j += 64) {
            const float v = to_f32(g[base + j]);
            const float x = (amax > 0.0f) ? v / amax : 0.0f;
            const int k = lloyd_index(x, L.thr, L.bucket, K, cb_prev, cb_last);
            atomicAdd(&s_sum[k], x);
            atomicAdd(&s_cnt[k], 1u);
        }
    }
    __syncthreads();
    for (int k = threadIdx.x; k < K; k += 256) {
        if (s_cnt[k]) {
            atomicAdd(&sums[k], s_sum[k]);
            atomicAdd(&counts[k], (unsigned long long)s_cnt[k]);
        }
    }
}

template <typename G>
__global__ __launch_bounds__(256) void k_lloyd_mse(const G* __restrict__ g, int64_t nrows, int64_t period,
                                                   const CodebookTables* __restrict__ T,
                                                   const float* __restrict__ new_cb, float* __restrict__ mse_norm,
                                                   float* __restrict__ mse_orig) {
    __shared__ LloydLds L;
    __shared__ float red[2][4];
    const int K = T->K;
    const float cb_last = T->cb[K - 1], cb_prev = T->cb[K >= 2 ? K - 2 : 0];
    for (int i = threadIdx.x; i < 260; i += 256) L.thr[i] = T->thr[i];
    for (int i = threadIdx.x; i < 4100; i += 256) L.bucket[i] = T->bucket[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    float en = 0.0f, eo = 0.0f;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < nrows; row += (int64_t)gridDim.x * 4) {
        const int64_t base = row * period;
        float amax = 0.0f;
        for (int64_t j = lane; j < period; j += 64) amax = max_skip_nan(amax, fabsf(to_f32(g[base + j])));
        amax = group_max_skip_nan(amax, 64);
        for (int64_t j = lane; j < period; j += 64) {
            const float v = to_f32(g[base + j]);
            const float x = (amax > 0.0f) ? v / amax : 0.0f;
            const int k = lloyd_index(x, L.thr, L.bucket, K, cb_prev, cb_last);
            const float err = x - new_cb[k];
            const float e2 = err * err;
            en = en + e2;
            const float oe = err * amax;
            const float o2 = oe * oe;
            eo = eo + o2;
        }
    }
    en = group_sum(en, 64);
    eo = group_sum(eo, 64);
    if (lane == 0) { red[0][threadIdx.x >> 6] = en; red[1][threadIdx.x >> 6] = eo; }
    __syncthreads();
    if (threadIdx.x == 0) {
        atomicAdd(mse_norm, (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]));
        atomicAdd(mse_orig, (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]));
    }
}

namespace {
int grid_for_rows(int64_t units, int cap) {
    int64_t g = (units + 3) / 4;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}
int lpr_log2_for_len(int64_t len) {
    int l = 0;
    while ((1LL << l) < len && l < 6) ++l;
    return l;
}

struct TempTables {
    void* ptr = nullptr;
    hipStream_t st = nullptr;
    int init(const float* cb, int K, hipStream_t s) {
        st = s;
        hipError_t e = device_malloc_async(&ptr, sizeof(CodebookTables), s);
        if (e != hipSuccess) return hip_status(e, "hipMallocAsync(codebook tables)");
        return gefen_prepare_codebook(cb, K, ptr, reinterpret_cast<gefen_stream_t>(s));
    }
    ~TempTables() {
        if (ptr) (void)hipFreeAsync(ptr, st);
    }
};

int check_rows(const void* g, int dt, int64_t numel, int64_t period) {
    if (!valid_dtype(dt)) return fail_inval("unsupported gradient dtype %d", dt);
    if (period <= 0) return fail_inval("Expected period to be positive, got %lld", (long long)period);
    if (numel < 0 || numel % period)
        return fail_inval("Expected grad_flat.numel()=%lld to be divisible by period=%lld", (long long)numel,
                          (long long)period);
    if (numel > 0 && !g) return fail_inval("null gradient pointer");
    return GEFEN_OK;
}
}  // namespace
}  // namespace gefen

using namespace gefen;

extern "C" size_t gefen_codebook_tables_size(void) { return sizeof(CodebookTables); }

extern "C" int gefen_prepare_codebook(const float* codebook, int codebook_size, void* tables,
                                      gefen_stream_t stream) {
    if (!codebook || !tables) return fail_inval("null pointer");
    if (codebook_size <= 0 || codebook_size > 256)
        return fail_inval("Expected codebook to have at most 256 entries, got %d", codebook_size);
    hipLaunchKernelGGL(k_prepare_codebook, dim3(1), dim3(256), 0, reinterpret_cast<hipStream_t>(stream), codebook,
                       codebook_size, static_cast<CodebookTables*>(tables));
    return launch_status("gefen_prepare_codebook");
}

extern "C" int gefen_exact_histogram(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                                     int64_t* bin_counts, int bins, gefen_stream_t stream) {
    int rc = check_rows(grad, grad_dtype, numel, period);
    if (rc) return rc;
    if (bins <= 0 || bins > 4096) return fail_inval("Expected histogram bins in [1, 4096], got %d", bins);
    if (!bin_counts) return fail_inval("null bin_counts");
    if (numel == 0) return GEFEN_OK;
    const int64_t nrows = numel / period;
    const int l2 = lpr_log2_for_len(period);
    const int64_t units = (nrows + (64 >> l2) - 1) / (64 >> l2);
    const int grid = grid_for_rows(units, 2048);
    const float bw = (float)(2.0 / (double)bins);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    auto* cnt = reinterpret_cast<unsigned long long*>(bin_counts);
    if (grad_dtype == GEFEN_F32)
        hipLaunchKernelGGL(k_histogram<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(grad), nrows,
                           period, l2, bins, bw, cnt);
    else if (grad_dtype == GEFEN_BF16)
        hipLaunchKernelGGL(k_histogram<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(grad), nrows,
                           period, l2, bins, bw, cnt);
    else
        hipLaunchKernelGGL(k_histogram<f16_t>, dim3(grid), dim3(256), 0, st, static_cast<const f16_t*>(grad), nrows,
                           period, l2, bins, bw, cnt);
    return launch_status("gefen_exact_histogram");
}

extern "C" int gefen_accumulate_counts(float* acc, const int64_t* counts, int bins, gefen_stream_t stream) {
    if (!acc || !counts || bins <= 0) return fail_inval("invalid histogram accumulation arguments");
    hipLaunchKernelGGL(k_accumulate_counts, dim3((bins + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), acc, counts, bins);
    return launch_status("gefen_accumulate_counts");
}

extern "C" size_t gefen_exact_dp_workspace_size(int bins, int codebook_size) {
    if (bins <= 0 || codebook_size <= 0) return 0;
    return DpLayout(bins, codebook_size).total;
}

extern "C" int gefen_exact_dp(const float* counts, int bins, int codebook_size, int force_endpoints,
                              float* codebook_out, void* workspace, gefen_stream_t stream) {
    if (!counts || !codebook_out || !workspace) return fail_inval("null pointer");
    if (bins <= 0 || bins > 4096 || (bins & (bins - 1)))
        return fail_inval("exact DP needs a power-of-two bin count <= 4096, got %d", bins);
    if (codebook_size <= 0 || codebook_size > 256)
        return fail_inval("Expected codebook to have at most 256 entries, got %d", codebook_size);
    const int K = codebook_size;
    DpLayout L(bins, K);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    hipLaunchKernelGGL(k_dp_init, dim3(1), dim3(kDpInitThreads), 0, st, counts, bins, K, force_endpoints ? 1 : 0,
                       ws, L, codebook_out);
    int rc = launch_status("gefen_exact_dp init");
    if (rc) return rc;
    // enough waves for one pair of ends each at the largest level width (bins ends)
    const int grid = bins / 2 >= kDpWaves ? (bins / 2 + kDpWaves - 1) / kDpWaves : 1;
    for (int c = 1; c <= K; ++c) {
        hipLaunchKernelGGL(k_dp_level, dim3(grid), dim3(kDpThreads), 0, st, c, K, force_endpoints ? 1 : 0, bins, ws, L);
        rc = launch_status("gefen_exact_dp level");
        if (rc) return rc;
    }
    hipLaunchKernelGGL(k_dp_backtrack, dim3(1), dim3(64), 0, st, K, force_endpoints ? 1 : 0, bins, ws, L,
                       codebook_out);
    return launch_status("gefen_exact_dp backtrack");
}

extern "C" int gefen_lloyd_accumulate(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                                      const float* codebook, int codebook_size, float* sums, int64_t* counts,
                                      gefen_stream_t stream) {
    int rc = check_rows(grad, grad_dtype, numel, period);
    if (rc) return rc;
    if (!codebook || !sums || !counts) return fail_inval("null pointer");
    if (codebook_size <= 0 || codebook_size > 256)
        return fail_inval("Expected codebook to have at most 256 entries, got %d", codebook_size);
    if (numel == 0) return GEFEN_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    TempTables tt;
    rc = tt.init(codebook, codebook_size, st);
    if (rc) return rc;
    const int64_t nrows = numel / period;
    const int grid = grid_for_rows(nrows, 2048);
    auto* T = static_cast<const CodebookTables*>(tt.ptr);
    auto* cnt = reinterpret_cast<unsigned long long*>(counts);
    if (grad_dtype == GEFEN_F32)
        hipLaunchKernelGGL(k_lloyd_accumulate<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(grad),
                           nrows, period, T, sums, cnt);
    else if (grad_dtype == GEFEN_BF16)
        hipLaunchKernelGGL(k_lloyd_accumulate<bf16_t>, dim3(grid), dim3(256), 0, st,
                           static_cast<const bf16_t*>(grad), nrows, period, T, sums, cnt);
    else
        hipLaunchKernelGGL(k_lloyd_accumulate<f16_t>, dim3(grid), dim3(256), 0, st, static_cast<const f16_t*>(grad),
                           nrows, period, T, sums, cnt);
    return launch_status("gefen_lloyd_accumulate");
}

extern "C" int gefen_lloyd_mse(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                               const float* old_codebook, const float* new_codebook, int codebook_size,
                               float* mse_normalized_sum, float* mse_original_sum, gefen_stream_t stream) {
    int rc = check_rows(grad, grad_dtype, numel, period);
    if (rc) return rc;
    if (!old_codebook || !new_codebook || !mse_normalized_sum || !mse_original_sum) return fail_inval("null pointer");
    if (codebook_size <= 0 || codebook_size > 256)
        return fail_inval("Expected codebook to have at most 256 entries, got %d", codebook_size);
    if (numel == 0) return GEFEN_OK;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    TempTables tt;
    rc = tt.init(old_codebook, codebook_size, st);
    if (rc) return rc;
    const int64_t nrows = numel / period;
    const int grid = grid_for_rows(nrows, 2048);
    auto* T = static_cast<const CodebookTables*>(tt.ptr);
    if (grad_dtype == GEFEN_F32)
        hipLaunchKernelGGL(k_lloyd_mse<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(grad), nrows,
                           period, T, new_codebook, mse_normalized_sum, mse_original_sum);
    else if (grad_dtype == GEFEN_BF16)
        hipLaunchKernelGGL(k_lloyd_mse<bf16_t>, dim3(grid), dim3(256), 0, st, static_cast<const bf16_t*>(grad), nrows,
                           period, T, new_codebook, mse_normalized_sum, mse_original_sum);
    else
        hipLaunchKernelGGL(k_lloyd_mse<f16_t>, dim3(grid), dim3(256), 0, st, static_cast<const f16_t*>(grad), nrows,
                           period, T, new_codebook, mse_normalized_sum, mse_original_sum);
    return launch_status("gefen_lloyd_mse");
}

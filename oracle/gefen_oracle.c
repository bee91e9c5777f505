/*
 * gefen_oracle.c -- CPU restatement of the reference Gefen CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in gefen_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product never does.
 *
 * It restates, operation by operation, the torch-CPU arithmetic of the
 * reference's non-fused path (ndvbd/Gefen 1.2.3):
 *   vmean EMA            gefen.py:116-119
 *   stepsize             gefen.py:1326-1327
 *   weight decay         gefen.py:1280-1281
 *   momentum / quantise  gefen.py:1153-1206 (+ nearest 122-143, dequant 146-169)
 *   packed 4-bit indices automatic_gefen_fused_kernel.cu:14-57 (layout only)
 *   parameter update     gefen.py:1328-1333
 *   histogram            gefen.py:350-366
 *   exact DP codebook    quantization.py:68-81, 151-258 (+ gefen.py:373-399)
 *   period scores        partitioning.py:43-78, 119-167 (numpy pairwise sums)
 *   GefenMuon momentum   gefen_muon.py:132-171, 302-316
 *   Lloyd-Max, block variance / CoV: the reference's CUDA kernels
 *                        (lloyd_max_fused_kernel.cu:17-195,
 *                        period_variance_kernel.cu:13-106), which have no CPU path
 *
 * Rounding conventions (verified against torch 2.10 CPU): lerp and
 * add(alpha=) are fused multiply-adds; tensor/scalar is a true division;
 * scalar/tensor is reciprocal() then multiply; bf16/f16 results are rounded to
 * nearest even from the fp32 result.  Build with -ffp-contract=off so no other
 * operation is fused.
 *
 * The vmean row mean is summed in double and rounded once; torch sums in fp32
 * in its own order, so vmean (and the parameters through the stepsize) agree
 * with the reference to tolerance only.  Every other output (codebook indices,
 * magnitudes, histogram counts, DP codebook) is computed by order-independent
 * or fully specified operations.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

/* ------------------------------------------------------------------ dtypes */
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = f_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0; /* torch: canonical quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static inline float bf16_to_f32(uint16_t h) { return bits_f((uint32_t)h << 16); }

/* float -> half, round to nearest even (subnormals handled by an exact
 * float addition that aligns the half ulp). */
static inline uint16_t f32_to_f16(float ff) {
    uint32_t f = f_bits(ff);
    const uint32_t sign = f & 0x80000000u;
    f ^= sign;
    uint16_t o;
    if (f >= (143u << 23)) {                 /* >= 2^16: inf or NaN */
        o = (f > (255u << 23)) ? 0x7e00 : 0x7c00;
    } else if (f < (113u << 23)) {           /* < 2^-14: half subnormal or zero */
        const uint32_t magic = 126u << 23;   /* 0.5: ulp of (x + 0.5) is 2^-24 */
        float t = bits_f(f) + bits_f(magic);
        o = (uint16_t)(f_bits(t) - magic);
    } else {
        uint32_t odd = (f >> 13) & 1u;
        f += ((uint32_t)(15 - 127) << 23) + 0xfffu;
        f += odd;
        o = (uint16_t)(f >> 13);
    }
    return (uint16_t)(o | (sign >> 16));
}
static inline float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((e + 112u) << 23) | (m << 13));
}

static inline float load_dt(const void* base, int dt, int64_t i) {
    switch (dt) {
    case DT_F32: return ((const float*)base)[i];
    case DT_F16: return f16_to_f32(((const uint16_t*)base)[i]);
    default: return bf16_to_f32(((const uint16_t*)base)[i]);
    }
}
static inline void store_dt(void* base, int dt, int64_t i, float v) {
    switch (dt) {
    case DT_F32: ((float*)base)[i] = v; break;
    case DT_F16: ((uint16_t*)base)[i] = f32_to_f16(v); break;
    default: ((uint16_t*)base)[i] = f32_to_bf16(v); break;
    }
}
/* round an fp32 value to dtype and back */
static inline float round_dt(float v, int dt) {
    switch (dt) {
    case DT_F32: return v;
    case DT_F16: return f16_to_f32(f32_to_f16(v));
    default: return bf16_to_f32(f32_to_bf16(v));
    }
}
/* NaN-propagating max of non-negative values (torch amax semantics) */
static inline float nanmax(float a, float b) { return (b > a || b != b) ? b : a; }

int orc_f32_to_bf16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
    return 0;
}
int orc_f32_to_f16(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = f32_to_f16(x[i]);
    return 0;
}

/* ------------------------------------------------------------------ nearest
 * gefen.py:122-143: k = searchsorted(cb, x) (first k with cb[k] >= x; NaN -> K),
 * right = clamp(k), left = clamp(k-1); left wins ties of |x - cb|. */
static inline int nearest_index(const float* cb, int K, float x) {
    int lo = 0, hi = K;
    while (lo < hi) {
        int mid = lo + ((hi - lo) >> 1);
        if (!(cb[mid] >= x)) lo = mid + 1; else hi = mid;
    }
    int right = lo > K - 1 ? K - 1 : lo;
    int left = lo - 1;
    if (left < 0) left = 0;
    if (left > K - 1) left = K - 1;
    float dl = fabsf(x - cb[left]);
    float dr = fabsf(x - cb[right]);
    return (dl <= dr) ? left : right;
}

int orc_nearest(const float* cb, int K, const float* x, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)nearest_index(cb, K, x[i]);
    return 0;
}

/* ------------------------------------------------------------------ vmean
 * gefen.py:116-119 for one row: ms = mean(f32(g)^2); v = fma(ms, 1-b2, v*b2). */
static inline float row_mean_sq(const void* g, int dt, int64_t start, int64_t len) {
    double acc = 0.0;
    for (int64_t j = 0; j < len; ++j) {
        float x = load_dt(g, dt, start + j);
        float sq = x * x;
        acc += (double)sq;
    }
    return (float)acc / (float)len;
}

int orc_vmean_update(int sdt, void* vmean, int gdt, const void* g,
                     int64_t rows, int64_t period, double beta2) {
    const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2);
    for (int64_t r = 0; r < rows; ++r) {
        float ms = row_mean_sq(g, gdt, r * period, period);
        float prev = load_dt(vmean, sdt, r) * b2;
        store_dt(vmean, sdt, r, fmaf(ms, omb2, prev));
    }
    return 0;
}

/* ------------------------------------------------------------------ update
 * Momentum, quantisation and parameter update of one magnitude block of `mblk`
 * elements starting at s0 (gefen.py:1153-1206, 1328-1333).  The stepsize of
 * element i is stepsize[i / period] when `stepsize` is non-null, else the
 * stepsize of vmean[i / period] (gefen.py:1326-1327). */
typedef struct {
    int ddt, sdt, qdt, vdt, K, do_wd;
    void* p;
    const void* g;
    uint8_t* idx;
    void* mag;
    const void* vmean;
    const float* stepsize;
    const float* cb;
    float cbd[256];
    int64_t period;
    float b1c, sqrt_bc2, eps_f, inv_bc1, lr_f, wd_f;
} StepCtx;

static void step_ctx_init(StepCtx* c, int ddt, int sdt, const float* cb, int K, double beta1, double lr,
                          double eps, double wd, double bc1, double bc2) {
    c->ddt = ddt;
    c->sdt = sdt;
    /* promote(D, S) of codebook[idx].to(D) * magnitude (gefen.py:1205-1206) */
    c->qdt = (ddt == sdt) ? ddt : DT_F32;
    c->cb = cb;
    c->K = K;
    /* codebook rounded to the parameter dtype (dequant, gefen.py:160-162, 1205) */
    for (int k = 0; k < K; ++k) c->cbd[k] = round_dt(cb[k], ddt);
    c->b1c = (float)(1.0 - beta1);
    c->sqrt_bc2 = (float)sqrt(bc2);
    c->eps_f = (float)eps;
    c->inv_bc1 = (float)(1.0 / bc1);
    c->lr_f = (float)lr;
    c->do_wd = wd > 0.0;
    c->wd_f = (float)(1.0 - lr * wd);
}

static void quantise_block(const StepCtx* c, int64_t b, int64_t s0, int64_t mblk) {
    const float mold = load_dt(c->mag, c->sdt, b);
    float mx = 0.0f;
    for (int64_t j = 0; j < mblk; ++j) {
        const int64_t i = s0 + j;
        float cur = c->cbd[c->idx[i]] * mold;
        float gf = load_dt(c->g, c->ddt, i);
        float upd = fmaf(c->b1c, gf - cur, cur);
        mx = nanmax(mx, fabsf(upd));
    }
    store_dt(c->mag, c->sdt, b, mx);
    const float mn = load_dt(c->mag, c->sdt, b);
    float ss_row = 0.0f;
    int64_t cur_vrow = -1;
    for (int64_t j = 0; j < mblk; ++j) {
        const int64_t i = s0 + j;
        float cur = c->cbd[c->idx[i]] * mold;
        float gf = load_dt(c->g, c->ddt, i);
        float upd = fmaf(c->b1c, gf - cur, cur);
        float x = (mn > 0.0f) ? upd / mn : 0.0f;
        int k = nearest_index(c->cb, c->K, x);
        c->idx[i] = (uint8_t)k;
        const int64_t vr = i / c->period;
        if (vr != cur_vrow) {
            if (c->stepsize) {
                ss_row = c->stepsize[vr];
            } else {
                float v = load_dt(c->vmean, c->vdt, vr);
                float h = sqrtf(v) / c->sqrt_bc2 + c->eps_f;
                ss_row = (1.0f / h) * c->inv_bc1;
            }
            cur_vrow = vr;
        }
        float q = round_dt(c->cbd[k] * mn, c->qdt);
        float u = (q * ss_row) * c->lr_f;
        float pv = load_dt(c->p, c->ddt, i);
        if (c->do_wd) pv = round_dt(pv * c->wd_f, c->ddt);
        store_dt(c->p, c->ddt, i, pv - u);
    }
}

/* One Gefen step of one tensor on the reference CPU path, after the caller has
 * advanced state["step"] and computed bc1 = 1 - beta1**step, bc2 = 1 - beta2**step
 * in double precision (gefen.py:1278-1284).
 *
 * period > 1: rows of `period` share vmean and m_magnitude.
 * period == 1: vmean is per element and m_magnitude is per block of `pod`
 * elements (pod = largest divisor of n that is <= 256, gefen.py:622-623). */
int orc_gefen_step(int ddt, int sdt, void* p, const void* g, uint8_t* idx,
                   void* mag, void* vmean, int64_t n, int64_t period, int64_t pod,
                   const float* cb, int K, double beta1, double beta2, double lr,
                   double eps, double wd, double bc1, double bc2, int nthreads) {
    if (n <= 0) return 0;
    if (period <= 0 || n % period != 0) return 1;
    const int64_t vrows = n / period;
    const int64_t mblk = (period == 1) ? pod : period;
    if (mblk <= 0 || n % mblk != 0) return 1;
    const int64_t mrows = n / mblk;
    const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2);
    StepCtx c;
    step_ctx_init(&c, ddt, sdt, cb, K, beta1, lr, eps, wd, bc1, bc2);
    c.p = p;
    c.g = g;
    c.idx = idx;
    c.mag = mag;
    c.vmean = vmean;
    c.vdt = sdt;
    c.stepsize = NULL;
    c.period = period;

#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif

    /* 1) vmean (gefen.py:1275-1276) */
#pragma omp parallel for schedule(static) num_threads(nthreads) if (vrows > 64)
    for (int64_t r = 0; r < vrows; ++r) {
        float ms = row_mean_sq(g, ddt, r * period, period);
        float prev = load_dt(vmean, sdt, r) * b2;
        store_dt(vmean, sdt, r, fmaf(ms, omb2, prev));
    }

    /* 2) momentum, quantisation and parameter update per magnitude block */
#pragma omp parallel for schedule(static) num_threads(nthreads) if (mrows > 16)
    for (int64_t b = 0; b < mrows; ++b) quantise_block(&c, b, b * mblk, mblk);
    return 0;
}

/* The update of the reference's given-stepsize and given-vmean entry points
 * (automatic_gefen_fused.py:10-249) with the CPU-path arithmetic: rows of
 * `period` elements share m_magnitude and a stepsize, which is stepsize[r] when
 * `stepsize` is non-null, else the stepsize (gefen.py:1326-1327) of vmean[r]
 * as given (not updated here).  No weight decay. */
int orc_gefen_update_given(int ddt, int sdt, void* p, const void* g, uint8_t* idx, void* mag,
                           const void* vmean, int vdt, const float* stepsize, int64_t n,
                           int64_t period, const float* cb, int K, double beta1, double lr,
                           double bc1, double bc2, double eps) {
    if (n <= 0) return 0;
    if (period <= 0 || n % period != 0) return 1;
    StepCtx c;
    step_ctx_init(&c, ddt, sdt, cb, K, beta1, lr, eps, 0.0, bc1, bc2);
    c.p = p;
    c.g = g;
    c.idx = idx;
    c.mag = mag;
    c.vmean = vmean;
    c.vdt = vdt;
    c.stepsize = stepsize;
    c.period = period;
    for (int64_t b = 0; b < n / period; ++b) quantise_block(&c, b, b * period, period);
    return 0;
}

/* ------------------------------------------------------------------ packed indices
 * The packed 4-bit layout of automatic_gefen_fused_kernel.cu:14-57: the index of
 * element i is the low nibble of byte i/2 when i is even and the high nibble when
 * i is odd; storing keeps an index's low four bits and leaves the other nibble of
 * its byte alone (so the high nibble of the last byte of an odd n is kept). */
int orc_unpack_nibbles(const uint8_t* packed, int64_t n, uint8_t* idx) {
    for (int64_t i = 0; i < n; ++i) idx[i] = (i & 1) ? (uint8_t)(packed[i >> 1] >> 4) : (uint8_t)(packed[i >> 1] & 15);
    return 0;
}

int orc_pack_nibbles(const uint8_t* idx, int64_t n, uint8_t* packed) {
    for (int64_t i = 0; i < n; ++i) {
        const int sh = (i & 1) ? 4 : 0;
        packed[i >> 1] = (uint8_t)((packed[i >> 1] & ~(15 << sh)) | ((idx[i] & 15) << sh));
    }
    return 0;
}

/* ------------------------------------------------------------------ histogram
 * gefen.py:350-366 for one tensor: per row absmax normalisation, then
 * bin = clamp(floor((x + 1) / f32(2/bins)), 0, bins-1).  counts are += int64. */
int orc_histogram(int gdt, const void* g, int64_t n, int64_t period, int bins,
                  int64_t* counts) {
    if (period <= 0 || n % period != 0 || bins <= 0) return 1;
    const float bw = (float)(2.0 / (double)bins);
    const int64_t rows = n / period;
    /* integer counts per thread, added at the end: exact in any order */
    int failed = 0;
#pragma omp parallel if (n > (1 << 20)) reduction(| : failed)
    {
        int64_t* local = (int64_t*)calloc((size_t)bins, sizeof(int64_t));
        if (!local) failed = 1;
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            if (!local) continue;
            float amax = 0.0f;
            for (int64_t j = 0; j < period; ++j) amax = nanmax(amax, fabsf(load_dt(g, gdt, r * period + j)));
            for (int64_t j = 0; j < period; ++j) {
                float v = load_dt(g, gdt, r * period + j);
                float x = (amax > 0.0f) ? v / amax : 0.0f;
                float y = floorf((x + 1.0f) / bw);
                int64_t b;
                if (y != y) b = INT64_MIN; /* torch .to(long) of NaN on x86 */
                else if (y >= 9.2e18f) b = INT64_MIN;
                else if (y <= -9.2e18f) b = INT64_MIN;
                else b = (int64_t)y;
                if (b < 0) b = 0;
                if (b > bins - 1) b = bins - 1;
                local[b] += 1;
            }
        }
        if (local) {
#pragma omp critical
            for (int b = 0; b < bins; ++b) counts[b] += local[b];
            free(local);
        }
    }
    return failed ? 2 : 0;
}

/* f32 accumulation of per-tensor counts in parameter order (gefen.py:331, 347, 365) */
int orc_accumulate_counts(float* acc, const int64_t* counts, int bins) {
    for (int b = 0; b < bins; ++b) acc[b] = acc[b] + (float)counts[b];
    return 0;
}

/* ------------------------------------------------------------------ exact DP
 * quantization.py:206-258 (+ _run_exact_dp_python 151-203, padding 68-81) on
 * the histogram built at gefen.py:373-387.  bins must be a power of two so
 * that the linspace bin centres are exact dyadic numbers. */
static int cmp_float(const void* a, const void* b) {
    float x = *(const float*)a, y = *(const float*)b;
    return (x > y) - (x < y);
}

int orc_exact_dp(const float* counts, int bins, int K, int force, float* out) {
    if (bins <= 0 || (bins & (bins - 1)) != 0 || K <= 0) return 1;
    int N = 0;
    float* centers = (float*)malloc(sizeof(float) * (size_t)bins);
    float* wts = (float*)malloc(sizeof(float) * (size_t)bins);
    for (int b = 0; b < bins; ++b) {
        if (counts[b] > 0.0f) {
            centers[N] = (float)(-1.0 + (2.0 * b + 1.0) / (double)bins);
            wts[N] = counts[b];
            ++N;
        }
    }
    if (N == 0) { free(centers); free(wts); return 2; }
    if (K > N) { /* _build_padded_codebook */
        for (int k = 0; k < K; ++k) out[k] = centers[k < N ? k : N - 1];
        if (force) { out[0] = -1.0f; out[K - 1] = 1.0f; }
        qsort(out, (size_t)K, sizeof(float), cmp_float);
        free(centers); free(wts);
        return 0;
    }
    double* pw = (double*)calloc((size_t)N + 1, sizeof(double));
    double* pwx = (double*)calloc((size_t)N + 1, sizeof(double));
    double* pwx2 = (double*)calloc((size_t)N + 1, sizeof(double));
    for (int i = 0; i < N; ++i) {
        double w = (double)wts[i], c = (double)centers[i];
        pw[i + 1] = pw[i] + w;
        pwx[i + 1] = pwx[i] + w * c;
        pwx2[i + 1] = pwx2[i] + w * (c * c);
    }
    const size_t stride = (size_t)K + 1;
    double* dp = (double*)malloc(sizeof(double) * ((size_t)N + 1) * stride);
    int32_t* bt = (int32_t*)malloc(sizeof(int32_t) * ((size_t)N + 1) * stride);
    for (size_t i = 0; i < ((size_t)N + 1) * stride; ++i) { dp[i] = INFINITY; bt[i] = -1; }
    dp[0] = 0.0;
    for (int c = 1; c <= K; ++c) {
        const int fixed_lo = force && c == 1;
        const int fixed_hi = force && c == K;
#pragma omp parallel for schedule(dynamic, 16)
        for (int e = c; e <= N; ++e) {
            double best = INFINITY;
            int bs = -1;
            for (int s = c; s <= e; ++s) {
                double sw = pw[e] - pw[s - 1];
                double swx = pwx[e] - pwx[s - 1];
                double swx2 = pwx2[e] - pwx2[s - 1];
                double cost;
                if (fixed_lo) {
                    const double fc = -1.0;
                    cost = (swx2 - (2.0 * fc) * swx) + (fc * fc) * sw;
                } else if (fixed_hi) {
                    const double fc = 1.0;
                    cost = (swx2 - (2.0 * fc) * swx) + (fc * fc) * sw;
                } else {
                    cost = swx2 - (swx * swx) / sw;
                }
                double cand = dp[(size_t)(s - 1) * stride + (size_t)(c - 1)] + cost;
                if (cand < best) { best = cand; bs = s; }
            }
            dp[(size_t)e * stride + (size_t)c] = best;
            bt[(size_t)e * stride + (size_t)c] = bs;
        }
    }
    int e = N;
    int rc = 0;
    for (int c = K; c >= 1; --c) {
        int s = bt[(size_t)e * stride + (size_t)c];
        if (s < 1) { rc = 3; break; }
        if (force && c == 1) out[c - 1] = -1.0f;
        else if (force && c == K) out[c - 1] = 1.0f;
        else out[c - 1] = (float)((pwx[e] - pwx[s - 1]) / (pw[e] - pw[s - 1]));
        e = s - 1;
    }
    if (rc == 0) qsort(out, (size_t)K, sizeof(float), cmp_float);
    free(dp); free(bt); free(pw); free(pwx); free(pwx2); free(centers); free(wts);
    return rc;
}

/* ------------------------------------------------------------------ periods
 * numpy's summation of a contiguous float64 run: zero plus, for each buffer
 * chunk of 8192 items, the pairwise sum of the chunk (8-way unrolled blocks of
 * at most 128, halves rounded down to a multiple of 8). */
static double pairwise(const double* a, int64_t n) {
    if (n < 8) {
        double r = 0.0;
        for (int64_t i = 0; i < n; ++i) r += a[i];
        return r;
    }
    if (n <= 128) {
        double r[8];
        for (int j = 0; j < 8; ++j) r[j] = a[j];
        int64_t i;
        for (i = 8; i < n - (n % 8); i += 8)
            for (int j = 0; j < 8; ++j) r[j] += a[i + j];
        double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
        for (; i < n; ++i) res += a[i];
        return res;
    }
    int64_t n2 = n / 2;
    n2 -= n2 % 8;
    return pairwise(a, n2) + pairwise(a + n2, n - n2);
}
static double np_sum(const double* a, int64_t n) {
    double r = 0.0;
    for (int64_t c = 0; c < n; c += 8192) r += pairwise(a + c, (n - c) < 8192 ? (n - c) : 8192);
    return r;
}

/* Scores of partitioning.average_within_block_variance_cpu for each divisor.
 * mode 0: x = f64(f32(v))            (input already squared)
 * mode 1: x = f64(f32(f32(v)*f32(v))) (Gefen step: grad.float().square())
 * mode 2: x = f64(f32(v))^2           (input_is_squared=False on the CPU path)
 * Returns 4 if some x + eps <= 0 (the reference raises ValueError). */
int orc_period_scores(int gdt, const void* g, int64_t n, const int64_t* divs, int nd,
                      int mode, double eps, double* scores) {
    double* L = (double*)malloc(sizeof(double) * (size_t)n);
    if (!L) return 2;
    int invalid = 0;
    /* every element and every divisor is computed on its own in a fixed order,
     * so the threads change nothing in the results */
#pragma omp parallel for schedule(static) reduction(| : invalid)
    for (int64_t i = 0; i < n; ++i) {
        float v = load_dt(g, gdt, i);
        double x;
        if (mode == 1) x = (double)(v * v);
        else if (mode == 2) { x = (double)v; x = x * x; }
        else x = (double)v;
        double y = x + eps;
        if (y <= 0.0) invalid = 1;
        L[i] = log(y);
    }
    if (invalid) { free(L); return 4; }
    int64_t maxb = 0;
    for (int d = 0; d < nd; ++d) if (n / divs[d] > maxb) maxb = n / divs[d];
    int rc = 0;
#pragma omp parallel
    {
        double* means = (double*)malloc(sizeof(double) * (size_t)(maxb > 0 ? maxb : 1));
        if (!means) {
#pragma omp atomic write
            rc = 2;
        }
#pragma omp for schedule(dynamic, 1)
        for (int d = 0; d < nd; ++d) {
            if (!means) continue;
            const int64_t p = divs[d];
            const int64_t nb = n / p;
            for (int64_t j = 0; j < nb; ++j) means[j] = np_sum(L + j * p, p) / (double)p;
            for (int64_t j = 0; j + 1 < nb; ++j) means[j] = fabs(means[j + 1] - means[j]);
            scores[d] = (nb >= 2) ? np_sum(means, nb - 1) / (double)(nb - 1) : NAN;
        }
        free(means);
    }
    free(L);
    return rc;
}

/* ------------------------------------------------------------------ GefenMuon
 * gefen_muon.py:302-316 (+ _quantize_momentum_ 132-171), all in dtype D with a
 * rounding after each torch op; state dtype S.  Writes the Nesterov (or plain)
 * momentum update in dtype D into `out`.  Rows of `mblk` share a magnitude. */
int orc_muon_momentum(int ddt, int sdt, const void* g, uint8_t* idx, void* mag,
                      void* out, int64_t n, int64_t mblk, const float* cb, int K,
                      double momentum, int nesterov) {
    if (mblk <= 0 || n % mblk != 0) return 1;
    const int64_t rows = n / mblk;
    const float w = (float)(1.0 - momentum);
    const float mom = (float)momentum;
    /* add_(alpha=1-momentum): vectorised reduced-float kernels round alpha to the
     * tensor dtype first; fp32 uses it as is. */
    const float alpha = round_dt((float)(1.0 - momentum), ddt);
    /* torch.finfo(D).tiny, applied to the S-typed magnitude (gefen_muon.py:149-151) */
    const float tiny = round_dt((ddt == DT_F16) ? 6.103515625e-05f : 1.17549435e-38f, sdt);
    float cbd[256];
    for (int k = 0; k < K; ++k) cbd[k] = round_dt(cb[k], ddt);
    float* mu = (float*)malloc(sizeof(float) * (size_t)mblk);
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t s0 = r * mblk;
        const float mold = load_dt(mag, sdt, r);
        float mx = 0.0f;
        for (int64_t j = 0; j < mblk; ++j) {
            const int64_t i = s0 + j;
            float m0 = round_dt(cbd[idx[i]] * mold, ddt);           /* dequant .mul_(mag) */
            float gf = load_dt(g, ddt, i);
            float m1 = round_dt(fmaf(w, gf - m0, m0), ddt);         /* lerp_ */
            mu[j] = m1;
            mx = nanmax(mx, fabsf(m1));
        }
        store_dt(mag, sdt, r, mx);
        const float ms = load_dt(mag, sdt, r);
        const float clamped = (ms < tiny) ? tiny : ms;              /* clamp(min=tiny) */
        for (int64_t j = 0; j < mblk; ++j) {
            const int64_t i = s0 + j;
            float x = round_dt(mu[j] / clamped, ddt);               /* div_ */
            if (ms <= 0.0f) x = 0.0f;                               /* masked_fill_(mag <= 0) */
            int k = nearest_index(cb, K, x);
            idx[i] = (uint8_t)k;
            float q = round_dt(cbd[k] * ms, ddt);                   /* copy_ then mul_(mag) */
            if (nesterov) {
                float gf = load_dt(g, ddt, i);
                float a = round_dt(q * mom, ddt);                   /* mul_(momentum) */
                float o = (ddt == DT_F32) ? fmaf(gf, alpha, a) : round_dt(a + gf * alpha, ddt);
                store_dt(out, ddt, i, o);
            } else {
                store_dt(out, ddt, i, q);
            }
        }
    }
    free(mu);
    return 0;
}

/* out[i] = fma(a[i], b, c[i]) in fp32 (torch fp32 add_(x, alpha=b) on CPU) */
int orc_fma32(const float* a, float b, const float* c, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = fmaf(a[i], b, c[i]);
    return 0;
}

/* ------------------------------------------------------------------ Lloyd-Max
 * The reference's CUDA semantics (lloyd_max_fused_kernel.cu:17-195; it has no
 * CPU counterpart): per block, absmax = running maximum of |g| that a NaN never
 * replaces (lines 78-95); x = g / absmax in float32, 0 when absmax is 0; the
 * codeword from the binary search of lines 17-48 (first k with cb[k] >= x, its
 * left neighbour, ties to the left; NaN takes index 0, x above the last
 * codeword compares the last two).  The kernels add the sums and squared errors
 * in float32 in their own order; here they are added in double. */
static inline int lloyd_index(const float* cb, int K, float x) {
    int left = 0, right = K;
    while (left < right) {
        const int mid = left + (right - left) / 2;
        if (cb[mid] < x) left = mid + 1; else right = mid;
    }
    int r = left;
    if (r < 0) r = 0; else if (r >= K) r = K - 1;
    int l = r - 1;
    if (l < 0) l = 0;
    const float dl = fabsf(x - cb[l]), dr = fabsf(x - cb[r]);
    return dl <= dr ? l : r;
}

static float lloyd_absmax(const void* g, int dt, int64_t s, int64_t len) {
    float m = 0.0f;
    for (int64_t j = 0; j < len; ++j) {
        const float a = fabsf(load_dt(g, dt, s + j));
        if (a > m) m = a;
    }
    return m;
}

int orc_lloyd_accumulate(int gdt, const void* g, int64_t n, int64_t period, const float* cb, int K,
                         double* sums, int64_t* counts) {
    if (period <= 0 || n % period || K <= 0 || K > 256) return 1;
    for (int64_t s = 0; s < n; s += period) {
        const float amax = lloyd_absmax(g, gdt, s, period);
        for (int64_t j = 0; j < period; ++j) {
            const float v = load_dt(g, gdt, s + j);
            const float x = amax > 0.0f ? v / amax : 0.0f;
            const int k = lloyd_index(cb, K, x);
            sums[k] += (double)x;
            counts[k] += 1;
        }
    }
    return 0;
}

/* out[0] += sum of (x - new[k])^2, out[1] += sum of ((x - new[k]) * absmax)^2,
 * each term formed in float32 as lines 166-175 do. */
int orc_lloyd_mse(int gdt, const void* g, int64_t n, int64_t period, const float* old_cb, const float* new_cb,
                  int K, double* out) {
    if (period <= 0 || n % period || K <= 0 || K > 256) return 1;
    for (int64_t s = 0; s < n; s += period) {
        const float amax = lloyd_absmax(g, gdt, s, period);
        for (int64_t j = 0; j < period; ++j) {
            const float v = load_dt(g, gdt, s + j);
            const float x = amax > 0.0f ? v / amax : 0.0f;
            const int k = lloyd_index(old_cb, K, x);
            const float err = x - new_cb[k];
            const float e2 = err * err;
            const float oe = err * amax;
            const float o2 = oe * oe;
            out[0] += (double)e2;
            out[1] += (double)o2;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ block variance / CoV
 * The reference's CUDA scorers (period_variance_kernel.cu:13-106, 177-318), in
 * double: per block, x = v (input_is_squared) or v*v in float32; mean and
 * E[x^2] over the block, var = max(E[x^2] - mean^2, 0).  variance: out[0] =
 * sqrt(mean of var over blocks).  CoV: out[0] = sum of sqrt(var)/mean over
 * blocks with mean > 0, out[1] = their count, out[2] = count of mean < 0. */
int orc_block_variance(int gdt, const void* v, int64_t n, int64_t period, int input_is_squared, int cov,
                       double* out) {
    if (period <= 0 || n % period) return 1;
    const int64_t nb = n / period;
    double acc = 0.0, cnt = 0.0, neg = 0.0;
    for (int64_t b = 0; b < nb; ++b) {
        double sx = 0.0, sx2 = 0.0;
        for (int64_t j = 0; j < period; ++j) {
            const float a = load_dt(v, gdt, b * period + j);
            const double x = input_is_squared ? (double)a : (double)(a * a);
            sx += x;
            sx2 += x * x;
        }
        const double mean = sx / (double)period;
        double var = sx2 / (double)period - mean * mean;
        if (var < 0.0) var = 0.0;
        if (!cov) {
            acc += var;
        } else if (mean < 0.0) {
            neg += 1.0;
        } else if (mean > 0.0) {
            acc += sqrt(var) / mean;
            cnt += 1.0;
        }
    }
    out[0] = cov ? acc : sqrt(acc / (double)nb);
    out[1] = cnt;
    out[2] = neg;
    return 0;
}

// Device code of the fused Gefen / GefenMuon step: task tables, the step,
// GefenMuon momentum and packed-index kernels, and the launch templates that
// pick a kernel instance from a task's key.  The launch templates are
// instantiated once per (parameter, state) dtype pair in step_inst_*.hip, so
// the kernel instances of the pairs compile in parallel; step.hip holds the
// host side and declares those instances extern.
//
// One pass over the parameters, gradients and 8-bit codebook indices per step.
// Work unit: a magnitude block ("row") of `rowlen` elements -- the automatic
// period P, or the period-one divisor d when P = 1.  A row is owned by a group
// of LPR lanes (LPR = power of two <= 64, so a wave64 holds 64/LPR rows); each
// lane keeps up to R vectors of W elements in registers, so the row is read
// once, reduced with xor-butterflies inside the lane group (absmax for the
// magnitude, sum of squares for vmean) and written once.  Rows longer than
// 64*R*W elements take a two-sweep workgroup-per-row kernel.
//
// The arithmetic is the reference's CPU path (gefen.py:116-119, 1153-1206,
// 1280-1281, 1326-1333; gefen_muon.py:132-171, 302-316), op by op.

#pragma once

#include <math.h>
#include <stddef.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "capi_internal.h"
#include "common.h"

namespace gefen {

#ifndef GEFEN_MUON_TAB_LOG2
#define GEFEN_MUON_TAB_LOG2 6  // GefenMuon row tables for lane groups of 64 lanes
#endif
#ifndef GEFEN_MUON_ITER
#define GEFEN_MUON_ITER 2  // two wave-units per wave: the Qwen3-1.7B momentum pass 1.58 -> 1.49 ms (3 and 4: 1.54)
#endif
#ifndef GEFEN_STEP_ITER_ROWS
#define GEFEN_STEP_ITER_ROWS 1
#endif
#ifndef GEFEN_STEP_ITER_P1
#define GEFEN_STEP_ITER_P1 2
#endif
#ifndef GEFEN_STEP_P1_LUT
#define GEFEN_STEP_P1_LUT 1  // period one, 16-bit state: stepsize from the table (0: computed)
#endif
#ifndef GEFEN_STEP_NT
#define GEFEN_STEP_NT 1
#endif
#ifndef GEFEN_STEP_WAVES
#define GEFEN_STEP_WAVES 4
#endif
constexpr int kThreads = 256;  // 4 waves: two-sweep, GefenMuon and vmean kernels
constexpr int kMuonIter = GEFEN_MUON_ITER;  // wave-units per wave in one GefenMuon workgroup
// wave-units per wave in one step workgroup: block rows, period-one rows
constexpr int kIterRows = GEFEN_STEP_ITER_ROWS;
constexpr int kIterP1 = GEFEN_STEP_ITER_P1;
template <bool P1> constexpr int step_iter() { return P1 ? kIterP1 : kIterRows; }
constexpr int kStepWaves = GEFEN_STEP_WAVES;  // waves per workgroup of the register-path step kernel
constexpr int kStepThreads = 64 * kStepWaves;

constexpr bool kStreamNT = GEFEN_STEP_NT != 0;  // non-temporal loads / stores of the streamed tensors

template <typename T, int W>
__device__ __forceinline__ Vec<T, W> sload(const T* base, uint32_t elem) {
    if constexpr (kStreamNT) return vload32_nt<T, W>(base, elem);
    else return vload32<T, W>(base, elem);
}
template <typename T, int W>
__device__ __forceinline__ void sstore(T* base, uint32_t elem, const Vec<T, W>& x) {
    if constexpr (kStreamNT) vstore32_nt<T, W>(base, elem, x);
    else vstore32<T, W>(base, elem, x);
}
constexpr int kMaxBatch = 30;  // tasks per launch (the task table is the kernel argument block, < 4 KB)

enum StepMode : int32_t { kVmeanUpdate = 0, kVmeanGiven = 1, kStepsizeGiven = 2 };

struct StepTask {
    void* p;
    const void* g;
    uint8_t* idx;
    void* mag;
    void* vmean;
    const float* stepsize;
    const float* lut;  // period one, 16-bit state: stepsize of every non-negative state value
    int64_t nrows;     // magnitude rows
    int64_t rowlen;    // elements per magnitude row
    int32_t period;    // elements per vmean row (rowlen if P > 1, 1 if P = 1)
    int32_t nvec;      // rowlen / W (register path)
    int32_t lpr_log2;  // log2(lanes per row)
    int32_t mode;      // StepMode
    float b1c, b2, omb2, sqrt_bc2, eps, inv_bc1, lr, wdf;
    int32_t do_wd;
    int32_t nwg;       // workgroups of this task
};

struct StepBatch {
    StepTask t[kMaxBatch];
    int32_t wg_begin[kMaxBatch + 1];
    int32_t ntasks;
    int32_t pad;
    const CodebookTables* tables;
};
static_assert(sizeof(StepBatch) <= 4000, "kernel arguments are limited to 4 KB");

// LDS copy of the codebook tables (6 KB; FINE: 10 KB): the codebook rounded to
// the parameter dtype, the thresholds and the byte bucket index (bucket8; FINE:
// bucket_fine, for a one-probe search).
template <bool FINE>
struct alignas(16) LdsTables {
    float thr[260];
    uint8_t bucket[FINE ? kFineBytes : kBucket8Bytes];
    float cbd[256];
};
static_assert(offsetof(CodebookTables, thr) % 16 == 0 && offsetof(CodebookTables, bucket8) % 16 == 0 &&
                  offsetof(CodebookTables, bucket_fine) % 16 == 0 && offsetof(CodebookTables, nb16) % 16 == 0,
              "codebook tables must allow 16-byte copies");

// The LDS tables are 16-byte pieces: thr (65 pieces, from piece 64 of
// CodebookTables), the bucket (257 pieces of bucket8 right after thr, or 513 of
// bucket_fine from piece 386) and the codebook (pieces 0..63).  Every piece of a
// thread is loaded before any is stored, so a workgroup waits for one round
// trip to L2, not one per table.
constexpr int kThrPieces = 65;
template <bool FINE> constexpr int bucket_pieces() { return FINE ? kFineBytes / 16 : kBucket8Bytes / 16; }
static_assert(offsetof(CodebookTables, thr) == 64 * 16 && offsetof(CodebookTables, bucket8) == (64 + kThrPieces) * 16 &&
                  offsetof(CodebookTables, bucket_fine) == 386 * 16 && sizeof(LdsTables<false>) == 386 * 16 &&
                  sizeof(LdsTables<true>) == 642 * 16 && offsetof(LdsTables<true>, bucket) == kThrPieces * 16 &&
                  offsetof(LdsTables<false>, cbd) == (kThrPieces + 257) * 16 &&
                  offsetof(LdsTables<true>, cbd) == (kThrPieces + 513) * 16,
              "table layout");

// Period-one stepsize of a bf16 state from a 384-entry square-root table
// (kRootTab floats, 96 16-byte pieces; layout at root_h), optionally
// loaded with the codebook tables (root != nullptr).
constexpr int kRootTab = 384;

// NB16: also copy the bf16 nearest-index table (CodebookTables::nb16) to nb16_lds.
template <typename D, int NT, bool NB16 = false, bool FINE>
__device__ __forceinline__ void load_tables(LdsTables<FINE>& L, const CodebookTables* T, int& K,
                                            const float* root = nullptr, float* root_lds = nullptr,
                                            uint8_t* nb16_lds = nullptr) {
    using U4 = RawVec<16>::type;
    constexpr int kThrBucketPieces = kThrPieces + bucket_pieces<FINE>();
    constexpr int kPieces = kThrBucketPieces + 64, kPer = (kPieces + NT - 1) / NT;
    // bucket_fine starts at piece 386, not right after thr
    constexpr int kFineShift = FINE ? (int)(offsetof(CodebookTables, bucket_fine) / 16) - kThrPieces - 64 : 0;
    constexpr int kRootPieces = kRootTab * 4 / 16;
    constexpr int kNbPieces = kNb16Bytes / 16, kNbPer = NB16 ? (kNbPieces + NT - 1) / NT : 0;
    static_assert(NT >= kRootPieces, "one root-table piece per thread");
    K = T->K;
    const U4* src = reinterpret_cast<const U4*>(T);
    U4* dst = reinterpret_cast<U4*>(&L);
    U4 v[kPer];
    U4 nv[kNbPer > 0 ? kNbPer : 1];
    U4 rv;
    const bool has_root = root != nullptr && threadIdx.x < kRootPieces;
    if (has_root) rv = reinterpret_cast<const U4*>(root)[threadIdx.x];
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int q = threadIdx.x + r * NT;
        if (q < kPieces)
            v[r] = src[q < kThrPieces ? q + 64 : (q < kThrBucketPieces ? q + 64 + kFineShift : q - kThrBucketPieces)];
    }
#pragma unroll
    for (int r = 0; r < kNbPer; ++r) {
        const int q = threadIdx.x + r * NT;
        if (q < kNbPieces) nv[r] = reinterpret_cast<const U4*>(T->nb16)[q];
    }
    if (has_root) reinterpret_cast<U4*>(root_lds)[threadIdx.x] = rv;
#pragma unroll
    for (int r = 0; r < kNbPer; ++r) {
        const int q = threadIdx.x + r * NT;
        if (q < kNbPieces) reinterpret_cast<U4*>(nb16_lds)[q] = nv[r];
    }
#pragma unroll
    for (int r = 0; r < kPer; ++r) {
        const int q = threadIdx.x + r * NT;
        if (q < kPieces) {
            if (q >= kThrBucketPieces) {
#pragma unroll
                for (int c = 0; c < 4; ++c) v[r][c] = __float_as_uint(round_to<D>(__uint_as_float(v[r][c])));
            }
            dst[q] = v[r];
        }
    }
    __syncthreads();
}

// Task of this workgroup: the last t with wg_begin[t] <= blockIdx.x (binary
// search over the launch's task table; wg_begin[0] = 0 and is non-decreasing).
__device__ __forceinline__ int find_task(const int32_t* wg_begin, int ntasks) {
    const int b = blockIdx.x;
    int lo = 0, hi = ntasks - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (wg_begin[mid] <= b) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// sum / n rounded once (the block mean of g^2, gefen.py:116-117): a power-of-two
// n (uniform) divides exactly by multiplying with 2^-log2(n), which rounds the
// same real number; other n take the IEEE division.
__device__ __forceinline__ float mean_of(float sum, int32_t n) {
    if ((n & (n - 1)) == 0) return sum * __int_as_float((127 - __builtin_ctz((uint32_t)n)) << 23);
    return sum / (float)n;
}

// stepsize of gefen.py:1326-1327: (1/bc1) * reciprocal(sqrt(v)/sqrt(bc2) + eps)
__device__ __forceinline__ float stepsize_of(float v, const StepTask& T) {
    float h = sqrtf(v) / T.sqrt_bc2 + T.eps;
    return (1.0f / h) * T.inv_bc1;
}

// ---------------------------------------------------------------------------
// Gefen step, register path.

// Period-one stepsize of an f16 state value from the 32768-entry table in
// global memory indexed by its bits (k_build_lut); fp32 states compute it.
template <typename S>
__device__ __forceinline__ float p1_stepsize(S v, const StepTask& T) {
    if constexpr (sizeof(S) == 2) {
        const uint16_t bits = reinterpret_cast<const uint16_t&>(v);
        if (GEFEN_STEP_P1_LUT && T.lut && !(bits & 0x8000u)) return T.lut[bits];
    }
    return stepsize_of(to_f32(v), T);
}

// Period-one stepsize of a bf16 state value (bits) from the LDS square-root
// table root.  A finite v >= 0 is M * 2^E with an integer M < 256 (128 +
// mantissa for normal v, the mantissa for subnormal v), E = max(exponent
// field, 1) - 134.  With par = E mod 2 and half = floor(E / 2) = (bits >> 8) - 67,
// sqrt(v) = sqrt(M * 2^par) * 2^half.  A launch reads the table only when
// 2^-60 <= sqrt_bc2 <= 2^30 and 2^-126 <= eps <= 2^100 (root_table_ok), so
// every value here is a normal float (2^-67 <= sqrt(v) < 2^64 and 2^-97 <=
// fl(sqrt(v)) / sqrt_bc2 <= 2^124 for v > 0, nonzero table entries in
// [2^-97, 2^-2]) and scaling by powers of two commutes with rounding:
//   fl(fl(sqrt(v)) / sqrt_bc2) = root[i] * 2^(bits >> 8)   exactly, with
//   i = bits & 0xff   for normal v (= par * 128 + mantissa; E and the exponent
//                     field have the same parity),
//   i = 256 + bits    for subnormal v and zero (par = 1),
//   root[i] = fl(fl(sqrt(M * 2^par)) / sqrt_bc2) * 2^-67   (k_build_root).
// root_h returns h = that + eps, in [2^-126, 2^126) by the same bounds (eps for
// v = 0, at least 2^-97 for v > 0, at most 2^124 + 2^100).
__device__ __forceinline__ float root_h(uint32_t bits, const StepTask& T, const float* root) {
    const uint32_t i = bits < 0x80u ? bits + 256u : (bits & 0xffu);
    return __builtin_ldexpf(root[i], (int)(bits >> 8)) + T.eps;
}

// The bounds of root_h on the table's settings (checked on the host per launch).
__host__ __device__ inline bool root_table_ok(float sqrt_bc2, float eps) {
    return sqrt_bc2 >= 0x1p-60f && sqrt_bc2 <= 0x1p30f && eps >= 0x1p-126f && eps <= 0x1p100f;
}

// root_h is exact for finite v >= 0 (bits < 0x7f80); negative, inf and NaN
// states take stepsize_of.  In root_h's range of h the reciprocal
// fma(fma(-h, r, 1), r, r) with r = v_rcp_f32(h) equals the IEEE quotient 1 / h
// (checked on gfx950 for every float h in [2^-126, 2^126)).
__device__ __forceinline__ bool root_ok(uint32_t bits) { return bits < 0x7f80u; }

__device__ __forceinline__ float root_stepsize(float h, const StepTask& T) {
    const float r = __builtin_amdgcn_rcpf(h);
    const float e = __builtin_fmaf(-h, r, 1.0f);
    return __builtin_fmaf(e, r, r) * T.inv_bc1;
}

// Bucket one below x's (an fma rounding up can only reach x's own bucket),
// clamped to the grid of bucket8 (FINE: bucket_fine): for finite x, the bucket
// counts the thresholds below x but at most max_probe (max_probe_fine) of them.
template <bool FINE>
__device__ __forceinline__ int bucket_below(float x) {
    constexpr float kHalf = FINE ? 4096.0f : 2048.0f;
    float y = __builtin_fmaf(x, kHalf, kHalf - 1.0f);  // (x + 1) * cells / 2 - 1, rounded once
    y = fminf(fmaxf(y, 0.0f), 2.0f * kHalf);
    return (int)y;
}

// Nearest index with at most two threshold probes (max_probe <= 2): one
// ds_read2 of thr[k+1], thr[k+2] after the bucket lookup.
template <bool FINE>
__device__ __forceinline__ int nearest_two_probe(float x, const float* thr, const uint8_t* bucket) {
    int k = bucket[bucket_below<FINE>(x)];
    const float t1 = thr[k + 1], t2 = thr[k + 2];
    k += (t1 < x ? 1 : 0) + (t2 < x ? 1 : 0);
    return k;
}

// Nearest index with one threshold probe (max_probe_fine <= 1).
__device__ __forceinline__ int nearest_one_probe(float x, const float* thr, const uint8_t* bucket_fine) {
    const int k = bucket_fine[bucket_below<true>(x)];
    return k + (thr[k + 1] < x ? 1 : 0);
}

// Second sweep of a row: quantise, dequantise, update p.  QROUND: the
// dequantised update cb[idx]*mag is rounded to D (param dtype == state dtype)
// or kept in fp32 (fp32 state).  PROBES 1 or 2: the block magnitude is finite
// and positive and the search with that many probes is exact (0: the general
// search).  Every lane computes all R
// vectors (out-of-row vectors hold a copy of the row's last vector); only
// in-row vectors of active rows are stored.  WD: weight decay
// (gefen.py:1280-1281) is applied to the parameter first.  root: the LDS
// square-root table of a period-one bf16 state, or nullptr.
template <typename D, typename S, int W, int R, bool P1, bool TAB, int PROBES, bool WD, bool FINE, typename UF>
__device__ __forceinline__ void step_sweep2(const StepTask& T, const LdsTables<FINE>& L, const float* utab,
                                            const float* root, const UF& upd_of, const Vec<D, W> (&gv)[R],
                                            const Vec<D, W> (&pv)[R], const Vec<S, W> (&vv)[R], uint8_t* idx, D* p,
                                            S* vm, uint32_t base, int lir, int lpr, bool active, int K, float mn,
                                            double rb, float ss) {
    constexpr bool QROUND = sizeof(D) == sizeof(S);
#pragma unroll
    for (int j = 0; j < R; ++j) {
        Vec<uint8_t, W> io;
        Vec<D, W> po;
        Vec<S, W> vo;
        float sw[W];  // period one: stepsize of each element's new vmean
        if constexpr (P1) {
            bool special = false;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float gf = to_f32(gv[j].v[w]);
                const float sq = gf * gf;  // mean over a one-element row
                const float prev = to_f32(vv[j].v[w]) * T.b2;
                const S vnew = from_f32<S>(__builtin_fmaf(sq, T.omb2, prev));
                vo.v[w] = vnew;
                if constexpr (std::is_same<S, bf16_t>::value) {
                    if (root) {
                        special = special || !root_ok(vnew.bits);
                        sw[w] = root_stepsize(root_h(vnew.bits, T, root), T);
                    } else {
                        sw[w] = stepsize_of(to_f32(vnew), T);
                    }
                } else {
                    sw[w] = p1_stepsize<S>(vnew, T);
                }
            }
            if constexpr (std::is_same<S, bf16_t>::value) {
                if (special) {  // one branch per vector for the rare values outside the table's range
#pragma unroll
                    for (int w = 0; w < W; ++w)
                        if (!root_ok(vo.v[w].bits))
                            sw[w] = stepsize_of(to_f32(vo.v[w]), T);
                }
            }
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
            int k;
            if constexpr (PROBES == 1) {
                static_assert(FINE, "a single probe needs the fine bucket");
                k = nearest_one_probe(div_by_block(upd_of(j, w), rb), L.thr, L.bucket);
            } else if constexpr (PROBES == 2) {
                k = nearest_two_probe<FINE>(div_by_block(upd_of(j, w), rb), L.thr, L.bucket);
            } else {
                const bool plain = (mn > 0.0f) && (mn < __builtin_inff());
                const float uj = upd_of(j, w);
                const float x = plain ? div_by_block(uj, rb) : ((mn > 0.0f) ? uj / mn : 0.0f);
                k = nearest_fast<FINE>(x, L.thr, L.bucket, K);
            }
            io.v[w] = (uint8_t)k;
            float u;
            if (TAB && !P1 && PROBES > 0) {
                u = utab[k];
            } else {
                float q = L.cbd[k] * mn;
                if (QROUND) q = round_to<D>(q);
                const float s = P1 ? sw[w] : ss;
                u = (q * s) * T.lr;
            }
            float pf = to_f32(pv[j].v[w]);
            if (WD) pf = round_to<D>(pf * T.wdf);
            po.v[w] = from_f32<D>(pf - u);
        }
        const int v = lir + j * lpr;
        if (active && v < T.nvec) {
            const uint32_t e = base + (uint32_t)(v * W);
            sstore<uint8_t, W>(idx, e, io);
            sstore<D, W>(p, e, po);
            if (P1) sstore<S, W>(vm, e, vo);
        }
    }
}

// TAB: a lane group of >= 32 lanes owns the row and keeps two row tables in
// LDS, cur[i] = cb_D[i] * old magnitude and upd[i] = the parameter step of
// codeword i (gefen.py:1205-1206, 1328-1332 for this row's magnitude and
// stepsize), so the element loops look both up instead of recomputing.
//
// Loads are unconditional and straight-line: a lane group past the last row
// reads the last row, a vector past the row end reads the row's last vector,
// so each lane has all of its row's bytes in flight at once.  Absmax is
// idempotent under such copies; the sum of squares masks them out.
template <typename D, typename S, int W, int R, bool P1, bool TAB>
__global__ __launch_bounds__(kStepThreads) void k_gefen_step(const StepBatch B) {
    constexpr bool kRoot = P1 && std::is_same<S, bf16_t>::value;
    // 16-bit parameters search the fine bucket with one probe where the codebook
    // allows; fp32 kernels keep the 6 KB tables, which leave them one more
    // workgroup per CU
    constexpr bool kFine = sizeof(D) == 2;
    __shared__ LdsTables<kFine> L;
    // row tables of the wave's rows: rows of at least two vectors per lane own a
    // whole wave (64 lanes), so one slot per wave; single-vector rows may take 32
    // lanes, two rows per wave (make_step_task keeps to this).  The smaller LDS
    // footprint lets more workgroups share a CU.
    constexpr int kRowSlots = (TAB && R == 1) ? 2 : 1;
    __shared__ float row_tab[TAB ? kStepWaves : 1][kRowSlots][2][256];
    __shared__ __attribute__((aligned(16))) float root_lds[kRoot ? kRootTab : 4];
    // every task of a launch has the same stepsize table (flush_steps)
    const float* root_src = kRoot ? B.t[0].lut : nullptr;
    const float* root = root_src ? root_lds : nullptr;  // uniform
    int K;
    load_tables<D, kStepThreads>(L, B.tables, K, root_src, root_lds);
    const int max_probe = kFine ? B.tables->max_probe_fine : B.tables->max_probe;
    const bool two_probe = max_probe <= 2, one_probe = kFine && max_probe <= 1;
    const int ti = find_task(B.wg_begin, B.ntasks);
    const StepTask T = B.t[ti];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lpr = 1 << T.lpr_log2;
    const int rpw = 64 >> T.lpr_log2;
    const int lir = lane & (lpr - 1);
    const int sub = lane >> T.lpr_log2;
    const int64_t lw = blockIdx.x - B.wg_begin[ti];
    float* ctab = row_tab[TAB ? wave : 0][kRowSlots == 2 ? (sub & 1) : 0][0];
    float* utab = row_tab[TAB ? wave : 0][kRowSlots == 2 ? (sub & 1) : 0][1];

    constexpr int kIt = step_iter<P1>();
    for (int it = 0; it < kIt; ++it) {
        const int64_t unit = (lw * kIt + it) * kStepWaves + wave;
        const int64_t row0 = unit * rpw;
        if (row0 >= T.nrows) break;  // uniform across the wave
        const int64_t row = row0 + sub;
        const bool active = row < T.nrows;
        const int rsub = active ? sub : (int)(T.nrows - 1 - row0);  // row within the unit
        // the unit's rows start here; lanes address them with 32-bit offsets
        // (64 rows of at most 64 * 8 * 8 elements)
        const int64_t ub = row0 * T.rowlen;
        D* __restrict__ p = static_cast<D*>(T.p) + ub;
        const D* __restrict__ g = static_cast<const D*>(T.g) + ub;
        uint8_t* __restrict__ idx = T.idx + ub;
        S* __restrict__ mag = static_cast<S*>(T.mag) + row0;
        S* __restrict__ vm = static_cast<S*>(T.vmean) + (P1 ? ub : row0);
        const float* stepsize = T.stepsize + row0;
        const uint32_t base = (uint32_t)rsub * (uint32_t)T.rowlen;

        // every element vector of the row, then the row scalars
        Vec<D, W> gv[R], pv[R];
        Vec<uint8_t, W> iv[R];
        Vec<S, W> vv[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int v = min(lir + j * lpr, T.nvec - 1);
            const uint32_t e = base + (uint32_t)(v * W);
            gv[j] = sload<D, W>(g, e);
            iv[j] = sload<uint8_t, W>(idx, e);
            pv[j] = sload<D, W>(p, e);
            if (P1) vv[j] = sload<S, W>(vm, e);
        }
        const S mold_s = mag[rsub];
        S vold_s = S();
        float step_given = 0.0f;
        if (!P1) {
            if (T.mode == kStepsizeGiven) step_given = stepsize[rsub];
            else vold_s = vm[rsub];
        }
        const float mold = to_f32(mold_s);
        // vmean (vmean modes) or stepsize (given-stepsize mode) of the row
        const float rowv = (T.mode == kStepsizeGiven) ? step_given : to_f32(vold_s);
        if (TAB) {
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = lir + t * lpr;
                if (i < 256) ctab[i] = L.cbd[i] * mold;
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        float upd[R][W];
        uint32_t mxk = 0;
        float sumsq = 0.0f;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            float sj = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float gf = to_f32(gv[j].v[w]);
                const float cur = TAB ? ctab[iv[j].v[w]] : L.cbd[iv[j].v[w]] * mold;
                const float u = __builtin_fmaf(T.b1c, gf - cur, cur);  // lerp, weight < 0.5
                upd[j][w] = u;
                const uint32_t key = abs_key(u);
                mxk = key > mxk ? key : mxk;
                if (!P1) sj = __builtin_fmaf(gf, gf, sj);
            }
            if (!P1) sumsq = sumsq + ((lir + j * lpr < T.nvec) ? sj : 0.0f);
        }
        const float mx = __uint_as_float(wave_group_max_u32(mxk, lpr));
        float ss = 0.0f;
        if (!P1) {
            if (T.mode == kVmeanUpdate) {
                const float tot = wave_group_sum(sumsq, lpr);
                const float ms = mean_of(tot, T.period);
                const S vnew = from_f32<S>(__builtin_fmaf(ms, T.omb2, rowv * T.b2));
                if (active && lir == 0) vm[rsub] = vnew;
                ss = stepsize_of(to_f32(vnew), T);
            } else if (T.mode == kVmeanGiven) {
                ss = stepsize_of(rowv, T);
            } else {
                ss = rowv;
            }
        }
        const S mag_s = from_f32<S>(mx);
        if (active && lir == 0) mag[rsub] = mag_s;
        const float mn = to_f32(mag_s);
        auto upd_of = [&](int j, int w) -> float { return upd[j][w]; };
        // x = upd / mn where mn > 0, else 0 (gefen.py:1184-1187).  A block whose
        // magnitude is 0, NaN or inf takes the general element path.
        const bool plain = (mn > 0.0f) && (mn < __builtin_inff());
        const double rb = plain ? 1.0 / (double)mn : 0.0;
        const bool fast = plain && two_probe;
        if (TAB && !P1) {
            if (fast) {
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const int i = lir + t * lpr;
                    if (i < 256) {
                        float q = L.cbd[i] * mn;
                        if (sizeof(D) == sizeof(S)) q = round_to<D>(q);
                        utab[i] = (q * ss) * T.lr;
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
#define GEFEN_SWEEP2(PROBES, WD)                                                                                 \
    step_sweep2<D, S, W, R, P1, TAB, PROBES, WD>(T, L, utab, root, upd_of, gv, pv, vv, idx, p, vm, base, lir, lpr, active, \
                                                 K, mn, rb, ss)
        // (one_probe is false without the fine bucket: kFine ? 1 : 2 only keeps
        // the single-probe sweep from being instantiated there)
        if (T.do_wd) {
            if (fast && one_probe) GEFEN_SWEEP2(kFine ? 1 : 2, true);
            else if (fast) GEFEN_SWEEP2(2, true);
            else GEFEN_SWEEP2(0, true);
        } else {
            if (fast && one_probe) GEFEN_SWEEP2(kFine ? 1 : 2, false);
            else if (fast) GEFEN_SWEEP2(2, false);
            else GEFEN_SWEEP2(0, false);
        }
#undef GEFEN_SWEEP2
    }
}

// ---------------------------------------------------------------------------
// Gefen step, two-sweep path for rows longer than the register path holds
// (P > 1 only): one workgroup per row, the second sweep re-reads g and idx.
template <typename D, typename S>
__global__ __launch_bounds__(kThreads) void k_gefen_step_long(const StepBatch B) {
    __shared__ LdsTables<false> L;
    __shared__ float red_mx[4], red_sum[4];
    int K;
    load_tables<D, kThreads>(L, B.tables, K);
    const int ti = find_task(B.wg_begin, B.ntasks);
    const StepTask& T = B.t[ti];
    constexpr bool QROUND = sizeof(D) == sizeof(S);
    const int64_t row = blockIdx.x - B.wg_begin[ti];
    if (row >= T.nrows) return;
    D* __restrict__ p = static_cast<D*>(T.p);
    const D* __restrict__ g = static_cast<const D*>(T.g);
    uint8_t* __restrict__ idx = T.idx;
    S* __restrict__ mag = static_cast<S*>(T.mag);
    S* __restrict__ vm = static_cast<S*>(T.vmean);
    const int64_t base = row * T.rowlen;
    const float mold = to_f32(mag[row]);
    float mx = 0.0f, sumsq = 0.0f;
    for (int64_t j = threadIdx.x; j < T.rowlen; j += kThreads) {
        const float gf = to_f32(g[base + j]);
        const float cur = L.cbd[idx[base + j]] * mold;
        const float u = __builtin_fmaf(T.b1c, gf - cur, cur);
        mx = nanmax(mx, fabsf(u));
        const float sq = gf * gf;
        sumsq = sumsq + sq;
    }
    mx = group_max(mx, 64);
    sumsq = group_sum(sumsq, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { red_mx[wave] = mx; red_sum[wave] = sumsq; }
    __syncthreads();
    mx = nanmax(nanmax(red_mx[0], red_mx[1]), nanmax(red_mx[2], red_mx[3]));
    const float tot = (red_sum[0] + red_sum[1]) + (red_sum[2] + red_sum[3]);
    float ss;
    if (T.mode == kVmeanUpdate) {
        const float ms = mean_of(tot, T.period);
        const float prev = to_f32(vm[row]) * T.b2;
        const S vnew = from_f32<S>(__builtin_fmaf(ms, T.omb2, prev));
        ss = stepsize_of(to_f32(vnew), T);
        __syncthreads();  // every thread has read vm[row] before it is replaced
        if (threadIdx.x == 0) vm[row] = vnew;
    } else if (T.mode == kVmeanGiven) {
        ss = stepsize_of(to_f32(vm[row]), T);
    } else {
        ss = T.stepsize[row];
    }
    const S mag_s = from_f32<S>(mx);
    const float mn = to_f32(mag_s);
    __syncthreads();  // every thread has read mag[row] (mold) before it is replaced
    if (threadIdx.x == 0) mag[row] = mag_s;
    for (int64_t j = threadIdx.x; j < T.rowlen; j += kThreads) {
        const float gf = to_f32(g[base + j]);
        const float cur = L.cbd[idx[base + j]] * mold;
        const float u = __builtin_fmaf(T.b1c, gf - cur, cur);
        const float x = (mn > 0.0f) ? u / mn : 0.0f;
        const int k = nearest_fast<false>(x, L.thr, L.bucket, K);
        idx[base + j] = (uint8_t)k;
        float q = L.cbd[k] * mn;
        if (QROUND) q = round_to<D>(q);
        const float uu = (q * ss) * T.lr;
        float pf = to_f32(p[base + j]);
        if (T.do_wd) pf = round_to<D>(pf * T.wdf);
        p[base + j] = from_f32<D>(pf - uu);
    }
}

// ---------------------------------------------------------------------------
// GefenMuon quantised momentum (gefen_muon.py:302-316 with 132-171): every op is
// a torch op on a D tensor, so each result is rounded to D.
struct MuonTask {
    const void* g;
    uint8_t* idx;
    void* mag;
    void* out;
    int64_t nrows;
    int64_t rowlen;
    int32_t nvec;
    int32_t lpr_log2;
    float w;       // f32(1 - momentum): lerp weight
    float mom;     // f32(momentum)
    float alpha;   // add_ alpha: f32(1 - momentum), rounded to D for reduced dtypes
    float tiny;    // finfo(D).tiny rounded to S
    int32_t nesterov;
    int32_t nwg;
    double* sumsq;  // if set: GEFEN_SUMSQ_SLOTS accumulators (16 doubles apart) of the sum of squares of the output
};

struct MuonBatch {
    MuonTask t[kMaxBatch];
    int32_t wg_begin[kMaxBatch + 1];
    int32_t ntasks;
    int32_t pad;
    const CodebookTables* tables;
};
static_assert(sizeof(MuonBatch) <= 4000, "kernel arguments are limited to 4 KB");

// Workgroup sum of the lanes' sums of squares (kThreads lanes), added to slot
// `key mod GEFEN_SUMSQ_SLOTS` of a task's accumulators (one 128-byte line each):
// one float64 atomic per workgroup, spread over separate lines.
__device__ __forceinline__ void add_sumsq(float v, double* sumsq, int64_t key) {
    __shared__ float red[kThreads / 64];
    v = group_sum(v, 64);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) t = t + red[w];
        atomicAdd(sumsq + 16 * (key & (GEFEN_SUMSQ_SLOTS - 1)), (double)t);
    }
}

// Nesterov blend of gefen_muon.py:312-316 on a = D(q * momentum): add_(g, alpha)
template <typename D>
__device__ __forceinline__ float muon_blend(float a, float gf, const MuonTask& T) {
    if (!T.nesterov) return a;
    // fp32: fma; reduced dtype: alpha is in D, so the product is exact and the
    // fma rounds once, as the unfused sum would
    return __builtin_fmaf(gf, T.alpha, a);
}

// bf16 bits of two floats (round to nearest even), a in the low half: one
// v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pk_bf16_bits(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 v = __builtin_convertvector((f2){a, b}, b2);
    uint32_t r;
    __builtin_memcpy(&r, &v, 4);
    return r;
}

// Per-half unsigned max of two packed 16-bit values (v_pk_max_u16).
__device__ __forceinline__ uint32_t max_u16x2(uint32_t a, uint32_t b) {
    typedef unsigned short u2 __attribute__((ext_vector_type(2)));
    u2 x, y;
    __builtin_memcpy(&x, &a, 4);
    __builtin_memcpy(&y, &b, 4);
    const u2 r = __builtin_elementwise_max(x, y);
    uint32_t o;
    __builtin_memcpy(&o, &r, 4);
    return o;
}

// acc + lo^2 + hi^2 of the two bf16 values packed in v (v_dot2c_f32_bf16; the
// products are exact in float32).
__device__ __forceinline__ float dot2_bf16(uint32_t v, float acc) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    b2 x;
    __builtin_memcpy(&x, &v, 4);
    return __builtin_amdgcn_fdot2_f32_bf16(x, x, acc, false);
}

template <typename D, typename S>
__device__ __forceinline__ float muon_out(float q, float gf, const MuonTask& T) {
    if (!T.nesterov) return q;
    return muon_blend<D>(round_to<D>(q * T.mom), gf, T);  // mul_(momentum), then the blend
}

// Register path: as k_gefen_step, a lane group per row and straight-line
// unconditional loads (a lane group past the last row reads the last row, a
// vector past the row end the row's last vector: the absmax is idempotent under
// such copies), non-temporal, addressed from the wave's unit base.  TAB: a lane
// group of >= 32 lanes keeps two row tables in LDS, cur[i] = D(cb_D[i] * old
// magnitude) and out[i] = the output of codeword i without the Nesterov
// gradient term, so the element loops look them up instead of recomputing.
template <typename D, typename S, int W, int R, bool TAB>
__global__ __launch_bounds__(kThreads) void k_muon(const MuonBatch B) {
    constexpr bool kNb = std::is_same<D, bf16_t>::value;  // bf16 quotients: the nb16 table
    constexpr bool kPk = kNb && W % 2 == 0;                // bf16 pairs: packed conversions
    __shared__ LdsTables<false> L;
    // one row table per wave: row tables are used for whole-wave rows only
    // (make_muon_task keeps to this)
    __shared__ float row_tab[TAB ? 4 : 1][2][256];
    __shared__ __attribute__((aligned(16))) uint8_t nb16[kNb ? kNb16Bytes : 16];
    int K;
    load_tables<D, kThreads, kNb>(L, B.tables, K, nullptr, nullptr, nb16);
    const int ti = find_task(B.wg_begin, B.ntasks);
    const MuonTask& T = B.t[ti];
    const bool two_probe = B.tables->max_probe <= 2;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lpr = 1 << T.lpr_log2;
    const int rpw = 64 >> T.lpr_log2;
    const int lir = lane & (lpr - 1);
    const int sub = lane >> T.lpr_log2;
    const int64_t lw = blockIdx.x - B.wg_begin[ti];
    float* ctab = row_tab[TAB ? wave : 0][0];
    float* otab = row_tab[TAB ? wave : 0][1];
    float wsq = 0.0f;  // this lane's sum of squares of the outputs it wrote

    for (int it = 0; it < kMuonIter; ++it) {
        const int64_t unit = (lw * kMuonIter + it) * 4 + wave;
        const int64_t row0 = unit * rpw;
        if (row0 >= T.nrows) break;  // uniform across the wave
        const int64_t row = row0 + sub;
        const bool active = row < T.nrows;
        const int rsub = active ? sub : (int)(T.nrows - 1 - row0);
        const int64_t ub = row0 * T.rowlen;
        const D* __restrict__ g = static_cast<const D*>(T.g) + ub;
        uint8_t* __restrict__ idx = T.idx + ub;
        D* __restrict__ out = static_cast<D*>(T.out) + ub;
        S* __restrict__ mag = static_cast<S*>(T.mag) + row0;
        const uint32_t base = (uint32_t)rsub * (uint32_t)T.rowlen;
        Vec<D, W> gv[R];
        Vec<uint8_t, W> iv[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
            const int v = min(lir + j * lpr, T.nvec - 1);
            const uint32_t e = base + (uint32_t)(v * W);
            gv[j] = sload<D, W>(g, e);
            iv[j] = sload<uint8_t, W>(idx, e);
        }
        const float mold = to_f32(mag[rsub]);
        if (TAB) {
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = lir + t * lpr;
                if (i < 256) ctab[i] = round_to<D>(L.cbd[i] * mold);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        float mu[R][W];
        uint32_t mxk = 0;  // ordered |m1|: the unsigned max is the NaN-propagating absmax
        if constexpr (kPk) {
            // bf16 pairs: one conversion rounds two lerps, and the absmax runs on
            // the packed |bf16| bits (the top halves of the float32 keys)
            uint32_t mx2 = 0;
#pragma unroll
            for (int j = 0; j < R; ++j) {
#pragma unroll
                for (int w = 0; w < W; w += 2) {
                    const float g0 = to_f32(gv[j].v[w]), g1 = to_f32(gv[j].v[w + 1]);
                    float c0, c1;  // dequant * mag
                    if (TAB) {
                        c0 = ctab[iv[j].v[w]];
                        c1 = ctab[iv[j].v[w + 1]];
                    } else {
                        const uint32_t c = pk_bf16_bits(L.cbd[iv[j].v[w]] * mold, L.cbd[iv[j].v[w + 1]] * mold);
                        c0 = __uint_as_float(c << 16);
                        c1 = __uint_as_float(c & 0xffff0000u);
                    }
                    const uint32_t pk = pk_bf16_bits(__builtin_fmaf(T.w, g0 - c0, c0), __builtin_fmaf(T.w, g1 - c1, c1));
                    mu[j][w] = __uint_as_float(pk << 16);
                    mu[j][w + 1] = __uint_as_float(pk & 0xffff0000u);
                    mx2 = max_u16x2(mx2, pk & 0x7fff7fffu);
                }
            }
            const uint32_t lo = mx2 & 0xffffu, hi = mx2 >> 16;
            mxk = (lo > hi ? lo : hi) << 16;
        } else {
#pragma unroll
            for (int j = 0; j < R; ++j) {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const float gf = to_f32(gv[j].v[w]);
                    const float m0 = TAB ? ctab[iv[j].v[w]] : round_to<D>(L.cbd[iv[j].v[w]] * mold);  // dequant * mag
                    const float m1 = round_to<D>(__builtin_fmaf(T.w, gf - m0, m0));                   // lerp_
                    mu[j][w] = m1;
                    const uint32_t key = abs_key(m1);
                    mxk = key > mxk ? key : mxk;
                }
            }
        }
        const float mx = __uint_as_float(wave_group_max_u32(mxk, lpr));
        const S mag_s = from_f32<S>(mx);
        if (active && lir == 0) mag[rsub] = mag_s;
        const float ms = to_f32(mag_s);
        const float clamped = (ms < T.tiny) ? T.tiny : ms;  // clamp(min=tiny) in S
        // FAST: a finite positive magnitude, the division as the float64 product
        // with the reciprocal (exact, see div_by_block) and the two-probe search
        const bool fast = two_probe && ms > 0.0f && clamped < __builtin_inff();
        const double rb = fast ? 1.0 / (double)clamped : 0.0;
        // The bf16 table path rounds the float32 product m1 * r32 instead: m1 and
        // the magnitude are bf16 values (8-bit significands), so m1 / magnitude is
        // never a bf16 rounding midpoint and lies at least 2^-17 (relative) away
        // from every midpoint, while the product is within 2^-23 of it as long as
        // r32 and the product are normal; then both round to the same bf16 value
        // as the IEEE quotient.  Rows with magnitudes from 2^100 (r32 near the
        // subnormal range) and quotients below the table (|x| < 2^-20) take the
        // float64 quotient.
        const float r32 = (float)rb;
        const bool fast32 = fast && clamped < 0x1p100f;
        // output of codeword k before the Nesterov gradient term: q = D(cb_D[k] * mag),
        // then D(q * momentum) with Nesterov
        auto out_base = [&](int k) -> float {
            const float q = round_to<D>(L.cbd[k] * ms);  // copy_(cb[idx]) then mul_(mag)
            return T.nesterov ? round_to<D>(q * T.mom) : q;
        };
        if (TAB) {
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const int i = lir + t * lpr;
                if (i < 256) otab[i] = out_base(i);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        float sq = 0.0f;  // sum of squares of the outputs this lane writes
        // every row of the wave fast (wave-uniform): the branch-free search below
        const bool all_fast = __builtin_amdgcn_ballot_w64(!fast32) == 0;
        // the element loop, instantiated for T.nesterov (uniform over the workgroup)
        auto elements = [&](auto nes_tag) {
        constexpr bool NES = decltype(nes_tag)::value;
#pragma unroll
        for (int j = 0; j < R; ++j) {
            Vec<uint8_t, W> io;
            Vec<D, W> oo;
            float sqj = 0.0f;
            int kw[W];
            if (kNb && all_fast) {
                // the bf16 quotient's bits index nb16 directly (two quotients per
                // conversion); the read index is clamped into the table, and a lane
                // with a quotient outside it (|x| < 2^-20) redoes its vector with
                // the two-probe search, once per wave
                bool miss = false;
#pragma unroll
                for (int w = 0; w < W; w += 2) {
                    const uint32_t xb2 = pk_bf16_bits(mu[j][w] * r32, w + 1 < W ? mu[j][w + 1] * r32 : 0.0f);
#pragma unroll
                    for (int h = 0; h < 2 && w + h < W; ++h) {
                        const uint32_t off = ((h ? xb2 >> 16 : xb2) & 0x7fffu) - kNb16Lo;
                        const int32_t sg = (int32_t)(h ? xb2 : xb2 << 16) >> 31;  // -1 for a negative x
                        miss |= off >= kNb16Side;
                        kw[w + h] = nb16[(int32_t)kNb16Side + ((int32_t)min(off, kNb16Side - 1u) ^ sg)];
                    }
                }
                if (__builtin_amdgcn_ballot_w64(miss) != 0 && miss) {
#pragma unroll
                    for (int w = 0; w < W; ++w)
                        kw[w] = nearest_two_probe<false>(round_to<D>(div_by_block(mu[j][w], rb)), L.thr, L.bucket);
                }
            } else {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    if (fast) {
                        kw[w] = nearest_two_probe<false>(round_to<D>(div_by_block(mu[j][w], rb)), L.thr, L.bucket);
                    } else {
                        float x = round_to<D>(mu[j][w] / clamped);  // div_
                        if (ms <= 0.0f) x = 0.0f;                   // masked_fill_(mag <= 0)
                        kw[w] = nearest_fast<false>(x, L.thr, L.bucket, K);
                    }
                }
            }
            // the output: a = D(q * momentum) of codeword k (q without Nesterov),
            // then the Nesterov blend a + g * alpha, one rounding (as muon_blend)
            if constexpr (kPk) {
#pragma unroll
                for (int w = 0; w < W; w += 2) {
                    io.v[w] = (uint8_t)kw[w];
                    io.v[w + 1] = (uint8_t)kw[w + 1];
                    float a0, a1;
                    if (TAB) {
                        a0 = otab[kw[w]];
                        a1 = otab[kw[w + 1]];
                    } else {  // out_base of both codewords, two values per conversion
                        uint32_t q = pk_bf16_bits(L.cbd[kw[w]] * ms, L.cbd[kw[w + 1]] * ms);
                        if (NES) q = pk_bf16_bits(__uint_as_float(q << 16) * T.mom, __uint_as_float(q & 0xffff0000u) * T.mom);
                        a0 = __uint_as_float(q << 16);
                        a1 = __uint_as_float(q & 0xffff0000u);
                    }
                    if (NES) {
                        a0 = __builtin_fmaf(to_f32(gv[j].v[w]), T.alpha, a0);
                        a1 = __builtin_fmaf(to_f32(gv[j].v[w + 1]), T.alpha, a1);
                    }
                    const uint32_t pk = pk_bf16_bits(a0, a1);
                    oo.v[w].bits = (uint16_t)pk;
                    oo.v[w + 1].bits = (uint16_t)(pk >> 16);
                    sqj = dot2_bf16(pk, sqj);  // + o0^2 + o1^2 (exact products)
                }
            } else {
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const int k = kw[w];
                    io.v[w] = (uint8_t)k;
                    const float a = TAB ? otab[k] : out_base(k);
                    oo.v[w] = from_f32<D>(muon_blend<D>(a, to_f32(gv[j].v[w]), T));
                    const float o = to_f32(oo.v[w]);
                    sqj = __builtin_fmaf(o, o, sqj);
                }
            }
            const int v = lir + j * lpr;
            if (active && v < T.nvec) {
                const uint32_t e = base + (uint32_t)(v * W);
                sstore<uint8_t, W>(idx, e, io);
                sstore<D, W>(out, e, oo);
                sq += sqj;
            }
        }
        };
        if (T.nesterov) elements(std::true_type{});
        else elements(std::false_type{});
        wsq += sq;
    }
    if (T.sumsq) add_sumsq(wsq, T.sumsq, lw);  // uniform: one task per workgroup
}

template <typename D, typename S>
__global__ __launch_bounds__(kThreads) void k_muon_long(const MuonBatch B) {
    __shared__ LdsTables<false> L;
    __shared__ float red_mx[4];
    int K;
    load_tables<D, kThreads>(L, B.tables, K);
    const int ti = find_task(B.wg_begin, B.ntasks);
    const MuonTask& T = B.t[ti];
    const int64_t row = blockIdx.x - B.wg_begin[ti];
    if (row >= T.nrows) return;
    const D* __restrict__ g = static_cast<const D*>(T.g);
    uint8_t* __restrict__ idx = T.idx;
    S* __restrict__ mag = static_cast<S*>(T.mag);
    D* __restrict__ out = static_cast<D*>(T.out);
    const int64_t base = row * T.rowlen;
    const float mold = to_f32(mag[row]);
    float mx = 0.0f;
    for (int64_t j = threadIdx.x; j < T.rowlen; j += kThreads) {
        const float gf = to_f32(g[base + j]);
        const float m0 = round_to<D>(L.cbd[idx[base + j]] * mold);
        const float m1 = round_to<D>(__builtin_fmaf(T.w, gf - m0, m0));
        mx = nanmax(mx, fabsf(m1));
    }
    mx = group_max(mx, 64);
    if ((threadIdx.x & 63) == 0) red_mx[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = nanmax(nanmax(red_mx[0], red_mx[1]), nanmax(red_mx[2], red_mx[3]));
    const S mag_s = from_f32<S>(mx);
    const float ms = to_f32(mag_s);
    const float clamped = (ms < T.tiny) ? T.tiny : ms;
    __syncthreads();
    if (threadIdx.x == 0) mag[row] = mag_s;
    float sq = 0.0f;
    for (int64_t j = threadIdx.x; j < T.rowlen; j += kThreads) {
        const float gf = to_f32(g[base + j]);
        const float m0 = round_to<D>(L.cbd[idx[base + j]] * mold);
        const float m1 = round_to<D>(__builtin_fmaf(T.w, gf - m0, m0));
        float x = round_to<D>(m1 / clamped);
        if (ms <= 0.0f) x = 0.0f;
        const int k = nearest_fast<false>(x, L.thr, L.bucket, K);
        idx[base + j] = (uint8_t)k;
        const float q = round_to<D>(L.cbd[k] * ms);
        const D o = from_f32<D>(muon_out<D, S>(q, gf, T));
        out[base + j] = o;
        const float of = to_f32(o);
        sq = __builtin_fmaf(of, of, sq);
    }
    if (T.sumsq) add_sumsq(sq, T.sumsq, row);
}

// ---------------------------------------------------------------------------
// Packed 4-bit codebook indices (automatic_gefen_fused_kernel.cu:14-57): the
// index of element e is the low nibble of byte e/2 when e is even and the high
// nibble when e is odd, and a stored index keeps its low four bits only.  A lane
// owns whole bytes, so both nibbles of a byte inside one row go out in one plain
// byte store.  A byte shared by two rows (odd period), or holding the last
// element of an odd-length tensor, is changed by one atomic xor of old ^ new on
// the row's own nibble: xors of disjoint nibbles commute, so both rows' nibbles
// land and the nibble past the tensor's end keeps its bits.  No other lane
// writes a lane's own nibble, so the byte it loaded holds that nibble's old value.
//
// G lanes per row (16, 64 or 256), kThreads / G rows per workgroup; the
// workgroups stride over the rows.
constexpr int kPackedMaxGrid = 65536;

__device__ __forceinline__ void store_nibbles(uint8_t* idx, int64_t b, uint32_t oldb, int k0, int k1, bool in0,
                                              bool in1) {
    if (in0 && in1) {
        idx[b] = (uint8_t)((k0 & 15) | ((k1 & 15) << 4));
        return;
    }
    const uint32_t x = in0 ? (((uint32_t)k0 ^ oldb) & 15u) : ((((uint32_t)k1 ^ (oldb >> 4)) & 15u) << 4);
    if (x == 0) return;
    const uintptr_t a = reinterpret_cast<uintptr_t>(idx + b);
    atomicXor(reinterpret_cast<unsigned int*>(a & ~(uintptr_t)3), x << (8u * (uint32_t)(a & 3)));
}

// Max over the G lanes of a row; for G = 256 through LDS, with a barrier on each
// side so every lane has read the row's old magnitude and red[] is free again.
template <int G>
__device__ __forceinline__ float packed_row_max(float mx, float* red) {
    if constexpr (G <= 64) {
        return group_max(mx, G);
    } else {
        mx = group_max(mx, 64);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
        __syncthreads();
        const float r = nanmax(nanmax(red[0], red[1]), nanmax(red[2], red[3]));
        __syncthreads();
        return r;
    }
}

// Gefen update with a given stepsize or given vmean (rows of `rowlen`), packed indices.
template <typename D, typename S, int G>
__global__ __launch_bounds__(kThreads) void k_gefen_step_packed(const StepBatch B) {
    __shared__ LdsTables<false> L;
    __shared__ float red[4];
    int K;
    load_tables<D, kThreads>(L, B.tables, K);
    const StepTask& T = B.t[0];
    constexpr bool QROUND = sizeof(D) == sizeof(S);
    constexpr int RPW = kThreads / G;
    const int sub = threadIdx.x / G, t = threadIdx.x % G;
    D* __restrict__ p = static_cast<D*>(T.p);
    const D* __restrict__ g = static_cast<const D*>(T.g);
    uint8_t* idx = T.idx;
    S* __restrict__ mag = static_cast<S*>(T.mag);
    const S* __restrict__ vm = static_cast<const S*>(T.vmean);
    for (int64_t r0 = (int64_t)blockIdx.x * RPW; r0 < T.nrows; r0 += (int64_t)gridDim.x * RPW) {
        const int64_t row = r0 + sub;
        const bool active = row < T.nrows;
        const int64_t e_lo = row * T.rowlen, e_hi = e_lo + T.rowlen;
        const int64_t b_lo = e_lo >> 1, b_hi = (e_hi + 1) >> 1;
        const float mold = active ? to_f32(mag[row]) : 0.0f;
        auto momentum = [&](int64_t e, uint32_t old) -> float {
            const float gf = to_f32(g[e]);
            const float cur = L.cbd[old] * mold;
            return __builtin_fmaf(T.b1c, gf - cur, cur);
        };
        float mx = 0.0f;
        if (active) {
            for (int64_t b = b_lo + t; b < b_hi; b += G) {
                const uint32_t ob = idx[b];
                const int64_t e0 = 2 * b;
                if (e0 >= e_lo) mx = nanmax(mx, fabsf(momentum(e0, ob & 15u)));
                if (e0 + 1 < e_hi) mx = nanmax(mx, fabsf(momentum(e0 + 1, ob >> 4)));
            }
        }
        mx = packed_row_max<G>(mx, red);
        if (!active) continue;
        const S mag_s = from_f32<S>(mx);
        const float mn = to_f32(mag_s);
        const float ss = T.mode == kVmeanGiven ? stepsize_of(to_f32(vm[row]), T) : T.stepsize[row];
        if (t == 0) mag[row] = mag_s;
        auto update = [&](int64_t e, uint32_t old) -> int {
            const float u = momentum(e, old);
            const float x = (mn > 0.0f) ? u / mn : 0.0f;
            const int k = nearest_fast<false>(x, L.thr, L.bucket, K);
            float q = L.cbd[k] * mn;
            if (QROUND) q = round_to<D>(q);
            const float uu = (q * ss) * T.lr;
            float pf = to_f32(p[e]);
            if (T.do_wd) pf = round_to<D>(pf * T.wdf);
            p[e] = from_f32<D>(pf - uu);
            return k;
        };
        for (int64_t b = b_lo + t; b < b_hi; b += G) {
            const uint32_t ob = idx[b];
            const int64_t e0 = 2 * b;
            const bool in0 = e0 >= e_lo, in1 = e0 + 1 < e_hi;
            const int k0 = in0 ? update(e0, ob & 15u) : 0;
            const int k1 = in1 ? update(e0 + 1, ob >> 4) : 0;
            store_nibbles(idx, b, ob, k0, k1, in0, in1);
        }
    }
}

// GefenMuon quantised momentum (as k_muon_long), packed indices.
template <typename D, typename S, int G>
__global__ __launch_bounds__(kThreads) void k_muon_packed(const MuonBatch B) {
    __shared__ LdsTables<false> L;
    __shared__ float red[4];
    int K;
    load_tables<D, kThreads>(L, B.tables, K);
    const MuonTask& T = B.t[0];
    constexpr int RPW = kThreads / G;
    const int sub = threadIdx.x / G, t = threadIdx.x % G;
    const D* __restrict__ g = static_cast<const D*>(T.g);
    uint8_t* idx = T.idx;
    S* __restrict__ mag = static_cast<S*>(T.mag);
    D* __restrict__ out = static_cast<D*>(T.out);
    for (int64_t r0 = (int64_t)blockIdx.x * RPW; r0 < T.nrows; r0 += (int64_t)gridDim.x * RPW) {
        const int64_t row = r0 + sub;
        const bool active = row < T.nrows;
        const int64_t e_lo = row * T.rowlen, e_hi = e_lo + T.rowlen;
        const int64_t b_lo = e_lo >> 1, b_hi = (e_hi + 1) >> 1;
        const float mold = active ? to_f32(mag[row]) : 0.0f;
        auto lerped = [&](int64_t e, uint32_t old) -> float {
            const float gf = to_f32(g[e]);
            const float m0 = round_to<D>(L.cbd[old] * mold);
            return round_to<D>(__builtin_fmaf(T.w, gf - m0, m0));
        };
        float mx = 0.0f;
        if (active) {
            for (int64_t b = b_lo + t; b < b_hi; b += G) {
                const uint32_t ob = idx[b];
                const int64_t e0 = 2 * b;
                if (e0 >= e_lo) mx = nanmax(mx, fabsf(lerped(e0, ob & 15u)));
                if (e0 + 1 < e_hi) mx = nanmax(mx, fabsf(lerped(e0 + 1, ob >> 4)));
            }
        }
        mx = packed_row_max<G>(mx, red);
        if (!active) continue;
        const S mag_s = from_f32<S>(mx);
        const float ms = to_f32(mag_s);
        const float clamped = (ms < T.tiny) ? T.tiny : ms;
        if (t == 0) mag[row] = mag_s;
        auto requant = [&](int64_t e, uint32_t old) -> int {
            float x = round_to<D>(lerped(e, old) / clamped);
            if (ms <= 0.0f) x = 0.0f;
            const int k = nearest_fast<false>(x, L.thr, L.bucket, K);
            const float q = round_to<D>(L.cbd[k] * ms);
            out[e] = from_f32<D>(muon_out<D, S>(q, to_f32(g[e]), T));
            return k;
        };
        for (int64_t b = b_lo + t; b < b_hi; b += G) {
            const uint32_t ob = idx[b];
            const int64_t e0 = 2 * b;
            const bool in0 = e0 >= e_lo, in1 = e0 + 1 < e_hi;
            const int k0 = in0 ? requant(e0, ob & 15u) : 0;
            const int k1 = in1 ? requant(e0 + 1, ob >> 4) : 0;
            store_nibbles(idx, b, ob, k0, k1, in0, in1);
        }
    }
}

// ---------------------------------------------------------------------------
// Launch templates (instantiated per dtype pair by GEFEN_STEP_INSTANCES)

// kernel key: dtype pair, W, R (0 = long rows), P1
struct Key {
    int d, s, W, R, p1, tab;
    bool operator==(const Key& o) const {
        return d == o.d && s == o.s && W == o.W && R == o.R && p1 == o.p1 && tab == o.tab;
    }
};

template <typename D, typename S>
hipError_t launch_step(const Key& k, const StepBatch& b, int grid, hipStream_t st) {
#define GEFEN_STEP_CASE(WW, RR)                                                                          \
    if (k.W == WW && k.R == RR) {                                                                       \
        if (k.p1) {                                                                                     \
            hipLaunchKernelGGL((k_gefen_step<D, S, WW, RR, true, false>), dim3(grid), dim3(kStepThreads), 0, st, b);           \
        } else {                                                                                        \
            if (k.tab) hipLaunchKernelGGL((k_gefen_step<D, S, WW, RR, false, true>), dim3(grid), dim3(kStepThreads), 0, st, b); \
            else hipLaunchKernelGGL((k_gefen_step<D, S, WW, RR, false, false>), dim3(grid), dim3(kStepThreads), 0, st, b);      \
        }                                                                                               \
        return hipGetLastError();                                                                       \
    }
    if (k.R == 0) {
        hipLaunchKernelGGL((k_gefen_step_long<D, S>), dim3(grid), dim3(kThreads), 0, st, b);
        return hipGetLastError();
    }
    if (sizeof(D) == 2) {
        GEFEN_STEP_CASE(8, 1) GEFEN_STEP_CASE(8, 2) GEFEN_STEP_CASE(8, 4) GEFEN_STEP_CASE(8, 8)
        GEFEN_STEP_CASE(4, 1) GEFEN_STEP_CASE(4, 2) GEFEN_STEP_CASE(4, 4) GEFEN_STEP_CASE(4, 8)
    } else {
        GEFEN_STEP_CASE(4, 1) GEFEN_STEP_CASE(4, 2) GEFEN_STEP_CASE(4, 4) GEFEN_STEP_CASE(4, 8)
    }
    GEFEN_STEP_CASE(1, 1) GEFEN_STEP_CASE(1, 2) GEFEN_STEP_CASE(1, 4) GEFEN_STEP_CASE(1, 8)
#undef GEFEN_STEP_CASE
    return hipErrorInvalidValue;
}

template <typename D, typename S>
hipError_t launch_muon(const Key& k, const MuonBatch& b, int grid, hipStream_t st) {
#define GEFEN_MUON_CASE(WW, RR)                                                                      \
    if (k.W == WW && k.R == RR) {                                                                   \
        if (k.tab) hipLaunchKernelGGL((k_muon<D, S, WW, RR, true>), dim3(grid), dim3(kThreads), 0, st, b);  \
        else hipLaunchKernelGGL((k_muon<D, S, WW, RR, false>), dim3(grid), dim3(kThreads), 0, st, b);       \
        return hipGetLastError();                                                                   \
    }
    if (k.R == 0) {
        hipLaunchKernelGGL((k_muon_long<D, S>), dim3(grid), dim3(kThreads), 0, st, b);
        return hipGetLastError();
    }
    if (sizeof(D) == 2) {
        GEFEN_MUON_CASE(8, 1) GEFEN_MUON_CASE(8, 2) GEFEN_MUON_CASE(8, 3) GEFEN_MUON_CASE(8, 4)
        GEFEN_MUON_CASE(8, 8)
        GEFEN_MUON_CASE(4, 1) GEFEN_MUON_CASE(4, 2) GEFEN_MUON_CASE(4, 4) GEFEN_MUON_CASE(4, 8)
    } else {
        GEFEN_MUON_CASE(4, 1) GEFEN_MUON_CASE(4, 2) GEFEN_MUON_CASE(4, 4) GEFEN_MUON_CASE(4, 8)
    }
    GEFEN_MUON_CASE(1, 1) GEFEN_MUON_CASE(1, 2) GEFEN_MUON_CASE(1, 4) GEFEN_MUON_CASE(1, 8)
#undef GEFEN_MUON_CASE
    return hipErrorInvalidValue;
}

// Packed-index kernels: lanes per row from the row's byte count, grid-stride over rows.
inline int packed_lanes(int64_t rowlen) {
    const int64_t bytes = rowlen / 2 + 1;
    return bytes <= 32 ? 16 : (bytes <= 512 ? 64 : 256);
}

inline int packed_grid(int64_t nrows, int lanes) {
    const int64_t rpw = kThreads / lanes;
    return (int)std::min<int64_t>((nrows + rpw - 1) / rpw, kPackedMaxGrid);
}

template <typename D, typename S, typename BatchT>
hipError_t launch_packed(const BatchT& b, int64_t rowlen, int64_t nrows, hipStream_t st) {
    const int G = packed_lanes(rowlen);
    const int grid = packed_grid(nrows, G);
#define GEFEN_PACKED_CASE(GG)                                                                                      \
    if (G == GG) {                                                                                                 \
        if constexpr (std::is_same<BatchT, MuonBatch>::value)                                                      \
            hipLaunchKernelGGL((k_muon_packed<D, S, GG>), dim3(grid), dim3(kThreads), 0, st, b);                    \
        else                                                                                                       \
            hipLaunchKernelGGL((k_gefen_step_packed<D, S, GG>), dim3(grid), dim3(kThreads), 0, st, b);              \
        return hipGetLastError();                                                                                  \
    }
    GEFEN_PACKED_CASE(16) GEFEN_PACKED_CASE(64) GEFEN_PACKED_CASE(256)
#undef GEFEN_PACKED_CASE
    return hipErrorInvalidValue;
}

// The launch templates of one (parameter, state) dtype pair: PREFIX is `template`
// for the explicit instantiation (step_inst_*.hip) or `extern template` for
// the declaration that keeps other files from instantiating them.
#define GEFEN_STEP_INSTANCES(PREFIX, D, S)                                                              \
    PREFIX hipError_t launch_step<D, S>(const Key&, const StepBatch&, int, hipStream_t);                 \
    PREFIX hipError_t launch_muon<D, S>(const Key&, const MuonBatch&, int, hipStream_t);                 \
    PREFIX hipError_t launch_packed<D, S, StepBatch>(const StepBatch&, int64_t, int64_t, hipStream_t);   \
    PREFIX hipError_t launch_packed<D, S, MuonBatch>(const MuonBatch&, int64_t, int64_t, hipStream_t);

}  // namespace gefen

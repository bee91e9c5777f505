// Host side of the fused Gefen / GefenMuon step for gfx950: task planning,
// batching of tasks into launches, the period-one stepsize tables, the C entry
// points, and the small table / fill / vmean kernels.  The step, GefenMuon
// momentum and packed-index kernels are in step_kernels.h (instantiated per
// dtype pair in step_inst_*.hip).
//
// The arithmetic is the reference's CPU path (gefen.py:116-119, 1153-1206,
// 1280-1281, 1326-1333; gefen_muon.py:132-171, 302-316), op by op.
#include <math.h>
#include <stddef.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <type_traits>
#include <vector>

#include "capi_internal.h"
#include "common.h"
#include "step_kernels.h"

// Scratch buffer of gefen_step_tasks_noalloc: the stepsize tables of one call,
// at most kNoAllocScratchFloats floats (1 MiB per device, held until the process
// ends).  Host code never passes `scratch` itself to a kernel or a copy: on the
// host the name is only a stand-in for the device variable.  Its device address
// comes from hipGetSymbolAddress, once per device with that device current
// (gefen::scratch_for_device), and only that address is used.
static constexpr size_t kNoAllocScratchFloats = size_t(1) << 18;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace gefen {

GEFEN_STEP_INSTANCES(extern template, float, float)
GEFEN_STEP_INSTANCES(extern template, bf16_t, bf16_t)
GEFEN_STEP_INSTANCES(extern template, f16_t, f16_t)
GEFEN_STEP_INSTANCES(extern template, bf16_t, float)
GEFEN_STEP_INSTANCES(extern template, f16_t, float)


// ---------------------------------------------------------------------------
// The bf16 square-root table of root_h: root[i] = fl(fl(sqrt(M * 2^par)) /
// sqrt_bc2) * 2^-67 with (par, M) = (i >> 7, 128 + (i & 127)) for i < 256 and
// (1, i - 256) for 256 <= i < 384.
__global__ __launch_bounds__(256) void k_build_root(float* __restrict__ root, StepTask T) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < kRootTab) {
        const int par = i < 256 ? (i >> 7) : 1;
        const int m = i < 256 ? 128 + (i & 127) : i - 256;
        root[i] = __builtin_ldexpf(sqrtf((float)m * (par ? 2.0f : 1.0f)) / T.sqrt_bc2, -67);
    }
}

// x[0, n) = 0 (the accumulator slots of gefen_muon_tasks_sumsq)
__global__ __launch_bounds__(256) void k_fill_f64(double* __restrict__ x, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = 0.0;
}

// Stepsize table of a period-one tensor with an f16 state: lut[b] is the
// stepsize (gefen.py:1326-1327) of the non-negative state value with bits b,
// computed by the same expression as the per-block path, so lookups are exact.
template <typename S>
__global__ __launch_bounds__(256) void k_build_lut(float* __restrict__ lut, StepTask T) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < 32768) {
        S v;
        const uint16_t bits = (uint16_t)i;
        __builtin_memcpy(&v, &bits, 2);
        lut[i] = stepsize_of(to_f32(v), T);
    }
}

// Stepsize of each block from a given vmean of another dtype than the
// magnitudes (gefen_automatic_fused_update_from_vmean): the expression the
// given-vmean kernels evaluate on to_f32(vmean), so the given-stepsize update
// that follows gives their results.
template <typename V>
__global__ __launch_bounds__(256) void k_block_stepsize(const V* __restrict__ vm, int64_t n, StepTask T,
                                                        float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = stepsize_of(to_f32(vm[i]), T);
}

// ---------------------------------------------------------------------------
// vmean only (automatic_vmean_update): one lane group per row, streaming.
template <typename G, typename S>
__global__ __launch_bounds__(kThreads) void k_vmean(S* __restrict__ vm, const G* __restrict__ g,
                                                     int64_t nrows, int64_t period, int lpr_log2,
                                                     float b2, float omb2) {
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int lir = lane & (lpr - 1);
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t row = unit * (64 >> lpr_log2) + (lane >> lpr_log2);
    const bool active = row < nrows;
    float s = 0.0f;
    if (active) {
        const int64_t base = row * period;
        for (int64_t j = lir; j < period; j += lpr) {
            const float gf = to_f32(g[base + j]);
            const float sq = gf * gf;
            s = s + sq;
        }
    }
    s = group_sum(s, lpr);
    if (active && lir == 0) {
        const float ms = s / (float)period;
        const float prev = to_f32(vm[row]) * b2;
        vm[row] = from_f32<S>(__builtin_fmaf(ms, omb2, prev));
    }
}

// ---------------------------------------------------------------------------
// host side
namespace {

int lpr_log2_for(int64_t nvec) {
    int l = 0;
    while ((1LL << l) < nvec && l < 6) ++l;
    return l;
}

int pick_width(int dsize, int64_t rowlen, std::initializer_list<const void*> ptrs, int idx_needed,
               const void* idx_ptr, int ssize, const void* vptr) {
    const int cands16[3] = {8, 4, 1};
    const int cands32[2] = {4, 1};
    const int* c = dsize == 2 ? cands16 : cands32;
    const int nc = dsize == 2 ? 3 : 2;
    for (int i = 0; i < nc; ++i) {
        const int W = c[i];
        if (rowlen % W) continue;
        bool ok = true;
        for (const void* q : ptrs) ok = ok && aligned(q, W * dsize);
        if (idx_needed) ok = ok && aligned(idx_ptr, W);
        if (vptr) ok = ok && aligned(vptr, W * ssize);
        if (ok) return W;
    }
    return 1;
}

int r_bucket(int64_t nvec, int lpr_log2) {
    const int64_t r = (nvec + (1LL << lpr_log2) - 1) >> lpr_log2;
    if (r <= 1) return 1;
    if (r <= 2) return 2;
    if (r <= 4) return 4;
    if (r <= 8) return 8;
    return 0;  // two-sweep path
}


hipError_t dispatch_step(const Key& k, const StepBatch& b, int grid, hipStream_t st) {
    if (k.d == GEFEN_F32) return launch_step<float, float>(k, b, grid, st);
    if (k.d == GEFEN_BF16 && k.s == GEFEN_BF16) return launch_step<bf16_t, bf16_t>(k, b, grid, st);
    if (k.d == GEFEN_F16 && k.s == GEFEN_F16) return launch_step<f16_t, f16_t>(k, b, grid, st);
    if (k.d == GEFEN_BF16 && k.s == GEFEN_F32) return launch_step<bf16_t, float>(k, b, grid, st);
    if (k.d == GEFEN_F16 && k.s == GEFEN_F32) return launch_step<f16_t, float>(k, b, grid, st);
    return hipErrorInvalidValue;
}


hipError_t dispatch_muon(const Key& k, const MuonBatch& b, int grid, hipStream_t st) {
    if (k.d == GEFEN_F32) return launch_muon<float, float>(k, b, grid, st);
    if (k.d == GEFEN_BF16 && k.s == GEFEN_BF16) return launch_muon<bf16_t, bf16_t>(k, b, grid, st);
    if (k.d == GEFEN_F16 && k.s == GEFEN_F16) return launch_muon<f16_t, f16_t>(k, b, grid, st);
    if (k.d == GEFEN_BF16 && k.s == GEFEN_F32) return launch_muon<bf16_t, float>(k, b, grid, st);
    if (k.d == GEFEN_F16 && k.s == GEFEN_F32) return launch_muon<f16_t, float>(k, b, grid, st);
    return hipErrorInvalidValue;
}


template <typename BatchT>
hipError_t dispatch_packed(int d, int s, const BatchT& b, int64_t rowlen, int64_t nrows, hipStream_t st) {
    if (d == GEFEN_F32) return launch_packed<float, float>(b, rowlen, nrows, st);
    if (d == GEFEN_BF16 && s == GEFEN_BF16) return launch_packed<bf16_t, bf16_t>(b, rowlen, nrows, st);
    if (d == GEFEN_F16 && s == GEFEN_F16) return launch_packed<f16_t, f16_t>(b, rowlen, nrows, st);
    if (d == GEFEN_BF16 && s == GEFEN_F32) return launch_packed<bf16_t, float>(b, rowlen, nrows, st);
    if (d == GEFEN_F16 && s == GEFEN_F32) return launch_packed<f16_t, float>(b, rowlen, nrows, st);
    return hipErrorInvalidValue;
}

bool valid_pair(int d, int s) { return valid_dtype(d) && valid_dtype(s) && (d == s || s == GEFEN_F32); }

// Workgroups of one launch: the dispatch's grid size in threads is 32-bit.
constexpr int64_t kMaxLaunchWgs = 0xFFFFFFFFLL / 256;
static_assert(kStepThreads <= 256 && kThreads <= 256, "launch cap assumes at most 256 threads per workgroup");

// Work of one task in workgroups for its kernel key; -1 when it exceeds one
// launch's grid (the caller rejects the tensor).
int32_t task_wgs(const Key& k, int64_t nrows, int lpr_log2, int waves, int iters) {
    int64_t wgs = nrows;
    if (k.R != 0) {
        const int64_t rpw = 64 >> lpr_log2;
        const int64_t units = (nrows + rpw - 1) / rpw;
        wgs = (units + waves * iters - 1) / (waves * iters);
    }
    return wgs <= kMaxLaunchWgs ? (int32_t)wgs : -1;
}

struct PendingStep {
    Key key;
    StepTask task;
};

// A second stream per device (default priority) for the small launches of a
// step, forked from and joined back to the caller's stream with events, so the
// launches of small tensors run beside the large ones instead of after them.
struct SideStream {
    std::mutex m;
    bool tried = false;
    hipStream_t s = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kMaxDevices = 64;
SideStream g_side[kMaxDevices];

// Launches of fewer elements than this go to the side stream.
constexpr int64_t kSmallLaunchElems = 1 << 20;

// The side stream of device dev (created on first use, with dev current), or
// nullptr when it could not be created.
SideStream* side_stream_of(int dev) {
    SideStream& ss = g_side[dev];
    std::lock_guard<std::mutex> lock(ss.m);
    if (!ss.tried) {
        ss.tried = true;
        if (hipStreamCreateWithFlags(&ss.s, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) != hipSuccess) {
            ss.s = nullptr;
            (void)hipGetLastError();
        }
    }
    return ss.s ? &ss : nullptr;
}

// The side stream of the current device, or nullptr (then everything runs on
// st): also when st belongs to another device than the current one.
SideStream* side_stream(hipStream_t st) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    if (st) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev) {
            (void)hipGetLastError();
            return nullptr;
        }
    }
    return side_stream_of(dev);
}

// One launch of the step kernels: a kernel key, its task table and grid.
struct StepLaunch {
    Key key;
    StepBatch b;
    int wg;
    int64_t elems;
};

// Group the pending tasks into launches: per kernel key, up to kMaxBatch tasks
// and one stepsize table per launch, in order of first appearance.  slot_of
// (optional) receives, for each pending task, launch index * kMaxBatch + its
// position in that launch's table.
void group_launches(const std::vector<PendingStep>& pend, const CodebookTables* tables,
                    std::vector<StepLaunch>& launches, std::vector<int>* slot_of = nullptr) {
    launches.clear();
    if (slot_of) slot_of->assign(pend.size(), -1);
    std::vector<bool> done(pend.size(), false);
    for (size_t i = 0; i < pend.size(); ++i) {
        if (done[i]) continue;
        StepLaunch L;
        memset(&L.b, 0, sizeof(L.b));
        L.key = pend[i].key;
        L.b.tables = tables;
        L.elems = 0;
        int n = 0;
        int64_t wg = 0;
        std::vector<size_t> members;
        for (size_t j = i; j < pend.size() && n < kMaxBatch; ++j) {
            if (done[j] || !(pend[j].key == pend[i].key)) continue;
            // one stepsize table per launch: workgroups load it before they find their task
            if (pend[j].task.lut != pend[i].task.lut) continue;
            if (wg + pend[j].task.nwg > kMaxLaunchWgs) break;
            L.b.t[n] = pend[j].task;
            L.b.wg_begin[n] = (int32_t)wg;
            wg += pend[j].task.nwg;
            L.elems += pend[j].task.nrows * pend[j].task.rowlen;
            members.push_back(j);
            ++n;
            done[j] = true;
        }
        L.b.wg_begin[n] = (int32_t)wg;
        L.b.ntasks = n;
        L.wg = (int)wg;
        if (wg > 0) {
            if (slot_of)
                for (int q = 0; q < n; ++q) (*slot_of)[members[q]] = (int)launches.size() * kMaxBatch + q;
            launches.push_back(L);
        }
    }
}

// Issue the launches on st; with allow_side, the launches of small tensors go
// to the device's side stream when the call also has large ones (side: that
// stream, or nullptr to look it up).  allow_side = false keeps every launch on
// st (no library-owned stream or event is created or used).
int issue_launches(const std::vector<StepLaunch>& launches, hipStream_t st, bool allow_side,
                   SideStream* side = nullptr) {
    bool any_small = false, any_large = false;
    for (const StepLaunch& L : launches) (L.elems < kSmallLaunchElems ? any_small : any_large) = true;
    if (!(allow_side && any_small && any_large)) side = nullptr;
    else if (!side) side = side_stream(st);
    std::unique_lock<std::mutex> lock;
    if (side) {
        lock = std::unique_lock<std::mutex>(side->m);
        if (hipEventRecord(side->fork, st) != hipSuccess || hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess)
            return launch_status("gefen step fork");
    }
    int rc = GEFEN_OK;
    for (const StepLaunch& L : launches) {
        hipStream_t ls = (side && L.elems < kSmallLaunchElems) ? side->s : st;
        hipError_t e = dispatch_step(L.key, L.b, L.wg, ls);
        if (e != hipSuccess) {
            rc = hip_status(e, "gefen step launch");
            break;
        }
    }
    // join even after a failed launch: st must stay ordered after the side-stream
    // launches already queued (they read the stepsize tables and write parameters)
    if (side) {
        const hipError_t e1 = hipEventRecord(side->join, side->s);
        const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(st, side->join, 0) : e1;
        if (e2 != hipSuccess && rc == GEFEN_OK) rc = hip_status(e2, "gefen step join");
    }
    return rc;
}

// Launch every pending task.
int flush_steps(std::vector<PendingStep>& pend, const CodebookTables* tables, hipStream_t st,
                bool allow_side = true) {
    std::vector<StepLaunch> launches;
    group_launches(pend, tables, launches);
    return issue_launches(launches, st, allow_side);
}

// The per-step scalars of a task as the kernels take them (float), from the
// caller's doubles: 1 - beta1, beta2, 1 - beta2, sqrt(bc2), eps, 1 / bc1, lr and
// the weight-decay factor 1 - lr * wd.
inline void set_step_scalars(const gefen_step_task& in, StepTask& t) {
    t.b1c = (float)(1.0 - in.beta1);
    t.b2 = (float)in.beta2;
    t.omb2 = (float)(1.0 - in.beta2);
    t.sqrt_bc2 = (float)sqrt(in.bias_correction_2);
    t.eps = (float)in.eps;
    t.inv_bc1 = (float)(1.0 / in.bias_correction_1);
    t.lr = (float)in.lr;
    t.do_wd = in.weight_decay > 0.0;
    t.wdf = (float)(1.0 - in.lr * in.weight_decay);
}

// Build the StepTask of one tensor.  mode / stepsize select the stepsize source.
int make_step_task(const gefen_step_task& in, int mode, const float* stepsize, PendingStep& out) {
    const int64_t n = in.numel;
    const int64_t P = in.period;
    if (P <= 0 || n % P) return fail_inval("period %lld does not divide numel %lld", (long long)P, (long long)n);
    // period-one mode (per-element vmean, magnitude per divisor block) is the fused
    // step of a P = 1 tensor; the stepsize / given-vmean entry points use rows of P
    const bool p1 = (P == 1 && mode == kVmeanUpdate);
    const int64_t rowlen = p1 ? in.period_one_divisor : P;
    if (rowlen <= 0 || n % rowlen) return fail_inval("magnitude block %lld does not divide numel %lld",
                                                     (long long)rowlen, (long long)n);
    if (p1 && rowlen > 256 * 64) return fail_inval("period_one_divisor %lld is too large", (long long)rowlen);
    if (P > INT32_MAX) return fail_inval("period %lld is too large", (long long)P);
    const int dsz = dtype_size(in.param_dtype), ssz = dtype_size(in.state_dtype);
    const int W = pick_width(dsz, rowlen, {in.p, in.grad}, 1, in.m_codebook, ssz, p1 ? in.vmean : nullptr);
    const int64_t nvec = rowlen / W;
    // period-one rows (at most 256 * 64 elements) take half the lanes with
    // twice the vectors per lane: more bytes in flight per lane
    int l2 = lpr_log2_for(nvec);
    if (p1 && l2 > 0) --l2;
    int R = r_bucket(nvec, l2);
    if (p1 && R == 0) return fail_inval("period_one_divisor %lld is too large", (long long)rowlen);
    // row tables pay off when a row has at least as many elements as codewords per lane group
    const int tab = (R != 0 && l2 >= 5 && !p1) ? 1 : 0;
    // the kernels keep one row table per wave when R >= 2 (whole-wave rows)
    if (tab && R >= 2 && l2 != 6) return fail_inval("internal: row tables of a %d-lane row", 1 << l2);
    Key k{in.param_dtype, in.state_dtype, R == 0 ? 1 : W, R, p1 ? 1 : 0, tab};
    StepTask& t = out.task;
    memset(&t, 0, sizeof(t));
    t.p = in.p;
    t.g = in.grad;
    t.idx = in.m_codebook;
    t.mag = in.m_magnitude;
    t.vmean = in.vmean;
    t.stepsize = stepsize;
    t.nrows = n / rowlen;
    t.rowlen = rowlen;
    t.period = (int32_t)(p1 ? 1 : P);
    t.nvec = (int32_t)std::min<int64_t>(nvec, INT32_MAX);
    t.lpr_log2 = l2;
    t.mode = mode;
    set_step_scalars(in, t);
    t.nwg = task_wgs(k, t.nrows, l2, kStepWaves, k.p1 ? kIterP1 : kIterRows);
    if (t.nwg < 0) return fail_inval("tensor of %lld elements is too large for one launch", (long long)n);
    out.key = k;
    return GEFEN_OK;
}

// Stepsize tables of the period-one tasks with a 16-bit state: one per distinct
// (state dtype, sqrt(bc2), eps, 1/bc1); the 384-entry square-root table for
// bf16 (k_build_root), the 32768-entry stepsize table for f16 (k_build_lut).
struct LutPlan {
    struct KeyT { int s; float a, b, c; };
    std::vector<KeyT> keys;
    std::vector<size_t> off;   // float offset of each key's table
    std::vector<int> which;    // key of each pending task, -1 if it takes no table
    size_t total = 0;          // floats of all tables
};

constexpr size_t kRootSlot = kRootTab;  // 1536 bytes: 256-byte aligned slots
constexpr size_t kLutSlot = 32768;
static_assert(kRootSlot % 64 == 0 && kLutSlot % 64 == 0, "table slots keep 256-byte alignment");

void plan_luts(const std::vector<PendingStep>& pend, LutPlan& lp) {
    lp.keys.clear();
    lp.off.clear();
    lp.total = 0;
    lp.which.assign(pend.size(), -1);
    for (size_t i = 0; i < pend.size(); ++i) {
        const Key& k = pend[i].key;
        if (!k.p1 || k.s == GEFEN_F32) continue;
        const StepTask& t = pend[i].task;
        // bf16 states outside the square-root table's bounds compute every stepsize
        if (k.s == GEFEN_BF16 && !root_table_ok(t.sqrt_bc2, t.eps)) continue;
        int found = -1;
        for (size_t j = 0; j < lp.keys.size(); ++j)
            if (lp.keys[j].s == k.s && memcmp(&lp.keys[j].a, &t.sqrt_bc2, 4) == 0 &&
                memcmp(&lp.keys[j].b, &t.eps, 4) == 0 && memcmp(&lp.keys[j].c, &t.inv_bc1, 4) == 0)
                found = (int)j;
        if (found < 0) {
            found = (int)lp.keys.size();
            lp.keys.push_back(LutPlan::KeyT{k.s, t.sqrt_bc2, t.eps, t.inv_bc1});
            lp.off.push_back(lp.total);
            lp.total += k.s == GEFEN_BF16 ? kRootSlot : kLutSlot;
        }
        lp.which[i] = found;
    }
}

// Build the planned tables at base (lp.total floats of device memory) on st and
// point the tasks at them.
int launch_luts(const LutPlan& lp, float* base, hipStream_t st) {
    for (size_t j = 0; j < lp.keys.size(); ++j) {
        StepTask t;
        memset(&t, 0, sizeof(t));
        t.sqrt_bc2 = lp.keys[j].a;
        t.eps = lp.keys[j].b;
        t.inv_bc1 = lp.keys[j].c;
        if (lp.keys[j].s == GEFEN_BF16)
            hipLaunchKernelGGL(k_build_root, dim3((kRootTab + 255) / 256), dim3(256), 0, st, base + lp.off[j], t);
        else
            hipLaunchKernelGGL(k_build_lut<f16_t>, dim3(128), dim3(256), 0, st, base + lp.off[j], t);
        int rc = launch_status("gefen stepsize table");
        if (rc) return rc;
    }
    return GEFEN_OK;
}

// Point the tasks at their tables in base.
void assign_luts(std::vector<PendingStep>& pend, const LutPlan& lp, float* base) {
    for (size_t i = 0; i < pend.size(); ++i)
        if (lp.which[i] >= 0) pend[i].task.lut = base + lp.off[(size_t)lp.which[i]];
}

int build_luts(std::vector<PendingStep>& pend, const LutPlan& lp, float* base, hipStream_t st) {
    int rc = launch_luts(lp, base, st);
    if (rc == GEFEN_OK) assign_luts(pend, lp, base);
    return rc;
}

// Device of a stream (the current device for the null stream).
int stream_device(hipStream_t st, int* dev) {
    if (hipGetDevice(dev) != hipSuccess) return launch_status("hipGetDevice");
    if (st) {
        hipDevice_t sd = -1;
        hipError_t e = hipStreamGetDevice(st, &sd);
        if (e != hipSuccess) return hip_status(e, "hipStreamGetDevice");
        *dev = sd;
    }
    if (*dev < 0 || *dev >= kMaxDevices) return fail_inval("device %d out of range", *dev);
    return GEFEN_OK;
}

// Makes `dev` current for its lifetime when it is not.
struct DeviceScope {
    int prev = -1;
    explicit DeviceScope(int dev) {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != dev && hipSetDevice(dev) == hipSuccess) prev = cur;
    }
    ~DeviceScope() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Orders the calls that share a device buffer (the stepsize tables): `done` is
// recorded on the stream of the last call after its launches, and a call on
// another stream waits for it before rewriting the buffer.  Not used while st
// is being captured into a graph (the graph's own edges order its nodes).
struct StreamOrder {
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool recorded = false;

    // Creates the event on first use (dev current); hipEventCreate allocates no device memory.
    int init(int dev) {
        if (done) return GEFEN_OK;
        DeviceScope scope(dev);
        hipError_t e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
        if (e != hipSuccess) {
            done = nullptr;
            return hip_status(e, "hipEventCreate(stepsize tables)");
        }
        return GEFEN_OK;
    }
    int wait(hipStream_t st) {
        if (!recorded || last == st) return GEFEN_OK;
        hipError_t e = hipStreamWaitEvent(st, done, 0);
        return e == hipSuccess ? GEFEN_OK : hip_status(e, "hipStreamWaitEvent(stepsize tables)");
    }
    // After the call's launches (and the join of the side stream): rc is the
    // call's status so far, returned unless the record itself fails.
    int record(hipStream_t st, int rc) {
        hipError_t e = hipEventRecord(done, st);
        if (e == hipSuccess) {
            recorded = true;
            last = st;
        } else if (rc == GEFEN_OK) {
            rc = hip_status(e, "hipEventRecord(stepsize tables)");
        }
        return rc;
    }
};

// True when st is capturing into a graph (then no event of a previous call may be waited on).
bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return cs != hipStreamCaptureStatusNone;
}

// Library-owned stepsize-table memory of a device, kept between calls and grown
// when a call needs more; calls on different streams are ordered by `order`.
struct LutPool {
    std::mutex m;
    float* buf = nullptr;
    size_t cap = 0;  // floats
    StreamOrder order;
};
LutPool g_lut_pool[kMaxDevices];

// Make the pool hold at least `floats` floats (pool.m held by the caller) and
// order st after the pool's last call on another stream.
int lut_pool_reserve(LutPool& pool, int dev, size_t floats, hipStream_t st) {
    int rc = pool.order.init(dev);
    if (rc) return rc;
    if (pool.cap < floats) {
        DeviceScope scope(dev);
        if (pool.buf) {
            if (pool.order.recorded) (void)hipEventSynchronize(pool.order.done);
            (void)hipFree(pool.buf);
            pool.buf = nullptr;
            pool.cap = 0;
        }
        const size_t want = std::max<size_t>(floats, 4 * kLutSlot);
        hipError_t e = device_malloc(reinterpret_cast<void**>(&pool.buf), want * sizeof(float));
        if (e != hipSuccess) {
            pool.buf = nullptr;
            return hip_status(e, "hipMalloc(stepsize tables)");
        }
        pool.cap = want;
    }
    return pool.order.wait(st);
}

// Stepsize tables in the device's pool, then the step launches.
int run_steps_pooled(std::vector<PendingStep>& pend, const CodebookTables* tables, hipStream_t st) {
    LutPlan lp;
    plan_luts(pend, lp);
    if (lp.keys.empty()) return flush_steps(pend, tables, st);
    int dev = 0;
    int rc = stream_device(st, &dev);
    if (rc) return rc;
    LutPool& pool = g_lut_pool[dev];
    std::lock_guard<std::mutex> lock(pool.m);
    rc = lut_pool_reserve(pool, dev, lp.total, st);
    if (rc) return rc;
    rc = build_luts(pend, lp, pool.buf, st);
    if (rc == GEFEN_OK) rc = flush_steps(pend, tables, st);
    // recorded after the join of the side stream: covers every launch that reads the tables
    return pool.order.record(st, rc);
}

// The scratch buffer of each device: its device address (from
// hipGetSymbolAddress, taken once with the device current) and the order of
// the no-allocation calls that write it.
struct ScratchSlot {
    std::mutex m;
    float* ptr = nullptr;
    StreamOrder order;
};
ScratchSlot g_scratch[kMaxDevices];

// Set-up of device dev's slot on its first use (slot.m held by the caller).
int scratch_init(ScratchSlot& slot, int dev) {
    if (!slot.ptr) {
        DeviceScope scope(dev);
        int cur = -1;
        if (hipGetDevice(&cur) != hipSuccess || cur != dev) return fail_inval("cannot make device %d current", dev);
        void* ptr = nullptr;
        hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(::scratch));
        if (e != hipSuccess || !ptr) return hip_status(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                       "hipGetSymbolAddress(scratch)");
        slot.ptr = static_cast<float*>(ptr);
    }
    return slot.order.init(dev);
}

int check_step_task(const gefen_step_task& t) {
    if (t.numel < 0) return fail_inval("numel must be non-negative");
    if (!valid_pair(t.param_dtype, t.state_dtype))
        return fail_inval("unsupported dtype pair (param %d, state %d)", t.param_dtype, t.state_dtype);
    if (t.numel == 0) return GEFEN_OK;
    if (!t.p || !t.grad || !t.m_codebook || !t.m_magnitude || !t.vmean)
        return fail_inval("null tensor pointer");
    if (!(t.bias_correction_1 > 0.0)) return fail_inval("Expected bias_correction_1 to be positive, got %g", t.bias_correction_1);
    if (!(t.bias_correction_2 > 0.0)) return fail_inval("Expected bias_correction_2 to be positive, got %g", t.bias_correction_2);
    if (t.eps < 0.0) return fail_inval("Expected eps to be non-negative, got %g", t.eps);
    return GEFEN_OK;
}

int check_codebook(const float* cb, int K) {
    if (!cb) return fail_inval("null codebook");
    if (K <= 0 || K > 256) return fail_inval("Expected codebook to have at most 256 entries, got %d", K);
    return GEFEN_OK;
}

// gefen_step_tasks: check and plan every row, then run them with the pooled
// stepsize tables.
int step_tasks_general(const gefen_step_task* tasks, int ntasks, const CodebookTables* tables, hipStream_t st) {
    std::vector<PendingStep> pend;
    pend.reserve(ntasks);
    for (int i = 0; i < ntasks; ++i) {
        int rc = check_step_task(tasks[i]);
        if (rc) return rc;
        if (tasks[i].numel == 0) continue;
        PendingStep ps;
        rc = make_step_task(tasks[i], kVmeanUpdate, nullptr, ps);
        if (rc) return rc;
        pend.push_back(ps);
    }
    return run_steps_pooled(pend, tables, st);
}

// Temporary codebook tables for the single-call entry points.
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

}  // namespace
}  // namespace gefen

using namespace gefen;

extern "C" int gefen_step_tasks(const gefen_step_task* tasks, int ntasks, const void* tables,
                                gefen_stream_t stream) {
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    if (!tables) return fail_inval("null codebook tables");
    return step_tasks_general(tasks, ntasks, static_cast<const CodebookTables*>(tables),
                              reinterpret_cast<hipStream_t>(stream));
}

extern "C" int gefen_step_tasks_noalloc(const gefen_step_task* tasks, int ntasks, const void* tables,
                                        gefen_stream_t stream) {
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    if (!tables) return fail_inval("null codebook tables");
    std::vector<PendingStep> pend;
    pend.reserve(ntasks);
    for (int i = 0; i < ntasks; ++i) {
        int rc = check_step_task(tasks[i]);
        if (rc) return rc;
        if (tasks[i].numel == 0) continue;
        PendingStep ps;
        rc = make_step_task(tasks[i], kVmeanUpdate, nullptr, ps);
        if (rc) return rc;
        pend.push_back(ps);
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    LutPlan lp;
    plan_luts(pend, lp);
    if (lp.total > kNoAllocScratchFloats)
        return fail_inval("the stepsize tables of this call need %zu bytes, more than the %zu-byte scratch buffer "
                          "(at most %zu f16-state or %zu bf16-state (sqrt(bc2), eps, 1/bc1) settings per call)",
                          lp.total * sizeof(float), kNoAllocScratchFloats * sizeof(float), kNoAllocScratchFloats / kLutSlot,
                          kNoAllocScratchFloats / kRootSlot);
    if (lp.keys.empty()) return flush_steps(pend, static_cast<const CodebookTables*>(tables), st, false);
    int dev = 0;
    int rc = stream_device(st, &dev);
    if (rc) return rc;
    ScratchSlot& slot = g_scratch[dev];
    std::lock_guard<std::mutex> lock(slot.m);
    rc = scratch_init(slot, dev);
    if (rc) return rc;
    // a call on another stream waits until the previous call's launches, which
    // read the tables, are done (not under graph capture: there the graph orders them)
    const bool cap = capturing(st);
    if (!cap) {
        rc = slot.order.wait(st);
        if (rc) return rc;
    }
    rc = build_luts(pend, lp, slot.ptr, st);
    if (rc == GEFEN_OK) rc = flush_steps(pend, static_cast<const CodebookTables*>(tables), st, false);
    return cap ? rc : slot.order.record(st, rc);
}

// ------------------------------------------------------------------------- step plan
// gefen_step_plan: the launches of one task table, kept between steps.  At
// creation the tasks are checked, their kernels chosen and grouped into
// launches exactly as gefen_step_tasks does; a run checks that each row still
// describes the same tensors (parameter and state pointers, sizes, period,
// dtypes, and a gradient aligned for the chosen kernel), writes the per-step
// values (gradient address and the scalars of set_step_scalars) into the kept
// launch tables, rebuilds the period-one stepsize tables and launches.  A run
// whose rows or stream do not fit the plan takes the gefen_step_tasks path.
struct gefen_step_plan {
    int dev = 0;
    const CodebookTables* tables = nullptr;
    int ntasks = 0;
    std::vector<gefen_step_task> shape;  // the creation rows
    std::vector<int> row;                // caller row of each pending task
    std::vector<int> galign;             // gradient alignment (bytes) each pending task's kernel needs
    std::vector<PendingStep> pend;
    std::vector<StepLaunch> launches;
    std::vector<int> slot;               // launch * kMaxBatch + position of each pending task
    LutPlan lp;                          // stepsize tables of the current run
    std::vector<int> launch_key;         // stepsize-table key of each launch in the current run
    SideStream* side = nullptr;
    bool timing = false, timed = false;
    hipEvent_t t0 = nullptr, t1 = nullptr;
};

namespace gefen {
namespace {

// The fields of a row that fix its kernel and launch slot.
bool same_tensors(const gefen_step_task& a, const gefen_step_task& b) {
    return a.p == b.p && a.m_codebook == b.m_codebook && a.m_magnitude == b.m_magnitude && a.vmean == b.vmean &&
           a.numel == b.numel && a.period == b.period &&
           (a.period != 1 || a.period_one_divisor == b.period_one_divisor) && a.param_dtype == b.param_dtype &&
           a.state_dtype == b.state_dtype;
}

// The plan's fast path: a GEFEN_* status, or -1 when the rows do not fit the
// plan (then nothing was launched).
// The hyperparameters and bias corrections of a task row, as compared between rows.
bool same_scalars(const gefen_step_task& a, const gefen_step_task& b) {
    return a.beta1 == b.beta1 && a.beta2 == b.beta2 && a.lr == b.lr && a.eps == b.eps &&
           a.weight_decay == b.weight_decay && a.bias_correction_1 == b.bias_correction_1 &&
           a.bias_correction_2 == b.bias_correction_2;
}

int plan_run_fast(gefen_step_plan& P, const gefen_step_task* tasks, hipStream_t st) {
    // rows of one group share their scalars: the float forms are computed once per run of equal rows
    const gefen_step_task* prev = nullptr;
    const StepTask* prev_t = nullptr;
    for (size_t i = 0; i < P.pend.size(); ++i) {
        const gefen_step_task& in = tasks[P.row[i]];
        if (!same_tensors(in, P.shape[P.row[i]]) || !in.grad || !aligned(in.grad, P.galign[i])) return -1;
        int rc = check_step_task(in);
        if (rc) return rc;
        StepTask& t = P.pend[i].task;
        t.g = in.grad;
        if (prev && same_scalars(in, *prev)) {
            t.b1c = prev_t->b1c; t.b2 = prev_t->b2; t.omb2 = prev_t->omb2; t.sqrt_bc2 = prev_t->sqrt_bc2;
            t.eps = prev_t->eps; t.inv_bc1 = prev_t->inv_bc1; t.lr = prev_t->lr; t.do_wd = prev_t->do_wd;
            t.wdf = prev_t->wdf;
        } else {
            set_step_scalars(in, t);
        }
        t.lut = nullptr;
        prev = &in;
        prev_t = &t;
    }
    // every row that must be stepped as a no-op (numel 0) is still empty
    for (int r = 0; r < P.ntasks; ++r)
        if (tasks[r].numel != P.shape[r].numel) return -1;
    plan_luts(P.pend, P.lp);
    // one stepsize table per launch, as the grouping assumed
    P.launch_key.assign(P.launches.size(), -2);
    for (size_t i = 0; i < P.pend.size(); ++i) {
        int& k = P.launch_key[(size_t)(P.slot[i] / kMaxBatch)];
        if (k == -2) k = P.lp.which[i];
        else if (k != P.lp.which[i]) return -1;
    }
    // stepsize tables: reserve the pool (ordered after its last use on another
    // stream) and point the tasks at their tables before the launch tables are filled
    int rc = GEFEN_OK;
    LutPool* pool = nullptr;
    std::unique_lock<std::mutex> pool_lock;
    if (!P.lp.keys.empty()) {
        pool = &g_lut_pool[P.dev];
        pool_lock = std::unique_lock<std::mutex>(pool->m);
        rc = lut_pool_reserve(*pool, P.dev, P.lp.total, st);
        if (rc) return rc;
        assign_luts(P.pend, P.lp, pool->buf);
    }
    for (size_t i = 0; i < P.pend.size(); ++i) {
        const int q = P.slot[i];
        P.launches[(size_t)(q / kMaxBatch)].b.t[q % kMaxBatch] = P.pend[i].task;
    }
    // Issue order, so that the first large launch goes out as early as possible:
    // the side stream's fork event (recorded before any launch, so the side
    // stream waits only for the work before this step), the large launches on st
    // with the stepsize tables built right before the first launch that reads
    // them, then the side stream's wait and the small launches (tables built
    // before the fork when a small launch reads them), and the join.
    bool any_small = false, any_large = false, small_lut = false;
    for (size_t l = 0; l < P.launches.size(); ++l) {
        const bool small = P.launches[l].elems < kSmallLaunchElems;
        (small ? any_small : any_large) = true;
        small_lut = small_lut || (small && P.launches[l].b.t[0].lut);
    }
    SideStream* side = (any_small && any_large) ? P.side : nullptr;
    const bool timing = P.timing;
    if (timing && hipEventRecord(P.t0, st) != hipSuccess) rc = launch_status("hipEventRecord(step plan)");
    bool luts_built = pool == nullptr;
    if (rc == GEFEN_OK && !luts_built && side && small_lut) {
        rc = launch_luts(P.lp, pool->buf, st);
        luts_built = true;
    }
    std::unique_lock<std::mutex> side_lock;
    if (rc == GEFEN_OK && side) {
        side_lock = std::unique_lock<std::mutex>(side->m);
        if (hipEventRecord(side->fork, st) != hipSuccess) rc = launch_status("gefen step fork");
    }
    for (size_t l = 0; rc == GEFEN_OK && l < P.launches.size(); ++l) {
        const StepLaunch& L = P.launches[l];
        if (side && L.elems < kSmallLaunchElems) continue;
        if (!luts_built && L.b.t[0].lut) {
            rc = launch_luts(P.lp, pool->buf, st);
            luts_built = true;
            if (rc) break;
        }
        hipError_t e = dispatch_step(L.key, L.b, L.wg, st);
        if (e != hipSuccess) rc = hip_status(e, "gefen step launch");
    }
    if (side) {
        bool waited = false;
        if (rc == GEFEN_OK) {
            if (hipStreamWaitEvent(side->s, side->fork, 0) != hipSuccess) rc = launch_status("gefen step fork");
            else waited = true;
        }
        for (size_t l = 0; rc == GEFEN_OK && l < P.launches.size(); ++l) {
            const StepLaunch& L = P.launches[l];
            if (L.elems >= kSmallLaunchElems) continue;
            hipError_t e = dispatch_step(L.key, L.b, L.wg, side->s);
            if (e != hipSuccess) rc = hip_status(e, "gefen step launch");
        }
        // join even after a failed launch: st stays ordered after what the side stream queued
        if (waited) {
            const hipError_t e1 = hipEventRecord(side->join, side->s);
            const hipError_t e2 = e1 == hipSuccess ? hipStreamWaitEvent(st, side->join, 0) : e1;
            if (e2 != hipSuccess && rc == GEFEN_OK) rc = hip_status(e2, "gefen step join");
        }
    }
    // recorded after the join: covers every launch that reads the stepsize tables
    if (pool) rc = pool->order.record(st, rc);
    if (timing) {
        hipError_t e = hipEventRecord(P.t1, st);
        if (e != hipSuccess && rc == GEFEN_OK) rc = hip_status(e, "hipEventRecord(step plan)");
        P.timed = e == hipSuccess;
    }
    return rc;
}

}  // namespace
}  // namespace gefen

extern "C" int gefen_step_plan_create(const gefen_step_task* tasks, int ntasks, const void* tables,
                                      gefen_step_plan** out) {
    if (!out) return fail_inval("null plan pointer");
    *out = nullptr;
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    if (!tables) return fail_inval("null codebook tables");
    int dev = 0;
    int rc = stream_device(nullptr, &dev);
    if (rc) return rc;
    gefen_step_plan* P = new (std::nothrow) gefen_step_plan();
    if (!P) return fail_inval("out of host memory");
    P->dev = dev;
    P->tables = static_cast<const CodebookTables*>(tables);
    P->ntasks = ntasks;
    P->shape.assign(tasks, tasks + ntasks);
    for (int i = 0; i < ntasks; ++i) {
        rc = check_step_task(tasks[i]);
        if (rc == GEFEN_OK && tasks[i].numel > 0) {
            PendingStep ps;
            rc = make_step_task(tasks[i], kVmeanUpdate, nullptr, ps);
            if (rc == GEFEN_OK) {
                P->pend.push_back(ps);
                P->row.push_back(i);
                P->galign.push_back((ps.key.R == 0 ? 1 : ps.key.W) * dtype_size(ps.key.d));
            }
        }
        if (rc) {
            delete P;
            return rc;
        }
    }
    // group as gefen_step_tasks would, with the creation rows' stepsize-table keys
    plan_luts(P->pend, P->lp);
    for (size_t i = 0; i < P->pend.size(); ++i)
        P->pend[i].task.lut = P->lp.which[i] >= 0 ? reinterpret_cast<const float*>((uintptr_t)(P->lp.which[i] + 1) * 256)
                                                  : nullptr;
    group_launches(P->pend, P->tables, P->launches, &P->slot);
    for (PendingStep& ps : P->pend) ps.task.lut = nullptr;
    P->side = side_stream_of(dev);
    *out = P;
    return GEFEN_OK;
}

extern "C" int gefen_step_plan_run(gefen_step_plan* plan, const gefen_step_task* tasks, int ntasks,
                                   gefen_stream_t stream) {
    if (!plan) return fail_inval("null step plan");
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    int dev = -1;
    int rc = stream_device(st, &dev);
    if (rc) return rc;
    if (ntasks == plan->ntasks && dev == plan->dev) {
        DeviceScope scope(dev);
        rc = plan_run_fast(*plan, tasks, st);
        if (rc != -1) return rc;
    }
    DeviceScope scope(dev);
    const bool timing = plan->timing && dev == plan->dev;
    if (timing && hipEventRecord(plan->t0, st) != hipSuccess) return launch_status("hipEventRecord(step plan)");
    rc = step_tasks_general(tasks, ntasks, plan->tables, st);
    if (timing) {
        hipError_t e = hipEventRecord(plan->t1, st);
        if (e != hipSuccess && rc == GEFEN_OK) rc = hip_status(e, "hipEventRecord(step plan)");
        plan->timed = e == hipSuccess;
    }
    return rc;
}

extern "C" int gefen_step_plan_time_runs(gefen_step_plan* plan, int enable) {
    if (!plan) return fail_inval("null step plan");
    if (enable && !plan->t0) {
        DeviceScope scope(plan->dev);
        hipError_t e = hipEventCreate(&plan->t0);
        if (e == hipSuccess) e = hipEventCreate(&plan->t1);
        if (e != hipSuccess) return hip_status(e, "hipEventCreate(step plan)");
    }
    plan->timing = enable != 0;
    plan->timed = false;
    return GEFEN_OK;
}

extern "C" int gefen_step_plan_last_ms(gefen_step_plan* plan, float* ms) {
    if (!plan || !ms) return fail_inval("null step plan or result pointer");
    if (!plan->timed) return fail_inval("no timed run: enable gefen_step_plan_time_runs before a run");
    hipError_t e = hipEventSynchronize(plan->t1);
    if (e == hipSuccess) e = hipEventElapsedTime(ms, plan->t0, plan->t1);
    return hip_status(e, "hipEventElapsedTime(step plan)");
}

extern "C" void gefen_step_plan_destroy(gefen_step_plan* plan) {
    if (!plan) return;
    if (plan->t0 || plan->t1) {
        DeviceScope scope(plan->dev);
        if (plan->t1) (void)hipEventSynchronize(plan->t1);
        if (plan->t0) (void)hipEventDestroy(plan->t0);
        if (plan->t1) (void)hipEventDestroy(plan->t1);
    }
    delete plan;
}

static int single_update(void* p, const void* grad, int param_dtype, uint8_t* m_sign, void* mag,
                         int mag_dtype, void* vmean, int vmean_dtype, const float* stepsize,
                         const float* codebook, int K, int packed, int64_t num_blocks, int64_t period,
                         int64_t pod, int mode, double beta1, double beta2, double lr, double bc1,
                         double bc2, double eps, gefen_stream_t stream) {
    int rc = check_codebook(codebook, K);
    if (rc) return rc;
    if (!valid_dtype(param_dtype)) return fail_inval("unsupported parameter dtype %d", param_dtype);
    if (!valid_pair(param_dtype, mag_dtype))
        return fail_inval("Expected m_magnitude to be float32, float16, or bfloat16 matching the parameters");
    if (mode != kStepsizeGiven && !valid_dtype(vmean_dtype))
        return fail_inval("Expected vmean to be float32, float16, or bfloat16, got %d", vmean_dtype);
    if (mode == kVmeanUpdate && vmean_dtype != mag_dtype)
        return fail_inval("the period-one update keeps vmean in the magnitude dtype: vmean dtype %d, "
                          "m_magnitude dtype %d", vmean_dtype, mag_dtype);
    if (num_blocks < 0 || period <= 0) return fail_inval("Expected a positive period, got %lld", (long long)period);
    if (mode == kVmeanGiven && vmean_dtype != mag_dtype && num_blocks > 0) {
        // a vmean of another dtype: each block's stepsize formed on the device, then
        // the given-stepsize update (the stepsize is all the kernels take from vmean)
        if (bc1 <= 0.0 || bc2 <= 0.0 || !(eps >= 0.0)) return fail_inval("invalid bias corrections or eps");
        if (!vmean) return fail_inval("null vmean");
        gefen_step_task in;
        memset(&in, 0, sizeof(in));
        in.beta1 = beta1;
        in.lr = lr;
        in.eps = eps;
        in.bias_correction_1 = bc1;
        in.bias_correction_2 = bc2;
        StepTask ts;
        memset(&ts, 0, sizeof(ts));
        set_step_scalars(in, ts);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        void* tmp = nullptr;
        hipError_t e = device_malloc_async(&tmp, (size_t)num_blocks * sizeof(float), st);
        if (e != hipSuccess) return hip_status(e, "hipMallocAsync(block stepsizes)");
        const unsigned grid = (unsigned)std::min<int64_t>((num_blocks + 255) / 256, 4096);
        float* ss = static_cast<float*>(tmp);
        if (vmean_dtype == GEFEN_F32)
            hipLaunchKernelGGL(k_block_stepsize<float>, dim3(grid), dim3(256), 0, st, static_cast<const float*>(vmean),
                               num_blocks, ts, ss);
        else if (vmean_dtype == GEFEN_BF16)
            hipLaunchKernelGGL(k_block_stepsize<bf16_t>, dim3(grid), dim3(256), 0, st,
                               static_cast<const bf16_t*>(vmean), num_blocks, ts, ss);
        else
            hipLaunchKernelGGL(k_block_stepsize<f16_t>, dim3(grid), dim3(256), 0, st,
                               static_cast<const f16_t*>(vmean), num_blocks, ts, ss);
        rc = launch_status("gefen block stepsize");
        if (rc == GEFEN_OK)
            rc = single_update(p, grad, param_dtype, m_sign, mag, mag_dtype, nullptr, mag_dtype, ss, codebook, K,
                               packed, num_blocks, period, 0, kStepsizeGiven, beta1, 0.0, lr, 1.0, 1.0, 0.0, stream);
        (void)hipFreeAsync(tmp, st);
        return rc;
    }
    gefen_step_task t;
    memset(&t, 0, sizeof(t));
    t.p = p;
    t.grad = grad;
    t.m_codebook = m_sign;
    t.m_magnitude = mag;
    t.vmean = mode == kStepsizeGiven ? (void*)stepsize : vmean;
    t.numel = num_blocks * period;
    t.period = period;
    t.period_one_divisor = pod;
    t.param_dtype = param_dtype;
    t.state_dtype = mag_dtype;
    t.beta1 = beta1;
    t.beta2 = beta2;
    t.lr = lr;
    t.eps = eps;
    t.weight_decay = 0.0;
    t.bias_correction_1 = bc1;
    t.bias_correction_2 = bc2;
    rc = check_step_task(t);
    if (rc) return rc;
    if (t.numel == 0) return GEFEN_OK;
    PendingStep ps;
    rc = make_step_task(t, mode, stepsize, ps);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    TempTables tt;
    rc = tt.init(codebook, K, st);
    if (rc) return rc;
    if (packed) {
        StepBatch b;
        memset(&b, 0, sizeof(b));
        b.t[0] = ps.task;
        b.ntasks = 1;
        b.tables = static_cast<const CodebookTables*>(tt.ptr);
        hipError_t e = dispatch_packed(param_dtype, mag_dtype, b, ps.task.rowlen, ps.task.nrows, st);
        return e == hipSuccess ? GEFEN_OK : hip_status(e, "gefen packed step launch");
    }
    std::vector<PendingStep> pend(1, ps);
    return run_steps_pooled(pend, static_cast<const CodebookTables*>(tt.ptr), st);
}

extern "C" int gefen_automatic_fused_update(void* p, const void* grad, int param_dtype, uint8_t* m_sign,
                                            void* m_magnitude, int magnitude_dtype, const float* stepsize,
                                            const float* codebook, int codebook_size, int packed_indices,
                                            int64_t num_blocks, int64_t period, double beta1, double lr,
                                            gefen_stream_t stream) {
    if (!stepsize && num_blocks > 0) return fail_inval("null stepsize");
    return single_update(p, grad, param_dtype, m_sign, m_magnitude, magnitude_dtype, nullptr,
                         magnitude_dtype, stepsize, codebook, codebook_size, packed_indices,
                         num_blocks, period, 0, kStepsizeGiven, beta1, 0.0, lr, 1.0, 1.0, 0.0, stream);
}

extern "C" int gefen_automatic_fused_update_from_vmean(
    void* p, const void* grad, int param_dtype, uint8_t* m_sign, void* m_magnitude, int magnitude_dtype,
    const void* vmean, int vmean_dtype, const float* codebook, int codebook_size, int packed_indices,
    int64_t num_blocks, int64_t period, double beta1, double lr, double bias_correction_1,
    double bias_correction_2, double eps, gefen_stream_t stream) {
    return single_update(p, grad, param_dtype, m_sign, m_magnitude, magnitude_dtype,
                         const_cast<void*>(vmean), vmean_dtype, nullptr, codebook, codebook_size,
                         packed_indices, num_blocks, period, 0, kVmeanGiven, beta1, 0.0, lr,
                         bias_correction_1, bias_correction_2, eps, stream);
}

extern "C" int gefen_automatic_period1_update(void* p, const void* grad, int param_dtype, uint8_t* m_sign,
                                              void* m_magnitude, int magnitude_dtype, void* vmean,
                                              int vmean_dtype, const float* codebook, int codebook_size,
                                              int64_t numel, int64_t period_one_divisor, double beta1,
                                              double beta2, double lr, double bias_correction_1,
                                              double bias_correction_2, double eps, gefen_stream_t stream) {
    if (period_one_divisor <= 0) return fail_inval("Expected period_one_divisor to be positive, got %lld",
                                                   (long long)period_one_divisor);
    if (!(beta2 >= 0.0 && beta2 <= 1.0)) return fail_inval("Expected beta2 to be in [0, 1], got %g", beta2);
    return single_update(p, grad, param_dtype, m_sign, m_magnitude, magnitude_dtype, vmean, vmean_dtype,
                         nullptr, codebook, codebook_size, 0, numel, 1, period_one_divisor, kVmeanUpdate,
                         beta1, beta2, lr, bias_correction_1, bias_correction_2, eps, stream);
}

// ------------------------------------------------------------------------- muon
namespace gefen {
namespace {
struct PendingMuon {
    Key key;
    MuonTask task;
};

int make_muon_task(const gefen_muon_task& in, PendingMuon& out) {
    const int64_t n = in.numel, rowlen = in.block;
    if (rowlen <= 0 || n % rowlen) return fail_inval("block %lld does not divide numel %lld",
                                                     (long long)rowlen, (long long)n);
    if (!valid_pair(in.grad_dtype, in.state_dtype))
        return fail_inval("unsupported dtype pair (grad %d, state %d)", in.grad_dtype, in.state_dtype);
    if (!(in.momentum >= 0.0 && in.momentum < 1.0))
        return fail_inval("Expected beta1 to be in [0, 1), got %g", in.momentum);
    if (n > 0 && (!in.grad || !in.m_codebook || !in.m_magnitude || !in.out)) return fail_inval("null tensor pointer");
    const int dsz = dtype_size(in.grad_dtype);
    const int W = pick_width(dsz, rowlen, {in.grad, in.out}, 1, in.m_codebook, 0, nullptr);
    const int64_t nvec = rowlen / W;
    // rows of at most 32 vectors take half the lanes with twice the vectors per
    // lane (measured 6% faster on the Qwen3-1.7B momentum, mostly period-one rows)
    int l2 = lpr_log2_for(nvec);
    if (l2 > 0 && l2 <= 5) --l2;
    int R = r_bucket(nvec, l2);
    // rows of exactly three vectors per lane (1536 bf16 elements on a whole wave)
    // get their own instance instead of the four-vector one with a clamped fourth
    if (R == 4 && W == 8 && ((nvec + (1LL << l2) - 1) >> l2) == 3) R = 3;
    // row tables pay off for whole-wave rows (measured: 5% faster there, none for 32-lane rows)
    const int tab = (R != 0 && l2 >= GEFEN_MUON_TAB_LOG2) ? 1 : 0;
    // k_muon keeps one row table per wave: whole-wave rows only
    static_assert(GEFEN_MUON_TAB_LOG2 >= 6, "GefenMuon row tables need whole-wave rows");
    Key k{in.grad_dtype, in.state_dtype, R == 0 ? 1 : W, R, 0, tab};
    MuonTask& t = out.task;
    memset(&t, 0, sizeof(t));
    t.g = in.grad;
    t.idx = in.m_codebook;
    t.mag = in.m_magnitude;
    t.out = in.out;
    t.nrows = n / rowlen;
    t.rowlen = rowlen;
    t.nvec = (int32_t)std::min<int64_t>(nvec, INT32_MAX);
    t.lpr_log2 = l2;
    t.w = (float)(1.0 - in.momentum);
    t.mom = (float)in.momentum;
    float alpha = (float)(1.0 - in.momentum);
    float tiny = in.grad_dtype == GEFEN_F16 ? 6.103515625e-05f : 1.17549435e-38f;
    // reduced-dtype add_(alpha=) rounds alpha to the tensor dtype; tiny lives in the state dtype
    auto round_host = [](float v, int dt) -> float {
        if (dt == GEFEN_F32) return v;
        if (dt == GEFEN_BF16) {
            uint32_t u;
            memcpy(&u, &v, 4);
            u += 0x7fffu + ((u >> 16) & 1u);
            u &= 0xffff0000u;
            float r;
            memcpy(&r, &u, 4);
            return r;
        }
        _Float16 h = (_Float16)v;
        return (float)h;
    };
    t.alpha = round_host(alpha, in.grad_dtype);
    t.tiny = round_host(tiny, in.state_dtype);
    t.nesterov = in.nesterov ? 1 : 0;
    t.nwg = task_wgs(k, t.nrows, l2, 4, kMuonIter);
    if (t.nwg < 0) return fail_inval("tensor of %lld elements is too large for one launch", (long long)n);
    out.key = k;
    return GEFEN_OK;
}

int flush_muon(std::vector<PendingMuon>& pend, const CodebookTables* tables, hipStream_t st) {
    std::vector<bool> done(pend.size(), false);
    for (size_t i = 0; i < pend.size(); ++i) {
        if (done[i]) continue;
        MuonBatch b;
        memset(&b, 0, sizeof(b));
        b.tables = tables;
        int n = 0;
        int64_t wg = 0;
        for (size_t j = i; j < pend.size() && n < kMaxBatch; ++j) {
            if (done[j] || !(pend[j].key == pend[i].key)) continue;
            if (wg + pend[j].task.nwg > kMaxLaunchWgs) break;
            b.t[n] = pend[j].task;
            b.wg_begin[n] = (int32_t)wg;
            wg += pend[j].task.nwg;
            ++n;
            done[j] = true;
        }
        b.wg_begin[n] = (int32_t)wg;
        b.ntasks = n;
        if (wg == 0) continue;
        hipError_t e = dispatch_muon(pend[i].key, b, (int)wg, st);
        if (e != hipSuccess) return hip_status(e, "gefen muon launch");
    }
    return GEFEN_OK;
}
}  // namespace
}  // namespace gefen

static int muon_tasks_common(const gefen_muon_task* tasks, int ntasks, const void* tables, double* sumsq,
                             gefen_stream_t stream) {
    if (ntasks < 0 || (ntasks > 0 && !tasks)) return fail_inval("invalid task array");
    if (!tables) return fail_inval("null codebook tables");
    std::vector<PendingMuon> pend;
    for (int i = 0; i < ntasks; ++i) {
        if (tasks[i].numel == 0) continue;
        PendingMuon pm;
        int rc = make_muon_task(tasks[i], pm);
        if (rc) return rc;
        pm.task.sumsq = sumsq ? sumsq + (size_t)i * GEFEN_SUMSQ_STRIDE : nullptr;
        pend.push_back(pm);
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (sumsq && ntasks > 0) {  // a fill kernel, not a memset node (callers may capture this)
        const int n = ntasks * GEFEN_SUMSQ_STRIDE;
        hipLaunchKernelGGL(k_fill_f64, dim3((n + 255) / 256), dim3(256), 0, st, sumsq, n);
        int rc = launch_status("gefen muon sumsq init");
        if (rc) return rc;
    }
    return flush_muon(pend, static_cast<const CodebookTables*>(tables), st);
}

extern "C" int gefen_muon_tasks(const gefen_muon_task* tasks, int ntasks, const void* tables,
                                gefen_stream_t stream) {
    return muon_tasks_common(tasks, ntasks, tables, nullptr, stream);
}

extern "C" int gefen_muon_tasks_sumsq(const gefen_muon_task* tasks, int ntasks, const void* tables, double* sumsq,
                                      gefen_stream_t stream) {
    if (!sumsq && ntasks > 0) return fail_inval("null sumsq");
    return muon_tasks_common(tasks, ntasks, tables, sumsq, stream);
}

extern "C" int gefen_automatic_muon_momentum(const void* grad, int grad_dtype, uint8_t* m_sign,
                                             void* m_magnitude, int magnitude_dtype, const float* codebook,
                                             int codebook_size, void* momentum_update, int packed_indices,
                                             int64_t num_blocks, int64_t period, double beta1,
                                             gefen_stream_t stream) {
    int rc = check_codebook(codebook, codebook_size);
    if (rc) return rc;
    if (num_blocks < 0 || period <= 0) return fail_inval("Expected a positive period, got %lld", (long long)period);
    gefen_muon_task t;
    memset(&t, 0, sizeof(t));
    t.grad = grad;
    t.m_codebook = m_sign;
    t.m_magnitude = m_magnitude;
    t.out = momentum_update;
    t.numel = num_blocks * period;
    t.block = period;
    t.grad_dtype = grad_dtype;
    t.state_dtype = magnitude_dtype;
    t.momentum = beta1;
    t.nesterov = 0;
    if (t.numel == 0) return GEFEN_OK;
    PendingMuon pm;
    rc = make_muon_task(t, pm);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    TempTables tt;
    rc = tt.init(codebook, codebook_size, st);
    if (rc) return rc;
    if (packed_indices) {
        MuonBatch b;
        memset(&b, 0, sizeof(b));
        b.t[0] = pm.task;
        b.ntasks = 1;
        b.tables = static_cast<const CodebookTables*>(tt.ptr);
        hipError_t e = dispatch_packed(grad_dtype, magnitude_dtype, b, pm.task.rowlen, pm.task.nrows, st);
        return e == hipSuccess ? GEFEN_OK : hip_status(e, "gefen packed muon launch");
    }
    std::vector<PendingMuon> pend(1, pm);
    return flush_muon(pend, static_cast<const CodebookTables*>(tt.ptr), st);
}

extern "C" int gefen_automatic_vmean_update(void* vmean, int vmean_dtype, const void* grad, int grad_dtype,
                                            int64_t num_blocks, int64_t period, double beta2,
                                            gefen_stream_t stream) {
    if (!valid_dtype(vmean_dtype))
        return fail_inval("Expected vmean to be float32, float16, or bfloat16, got %d", vmean_dtype);
    if (!valid_dtype(grad_dtype)) return fail_inval("unsupported grad dtype %d", grad_dtype);
    if (!(beta2 >= 0.0 && beta2 <= 1.0)) return fail_inval("Expected beta2 to be in [0, 1], got %g", beta2);
    if (num_blocks < 0 || period <= 0) return fail_inval("Expected a positive period, got %lld", (long long)period);
    if (num_blocks == 0) return GEFEN_OK;
    if (!vmean || !grad) return fail_inval("null tensor pointer");
    const int l2 = lpr_log2_for(period);
    const int64_t rpw = 64 >> l2;
    const int64_t units = (num_blocks + rpw - 1) / rpw;
    const int64_t grid = (units + 3) / 4;
    if (grid > INT32_MAX) return fail_inval("tensor too large");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const float b2 = (float)beta2, omb2 = (float)(1.0 - beta2);
#define GEFEN_VMEAN(G, S)                                                                               \
    hipLaunchKernelGGL((k_vmean<G, S>), dim3((unsigned)grid), dim3(kThreads), 0, st, static_cast<S*>(vmean), \
                       static_cast<const G*>(grad), num_blocks, period, l2, b2, omb2)
    auto launch_s = [&](auto gtag) {
        using G = decltype(gtag);
        if (vmean_dtype == GEFEN_F32) GEFEN_VMEAN(G, float);
        else if (vmean_dtype == GEFEN_BF16) GEFEN_VMEAN(G, bf16_t);
        else GEFEN_VMEAN(G, f16_t);
    };
    if (grad_dtype == GEFEN_F32) launch_s(float{});
    else if (grad_dtype == GEFEN_BF16) launch_s(bf16_t{});
    else launch_s(f16_t{});
#undef GEFEN_VMEAN
    return launch_status("gefen vmean launch");
}

// bf16 GEMM with fp32 accumulation on gfx950 MFMA for GefenMuon's
// Newton-Schulz iteration (gefen_muon.py:33-47):
//
//   C = alpha * A @ op(B) + beta * D      (rounded to bf16 once)
//
// A is [M, K] row-major.  op(B) is B^T for B given [N, K] row-major (the Gram
// matrix X X^T) or B for B given [K, N] row-major (A A and B X).
//
// Tiling: a 256-thread workgroup owns a 128x128 tile of C; its four waves each
// own 64x64 as 2x2 v_mfma_f32_32x32x16_bf16 tiles (16 fp32 accumulators per
// lane per tile).  K advances 32 at a time through LDS, double-buffered: the
// global loads of step k+1 are issued into registers before the MFMAs of step
// k and written to the other LDS buffer afterwards.  Operands are stored in LDS
// K-contiguous ([row][k], padded rows), so every MFMA operand is one 16-byte
// LDS read.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <type_traits>

#include "capi_internal.h"
#include "common.h"

namespace gefen {
namespace ns {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDK = BK + 8;  // padded LDS row (bf16 elements): 80 bytes
constexpr int NT = 256;

struct alignas(16) U4 { uint32_t x, y, z, w; };

// Stage of global data held in registers between the load and the LDS write.
struct Stage {
    U4 a[2];
    U4 b[2];
};

__device__ __forceinline__ U4 zero4() { return U4{0u, 0u, 0u, 0u}; }

// A or B(kcontig) tile: `rows` x BK from a row-major [R, K] matrix, 512 16-byte
// vectors, two per thread.  Out-of-range elements read as zero.
__device__ __forceinline__ void load_rows(const uint16_t* __restrict__ src, int64_t ld, int R, int K, int r0, int k0,
                                          bool vec_ok, U4 out[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int v = threadIdx.x + NT * i;
        const int row = v >> 2;
        const int kv = (v & 3) * 8;
        const int gr = r0 + row, gk = k0 + kv;
        if (vec_ok && gr < R && gk + 8 <= K) {
            out[i] = *reinterpret_cast<const U4*>(src + (int64_t)gr * ld + gk);
        } else {
            uint16_t tmp[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) tmp[e] = (gr < R && gk + e < K) ? src[(int64_t)gr * ld + gk + e] : (uint16_t)0;
            __builtin_memcpy(&out[i], tmp, 16);
        }
    }
}

// B tile of a row-major [K, N] matrix: BK rows of 128 columns, vectors of 8 columns.
__device__ __forceinline__ void load_kn(const uint16_t* __restrict__ src, int64_t ld, int K, int N, int k0, int n0,
                                        bool vec_ok, U4 out[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int v = threadIdx.x + NT * i;
        const int kr = v >> 4;        // 0..31
        const int nv = (v & 15) * 8;  // 0..120
        const int gk = k0 + kr, gn = n0 + nv;
        if (vec_ok && gk < K && gn + 8 <= N) {
            out[i] = *reinterpret_cast<const U4*>(src + (int64_t)gk * ld + gn);
        } else {
            uint16_t tmp[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) tmp[e] = (gk < K && gn + e < N) ? src[(int64_t)gk * ld + gn + e] : (uint16_t)0;
            __builtin_memcpy(&out[i], tmp, 16);
        }
    }
}

__device__ __forceinline__ void store_rows(uint16_t* lds, const U4 in[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int v = threadIdx.x + NT * i;
        *reinterpret_cast<U4*>(lds + (v >> 2) * LDK + (v & 3) * 8) = in[i];
    }
}

__device__ __forceinline__ void store_kn(uint16_t* lds, const U4 in[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int v = threadIdx.x + NT * i;
        const int kr = v >> 4, nv = (v & 15) * 8;
        uint16_t tmp[8];
        __builtin_memcpy(tmp, &in[i], 16);
#pragma unroll
        for (int e = 0; e < 8; ++e) lds[(nv + e) * LDK + kr] = tmp[e];
    }
}

template <bool B_KCONTIG>
__global__ __launch_bounds__(NT) void k_gemm(const uint16_t* __restrict__ A, int64_t lda,
                                             const uint16_t* __restrict__ B, int64_t ldb,
                                             uint16_t* __restrict__ C, int64_t ldc,
                                             const uint16_t* __restrict__ D, int64_t ldd, int M, int N, int K,
                                             float alpha, float beta, int vec_a, int vec_b) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    Stage s;
    load_rows(A, lda, M, K, m0, 0, vec_a, s.a);
    if (B_KCONTIG) load_rows(B, ldb, N, K, n0, 0, vec_b, s.b);
    else load_kn(B, ldb, K, N, 0, n0, vec_b, s.b);
    store_rows(As[0], s.a);
    if (B_KCONTIG) store_rows(Bs[0], s.b);
    else store_kn(Bs[0], s.b);
    __syncthreads();

    const int nk = (K + BK - 1) / BK;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            const int k0 = (kt + 1) * BK;
            load_rows(A, lda, M, K, m0, k0, vec_a, s.a);
            if (B_KCONTIG) load_rows(B, ldb, N, K, n0, k0, vec_b, s.b);
            else load_kn(B, ldb, K, N, k0, n0, vec_b, s.b);
        }
        const uint16_t* as = As[cur];
        const uint16_t* bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            bf16x8 af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const bf16x8*>(as + (wm + i * 32 + (lane & 31)) * LDK + kk + 8 * (lane >> 5));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8*>(bs + (wn + j * 32 + (lane & 31)) * LDK + kk + 8 * (lane >> 5));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            store_rows(As[cur ^ 1], s.a);
            if (B_KCONTIG) store_rows(Bs[cur ^ 1], s.b);
            else store_kn(Bs[cur ^ 1], s.b);
        }
        __syncthreads();
    }
    // epilogue: C = alpha * acc + beta * D, one rounding to bf16
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int col = n0 + wn + j * 32 + (lane & 31);
                if (row < M && col < N) {
                    float v = alpha * acc[i][j][r];
                    if (beta != 0.0f) {
                        const float d = __uint_as_float((uint32_t)D[(int64_t)row * ldd + col] << 16);
                        v = v + beta * d;
                    }
                    const bf16_t o = from_f32<bf16_t>(v);
                    C[(int64_t)row * ldc + col] = o.bits;
                }
            }
}

// ---------------------------------------------------------------------------
// Large-tile batched GEMM for the Newton-Schulz products, all in "A B^T" form:
//
//   C_b = alpha * A_b @ B_b^T + beta * D_b     (bf16 out, one rounding)
//
// A_b [M, K] and B_b [N, K] are row-major, so both operands are K-contiguous
// (the Gram matrix X X^T, A A with A symmetric, and B X with X^T kept beside X).
// A 512-thread workgroup owns a 256x256 tile; its eight waves (2 x 4) each own
// 128x64 as 4x2 v_mfma_f32_32x32x16_bf16 tiles (128 fp32 accumulators per
// lane).  K moves TK (64) at a time through one register stage and two LDS
// stages (global loads run two steps ahead of the MFMAs that use them).  Symmetric outputs (X X^T, b A + c A A)
// compute only the tiles on and above the diagonal and mirror them; CT
// (optional) receives C^T.  Each XCD takes a contiguous run of tiles, in bands
// of kGroupM tile rows, so workgroups that share operand panels share an L2.
// M and N must be multiples of 256, K a multiple of TK, every row 16-byte
// aligned; other shapes take k_gemm.
#ifndef GEFEN_NS_TK
#define GEFEN_NS_TK 64
#endif
constexpr int TM = 256, TN = 256, TK = GEFEN_NS_TK;
constexpr int TLD = TK + 8;  // padded LDS row (bf16 elements)
constexpr int CPR = TK / 8;  // 16-byte chunks per tile row
#ifndef GEFEN_NS_WJ
#define GEFEN_NS_WJ 2
#endif
constexpr int WI = 4, WJ = GEFEN_NS_WJ;  // 32x32 MFMA tiles per wave (rows, columns)
constexpr int WAVES_N = TN / (32 * WJ), WAVES_M = TM / (32 * WI);
constexpr int TT = 64 * WAVES_M * WAVES_N;
constexpr int TCH = TM * TK / 8 / TT;  // 16-byte chunks per thread per operand tile

struct TileGemm {
    const uint16_t* A;
    const uint16_t* B;
    uint16_t* C;
    uint16_t* CT;
    const uint16_t* D;
    int64_t lda, ldb, ldc, ldct, ldd;
    int64_t sa, sb, sc, sct, sd;  // batch strides (elements)
    int M, N, K;
    float alpha, beta;
    int tiles_n;   // N / TN
    int tiles;     // tiles per matrix
    int symmetric;
    int d_t;       // D is given as D^T [N, M] (row stride ldd): four rows of one column are one 8-byte load
};

// Buffer resource over the 256 rows of one operand tile (rows r0 .. r0 + 255 of
// a row-major matrix with row stride ld): the loads address it with a 32-bit
// per-thread offset and a scalar offset, so no 64-bit address is formed per
// load (the entry point checks that 256 rows fit in 2^31 bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const uint16_t* rows, int64_t ld) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(rows), (short)0, (int)(TM * ld * 2), 0x00020000);
}
// The TCH 16-byte chunks of this thread in a 256 x TK operand tile at column k0:
// chunk q = threadIdx.x + TT i is row q / CPR, k-chunk q % CPR.  voff is the
// byte offset of chunk 0 (row threadIdx.x / CPR); chunk i is TT / CPR rows on.
__device__ __forceinline__ void tile_load(__amdgpu_buffer_rsrc_t rs, int voff, int64_t ld, int k0, u32x4 out[TCH]) {
#pragma unroll
    for (int i = 0; i < TCH; ++i)
        out[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, (int)(((int64_t)(TT / CPR) * i * ld + k0) * 2), 0));
}
__device__ __forceinline__ void tile_store(uint16_t* lds, const u32x4 in[TCH]) {
#pragma unroll
    for (int i = 0; i < TCH; ++i) {
        const int q = threadIdx.x + TT * i;
        *reinterpret_cast<u32x4*>(lds + (q / CPR) * TLD + (q % CPR) * 8) = in[i];
    }
}

// MN-major operand (the Gram product X X^T with only X^T stored): the operand is
// given as its transpose [K, 256-column block], and a K step of the tile is
// rows k0 .. k0 + TK of it, 256 elements each.  LDS keeps that layout, [k][m]
// in rows of TLDM elements (576 bytes: consecutive rows start 16 banks apart,
// so the transposed fragment reads below are conflict-free), and fragments come
// out of ds_read_b64_tr_b16.  Chunk q = threadIdx.x + TT i is row q / MCPR,
// column chunk q % MCPR; chunk i is TT / MCPR rows on.
constexpr int MCPR = TM / 8;   // 16-byte chunks per K row of the tile
constexpr int TLDM = TM + 32;  // LDS row of an MN-major stage (bf16)
static_assert(TK * TLDM == TM * TLD, "an MN-major stage has the size of a K-major one");
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc_mn(const uint16_t* cols, int64_t ld, int K) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(cols), (short)0, (int)(K * ld * 2), 0x00020000);
}
__device__ __forceinline__ void tile_load_mn(__amdgpu_buffer_rsrc_t rs, int voff, int64_t ld, int k0, u32x4 out[TCH]) {
#pragma unroll
    for (int i = 0; i < TCH; ++i)
        out[i] = __builtin_bit_cast(
            u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, (int)(((int64_t)(TT / MCPR) * i + k0) * ld * 2), 0));
}
__device__ __forceinline__ void tile_store_mn(uint16_t* lds, const u32x4 in[TCH]) {
#pragma unroll
    for (int i = 0; i < TCH; ++i) {
        const int q = threadIdx.x + TT * i;
        *reinterpret_cast<u32x4*>(lds + (q / MCPR) * TLDM + (q % MCPR) * 8) = in[i];
    }
}
// ds_read_b64_tr_b16: in each group of 16 lanes, lane 4 j + q gives the address
// of 4 elements (row j, columns 4 q .. 4 q + 3 of a 4 x 16 block) and lane i
// receives column i, rows 0 .. 3.  The MFMA operand of lane l (row l % 32, k =
// 8 (l / 32) + 0..7) is two such reads: lane l points at K row kk + 8 (l / 32) +
// (l % 16) / 4 (+ 4 for the second read), column 16 ((l / 16) % 2) + 4 (l % 4).
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int mn_lane_offset(int lane) {
    const int g = lane >> 4, r = lane & 15;
    return (8 * (g >> 1) + (r >> 2)) * TLDM + 16 * (g & 1) + 4 * (r & 3);
}
__device__ __forceinline__ bf16x8 mn_frag(const uint16_t* p) {
    typedef __attribute__((address_space(3))) bf16x4 lds_v4;
    const auto* q = (const __attribute__((address_space(3))) uint16_t*)p;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4*)q);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_v4*)(q + 4 * TLDM));
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

#ifndef GEFEN_NS_XCD
#define GEFEN_NS_XCD 1
#endif
#ifndef GEFEN_NS_GROUP_M
#define GEFEN_NS_GROUP_M 8
#endif
constexpr int kXcds = 8;                 // workgroups go round-robin to the 8 XCDs
constexpr int kGroupM = GEFEN_NS_GROUP_M;  // tile rows per band of the tile order

// Logical tile index of this workgroup: consecutive logical tiles run on one
// XCD (which shares one L2), instead of the hardware's round-robin.
__device__ __forceinline__ int logical_block(int b, int nwg) {
    if (!GEFEN_NS_XCD) return b;
    const int q = nwg / kXcds, r = nwg % kXcds;
    const int x = b % kXcds, k = b / kXcds;
    return x < r ? x * (q + 1) + k : r * (q + 1) + (x - r) * q + k;
}

// Workgroup barrier for LDS traffic only: this wave's LDS reads and writes are
// complete, global loads may still be in flight (__syncthreads would also wait
// for them, which would cut the prefetch short).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


// Epilogue tile in LDS: T[c][r] = C[r][c] (the C^T orientation) in rows of LDT
// bf16.  LDT / 2 = 130 dwords = 2 (mod 32): the 8-byte accesses of 16
// consecutive columns cover all 32 banks once, and gathering one row from
// two column chunks 8 apart (1040 dwords = 16 mod 32) is conflict-free too.
constexpr int LDT = TM + 4;
static_assert(TM == TN, "square tiles");
static_assert(TN * LDT <= 4 * TM * TLD, "the epilogue tile fits in the operand stages");

// GefenMuon's parameter update fused into the last Newton-Schulz product
// (gefen_gemm_bf16_nt_batched_apply): matrix b of a launch is the update U of
// parameter p[b], whose layout is U (rows of N elements) or, when transposed, U^T
// (rows of M elements); the other entries are the scalars of muon_apply_value.
constexpr int kMaxFuse = 64;  // matrices per launch (the table travels in the kernel arguments)
struct FusedApply {
    void* p[kMaxFuse];
    float wdf[kMaxFuse];
    float alpha[kMaxFuse];
    uint8_t do_wd[kMaxFuse];
    uint8_t round_prod[kMaxFuse];
    int32_t transposed;
};

// MN: both operands MN-major (the symmetric Gram product from X^T; no D, no C^T).
// PD: void, or the parameter type of a fused update (fa != nullptr; C and C^T
// are then not stored).
template <bool MN, typename PD>
__device__ __forceinline__ void gemm_tile_body(const TileGemm& g, const FusedApply* fa) {
    // operand stages: A in [0, 2) and B in [2, 4) of TM x TLD each; the epilogue reuses them
    __shared__ __attribute__((aligned(16))) uint16_t smem[4 * TM * TLD];
    uint16_t* const As[2] = {smem, smem + TM * TLD};
    uint16_t* const Bs[2] = {smem + 2 * TM * TLD, smem + 3 * TM * TLD};
    const int lb = logical_block(blockIdx.x, gridDim.x);
    const int batch = lb / g.tiles;
    int t = lb - batch * g.tiles;
    int ti, tj;
    if (g.symmetric) {  // tiles (ti, tj), ti <= tj, row by row
        ti = 0;
        while (t >= g.tiles_n - ti) {
            t -= g.tiles_n - ti;
            ++ti;
        }
        tj = ti + t;
    } else {  // bands of kGroupM tile rows, column by column within a band
        const int tiles_m = g.M / TM;
        const int band = t / (kGroupM * g.tiles_n);
        const int rows_in = min(kGroupM, tiles_m - band * kGroupM);
        const int w = t - band * kGroupM * g.tiles_n;
        ti = band * kGroupM + w % rows_in;
        tj = w / rows_in;
    }
    const int m0 = ti * TM, n0 = tj * TN;
    const uint16_t* __restrict__ A = g.A + batch * g.sa;
    const uint16_t* __restrict__ B = g.B + batch * g.sb;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = (wave / WAVES_N) * (32 * WI), wn = (wave % WAVES_N) * (32 * WJ);
    f32x16 acc[WI][WJ];
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    const int nk = g.K / TK;
    u32x4 ra[TCH], rb[TCH];  // register stage of the global -> LDS pipeline
    const __amdgpu_buffer_rsrc_t rsa = MN ? tile_rsrc_mn(A + m0, g.lda, g.K) : tile_rsrc(A + (int64_t)m0 * g.lda, g.lda);
    const __amdgpu_buffer_rsrc_t rsb = MN ? tile_rsrc_mn(B + n0, g.ldb, g.K) : tile_rsrc(B + (int64_t)n0 * g.ldb, g.ldb);
    const int voa = MN ? (int)(((threadIdx.x / MCPR) * g.lda + (threadIdx.x % MCPR) * 8) * 2)
                       : (int)(((threadIdx.x / CPR) * g.lda + (threadIdx.x % CPR) * 8) * 2);
    const int vob = MN ? (int)(((threadIdx.x / MCPR) * g.ldb + (threadIdx.x % MCPR) * 8) * 2)
                       : (int)(((threadIdx.x / CPR) * g.ldb + (threadIdx.x % CPR) * 8) * 2);
    auto load_ops = [&](int k0) {
        if (MN) {
            tile_load_mn(rsa, voa, g.lda, k0, ra);
            tile_load_mn(rsb, vob, g.ldb, k0, rb);
        } else {
            tile_load(rsa, voa, g.lda, k0, ra);
            tile_load(rsb, vob, g.ldb, k0, rb);
        }
    };
    auto store_ops = [&](int stage) {
        if (MN) {
            tile_store_mn(As[stage], ra);
            tile_store_mn(Bs[stage], rb);
        } else {
            tile_store(As[stage], ra);
            tile_store(Bs[stage], rb);
        }
    };
    const int mn_lofs = MN ? mn_lane_offset(lane) : 0;
    load_ops(0);
    store_ops(0);
    if (nk > 1) load_ops(TK);
    __syncthreads();
    // One K step from LDS stage CUR.  It first stores step kt + 1 (loaded during
    // step kt - 1) into the other LDS stage, which every wave finished reading
    // before the last barrier, then reloads the registers with step kt + 2
    // (clamped to the last step: the loads are unconditional).  Fragments of the
    // next 16-deep slice are read while the current slice's MFMAs run, in the
    // order GEFEN_SCHED_STEP fixes: the first slice's fragments, then each MFMA
    // followed by one fragment read of the next slice and, during the first
    // slice, one of the step's global loads.  (Left to the compiler, the loads
    // sank to the end of the step and the reads bunched up: 8% slower.  A
    // second register stage, loads two steps ahead with the stores after the
    // MFMAs, measured 5% slower: the stores then wait at the end of every step.)
#define GEFEN_LOAD_FRAGS(AS, BS, KK, AF, BF)                                                                      \
    {                                                                                                             \
    if (MN) {                                                                                                     \
        _Pragma("unroll") for (int i = 0; i < WI; ++i) AF[i] = mn_frag((AS) + (KK) * TLDM + mn_lofs + wm + i * 32); \
        _Pragma("unroll") for (int j = 0; j < WJ; ++j) BF[j] = mn_frag((BS) + (KK) * TLDM + mn_lofs + wn + j * 32); \
    } else {                                                                                                      \
        _Pragma("unroll") for (int i = 0; i < WI; ++i) AF[i] =                                                    \
            *reinterpret_cast<const bf16x8*>((AS) + (wm + i * 32 + (lane & 31)) * TLD + (KK) + 8 * (lane >> 5));  \
        _Pragma("unroll") for (int j = 0; j < WJ; ++j) BF[j] =                                                    \
            *reinterpret_cast<const bf16x8*>((BS) + (wn + j * 32 + (lane & 31)) * TLD + (KK) + 8 * (lane >> 5));  \
    }                                                                                                             \
    }
#define GEFEN_MFMAS(AF, BF)                                                                                       \
    _Pragma("unroll") for (int i = 0; i < WI; ++i) _Pragma("unroll") for (int j = 0; j < WJ; ++j) acc[i][j] =     \
        __builtin_amdgcn_mfma_f32_32x32x16_bf16(AF[i], BF[j], acc[i][j], 0, 0, 0);
    // instruction groups in issue order (masks: 0x008 MFMA, 0x100 LDS read, 0x020 global read)
#define GEFEN_SCHED_STEP                                                                                          \
    {                                                                                                             \
        __builtin_amdgcn_sched_group_barrier(0x100, (WI + WJ) * (MN ? 2 : 1), 0);                                 \
        _Pragma("unroll") for (int s_ = 0; s_ < TK / 16; ++s_) {                                                  \
            _Pragma("unroll") for (int t_ = 0; t_ < WI * WJ; ++t_) {                                              \
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                                \
                if (s_ + 1 < TK / 16 && t_ < WI + WJ) __builtin_amdgcn_sched_group_barrier(0x100, MN ? 2 : 1, 0); \
                if (s_ == 0 && t_ < 2 * TCH) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                   \
            }                                                                                                     \
        }                                                                                                         \
    }
#define GEFEN_TILE_STEP(KT, CUR)                                                                                  \
    {                                                                                                             \
        if ((KT) + 1 < nk) store_ops((CUR) ^ 1);                                                                  \
        load_ops(min((KT) + 2, nk - 1) * TK);                                                                     \
        const uint16_t* as = As[CUR];                                                                             \
        const uint16_t* bs = Bs[CUR];                                                                             \
        bf16x8 af0[WI], bf0[WJ], af1[WI], bf1[WJ];                                                                \
        GEFEN_LOAD_FRAGS(as, bs, 0, af0, bf0)                                                                     \
        _Pragma("unroll") for (int kk = 0; kk < TK; kk += 32) {                                                   \
            GEFEN_LOAD_FRAGS(as, bs, kk + 16, af1, bf1)                                                           \
            GEFEN_MFMAS(af0, bf0)                                                                                 \
            if (kk + 32 < TK) GEFEN_LOAD_FRAGS(as, bs, kk + 32, af0, bf0)                                         \
            GEFEN_MFMAS(af1, bf1)                                                                                 \
        }                                                                                                         \
        GEFEN_SCHED_STEP                                                                                          \
        lds_barrier();                                                                                            \
    }
    int kt = 0;
    for (; kt + 1 < nk; kt += 2) {
        GEFEN_TILE_STEP(kt, 0)
        GEFEN_TILE_STEP(kt + 1, 1)
    }
    if (kt < nk) GEFEN_TILE_STEP(kt, 0)
#undef GEFEN_TILE_STEP
#undef GEFEN_SCHED_STEP
#undef GEFEN_MFMAS
#undef GEFEN_LOAD_FRAGS
    // epilogue: C = alpha * acc + beta * D rounded once, assembled in LDS as
    // T = C^T (every wave is past its last fragment read: the last K step ended
    // with a barrier), then written with 16-byte stores: T's rows are rows of
    // C^T (CT, or the mirror tile of a symmetric product), and C's rows are
    // gathered from two column chunks per wave instruction.  D given as D^T is
    // staged through T the same way; a row-major D is read directly.
    uint16_t* __restrict__ C = g.C ? g.C + batch * g.sc : nullptr;
    uint16_t* __restrict__ CT = g.CT ? g.CT + batch * g.sct : nullptr;
    const uint16_t* __restrict__ D = g.D ? g.D + batch * g.sd : nullptr;
    const bool mirror = g.symmetric && ti != tj;
    uint16_t* const T = smem;
    constexpr int kChunks = TM * TN / 8 / TT;  // 16-byte chunks per thread
    const bool d_lds = D && g.d_t;
    if (d_lds) {
        constexpr int kBatch = kChunks < 16 ? kChunks : 16;  // loads in flight per thread
#pragma unroll
        for (int i0 = 0; i0 < kChunks; i0 += kBatch) {
            u32x4 dv[kBatch];
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int q = threadIdx.x + TT * (i0 + i);
                const int c = q >> 5, r8 = (q & 31) * 8;
                dv[i] = *reinterpret_cast<const u32x4*>(D + (int64_t)(n0 + c) * g.ldd + m0 + r8);
            }
#pragma unroll
            for (int i = 0; i < kBatch; ++i) {
                const int q = threadIdx.x + TT * (i0 + i);
                const int c = q >> 5, r8 = (q & 31) * 8;
                uint2* t = reinterpret_cast<uint2*>(T + c * LDT + r8);
                t[0] = make_uint2(dv[i].x, dv[i].y);
                t[1] = make_uint2(dv[i].z, dv[i].w);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < WI; ++i)
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const int c = wn + j * 32 + (lane & 31);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int r0 = wm + i * 32 + 8 * r4 + 4 * (lane >> 5);
                uint2* t = reinterpret_cast<uint2*>(T + c * LDT + r0);
                float dv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (d_lds) {
                    const uint2 w = *t;
                    dv[0] = __uint_as_float(w.x << 16);
                    dv[1] = __uint_as_float(w.x & 0xffff0000u);
                    dv[2] = __uint_as_float(w.y << 16);
                    dv[3] = __uint_as_float(w.y & 0xffff0000u);
                } else if (D) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dv[r] = __uint_as_float((uint32_t)D[(int64_t)(m0 + r0 + r) * g.ldd + n0 + c] << 16);
                }
                uint32_t o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = g.alpha * acc[i][j][4 * r4 + r];
                    if (D) v = v + g.beta * dv[r];
                    o[r] = from_f32<bf16_t>(v).bits;
                }
                *t = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
            }
        }
    __syncthreads();
    if constexpr (!std::is_void<PD>::value) {
        // T holds the update tile as U^T (bf16): p <- muon_apply_value(p, U) with
        // 8-element chunks of parameter rows, read and written once; every chunk's
        // load is issued before the first update (the accumulators are dead here)
        PD* __restrict__ P = static_cast<PD*>(fa->p[batch]);
        const float wdf = fa->wdf[batch], al = fa->alpha[batch];
        const bool dwd = fa->do_wd[batch] != 0, rp = fa->round_prod[batch] != 0;
        const bool tr = fa->transposed != 0;
        int64_t e[kChunks];
        Vec<PD, 8> pv[kChunks];
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int q = threadIdx.x + TT * i;
            // transposed: parameter rows are rows of U^T, T row c -> row n0 + c;
            // else rows of U, gathered from two column chunks of T as C below
            e[i] = tr ? (int64_t)(n0 + (q >> 5)) * g.M + m0 + (q & 31) * 8
                      : (int64_t)(m0 + (q & 31) + 32 * (q >> 10)) * g.N + n0 + ((q >> 5) & 31) * 8;
            pv[i] = vload<PD, 8>(P, e[i]);
        }
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int q = threadIdx.x + TT * i;
            uint32_t w[4];
            if (tr) {
                const uint2* t = reinterpret_cast<const uint2*>(T + (q >> 5) * LDT + (q & 31) * 8);
                const uint2 lo = t[0], hi = t[1];
                w[0] = lo.x; w[1] = lo.y; w[2] = hi.x; w[3] = hi.y;
            } else {
                const uint16_t* t = T + ((q >> 5) & 31) * 8 * LDT + (q & 31) + 32 * (q >> 10);
                uint32_t h[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) h[u] = t[u * LDT];
                w[0] = h[0] | (h[1] << 16); w[1] = h[2] | (h[3] << 16);
                w[2] = h[4] | (h[5] << 16); w[3] = h[6] | (h[7] << 16);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float uf = __uint_as_float((u & 1) ? (w[u >> 1] & 0xffff0000u) : (w[u >> 1] << 16));
                pv[i].v[u] = from_f32<PD>(muon_apply_value<PD>(to_f32(pv[i].v[u]), uf, wdf, al, dwd, rp));
            }
            vstore<PD, 8>(P, e[i], pv[i]);
        }
        return;
    }
    if (CT || mirror) {  // rows of C^T: T row c -> row n0 + c
        uint16_t* __restrict__ dst = CT ? CT : C;
        const int64_t ld = CT ? g.ldct : g.ldc;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int q = threadIdx.x + TT * i;
            const int c = q >> 5, r8 = (q & 31) * 8;
            const uint2* t = reinterpret_cast<const uint2*>(T + c * LDT + r8);
            const uint2 lo = t[0], hi = t[1];
            u32x4 v;
            v.x = lo.x; v.y = lo.y; v.z = hi.x; v.w = hi.y;
            *reinterpret_cast<u32x4*>(dst + (int64_t)(n0 + c) * ld + m0 + r8) = v;
        }
    }
    // rows of C: lanes 0-31 take 32 consecutive rows of column chunk k, lanes
    // 32-63 the same rows of chunk k + 1 (C may be absent when only C^T is wanted)
    if (!g.C) return;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int q = threadIdx.x + TT * i;
        const int r = (q & 31) + 32 * (q >> 10), c8 = ((q >> 5) & 31) * 8;
        const uint16_t* t = T + c8 * LDT + r;
        uint32_t h[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) h[u] = t[u * LDT];
        u32x4 v;
        v.x = h[0] | (h[1] << 16);
        v.y = h[2] | (h[3] << 16);
        v.z = h[4] | (h[5] << 16);
        v.w = h[6] | (h[7] << 16);
        *reinterpret_cast<u32x4*>(C + (int64_t)(m0 + r) * g.ldc + n0 + c8) = v;
    }
}

template <bool MN>
__global__ __launch_bounds__(TT) void k_gemm_tile(const TileGemm g) {
    gemm_tile_body<MN, void>(g, nullptr);
}

template <typename PD>
__global__ __launch_bounds__(TT) void k_gemm_tile_apply(const TileGemm g, const FusedApply fa) {
    gemm_tile_body<false, PD>(g, &fa);
}

}  // namespace ns
}  // namespace gefen

using namespace gefen;

extern "C" int gefen_gemm_bf16(const void* a, int64_t lda, const void* b, int64_t ldb, int b_kcontig, void* c,
                               int64_t ldc, const void* d, int64_t ldd, int m, int n, int k, double alpha, double beta,
                               gefen_stream_t stream) {
    if (m < 0 || n < 0 || k < 0) return fail_inval("negative GEMM size");
    if (m == 0 || n == 0) return GEFEN_OK;
    if (!a || !b || !c || (beta != 0.0 && !d)) return fail_inval("null GEMM operand");
    if (lda < k || ldc < n || (b_kcontig ? ldb < k : ldb < n) || (beta != 0.0 && ldd < n))
        return fail_inval("GEMM leading dimension too small");
    const int vec_a = aligned(a, 16) && (lda % 8 == 0);
    const int vec_b = aligned(b, 16) && (ldb % 8 == 0);
    dim3 grid((n + ns::BN - 1) / ns::BN, (m + ns::BM - 1) / ns::BM);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    auto* A = static_cast<const uint16_t*>(a);
    auto* B = static_cast<const uint16_t*>(b);
    auto* C = static_cast<uint16_t*>(c);
    auto* D = static_cast<const uint16_t*>(d);
    if (b_kcontig)
        hipLaunchKernelGGL(ns::k_gemm<true>, grid, dim3(ns::NT), 0, st, A, lda, B, ldb, C, ldc, D, ldd, m, n, k,
                           (float)alpha, (float)beta, vec_a, vec_b);
    else
        hipLaunchKernelGGL(ns::k_gemm<false>, grid, dim3(ns::NT), 0, st, A, lda, B, ldb, C, ldc, D, ldd, m, n, k,
                           (float)alpha, (float)beta, vec_a, vec_b);
    return launch_status("gefen_gemm_bf16");
}

extern "C" int gefen_gemm_bf16_nt_batched(const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
                                          int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, void* ct,
                                          int64_t ldct, int64_t stride_ct, const void* d, int64_t ldd,
                                          int64_t stride_d, int d_transposed, int batch, int m, int n, int k,
                                          double alpha, double beta, int symmetric, gefen_stream_t stream) {
    if (m < 0 || n < 0 || k < 0 || batch < 0) return fail_inval("negative GEMM size");
    if (m == 0 || n == 0 || batch == 0) return GEFEN_OK;
    if (!a || !b || (!c && !ct) || (beta != 0.0 && !d)) return fail_inval("null GEMM operand");
    if (!c && symmetric) return fail_inval("a symmetric GEMM needs C");
    if (lda < k || ldb < k || (c && ldc < n) || (ct && ldct < m) || (d && ldd < (d_transposed ? m : n)))
        return fail_inval("GEMM leading dimension too small");
    if (symmetric && m != n) return fail_inval("a symmetric GEMM must be square");
    if (symmetric && ct) return fail_inval("a symmetric GEMM has no separate transposed output (C^T = C)");
    if ((int64_t)ns::TM * lda * 2 > INT32_MAX || (int64_t)ns::TN * ldb * 2 > INT32_MAX)
        return fail_inval("batched GEMM operand rows too long (256 rows must span less than 2^31 bytes)");
    if (m % ns::TM || n % ns::TN || k % ns::TK || k == 0)
        return fail_inval("batched GEMM needs M, N multiples of 256 and K a multiple of %d (got %d, %d, %d)", ns::TK, m, n, k);
    const void* ptrs[5] = {a, b, c, ct, d};
    const int64_t lds_[5] = {lda, ldb, ldc, ldct, ldd};
    const int64_t strides[5] = {stride_a, stride_b, stride_c, stride_ct, stride_d};
    for (int i = 0; i < 5; ++i) {
        if (!ptrs[i]) continue;
        if (!aligned(ptrs[i], 16) || lds_[i] % 8 || strides[i] % 8)
            return fail_inval("batched GEMM operands need 16-byte aligned rows");
    }
    ns::TileGemm g;
    g.A = static_cast<const uint16_t*>(a);
    g.B = static_cast<const uint16_t*>(b);
    g.C = static_cast<uint16_t*>(c);
    g.CT = static_cast<uint16_t*>(ct);
    g.D = beta != 0.0 ? static_cast<const uint16_t*>(d) : nullptr;
    g.lda = lda; g.ldb = ldb; g.ldc = ldc; g.ldct = ldct; g.ldd = ldd;
    g.sa = stride_a; g.sb = stride_b; g.sc = stride_c; g.sct = stride_ct; g.sd = stride_d;
    g.M = m; g.N = n; g.K = k;
    g.alpha = (float)alpha;
    g.beta = (float)beta;
    g.tiles_n = n / ns::TN;
    g.symmetric = symmetric ? 1 : 0;
    g.tiles = symmetric ? g.tiles_n * (g.tiles_n + 1) / 2 : (m / ns::TM) * g.tiles_n;
    g.d_t = d_transposed ? 1 : 0;
    if (g.D && d_transposed && ldd % 4) return fail_inval("D^T rows must be 8-byte aligned");
    const int64_t grid = (int64_t)g.tiles * batch;
    if (grid > INT32_MAX) return fail_inval("batched GEMM grid too large");
    hipLaunchKernelGGL(ns::k_gemm_tile<false>, dim3((unsigned)grid), dim3(ns::TT), 0, reinterpret_cast<hipStream_t>(stream),
                       g);
    return launch_status("gefen_gemm_bf16_nt_batched");
}

extern "C" int gefen_gram_bf16_batched(const void* xt, int64_t ldxt, int64_t stride_xt, void* c, int64_t ldc,
                                       int64_t stride_c, int batch, int m, int k, double alpha,
                                       gefen_stream_t stream) {
    if (m < 0 || k < 0 || batch < 0) return fail_inval("negative GEMM size");
    if (m == 0 || batch == 0) return GEFEN_OK;
    if (!xt || !c) return fail_inval("null GEMM operand");
    if (ldxt < m || ldc < m) return fail_inval("GEMM leading dimension too small");
    if (m % ns::TM || k % ns::TK || k == 0)
        return fail_inval("batched Gram product needs m a multiple of 256 and k a multiple of %d (got %d, %d)", ns::TK,
                          m, k);
    if ((int64_t)k * ldxt * 2 > INT32_MAX)
        return fail_inval("batched Gram product operand too large (k rows must span less than 2^31 bytes)");
    if (!aligned(xt, 16) || !aligned(c, 16) || ldxt % 8 || ldc % 8 || stride_xt % 8 || stride_c % 8)
        return fail_inval("batched GEMM operands need 16-byte aligned rows");
    ns::TileGemm g;
    memset(&g, 0, sizeof(g));
    g.A = g.B = static_cast<const uint16_t*>(xt);
    g.C = static_cast<uint16_t*>(c);
    g.lda = g.ldb = ldxt;
    g.ldc = ldc;
    g.sa = g.sb = stride_xt;
    g.sc = stride_c;
    g.M = g.N = m;
    g.K = k;
    g.alpha = (float)alpha;
    g.beta = 0.0f;
    g.tiles_n = m / ns::TN;
    g.symmetric = 1;
    g.tiles = g.tiles_n * (g.tiles_n + 1) / 2;
    const int64_t grid = (int64_t)g.tiles * batch;
    if (grid > INT32_MAX) return fail_inval("batched GEMM grid too large");
    hipLaunchKernelGGL(ns::k_gemm_tile<true>, dim3((unsigned)grid), dim3(ns::TT), 0, reinterpret_cast<hipStream_t>(stream),
                       g);
    return launch_status("gefen_gram_bf16_batched");
}

extern "C" int gefen_gemm_bf16_nt_batched_apply(const void* a, int64_t lda, int64_t stride_a, const void* b,
                                                int64_t ldb, int64_t stride_b, const void* d_t, int64_t ldd,
                                                int64_t stride_d, int batch, int m, int n, int k, double alpha,
                                                double beta, const gefen_muon_apply_task* tasks,
                                                gefen_stream_t stream) {
    if (m < 0 || n < 0 || k < 0 || batch < 0) return fail_inval("negative GEMM size");
    if (m == 0 || n == 0 || batch == 0) return GEFEN_OK;
    if (!a || !b || !tasks || (beta != 0.0 && !d_t)) return fail_inval("null GEMM operand");
    if (lda < k || ldb < k || (beta != 0.0 && ldd < m)) return fail_inval("GEMM leading dimension too small");
    if ((int64_t)ns::TM * lda * 2 > INT32_MAX || (int64_t)ns::TN * ldb * 2 > INT32_MAX)
        return fail_inval("batched GEMM operand rows too long (256 rows must span less than 2^31 bytes)");
    if (m % ns::TM || n % ns::TN || k % ns::TK || k == 0)
        return fail_inval("batched GEMM needs M, N multiples of 256 and K a multiple of %d (got %d, %d, %d)", ns::TK, m, n, k);
    const void* ptrs[3] = {a, b, beta != 0.0 ? d_t : nullptr};
    const int64_t lds_[3] = {lda, ldb, ldd};
    const int64_t strides[3] = {stride_a, stride_b, stride_d};
    for (int i = 0; i < 3; ++i) {
        if (!ptrs[i]) continue;
        if (!aligned(ptrs[i], 16) || lds_[i] % 8 || strides[i] % 8)
            return fail_inval("batched GEMM operands need 16-byte aligned rows");
    }
    const int dt = tasks[0].param_dtype;
    const int transposed = tasks[0].transposed ? 1 : 0;
    if (!valid_dtype(dt)) return fail_inval("unsupported parameter dtype %d", dt);
    for (int i = 0; i < batch; ++i) {
        const gefen_muon_apply_task& t = tasks[i];
        if (t.param_dtype != dt) return fail_inval("the parameters of one call must share a dtype");
        if ((t.transposed ? 1 : 0) != transposed) return fail_inval("the parameters of one call must share an orientation");
        if (t.numel != (int64_t)m * n) return fail_inval("parameter %d has %lld elements, the product %lld", i,
                                                        (long long)t.numel, (long long)m * n);
        if (!t.p) return fail_inval("null parameter pointer");
        if (!aligned(t.p, 8 * dtype_size(dt))) return fail_inval("parameters need %d-byte alignment", 8 * dtype_size(dt));
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int tiles = (m / ns::TM) * (n / ns::TN);
    for (int c0 = 0; c0 < batch; c0 += ns::kMaxFuse) {
        const int nb = batch - c0 < ns::kMaxFuse ? batch - c0 : ns::kMaxFuse;
        ns::TileGemm g;
        memset(&g, 0, sizeof(g));
        g.A = static_cast<const uint16_t*>(a) + c0 * stride_a;
        g.B = static_cast<const uint16_t*>(b) + c0 * stride_b;
        g.D = beta != 0.0 ? static_cast<const uint16_t*>(d_t) + c0 * stride_d : nullptr;
        g.lda = lda; g.ldb = ldb; g.ldd = ldd;
        g.sa = stride_a; g.sb = stride_b; g.sd = stride_d;
        g.M = m; g.N = n; g.K = k;
        g.alpha = (float)alpha;
        g.beta = (float)beta;
        g.tiles_n = n / ns::TN;
        g.symmetric = 0;
        g.tiles = tiles;
        g.d_t = 1;
        if (g.D && ldd % 4) return fail_inval("D^T rows must be 8-byte aligned");
        ns::FusedApply fa;
        memset(&fa, 0, sizeof(fa));
        fa.transposed = transposed;
        for (int i = 0; i < nb; ++i) {
            const MuonApplyScalars sc = muon_apply_scalars(tasks[c0 + i]);
            fa.p[i] = tasks[c0 + i].p;
            fa.wdf[i] = sc.wdf;
            fa.alpha[i] = sc.alpha;
            fa.do_wd[i] = (uint8_t)sc.do_wd;
            fa.round_prod[i] = (uint8_t)sc.round_prod;
        }
        const int64_t grid = (int64_t)tiles * nb;
        if (grid > INT32_MAX) return fail_inval("batched GEMM grid too large");
        if (dt == GEFEN_F32)
            hipLaunchKernelGGL(ns::k_gemm_tile_apply<float>, dim3((unsigned)grid), dim3(ns::TT), 0, st, g, fa);
        else if (dt == GEFEN_BF16)
            hipLaunchKernelGGL(ns::k_gemm_tile_apply<bf16_t>, dim3((unsigned)grid), dim3(ns::TT), 0, st, g, fa);
        else
            hipLaunchKernelGGL(ns::k_gemm_tile_apply<f16_t>, dim3((unsigned)grid), dim3(ns::TT), 0, st, g, fa);
        const int rc = launch_status("gefen_gemm_bf16_nt_batched_apply");
        if (rc) return rc;
    }
    return GEFEN_OK;
}

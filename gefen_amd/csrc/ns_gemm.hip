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

#include "capi_internal.h"
#include "common.h"

namespace gefen {
namespace ns {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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

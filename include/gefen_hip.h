/*
 * gefen_hip.h -- C ABI of the MI355X-native Gefen optimizer step.
 *
 * Every entry point takes raw device pointers, element counts, dtype codes and
 * scalars as double, launches asynchronously on `stream` (a hipStream_t; 0 is
 * the null stream) and returns
 *   GEFEN_OK (0), GEFEN_EINVAL (1: invalid argument, ValueError in Python),
 *   GEFEN_ERUNTIME (2: HIP or runtime failure, RuntimeError in Python).
 * gefen_last_error() returns the message of the calling thread's last failure.
 *
 * Numerics follow the reference's CPU path (fused=False) of ndvbd/Gefen 1.2.3,
 * not its CUDA kernels: codebook indices, magnitudes and histogram counts are
 * bit-identical to that path; parameters agree within the stated tolerances.
 *
 * The eleven functions of the reference's extension module
 * (kernels/gefen_cuda_binding.cpp:107-217) each have one counterpart here;
 * the comment above each names the reference interface it replaces.
 */
#ifndef GEFEN_HIP_H
#define GEFEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* gefen_stream_t; /* == hipStream_t */

enum { GEFEN_OK = 0, GEFEN_EINVAL = 1, GEFEN_ERUNTIME = 2 };
/* element types of parameters, gradients and optimizer state */
enum { GEFEN_F32 = 0, GEFEN_F16 = 1, GEFEN_BF16 = 2 };

const char* gefen_last_error(void);
int gefen_abi_version(void);
/* Number of device-memory allocations the library has made since it was loaded
 * (its pools, workspaces and temporaries; never the caller's tensors).  A
 * diagnostic: gefen_step_tasks_noalloc leaves it unchanged. */
int64_t gefen_device_allocations(void);
/* sizeof(gefen_step_task) for which = 0, sizeof(gefen_muon_task) for which = 1,
 * sizeof(gefen_muon_apply_task) for which = 2:
 * lets bindings check their mirror of the structs. */
size_t gefen_struct_size(int which);

/* ------------------------------------------------------------------ codebook tables
 * Size in bytes of the prepared lookup tables of one codebook (sorted, <= 256
 * entries); gefen_prepare_codebook fills them on `stream`.  Every update entry
 * point that takes `tables` reads the codebook from them. */
size_t gefen_codebook_tables_size(void);
int gefen_prepare_codebook(const float* codebook, int codebook_size, void* tables,
                           gefen_stream_t stream);

/* ------------------------------------------------------------------ vmean
 * Replaces automatic_vmean_update_cuda (kernels/automatic_vmean.py:10-55,
 * automatic_vmean_kernel.cu:66-158).  vmean[r] = fma(mean_j f32(g[r,j])^2, 1-beta2,
 * f32(vmean[r]) * beta2) rounded to vmean_dtype, as gefen.py:116-119. */
int gefen_automatic_vmean_update(void* vmean, int vmean_dtype, const void* grad, int grad_dtype,
                                 int64_t num_blocks, int64_t period, double beta2,
                                 gefen_stream_t stream);

/* ------------------------------------------------------------------ fused updates
 * packed_indices != 0 (here and in gefen_automatic_muon_momentum) selects the
 * packed 4-bit layout of automatic_gefen_fused_kernel.cu:14-57: m_sign holds
 * (numel + 1) / 2 bytes; element i's index is the low nibble of byte i/2 for even
 * i and the high nibble for odd i; a stored index keeps its low four bits (a
 * codebook of at most 16 entries is the meaningful use) and the other nibble of
 * its byte is left as it was.
 *
 * Replaces automatic_gefen_fused_update_cuda (automatic_gefen_fused.py:10-117,
 * automatic_gefen_fused_kernel.cu:568-674): stepsize given per block (f32). */
int gefen_automatic_fused_update(void* p, const void* grad, int param_dtype, uint8_t* m_sign,
                                 void* m_magnitude, int magnitude_dtype, const float* stepsize,
                                 const float* codebook, int codebook_size, int packed_indices,
                                 int64_t num_blocks, int64_t period, double beta1, double lr,
                                 gefen_stream_t stream);

/* Replaces automatic_gefen_fused_update_from_vmean_cuda (automatic_gefen_fused.py:120-249,
 * automatic_gefen_fused_kernel.cu:676-833): stepsize from the (already updated)
 * vmean with gefen.py:1326-1327; momentum, quantisation and p update as
 * gefen.py:1153-1206, 1328-1333. */
int gefen_automatic_fused_update_from_vmean(void* p, const void* grad, int param_dtype,
                                            uint8_t* m_sign, void* m_magnitude, int magnitude_dtype,
                                            const void* vmean, int vmean_dtype,
                                            const float* codebook, int codebook_size,
                                            int packed_indices, int64_t num_blocks, int64_t period,
                                            double beta1, double lr, double bias_correction_1,
                                            double bias_correction_2, double eps,
                                            gefen_stream_t stream);

/* Replaces automatic_gefen_period1_update_cuda (automatic_gefen_fused.py:252-388,
 * automatic_gefen_fused_kernel.cu:835-1000): per-element vmean and stepsize,
 * one magnitude per block of period_one_divisor elements. */
int gefen_automatic_period1_update(void* p, const void* grad, int param_dtype, uint8_t* m_sign,
                                   void* m_magnitude, int magnitude_dtype, void* vmean,
                                   int vmean_dtype, const float* codebook, int codebook_size,
                                   int64_t numel, int64_t period_one_divisor, double beta1,
                                   double beta2, double lr, double bias_correction_1,
                                   double bias_correction_2, double eps, gefen_stream_t stream);

/* Replaces automatic_gefen_muon_momentum_cuda (automatic_gefen_fused.py:391-489,
 * automatic_gefen_fused_kernel.cu:1002-1103): quantised momentum EMA of
 * gefen_muon.py:302-308 and 132-171 (every op rounded to the gradient dtype);
 * writes the dequantised momentum into momentum_update. */
int gefen_automatic_muon_momentum(const void* grad, int grad_dtype, uint8_t* m_sign,
                                  void* m_magnitude, int magnitude_dtype, const float* codebook,
                                  int codebook_size, void* momentum_update, int packed_indices,
                                  int64_t num_blocks, int64_t period, double beta1,
                                  gefen_stream_t stream);

/* ------------------------------------------------------------------ whole step
 * One tensor of Gefen._step_automatic (gefen.py:1270-1333) in one kernel pass:
 * vmean EMA, weight decay, bias-corrected stepsize, momentum, quantisation and
 * parameter update.  No reference counterpart as a single call: the reference
 * issues vmean + update (+ a weight-decay pass) per tensor. */
typedef struct gefen_step_task {
    void* p;                    /* parameter, numel elements of param_dtype      */
    const void* grad;           /* gradient, same dtype                          */
    uint8_t* m_codebook;        /* codebook indices, numel bytes                 */
    void* m_magnitude;          /* one per magnitude block, state_dtype          */
    void* vmean;                /* one per period block (per element if P = 1)   */
    int64_t numel;
    int64_t period;             /* automatic period P (1 = period-one mode)      */
    int64_t period_one_divisor; /* magnitude block for P = 1 (ignored if P > 1)  */
    int32_t param_dtype;
    int32_t state_dtype;
    double beta1, beta2, lr, eps, weight_decay;
    double bias_correction_1;   /* 1 - beta1**step, computed by the caller       */
    double bias_correction_2;   /* 1 - beta2**step                               */
} gefen_step_task;

/* All tasks of one call, batched into a few launches.  Launches of small
 * tensors may run on a library-owned second stream of the device, forked from
 * `stream` and joined back to it with events: the work is still ordered on
 * `stream`, but tasks of one call must not share memory. */
int gefen_step_tasks(const gefen_step_task* tasks, int ntasks, const void* tables,
                     gefen_stream_t stream);

/* The same step as gefen_step_tasks, allocating nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The period-one stepsize tables of 16-bit states go to a library-owned static
 * device buffer of 1 MiB per device (held until the process ends): at most 8
 * distinct f16-state or 682 distinct bf16-state (sqrt(bias_correction_2), eps,
 * 1/bias_correction_1) settings per call, else GEFEN_EINVAL before anything is
 * launched.  Every launch runs on `stream` (no side stream).  Calls on one
 * device share that buffer, which keeps the last call's tables: a call on
 * another stream than the previous call that wrote the tables waits for that
 * call's launches (an event per device, created on first use), and calls from
 * several threads are serialised.  Under graph capture no such wait is
 * recorded: a captured call and calls outside the graph that overlap with its
 * replays on one device race. */
int gefen_step_tasks_noalloc(const gefen_step_task* tasks, int ntasks, const void* tables,
                             gefen_stream_t stream);

/* A prepared step: gefen_step_tasks for a task table whose tensors stay the
 * same from step to step (the optimizer's cached plan).  No single counterpart
 * in the reference: it replaces the per-parameter loop of Gefen.step
 * (gefen.py:1409-1415) and its one or two launches per tensor, like
 * gefen_step_tasks, and keeps what gefen_step_tasks redoes on every call: the
 * row checks, kernel choices, grouping into launches and the launch tables.
 *
 * gefen_step_plan_create: tasks as for gefen_step_tasks (checked the same way);
 * `tables` is kept by pointer; the plan belongs to the current device.
 * gefen_step_plan_run: steps `tasks` (ntasks rows) exactly as gefen_step_tasks
 * would.  Only the gradient address and the scalars (betas, lr, eps, weight
 * decay, bias corrections) of a row may change cheaply; a table whose rows name
 * other tensors (parameter or state pointers, sizes, period, dtypes), whose
 * gradients lose the alignment their kernels were chosen for, or a stream of
 * another device takes the gefen_step_tasks path.  One plan must not be run
 * from two threads at once.
 * gefen_step_plan_time_runs: enable != 0 makes each later run record two
 * timing events on its stream, right before its first launch and after its
 * last; gefen_step_plan_last_ms waits for the last timed run to finish and
 * gives the GPU time between them in milliseconds. */
typedef struct gefen_step_plan gefen_step_plan;
int gefen_step_plan_create(const gefen_step_task* tasks, int ntasks, const void* tables, gefen_step_plan** plan);
int gefen_step_plan_run(gefen_step_plan* plan, const gefen_step_task* tasks, int ntasks, gefen_stream_t stream);
int gefen_step_plan_time_runs(gefen_step_plan* plan, int enable);
int gefen_step_plan_last_ms(gefen_step_plan* plan, float* ms);
void gefen_step_plan_destroy(gefen_step_plan* plan);

/* GefenMuon momentum of many tensors with the Nesterov blend fused
 * (gefen_muon.py:302-316): out = D(D(q*mu) + g*(1-mu)) if nesterov, else q. */
typedef struct gefen_muon_task {
    const void* grad;
    uint8_t* m_codebook;
    void* m_magnitude;
    void* out;                  /* momentum update, numel elements of grad dtype */
    int64_t numel;
    int64_t block;              /* magnitude block length (P, or divisor if P=1) */
    int32_t grad_dtype;
    int32_t state_dtype;
    double momentum;
    int32_t nesterov;
    int32_t pad;
} gefen_muon_task;

int gefen_muon_tasks(const gefen_muon_task* tasks, int ntasks, const void* tables,
                     gefen_stream_t stream);

/* gefen_muon_tasks, and the sum of squares of task i's output values: the
 * input of the Frobenius norm that gefen_ns_prepare_sumsq divides by, gathered
 * while the output is written instead of by another pass over it.  sumsq holds
 * GEFEN_SUMSQ_STRIDE float64 entries per task (device, ntasks * GEFEN_SUMSQ_STRIDE
 * entries, which the call sets to zero on `stream` by a fill kernel before the
 * momentum launches), of which GEFEN_SUMSQ_SLOTS partial sums, one per
 * 128-byte line: task i's sum is the sum over s of
 * sumsq[i * GEFEN_SUMSQ_STRIDE + 16 * s].  Each workgroup adds its float32 sum
 * to one slot with a float64 atomic, so the last bits may vary between runs;
 * the norm is rounded to bf16 from them. */
#define GEFEN_SUMSQ_SLOTS 8
#define GEFEN_SUMSQ_STRIDE (16 * GEFEN_SUMSQ_SLOTS)
int gefen_muon_tasks_sumsq(const gefen_muon_task* tasks, int ntasks, const void* tables, double* sumsq,
                           gefen_stream_t stream);

/* Replaces the bf16 normalisation before Newton-Schulz (gefen_muon.py:37,
 * ortho_grad.div_(ortho_grad.norm().clamp(min=eps)), done by torch in the
 * reference) for a stack of `batch` bf16 matrices [rows, cols] (contiguous):
 * x[g] = bf16(x[g] / max(bf16(||x[g]||), bf16(eps))) in place, and
 * xt[g] = x[g]^T [cols, rows].  rows and cols multiples of 64. */
int gefen_ns_prepare(void* x, void* xt, int batch, int rows, int cols, double eps, gefen_stream_t stream);

/* gefen_ns_prepare with each matrix's sum of squares given as the partial sums
 * gefen_muon_tasks_sumsq leaves for the bf16 outputs it wrote into the stack:
 * matrix g's norm is the square root of the sum over s of
 * sumsq[t * GEFEN_SUMSQ_STRIDE + 16 * s], t = index[g] (t = g when index is
 * NULL; both device arrays). */
int gefen_ns_prepare_sumsq(void* x, void* xt, int batch, int rows, int cols, double eps, const double* sumsq,
                           const int32_t* index, gefen_stream_t stream);

/* The same normalisation written in one orientation only: transpose = 1,
 * out[g] = (x[g] / max(bf16(||x[g]||), bf16(eps)))^T [cols, rows], x unchanged;
 * transpose = 0, x[g] normalised in place (out NULL or x).  The norms come
 * from the partial sums as in gefen_ns_prepare_sumsq. */
int gefen_ns_normalize_sumsq(void* x, void* out, int batch, int rows, int cols, double eps, const double* sumsq,
                             const int32_t* index, int transpose, gefen_stream_t stream);

/* Replaces the parameter update of gefen_muon.py:325-329 (p.mul_(1 - lr*wd);
 * p.add_(update, alpha=-lr_adj)) with the reference's CPU rounding: reduced
 * dtypes round alpha to the dtype, and round the product first when the
 * update came back transposed (rows > cols); fp32 is one fused multiply-add.
 * update: numel bf16 values in the parameter's layout. */
typedef struct gefen_muon_apply_task {
    void* p;
    const void* update;
    int64_t numel;
    int32_t param_dtype;
    int32_t transposed;
    double lr;
    double weight_decay;
    double adjusted_lr;
} gefen_muon_apply_task;

int gefen_muon_apply_tasks(const gefen_muon_apply_task* tasks, int ntasks, gefen_stream_t stream);

/* The last Newton-Schulz product of a stack applied as GefenMuon's parameter
 * update instead of being stored (no single reference counterpart: it is
 * gefen_muon.py:47 followed by gefen_muon.py:325-329 in one pass, so the update
 * is never written to memory and read back).  For each matrix i of the stack,
 *   U_i = bf16(alpha * A_i @ B_i^T + beta * D_i)
 * as gefen_gemm_bf16_nt_batched forms it (D given as its transpose d_t [n, m]),
 * and parameter tasks[i].p (numel m * n; layout U_i, or U_i^T when
 * tasks[i].transposed) is updated exactly as gefen_muon_apply_tasks updates it
 * with update = U_i (tasks[i].update is not read).  All tasks share one
 * parameter dtype and orientation; parameters are 8-element aligned. */
int gefen_gemm_bf16_nt_batched_apply(const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
                                     int64_t stride_b, const void* d_t, int64_t ldd, int64_t stride_d, int batch,
                                     int m, int n, int k, double alpha, double beta,
                                     const gefen_muon_apply_task* tasks, gefen_stream_t stream);

/* ------------------------------------------------------------------ first step
 * Replaces gefen_exact_histogram_cuda (exact_histogram_fused.py:10-58,
 * exact_histogram_fused_kernel.cu:131-160): per block absmax normalisation,
 * bin = clamp(floor((x + 1) / f32(2/bins)), 0, bins-1) as gefen.py:350-366;
 * bin_counts (int64, bins <= 4096) is accumulated (+=). */
int gefen_exact_histogram(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                          int64_t* bin_counts, int bins, gefen_stream_t stream);

/* acc[b] = f32(acc[b] + f32(counts[b])): the fp32 host accumulation of
 * gefen.py:331, 347 performed on the device. */
int gefen_accumulate_counts(float* acc, const int64_t* counts, int bins, gefen_stream_t stream);

/* Exact DP codebook (quantization.py:206-258, gefen.py:373-399) of a 4096-bin
 * fp32 histogram, on the device.  workspace: gefen_exact_dp_workspace_size() bytes. */
size_t gefen_exact_dp_workspace_size(int bins, int codebook_size);
int gefen_exact_dp(const float* counts, int bins, int codebook_size, int force_endpoints,
                   float* codebook_out, void* workspace, gefen_stream_t stream);

/* Replaces average_adjacent_log_block_mean_difference_cuda (period_variance.py:127-161,
 * period_variance_kernel.cu:320-396): out[0] = mean_j |m_{j+1} - m_j| of the
 * block means of log(x + epsilon), out[1] = count of x + epsilon <= 0 (the
 * caller raises when it is non-zero).  x = f64(f32(v)) if input_is_squared,
 * else f64(f32(v))^2.  out: 2 doubles of device memory. */
int gefen_average_adjacent_log_block_mean_difference(const void* values, int dtype, int64_t numel,
                                                     int64_t period, int input_is_squared,
                                                     double epsilon, double* out,
                                                     gefen_stream_t stream);

/* All period scores of one gradient at once (partitioning.py:119-167): for each
 * divisor divs[d] (host array), scores[d] as above; scores[ndiv] = invalid count.
 * mode 1 squares in fp32 first (Gefen._predict_period_from_grad_sq,
 * gefen.py:812-813); mode 0 / 2 as input_is_squared true / false.
 * workspace: gefen_period_scores_workspace_size() bytes. */
size_t gefen_period_scores_workspace_size(int64_t numel, const int64_t* divs, int ndiv);
int gefen_period_scores(const void* values, int dtype, int64_t numel, const int64_t* divs,
                        int ndiv, int mode, double epsilon, double* scores, void* workspace,
                        gefen_stream_t stream);

/* Replace average_within_block_variance_cuda and
 * average_within_block_coefficient_of_variation_cuda (period_variance.py:12-124,
 * period_variance_kernel.cu:177-318).  out: variance -> out[0] = sqrt(mean of
 * block variances); CoV -> out[0] = mean std/mean over blocks with a positive
 * mean, out[1] = count of such blocks, out[2] = count of negative means. */
int gefen_average_within_block_variance(const void* values, int dtype, int64_t numel,
                                        int64_t period, int input_is_squared, double* out,
                                        gefen_stream_t stream);
int gefen_average_within_block_coefficient_of_variation(const void* values, int dtype,
                                                        int64_t numel, int64_t period,
                                                        int input_is_squared, double* out,
                                                        gefen_stream_t stream);

/* Replace gefen_lloyd_accumulate_cuda and gefen_lloyd_mse_cuda (lloyd_max_fused.py:10-143,
 * lloyd_max_fused_kernel.cu:244-356): block absmax normalisation, nearest
 * codeword; sums (f32) / counts (int64) and the two squared-error sums (f32)
 * are accumulated (+=). */
int gefen_lloyd_accumulate(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                           const float* codebook, int codebook_size, float* sums, int64_t* counts,
                           gefen_stream_t stream);
int gefen_lloyd_mse(const void* grad, int grad_dtype, int64_t numel, int64_t period,
                    const float* old_codebook, const float* new_codebook, int codebook_size,
                    float* mse_normalized_sum, float* mse_original_sum, gefen_stream_t stream);

/* ------------------------------------------------------------------ Newton-Schulz GEMM
 * Replaces the three bf16 products of each Newton-Schulz iteration
 * (gefen_muon.py:39-47: X @ X.T, torch.addmm(A, A, A, beta=b, alpha=c),
 * torch.addmm(X, B, X, beta=a)), which the reference leaves to torch / the
 * vendor BLAS: C = alpha * A @ op(B) + beta * D with fp32 accumulation on MFMA
 * and one rounding to bf16.  A: [m, k] row-major; op(B) = B^T for B [n, k]
 * row-major (b_kcontig = 1) or B for B [k, n] row-major (b_kcontig = 0);
 * C, D: [m, n] row-major; D is not read when beta == 0.  All bf16. */
int gefen_gemm_bf16(const void* a, int64_t lda, const void* b, int64_t ldb, int b_kcontig, void* c,
                    int64_t ldc, const void* d, int64_t ldd, int m, int n, int k, double alpha, double beta,
                    gefen_stream_t stream);

/* Batched form of the same products for many same-shaped matrices at once
 * (the reference runs them one tensor at a time, gefen_muon.py:302-329), all
 * as A @ B^T: for b < batch,
 *   C_b = alpha * A_b @ B_b^T + beta * D_b,  A_b [m, k], B_b [n, k], C_b, D_b [m, n]
 * row-major bf16 with matrix strides stride_* (elements); fp32 accumulation on
 * MFMA, one rounding to bf16.  ct (optional, may be NULL) receives C_b^T
 * [n, m].  d_transposed = 1: d holds D_b^T [n, m] (row stride ldd), which the
 * kernel reads four rows at a time (the Gram matrix is its own transpose, and
 * Newton-Schulz keeps X^T beside X).  symmetric = 1 declares C_b symmetric
 * (m == n, e.g. X X^T, or
 * b A + c A A for a symmetric A): only tiles on and above the diagonal are
 * computed and mirrored (ct must then be NULL: C^T = C).  c may be NULL for a
 * non-symmetric product when ct is given (only C^T is written).  m and n must
 * be multiples of 256, k a multiple of 64,
 * rows 16-byte aligned (else ValueError; gefen_gemm_bf16 takes any shape). */
int gefen_gemm_bf16_nt_batched(const void* a, int64_t lda, int64_t stride_a, const void* b, int64_t ldb,
                               int64_t stride_b, void* c, int64_t ldc, int64_t stride_c, void* ct,
                               int64_t ldct, int64_t stride_ct, const void* d, int64_t ldd, int64_t stride_d,
                               int d_transposed, int batch, int m, int n, int k, double alpha, double beta,
                               int symmetric, gefen_stream_t stream);

/* The Gram product of Newton-Schulz (A = X @ X.T, gefen_muon.py:41) from X^T
 * alone: for b < batch, C_b = bf16(alpha * X_b @ X_b^T) [m, m], with X_b^T given
 * row-major [k, m] (row stride ldxt, matrix stride stride_xt); the result is
 * bit-identical to gefen_gemm_bf16_nt_batched(X, X, symmetric = 1), so
 * Newton-Schulz keeps only X^T between iterations.  m a multiple of 256, k of
 * 64, k * ldxt * 2 < 2^31, rows 16-byte aligned (else ValueError). */
int gefen_gram_bf16_batched(const void* xt, int64_t ldxt, int64_t stride_xt, void* c, int64_t ldc,
                            int64_t stride_c, int batch, int m, int k, double alpha, gefen_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* GEFEN_HIP_H */

/*
 * dmuon_amd.h -- C ABI of libdmuon_amd.so, the MI355X (gfx950) kernels behind the owner-rank
 * Muon update of X-Square-Robot/dmuon.
 *
 * Conventions (all entry points):
 *   - Every pointer is a device pointer unless stated otherwise; outputs are caller-allocated
 *     and written in place.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t passed as void*; NULL is the
 *     default stream). No entry point synchronises the host and none allocates device memory
 *     (scratch is the caller's `workspace`).
 *   - Return value: 0 on success, nonzero on a rejected argument or a failed launch; the text
 *     of the last error on the calling thread is returned by dmuon_last_error().
 *   - bf16 matrices are row-major with 16-byte aligned base pointers and leading dimensions
 *     that are multiples of 8 elements. Batched operands are [batch][rows][ld] with a batch
 *     stride in elements.
 *   - Per-matrix user tensors (gradients, momentum buffers, weights, outputs) are passed as
 *     DEVICE arrays of `batch` pointers, because they are separate allocations.
 *
 * Reference interfaces replaced (paths relative to the dmuon source tree):
 *   dmuon_syrk               dmuon/optim/syrk_dispatch.py:582-651   syrk_or_cublas(A, D, B, C,
 *                                                                   alpha, beta, diag_add) on the
 *                                                                   fp16 operands of
 *                                                                   newton_schulz.py:376-433
 *                            dmuon/kernels/syrk_sm80.py:465-569     syrk_sm80(...) kernel call
 *   dmuon_syrk_workspace_size (the padded path's scratch for shapes syrk_or_cublas hands to
 *                            cuBLAS, syrk_dispatch.py:644-651)
 *   dmuon_ns_gemm            dmuon/optim/newton_schulz.py:268-270   X = a*X + B @ X
 *                            dmuon/optim/newton_schulz.py:405-410   X = Q @ X (restart)
 *   dmuon_ns_gemm_final      dmuon/optim/newton_schulz.py:270-273,446 + dmuon/optim/muon.py:1728-1740
 *                                                                   last NS product fused with
 *                                                                   W *= 1-lr*wd; W += -lr*s*U
 *   dmuon_syrk_bf16, dmuon_ns_gemm_bf16, dmuon_ns_gemm_final_bf16: the three above with bf16
 *                            operands (kept from ABI 103)
 *   dmuon_muon_pre           dmuon/optim/muon.py:1683-1694 + newton_schulz.py:257-266
 *                                                                   momentum, Nesterov, float(),
 *                                                                   orientation, cast, ||X||^2
 *   dmuon_norm_finalize      dmuon/optim/newton_schulz.py:265       X / (X.norm() + eps)
 *   dmuon_muon_update        dmuon/optim/muon.py:1728-1740          owned.mul_/add_ update
 *   dmuon_muon_stage_group / dmuon_muon_apply_group  the two halves of dmuon_muon_step_group
 *   dmuon_muon_step_group    dmuon/optim/muon.py:1683-1740          one owner's per-param Muon
 *                                                                   math for `batch` same-shape
 *                                                                   params (direct NS, T steps)
 *                            + dmuon/_backends/fsdp2/group.py:766-781 owner publish copy-in
 *   dmuon_newton_schulz_group dmuon/optim/newton_schulz.py:225-273  direct_newton_schulz(G) /
 *                            dmuon/optim/newton_schulz.py:333-448  gram_newton_schulz(G) for
 *                                                                   `batch` same-shape matrices
 *   dmuon_adamw_multi        dmuon/optim/muon.py:1857-1916          _adamw_update_batch: the
 *                                                                   torch._foreach AdamW of one
 *                                                                   (step, dtype) bucket
 *   dmuon_segmented_l2_norm_sq dmuon/csrc/fast_clip_kernel.cu:116-155 segmented_l2_norm_sq
 *   dmuon_segmented_scale    dmuon/csrc/fast_clip_kernel.cu:157-195 segmented_scale
 *                            (both bound by dmuon/fast_clip.py:267,301)
 */
#ifndef DMUON_AMD_H_
#define DMUON_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DMUON_DTYPE_F32 0
#define DMUON_DTYPE_BF16 1
#define DMUON_DTYPE_F16 2 /* 16-bit product operands only (dmuon_syrk, dmuon_ns_gemm*) */

/* Newton-Schulz device algorithms (the `backend` argument below). */
#define DMUON_NS_DIRECT 0 /* X <- a X + (b A + c A A^T) X, A = X X^T, every step */
#define DMUON_NS_GRAM 1   /* Gram-space iteration with restarts (gram_newton_schulz) */

/* Text of the last error raised on this thread ("" if none). */
const char* dmuon_last_error(void);

/* ABI version (major*100 + minor): DMUON_ABI_VERSION of the header the library was built with. */
#define DMUON_ABI_VERSION 108
int dmuon_abi_version(void);

/*
 * Launch profiler (no reference counterpart; measurement support for the benchmark harness).
 * While enabled, every kernel launched by dmuon_muon_step_group / dmuon_newton_schulz_group /
 * dmuon_adamw_multi / the segmented clip entry points is bracketed by hipEvents on its stream.
 * dmuon_profile_collect synchronises on those events and returns, per kernel class (0 pre,
 * 1 norm-finalize, 2 SYRK X X^T (Gram: R = X X^T), 3 SYRK-poly (Gram: the m x m products),
 * 4 NS GEMM (Gram: restart Q X), 5 final GEMM + update, 6 AdamW, 7 segmented clip), the
 * summed milliseconds, launch counts, useful FLOPs and algorithmic bytes, then clears the
 * records. n_classes must be >= 8. Not thread-safe.
 */
int dmuon_profile_enable(int on);
int dmuon_profile_collect(double* ms, int64_t* launches, double* flops, double* bytes,
                          int n_classes);

/*
 * dst = src, `bytes` bytes (no reference counterpart; measurement support for the benchmark
 * harness): one 16-byte chunk per thread with non-temporal loads and stores, the pattern that
 * reaches this HBM's streaming ceiling, so bench.py can report the bandwidth-bound kernels
 * against what the device actually sustains. Both buffers 16-byte aligned, `bytes` a multiple
 * of 16, no overlap. Asynchronous on `stream`.
 */
int dmuon_stream_copy(const void* src, void* dst, int64_t bytes, void* stream);

/*
 * D[l] = alpha * s_l * A[l] @ B[l]^T + beta * C[l] + diag_add * I     for l < batch
 * where s_l = alpha_dev[l] if alpha_dev != NULL else 1, on 16-bit operands of type `dtype`
 * (DMUON_DTYPE_F16, as gram_newton_schulz calls syrk_or_cublas on X.half(), or
 * DMUON_DTYPE_BF16); fp32 accumulation, the epilogue in fp32, D rounded to `dtype`.
 * A, B: [M][K] (row stride lda / ldb); C, D: [M][M]. B == NULL means B = A. The result must be
 * symmetric (always true for B = A; the caller guarantees it when B != A, as syrk_or_cublas
 * requires). Only the upper triangle of tiles is computed; the lower triangle is written as its
 * mirror. C may be NULL (then beta is ignored) and may alias A, but D must not alias A, B or C.
 * tile: 0 (automatic), 128 or 256 (output tile edge of the plan: padding and operand
 * alignment). A launch of a 128-tile plan may run on 64- or 256-tiles when those fit the device
 * better, with the same bits as the 128-tile kernel.
 * Any M >= 0 and K >= 0 are accepted. When M is a multiple of the tile, K of 64, and every base
 * is 16-byte aligned with leading dimensions and batch strides that are multiples of 8, the
 * kernel reads the operands in place and `workspace` may be NULL; otherwise the call runs on
 * zero-padded copies in `workspace` (device memory of dmuon_syrk_workspace_size bytes, at least
 * 16-byte aligned; contents need no initialisation) and copies the M x M result into D.
 */
int dmuon_syrk(int dtype, const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
               int64_t strideB, const void* C, int64_t ldc, int64_t strideC, void* D, int64_t ldd,
               int64_t strideD, int M, int K, int batch, float alpha, float beta, float diag_add,
               const float* alpha_dev, int tile, void* workspace, int64_t workspace_bytes,
               void* stream);

/* Bytes of workspace dmuon_syrk needs for these arguments (0 when it reads the operands in
 * place). Host-only; the pointers are inspected for alignment, never dereferenced. */
int dmuon_syrk_workspace_size(int dtype, const void* A, int64_t lda, int64_t strideA,
                              const void* B, int64_t ldb, int64_t strideB, const void* C,
                              int64_t ldc, int64_t strideC, const void* D, int64_t ldd,
                              int64_t strideD, int M, int K, int batch, int tile,
                              int64_t* workspace_bytes);

/* dmuon_syrk with bf16 operands, tile 128 or 256, M % tile == 0, K % 64 == 0 and aligned
 * operands (no padded path). */
int dmuon_syrk_bf16(const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
                    int64_t strideB, const void* C, int64_t ldc, int64_t strideC, void* D,
                    int64_t ldd, int64_t strideD, int M, int K, int batch, float alpha, float beta,
                    float diag_add, const float* alpha_dev, int tile, void* stream);

/*
 * One Newton-Schulz step X' = s_l * (P @ X + beta * X) for l < batch, given P ([M][M], the
 * polynomial b*A + c*A@A of A = X X^T) and XT = X^T ([N][M]); s_l = alpha * alpha_dev[l] (or
 * alpha). Writes X' into Xout ([M][N], may alias X) and, when XTout != NULL, X'^T into XTout
 * ([N][M], must not alias XT). XT == NULL: the product reads X ([M][N] as stored, like the
 * reference's torch.mm(P, X)) as its B operand through transposing LDS loads -- same result,
 * no transposed copy needed; Xout must then not alias X. Operands, X, Xout and XTout are
 * 16-bit words of `dtype` (DMUON_DTYPE_F16 or DMUON_DTYPE_BF16). tile 128 or 256;
 * M % tile == 0, N % tile == 0 (the NS planner pads).
 */
int dmuon_ns_gemm(int dtype, const void* P, int64_t ldp, int64_t strideP, const void* XT,
                  int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx, int64_t strideX,
                  void* Xout, int64_t ldxo, int64_t strideXo, void* XTout, int64_t ldxto,
                  int64_t strideXTo, int M, int N, int batch, float alpha, float beta,
                  const float* alpha_dev, int tile, void* stream);
/* dmuon_ns_gemm with bf16 operands */
int dmuon_ns_gemm_bf16(const void* P, int64_t ldp, int64_t strideP, const void* XT, int64_t ldxt,
                       int64_t strideXT, const void* X, int64_t ldx, int64_t strideX, void* Xout,
                       int64_t ldxo, int64_t strideXo, void* XTout, int64_t ldxto,
                       int64_t strideXTo, int M, int N, int batch, float alpha, float beta,
                       const float* alpha_dev, int tile, void* stream);

/*
 * Last Newton-Schulz step fused with the Muon weight update. U = s_l*(P @ X + beta*X) is formed
 * in fp32 for the m_real x n_real corner of the padded [M][N] problem and, in the original
 * orientation (transposed != 0: the original matrix is U^T, n_real x m_real):
 *   out_ptrs != NULL: out[l] <- U                      (dtype out_dtype)
 *   w_ptrs   != NULL: W[l] <- round(W*decay) - lrs*U    (dtype w_dtype; decay == 1 skips the
 *                                                       decay rounding)
 *   pub_ptrs != NULL: pub[l] <- round(new W[l])         (dtype pub_dtype; needs w_ptrs): the
 *     forward copy of an owner's master weight, written in the same pass (the reference copies
 *     _owned_data into the packed forward buffer afterwards, fsdp2/group.py:766-781)
 * P, XT and X are 16-bit words of `dtype` (DMUON_DTYPE_F16 or DMUON_DTYPE_BF16); XT may be NULL
 * (X is then the B operand, as in dmuon_ns_gemm). U stays fp32
 * up to the update (W <- round(fma(-lrs, U, round(W*decay))): one rounding, as add_(alpha=)).
 */
int dmuon_ns_gemm_final(int dtype, const void* P, int64_t ldp, int64_t strideP, const void* XT,
                        int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx,
                        int64_t strideX, int M, int N, int batch, float alpha, float beta,
                        const float* alpha_dev, int m_real, int n_real, int transposed,
                        void* const* out_ptrs, int out_dtype, void* const* w_ptrs, int w_dtype,
                        void* const* pub_ptrs, int pub_dtype, float decay, float lrs, int tile,
                        void* stream);
/* dmuon_ns_gemm_final with bf16 operands */
int dmuon_ns_gemm_final_bf16(const void* P, int64_t ldp, int64_t strideP, const void* XT,
                             int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx,
                             int64_t strideX, int M, int N, int batch, float alpha, float beta,
                             const float* alpha_dev, int m_real, int n_real, int transposed,
                             void* const* out_ptrs, int out_dtype, void* const* w_ptrs,
                             int w_dtype, void* const* pub_ptrs, int pub_dtype, float decay,
                             float lrs, int tile, void* stream);

/* Number of partial sums per matrix that dmuon_muon_pre writes for a padded Rp x Cp matrix. */
int dmuon_muon_pre_partials(int Rp, int Cp);

/*
 * Momentum + Nesterov + NS-input staging for `batch` rows x cols matrices:
 *   buf <- g (first_step) | fp32(mu*buf) + g        (buf_ptrs may be NULL: ns_in = g)
 *   ns_in = g + mu*buf (nesterov) | buf
 *   Y[l]  <- bf16(ns_in)    [Rp][ldy]  zero outside rows x cols    (Y NULL: not written)
 *   YT[l] <- bf16(ns_in)^T  [Cp][ldyt] zero outside cols x rows    (YT NULL: not written;
 *                                                                   one of the two is needed)
 *   partials[l][p] <- partial sums of ns_in^2 (fp32), p < dmuon_muon_pre_partials(Rp, Cp)
 * g dtype: g_dtype; buf: fp32. Rp, Cp: multiples of 64, Rp >= rows, Cp >= cols.
 */
int dmuon_muon_pre(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs, void* Y, int64_t ldy,
                   int64_t strideY, void* YT, int64_t ldyt, int64_t strideYT, float* partials,
                   int rows, int cols, int Rp, int Cp, int batch, float mu, int first_step,
                   int nesterov, void* stream);

/* scale[l] = 1 / (sqrt(sum_p partials[l][p]) + eps); scale_sq[l] = scale[l]^2. Deterministic. */
int dmuon_norm_finalize(const float* partials, int nparts, int batch, float eps, float* scale,
                        float* scale_sq, void* stream);

/* W[l] <- round(W[l]*decay) - lrs*U[l] elementwise over numel elements (decay == 1: no decay). */
int dmuon_muon_update(void* const* w_ptrs, int w_dtype, const void* const* u_ptrs, int u_dtype,
                      int64_t numel, int batch, float decay, float lrs, void* stream);

/*
 * Planning for a group of `batch` same-shape rows x cols matrices: NS dims m = min, n = max,
 * chosen output tile (tile_req 0 = automatic, else 128 or 256), padded m_pad / n_pad and the
 * workspace bytes dmuon_muon_step_group / dmuon_newton_schulz_group need for `backend` (per
 * group member two m_pad x n_pad fp16 matrices, X and the next X, and two m_pad x m_pad ones
 * for DMUON_NS_DIRECT, five for DMUON_NS_GRAM). A padded matrix holds at most 2^30 values
 * (m_pad * n_pad; the NS products read X k-major through 32-bit offsets): larger shapes are
 * refused with an error. Host-only.
 */
int dmuon_ns_plan(int rows, int cols, int batch, int tile_req, int num_cus, int backend,
                  int* tile, int* m_pad, int* n_pad, int64_t* workspace_bytes);

/*
 * Full Muon update for `batch` params of one oriented NS shape (one owner's group): the first
 * batch - n_transposed are rows x cols, the last n_transposed are cols x rows (their momentum
 * buffers, weights and forward copies too). Both orientations share the m x n NS products
 * (m = min(rows, cols)); each param's update is written in its own orientation. Square shapes
 * ignore the split. Steps:
 *   momentum (+Nesterov), normalise, T Newton-Schulz steps with per-step coefficients
 *   coeffs[3*t .. 3*t+2] = (a, b, c) (HOST array), then
 *   W <- round(W*(1 - lr*wd)) - lr*0.2*sqrt(max(rows, cols)) * U    (decay skipped if wd <= 0)
 * and, when pub_ptrs != NULL, pub[l] <- round_to_pub_dtype(new W[l]) in the same epilogue (the
 * owner's forward copy when W is a master in another dtype; NULL when W is the forward tensor).
 * backend DMUON_NS_DIRECT: each step is SYRK (A = X X^T) -> SYRK-poly (b*A + c*A A^T) -> GEMM
 *   (a*X + P X) on fp16 MFMA (direct_newton_schulz, newton_schulz.py:225-273).
 * backend DMUON_NS_GRAM: gram_newton_schulz (newton_schulz.py:333-448): R = X X^T once; per step
 *   P = a I + b R + c R R, Q <- P Q, R <- (R P) P, all m x m; at each step index listed in
 *   restarts[0 .. n_restarts-1] (HOST array; index 0 ignored) X <- Q X and R = X X^T again;
 *   finally U = Q X. Fewer flops than direct when n > m.
 * est_ptrs (optional, device array of `batch` pointers to one fp32 each, kept by the caller per
 *   param across steps, initially 0): single-pass staging. Each holds the param's previous
 *   1 / (||ns_in|| + eps); the momentum pass then also writes the fp16 NS operand with that
 *   scale, the first products correct it by r = scale / est when r is within [1/4, 4], and a
 *   param outside that range (or with est <= 0) is staged again exactly; *est_ptrs[l] is
 *   updated in place. NULL: two staging passes, the operand always exactly scaled. The results
 *   of the two modes differ by the fp16 rounding of that operand. No reference counterpart
 *   (the reference stages per param with torch ops).
 * workspace: device memory of at least the planned bytes; its contents need no initialisation.
 */
int dmuon_muon_step_group(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                          float* const* est_ptrs, void* const* w_ptrs, int w_dtype,
                          void* const* pub_ptrs, int pub_dtype, int rows, int cols, int batch,
                          int n_transposed, double lr, double mu, double wd, int nesterov,
                          int first_step, const float* coeffs, int T, int backend,
                          const int* restarts, int n_restarts, float eps, void* workspace,
                          int64_t workspace_bytes, int tile, void* stream);

/*
 * dmuon_muon_step_group in two halves, for callers that overlap the bandwidth-bound half of one
 * group with the MFMA-bound half of another on two streams (each half enqueues on its own
 * stream; order them with events):
 *   stage: momentum (+Nesterov), the Frobenius norm and the NS operands of `batch` params,
 *          written into `workspace`;
 *   apply: the NS products from that staged workspace and the fused weight update (+ optional
 *          forward copy), as dmuon_muon_step_group's second half.
 * Both calls of one group must pass the same rows, cols, batch, n_transposed, backend, tile and
 * workspace; the workspace must not be staged again before its apply has run. Results equal
 * dmuon_muon_step_group's bit for bit. No reference counterpart (the reference runs the step
 * per parameter on one stream); it serves the same seam, muon.py:1683-1740.
 */
int dmuon_muon_stage_group(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                           float* const* est_ptrs, int rows, int cols, int batch,
                           int n_transposed, double mu, int nesterov, int first_step,
                           int backend, float eps, void* workspace, int64_t workspace_bytes,
                           int tile, void* stream);
int dmuon_muon_apply_group(void* const* w_ptrs, int w_dtype, void* const* pub_ptrs,
                           int pub_dtype, int rows, int cols, int batch, int n_transposed,
                           double lr, double wd, const float* coeffs, int T, int backend, const int* restarts,
                           int n_restarts, void* workspace, int64_t workspace_bytes, int tile,
                           void* stream);

/*
 * dmuon_muon_step_group for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference (its step allocates through torch). The arguments are dmuon_muon_step_group's minus
 * the workspace: the scratch is one static device array of DMUON_NOALLOC_SCRATCH_BYTES per GPU
 * (512 MiB: any single Muon matrix of Llama-3-8B in either NS form; a GPU holds it from the first
 * resolution of its address, below, until the process ends -- the library's other entry points
 * do not load it), and a group whose planned workspace (dmuon_ns_plan) exceeds it is rejected
 * with an error before any launch. The call
 * allocates nothing: no hipMalloc / hipFree, no library allocation, no profiler events. Every
 * call on one GPU shares that GPU's array and leaves its contents behind; a step needs none of
 * them (it writes every scratch byte it reads), but calls that overlap on one GPU (two streams,
 * two threads) race. `stream` must belong to the current device. Results equal
 * dmuon_muon_step_group's bit for bit. The scratch address of each GPU is resolved once, by
 * dmuon_noalloc_init or the first call on that GPU; that first resolution loads the code object
 * that holds the array (reserving the array on that GPU), so a caller that captures the step must
 * make it happen before capturing (a first call on a capturing stream is refused with an error).
 */
#define DMUON_NOALLOC_SCRATCH_BYTES (512LL << 20)
int dmuon_muon_step_group_noalloc(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                                  float* const* est_ptrs, void* const* w_ptrs, int w_dtype,
                                  void* const* pub_ptrs, int pub_dtype, int rows, int cols,
                                  int batch, int n_transposed, double lr, double mu, double wd,
                                  int nesterov, int first_step, const float* coeffs, int T, int backend,
                                  const int* restarts, int n_restarts, float eps, int tile,
                                  void* stream);

/* Set-up of dmuon_muon_step_group_noalloc on the current device (no counterpart in the
 * reference; for the same callers, those that cannot allocate): resolves the device address of
 * this GPU's scratch array outside any capture and returns it (*scratch_out, may be NULL) with
 * its size in bytes (*scratch_bytes, may be NULL). Call it once per device before capturing the
 * allocation-free step. Allocates no device memory besides the array itself, which the loader
 * reserves on this GPU with its code object at the first resolution. */
int dmuon_noalloc_init(void** scratch_out, int64_t* scratch_bytes);

/* direct_newton_schulz / gram_newton_schulz (by `backend`, as above) for `batch` matrices of one
 * oriented shape (the last n_transposed are cols x rows, as above): out[l] <- NS(g[l]). */
int dmuon_newton_schulz_group(void* const* g_ptrs, int g_dtype, void* const* out_ptrs,
                              int out_dtype, int rows, int cols, int batch, int n_transposed,
                              const float* coeffs,
                              int T, int backend, const int* restarts, int n_restarts, float eps,
                              void* workspace, int64_t workspace_bytes, int tile, void* stream);

/*
 * Decoupled AdamW over n tensors in one pass (one bucket of the reference's
 * _adamw_update_batch: same step count, same param dtype, same grad dtype).
 *   p_ptrs, g_ptrs, m_ptrs, v_ptrs: DEVICE arrays of n int64 addresses of the contiguous
 *     param, grad, exp_avg and exp_avg_sq tensors; p, exp_avg, exp_avg_sq have p_dtype.
 *   pub_ptrs: NULL, or a DEVICE array of n addresses of forward copies that receive
 *     round_to_pub_dtype(new p) in the same pass (an owner's master -> forward publish).
 *   offsets: DEVICE array of n+1 int64 prefix sums of the tensor sizes (offsets[0] = 0,
 *     offsets[n] = total).
 *   Scalars, as the reference derives them in double and hands them to the foreach ops:
 *     wd_scale = 1 - lr*wd (applied only if apply_wd), beta1, alpha1 = 1 - beta1, beta2,
 *     alpha2 = 1 - beta2, bc2_sqrt = sqrt(1 - beta2^step), eps, neg_step = -lr/(1 - beta1^step).
 * Per element: p = R(p*wd_scale); m = R(R(m*beta1) + alpha1*g); v = R(R(v*beta2) + alpha2*g*g);
 * d = R(R(R(sqrt(v))/bc2_sqrt) + eps); p = R(p + neg_step*(m/d)), R = rounding to p_dtype.
 */
int dmuon_adamw_multi(const int64_t* p_ptrs, const int64_t* g_ptrs, const int64_t* m_ptrs,
                      const int64_t* v_ptrs, const int64_t* pub_ptrs, const int64_t* offsets,
                      int n, int64_t total, int p_dtype, int g_dtype, int pub_dtype, int apply_wd,
                      float wd_scale, float beta1, float alpha1, float beta2, float alpha2,
                      float bc2_sqrt, float eps, float neg_step, void* stream);

/*
 * Segmented gradient clipping, the two device operations of the reference's fast-clip path,
 * with its argument list. Tensor t (of n) is the contiguous device buffer at address ptrs[t]
 * with numels[t] elements of dtype dtypes[t] (DMUON_CLIP_*: the reference's codes) belonging
 * to segment segments[t]. Job j covers elements [job_offsets[j], job_offsets[j] + chunk_size)
 * of tensor job_tensor_ids[j], clipped to its size; every array is DEVICE-resident (int64 or
 * int32 as typed) and the job table must reference valid tensors only.
 *   dmuon_segmented_l2_norm_sq: local_sq[segments[t]] += sum of float(x)^2 over every job
 *     (fp32 device array, caller-initialised; float atomics, so the addition order between
 *     jobs is not fixed).
 *   dmuon_segmented_scale: x <- dtype(float(x) * coefs[segments[t]]) in place.
 */
#define DMUON_CLIP_F32 0
#define DMUON_CLIP_F16 1
#define DMUON_CLIP_BF16 2
int dmuon_segmented_l2_norm_sq(const int64_t* ptrs, const int64_t* numels, const int32_t* dtypes,
                               const int32_t* segments, const int32_t* job_tensor_ids,
                               const int64_t* job_offsets, int64_t n_jobs, int64_t chunk_size,
                               float* local_sq, void* stream);
int dmuon_segmented_scale(const int64_t* ptrs, const int64_t* numels, const int32_t* dtypes,
                          const int32_t* segments, const int32_t* job_tensor_ids,
                          const int64_t* job_offsets, int64_t n_jobs, int64_t chunk_size,
                          const float* coefs, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DMUON_AMD_H_ */

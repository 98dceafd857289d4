// Internal declarations shared by the HIP translation units of libdmuon_amd.
// Not part of the public C-ABI (that is include/dmuon_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmuon {

// dtype codes used across the C-ABI (mirrors DMUON_DTYPE_* in dmuon_amd.h); DT_F16 only names
// 16-bit product operands (SYRK / NS-GEMM entry points).
enum DType : int { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

// Epilogue of the NT-form MFMA product  acc[i][j] = sum_k A[i][k] * B[j][k].
//   EPI_SYM   D = s*acc + beta*C + diag*I          (symmetric result, upper tiles + mirror)
//   EPI_NS    D = s*(acc + beta*C), also D^T        (Newton-Schulz X <- a*X + B*X step)
//   EPI_FINAL U = s*(acc + beta*C) -> out[] and/or W <- W*decay - lrs*U, original orientation
enum EpiMode : int { EPI_SYM = 0, EPI_NS = 1, EPI_FINAL = 2 };

// 16-bit element type of the NT product operands, addend and outputs
enum { ELT_BF16 = 0, ELT_F16 = 1 };

struct NtArgs {
  const uint16_t* A; long long lda, sA;   // elt [L][M][K], row stride lda, batch stride sA
  const uint16_t* B; long long ldb, sB;   // elt [L][N][K]
  int M, N, K, L;                         // multiples of the tile sizes (host pads)
  // K elements the loop multiplies (0: K), a multiple of 64: the operands are zero-padded
  // past it, so the slices beyond add nothing (an m x m product padded to a tile multiple
  // loops over m rounded up to 64 only)
  int k_loop;
  int mt, nt, tiles_per_mat, tri;         // tile grid; tri: upper-triangle tiles of an MxM result
  int mode;
  float alpha, beta, diag;
  const float* alpha_dev;                 // optional per-matrix multiplier of alpha
  const uint16_t* C; long long ldc, sC;   // optional elt [L][M][N] addend
  uint16_t* D; long long ldd, sD;         // elt [L][M][N]
  uint16_t* DT; long long lddt, sDT;      // elt [L][N][M] (EPI_NS, optional)
  void* const* out_ptrs; int out_dtype;   // EPI_FINAL: per-matrix U outputs (original shape)
  void* const* w_ptrs; int w_dtype;       // EPI_FINAL: per-matrix weights updated in place
  void* const* pub_ptrs; int pub_dtype;   // EPI_FINAL: optional forward copies of the new W
  float decay, lrs;                       // W <- round(W*decay) - lrs*U   (decay==1: no decay rounding)
  int m_real, n_real, transposed;         // true NS dims; transposed: original = X^T (n_real x m_real)
  int n_flip;                             // the last n_flip matrices take the other orientation
  int elt;                                // ELT_BF16 / ELT_F16 (A, B, C, D, DT)
  int sym_exact;                          // EPI_SYM + tri: diagonal tiles stored exactly symmetric
  uint16_t* D2; float diag2;              // EPI_SYM + tri + sym_exact: also D2 = D + diag2 * I
  // K-loop rotation of an M x M product (K == M) whose addend C is one of its own operands
  // (C_IS_A: C is A, C_IS_B: C is B, the matrix symmetric): the slices of the 256-column block
  // that holds the tile's C values run last, so the epilogue reads C from lines the block has
  // just brought into L2. Per-element summation order depends only on the 256-block, so the
  // 128- and 256-tile kernels give the same bits for the same K (a K padded differently for the
  // two tile sizes moves the start).
  int c_in;
  // B stored k-major, [L][K][N] with row stride ldb (X itself rather than a transposed copy):
  // the kernels stage its slices as BK rows of the tile's N values and assemble the MFMA
  // operand with transposing LDS reads. C_IS_B then means C is B as stored.
  int b_kmajor;
  // EPI_SYM + tri + sym_exact, 256-tiles: how much of a diagonal tile's work below the diagonal
  // (whose values the epilogue drops) is skipped. DIAG_SKIP_NONE computes every block;
  // DIAG_SKIP_WAVES skips the two waves that hold no kept value; DIAG_SKIP_BLOCKS also skips the
  // 16x16 blocks strictly below the diagonal in the waves that straddle it. Same bits each way.
  int diag_skip;
  // 256-tiles: output rows from live_rows on and columns from live_cols on are padding that no
  // later product reads (every K loop stops before it; 0: none). A wave whose 128 x 64
  // sub-tile lies wholly in it does no MFMA work and stores nothing; the padding then holds
  // whatever it held.
  int live_rows, live_cols;
};
enum { DIAG_SKIP_NONE = 0, DIAG_SKIP_WAVES = 1, DIAG_SKIP_BLOCKS = 2 };
enum { C_NONE = 0, C_IS_A = 1, C_IS_B = 2 };

// Launches the NT MFMA kernel; picks the tile configuration from args (tile = 256 or 128).
hipError_t launch_nt(const NtArgs& a, int tile, hipStream_t stream);
// The logical tile the NT kernels give hardware block b of a launch of nb blocks (host copy of
// the device mapping, for tests: it must be a permutation of 0 .. nb - 1).
int nt_block_tile(int b, int nb);

// What one launch of the pre kernel does:
//   PRE_BF16  momentum update, bf16 ns_in into Y / YT, norm partials (direct NS staging)
//   PRE_NORM  momentum update and norm partials only
//   PRE_F16   after PRE_NORM + norm finalise: recompute ns_in from g and the updated buffer
//             and write fp16(kx * scale * ns_in) into Y / YT; no buffer write. With `restage`,
//             only the matrices whose flag is set (the others return at once)
//   PRE_EST   momentum update, norm partials and fp16(kx * est * ns_in) into Y / YT, est being
//             the matrix's previous 1/(||ns_in|| + eps) (*est_ptrs[l]); est <= 0: no copy
enum { PRE_BF16 = 0, PRE_NORM = 1, PRE_F16 = 2, PRE_EST = 3 };

struct PreArgs {
  void* const* g_ptrs; int g_dtype;       // per-matrix gradient (rows x cols, row-major)
  float* const* buf_ptrs;                 // per-matrix fp32 momentum buffer (rows x cols)
  uint16_t* Y; long long ldy, sY;         // 16-bit ns_in in the gradient's layout, padded [L][Rp][Cp]
  uint16_t* YT; long long ldyt, sYT;      // 16-bit ns_in transposed, padded [L][Cp][Rp]
  float* partials;                        // [L][blocks_per_mat] sum of squares of ns_in
  int rows, cols, Rp, Cp, L;
  float mu; int first_step, nesterov;
  int stage;                              // PRE_*
  const float* scale; float kx;           // PRE_F16: per-matrix 1/(||ns_in|| + eps), power of 2
  float* const* est_ptrs;                 // PRE_EST: per-matrix scale estimate (device float)
  const int* restage;                     // PRE_F16: optional per-matrix "copy needed" flags
  // copies not written (the consumer reads the other one): skip_y -- Y, skip_yt -- YT
  int skip_y, skip_yt;
};
hipError_t launch_pre(const PreArgs& a, hipStream_t stream);
int pre_blocks_per_mat(int Rp, int Cp);


// scale[l] = 1/(sqrt(sum partials[l]) + eps), scale_sq[l] = scale^2
hipError_t launch_norm_finalize(const float* partials, int nparts, int L, float eps,
                                float* scale, float* scale_sq, hipStream_t stream);

// The same, plus the correction of a copy staged with an estimated scale: with est_ptrs and
// est = *est_ptrs[l] > 0 and r = scale / est in [1/4, 4], ratio[l] = r, ratio_sq[l] = r^2 and
// restage[l] = 0 (the staged copy times r is the exactly scaled one); otherwise ratio = 1,
// ratio_sq = 1, restage = 1 (stage again with the exact scale). *est_ptrs[l] becomes scale.
hipError_t launch_norm_finalize_est(const float* partials, int nparts, int L, float eps,
                                    float* scale, float* scale_sq, float* const* est_ptrs,
                                    float* ratio, float* ratio_sq, int* restage,
                                    hipStream_t stream);

// dst[l][r][c] = r < rows && c < cols ? src[l][r][c] : 0 over rows_out x cols_out (16-bit)
// dst = src, n16 chunks of 16 bytes (both 16-byte aligned, not overlapping)
hipError_t launch_stream_copy(const void* src, void* dst, long long n16, hipStream_t stream);
hipError_t launch_pad_copy(const uint16_t* src, long long lds, long long ss, uint16_t* dst,
                           long long ldd, long long sd, int rows, int cols, int rows_out,
                           int cols_out, int L, hipStream_t stream);

struct UpdateArgs {
  void* const* w_ptrs; int w_dtype;
  const void* const* u_ptrs; int u_dtype;
  long long numel; int L;
  float decay, lrs;
};
hipError_t launch_update(const UpdateArgs& a, hipStream_t stream);

// Fused decoupled AdamW over n tensors concatenated into one index space of `total` elements.
// Arrays are device-resident; p/m/v share p_dtype, g has g_dtype.
struct AdamWArgs {
  const int64_t* p_ptrs; const int64_t* g_ptrs; const int64_t* m_ptrs; const int64_t* v_ptrs;
  const int64_t* pub_ptrs;                // optional forward copies of the new p (pub_dtype)
  const int64_t* offsets;                 // [n+1] prefix sums of the tensor sizes
  int n; long long total;
  int p_dtype, g_dtype, pub_dtype;
  int apply_wd;
  float wd_scale, beta1, alpha1, beta2, alpha2, bc2_sqrt, eps, neg_step;
  long long per_block;                    // set by launch_adamw
};
hipError_t launch_adamw(AdamWArgs a, hipStream_t stream);

// Segmented clip job table (device arrays, the reference's fast-clip layout).
struct ClipArgs {
  const int64_t* ptrs; const int64_t* numels; const int32_t* dtypes; const int32_t* segments;
  const int32_t* job_tensor_ids; const int64_t* job_offsets;
  long long n_jobs, chunk;
  float* local_sq;                        // sumsq: per-segment accumulators (added to)
  const float* coefs;                     // scale: per-segment coefficients
  long long piece;                        // scale: elements per block (set by launch_clip_scale)
};
hipError_t launch_clip_sumsq(const ClipArgs& a, hipStream_t stream);
hipError_t launch_clip_scale(ClipArgs a, hipStream_t stream);

}  // namespace dmuon

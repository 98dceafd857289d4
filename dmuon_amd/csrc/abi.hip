// extern "C" entry points of libdmuon_amd.so (declared in include/dmuon_amd.h): argument
// validation, workspace planning and the launch sequence of one Muon group step.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/dmuon_amd.h"
#include "dmuon_amd_internal.h"

using namespace dmuon;

// Scratch of dmuon_muon_step_group_noalloc: one static device array, of which the loader gives
// every GPU its own copy, held until the process ends. This file holds no kernels, so its code
// object -- the array with it -- is loaded onto a GPU by the first hipGetSymbolAddress there,
// not by the kernels of the other entry points. Host code never uses the array's name as an
// address (on the host it is a stand-in symbol): the device address of the current GPU's copy
// comes from hipGetSymbolAddress on the first call on that GPU and is kept per device
// (scratch_of_current_device).
static __device__ __align__(256) char scratch[DMUON_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return 1;
}

int check_launch(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool ld_ok(int64_t ld) { return ld > 0 && (ld % 8) == 0; }
bool stride_ok(int64_t s, int batch) { return batch <= 1 || (s >= 0 && (s % 8) == 0); }

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
int64_t align256(int64_t b) { return round_up(b, 256); }

// Diagonal-tile work skipped by the exactly symmetric products (NtArgs::diag_skip): the
// m x m polynomials (K = m) skip every 16x16 block below the diagonal, the products X X^T
// (K = n, up to 14336) none. Measured on the c5 step, same box, against no skipping anywhere:
// polynomial class -3.1 ms (-2%); for X X^T skipping only the two idle waves cost +0.7 ms and
// skipping blocks +1.6 ms (a diagonal tile that finishes early takes its CU out of step with
// the tiles that share its operand panels in L2).
constexpr int kDiagSkipPoly = DIAG_SKIP_BLOCKS;
constexpr int kDiagSkipGram = DIAG_SKIP_NONE;

// The products X' = P X (direct) and Q X (Gram) read X itself as their k-major B operand
// (transposing LDS reads) instead of a transposed copy: the staging writes one fp16 copy of
// ns_in (12 B per element, not 14), and X ping-pongs between two buffers (such a product reads
// the current X across the whole K range, so the new X cannot overwrite it). The k-major loads
// address a matrix's whole X through one 32-bit buffer range, so m_pad * n_pad * 2 < 2^31
// bytes: 2^30 fp16 values per padded matrix, which plan() enforces.
constexpr int64_t kMaxXBytes = int64_t(1) << 31;

// Power-of-two scale of the fp16 NS operand X, both backends (entries of the normalised X are at
// most 1; the scale keeps the typical ~1/sqrt(mn) entries out of the fp16 subnormal range)
constexpr float kNsKx = 4096.f;

struct Workspace {
  uint16_t *X, *X2, *Am, *Pm;
  // Gram backend only: the two slots of the accumulated polynomial Q (or its transpose), P R
  uint16_t *Q0, *Q1, *Wm;
  float *partials, *scale, *scale_sq;
  // correction of a copy staged with an estimated scale (1 when staged exactly), and the
  // per-matrix "stage again" flags
  float *ratio, *ratio_sq;
  int* restage;
  int nparts;
  int64_t bytes;
};

// Carves the workspace of a group; base == nullptr only computes the size.
Workspace carve(char* base, int m_pad, int n_pad, int Rp, int Cp, int batch, int gram) {
  Workspace w{};
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    char* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  const int64_t L = batch;
  const int64_t xs = (int64_t)m_pad * n_pad * 2;
  const int64_t as = (int64_t)m_pad * m_pad * 2;
  // X and the second X buffer the NS products write the next X into, both backends; Gram adds
  // the two Q slots and P R
  w.X = reinterpret_cast<uint16_t*>(take(L * xs));
  w.X2 = reinterpret_cast<uint16_t*>(take(L * xs));
  w.Am = reinterpret_cast<uint16_t*>(take(L * as));
  w.Pm = reinterpret_cast<uint16_t*>(take(L * as));
  if (gram) {
    w.Q0 = reinterpret_cast<uint16_t*>(take(L * as));
    w.Q1 = reinterpret_cast<uint16_t*>(take(L * as));
    w.Wm = reinterpret_cast<uint16_t*>(take(L * as));
  }
  w.nparts = pre_blocks_per_mat(Rp, Cp);
  w.partials = reinterpret_cast<float*>(take(L * w.nparts * 4));
  w.scale = reinterpret_cast<float*>(take(L * 4));
  w.scale_sq = reinterpret_cast<float*>(take(L * 4));
  w.ratio = reinterpret_cast<float*>(take(L * 4));
  w.ratio_sq = reinterpret_cast<float*>(take(L * 4));
  w.restage = reinterpret_cast<int*>(take(L * 4));
  w.bytes = off;
  return w;
}

// ---- launch profiler: optional hipEvent pairs around every kernel of run_group ----------------
// Single-threaded use only (like the launch path itself). Events are host objects; no device
// memory is allocated.
enum ProfClass {
  PC_PRE = 0, PC_NORM, PC_SYRK, PC_POLY, PC_GEMM, PC_FINAL, PC_ADAMW, PC_CLIP, PC_COUNT
};
struct ProfRec {
  int cls;
  hipEvent_t a, b;
  double flops, bytes;
};
struct Profiler {
  bool on = false;
  std::vector<hipEvent_t> pool;
  std::vector<ProfRec> recs;
  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};
Profiler g_prof;
// set while an entry point that must not allocate runs: the profiler records no events then
thread_local bool g_no_events = false;

template <class F>
int timed(int cls, double flops, double bytes, hipStream_t stream, const char* who, F&& launch) {
  if (!g_prof.on || g_no_events) return check_launch(launch(), who);
  hipEvent_t a = g_prof.take(), b = g_prof.take();
  if (!a || !b) return fail("%s: hipEventCreate failed", who);
  if (hipEventRecord(a, stream) != hipSuccess) return fail("%s: hipEventRecord failed", who);
  const int rc = check_launch(launch(), who);
  if (hipEventRecord(b, stream) != hipSuccess) return fail("%s: hipEventRecord failed", who);
  g_prof.recs.push_back({cls, a, b, flops, bytes});
  return rc;
}

int tri_tiles(int m_pad, int tile) {
  const int mt = m_pad / tile;
  return mt * (mt + 1) / 2;
}

// Output tile of a group's products, by the estimated time of its triangle products (the bulk
// of the work) in units of one 256-tile of work: a wave of 256-tiles gives every CU one tile (4
// units of 128-tile work), a wave of 128-tiles gives it two (2 units) at about 1/1.35 of the
// 256-tile rate (fitted to grouped Gram runs: 32 x 4096^2, 64 x 1024x4096, 64 and 128 x
// 1408x2048, one 2048x8192). Ceil'd waves charge the last, partial wave in full; the padding
// each tile size adds to m and n counts too. Measured on MI355X: one 4096^2 matrix runs 20%
// faster on 256-tiles (136 tiles on 256 CUs) than on 128-tiles (528 tiles on 512 slots), one
// 1024x16384 or 2048x8192 matrix 25-55% faster on 128-tiles, 128 experts of 1408x2048 5% faster
// on 256-tiles padded to 1536.
int auto_tile(int64_t m, int64_t n, int64_t batch, int num_cus) {
  const int64_t m256 = round_up(m, 256) / 256, m128 = round_up(m, 128) / 128;
  const int64_t t256 = batch * m256 * (m256 + 1) / 2, t128 = batch * m128 * (m128 + 1) / 2;
  const double npad = (double)round_up(n, 256) / (double)round_up(n, 128);
  const double c256 = 4.0 * (double)((t256 + num_cus - 1) / num_cus) * npad;
  const double c128 = 2.7 * (double)((t128 + 2 * num_cus - 1) / (2 * num_cus));
  return c256 <= c128 ? 256 : 128;
}

int plan(int rows, int cols, int batch, int tile_req, int num_cus, int gram, int* tile,
         int* m_pad, int* n_pad, int64_t* bytes) {
  if (rows <= 0 || cols <= 0 || batch <= 0)
    return fail("dmuon_ns_plan: rows, cols and batch must be positive (got %d, %d, %d)", rows,
                cols, batch);
  if (tile_req != 0 && tile_req != 128 && tile_req != 256)
    return fail("dmuon_ns_plan: tile must be 0 (auto), 128 or 256, got %d", tile_req);
  const int m = rows < cols ? rows : cols;
  const int n = rows < cols ? cols : rows;
  if (num_cus <= 0) num_cus = 256;
  int t = tile_req;
  if (t == 0) t = auto_tile(m, n, batch, num_cus);
  const int mp = (int)round_up(m, t), np = (int)round_up(n, t);
  if ((int64_t)mp * np * 2 >= kMaxXBytes)
    return fail("dmuon_ns_plan: a %d x %d matrix pads to %d x %d, %lld fp16 values; the NS "
                "kernels take at most 2^30 per matrix", rows, cols, mp, np, (long long)mp * np);
  const bool tall = rows > cols;
  const int Rp = tall ? np : mp, Cp = tall ? mp : np;
  Workspace w = carve(nullptr, mp, np, Rp, Cp, batch, gram);
  *tile = t;
  *m_pad = mp;
  *n_pad = np;
  *bytes = w.bytes;
  return 0;
}

// Gram-space NS (the reference's gram_newton_schulz, newton_schulz.py:333-448) on the fp16 NT
// kernels, for X (m x n, m <= n) staged as fp16(KX * ns_in / ||ns_in||). With R = X X^T and
// Z_i = c_i R^2 + b_i R, one NS step maps X to P_i X, P_i = Z_i + a_i I, so per step
//   Q <- P_i Q  (Q = P_i after a start or restart), the accumulated polynomial: Z Q^T + a Q
//   R <- P_i R P_i  when the next step is neither the last nor a restart:
//        W = Z R + a R, R = W Z + a W
//   restart at step i: X <- Q X, R = X X^T, Q reset;   finally U = Q X / KX
// Every symmetric product (R, Z, W, a fresh Q) is computed on the upper-triangle tiles and
// stored exactly symmetric (diagonal tiles included), so R R^T = R R and Z R^T = Z R hold to the
// bit; an R that is symmetric only to rounding costs up to 10x accuracy in fp16 emulation. Q's
// update is a full product: Q is a product of polynomials that no longer commute once rounded,
// and symmetrising it costs 3-8x accuracy on square matrices. fp16 as in the reference (bf16
// loses the small eigenvalues of R). Power-of-two scales keep every operand normal in fp16:
// X carries KX = 2^12 throughout, the first R (eigenvalues ~1/m) carries kr = 2^floor(log2 m)
// (at most 2^12) until its first update; all scale changes are folded into alpha / beta.
int run_gram(const Workspace& w, int m, int n, int m_pad, int n_pad, int tile, int batch, bool tall,
             int n_flip,
             const float* coeffs, int T, const int* restarts, int n_restarts,
             void* const* w_ptrs, int w_dtype, void* const* pub_ptrs, int pub_dtype,
             void* const* out_ptrs, int out_dtype, float decay, float lrs, double syrk_flops,
             double tri_sq_flops, double gemm_flops, double final_bytes, hipStream_t stream,
             const char* who) {
  const long long xs = (long long)m_pad * n_pad, as = (long long)m_pad * m_pad;
  const double full_sq_flops = 2.0 * batch * (double)m * m * m;
  // K loop lengths: the operands are zero past m (n), so the products multiply only m (n)
  // rounded up to the 64-wide slice, not the tile-padded m_pad (n_pad)
  const int km = (int)round_up(m, 64), kn = (int)round_up(n, 64);
  auto is_restart = [&](int it) {
    for (int r = 0; r < n_restarts; ++r)
      if (restarts[r] == it) return true;
    return false;
  };
  // D = alpha * A B^T + beta * C + diag * I, m x m; tri: upper tiles mirrored (symmetric result)
  auto sq = [&](const uint16_t* A, const uint16_t* B, const uint16_t* C, uint16_t* D, float alpha,
                float beta, float diag, bool tri, uint16_t* D2 = nullptr,
                float diag2 = 0.f) -> int {
    NtArgs s{};
    s.elt = ELT_F16;
    s.A = A; s.lda = m_pad; s.sA = as;
    s.B = B; s.ldb = m_pad; s.sB = as;
    s.M = m_pad; s.N = m_pad; s.K = m_pad; s.L = batch; s.k_loop = km;
    s.mt = s.nt = m_pad / tile;
    s.tiles_per_mat = tri ? tri_tiles(m_pad, tile) : s.mt * s.nt; s.tri = tri ? 1 : 0;
    s.sym_exact = 1; s.diag_skip = kDiagSkipPoly;
    s.live_rows = s.live_cols = km < m_pad ? km : 0;   // rows and columns past m: never read
    s.mode = EPI_SYM; s.alpha = alpha; s.beta = C ? beta : 0.f; s.diag = diag;
    s.C = C; s.ldc = m_pad; s.sC = as;
    s.c_in = (C && C == A) ? C_IS_A : C_NONE;   // C's tile is the A panel's last slices
    s.D = D; s.ldd = m_pad; s.sD = as;
    s.D2 = D2; s.diag2 = diag2;
    return timed(PC_POLY, tri ? tri_sq_flops : full_sq_flops, 0.0, stream, who,
                 [&] { return launch_nt(s, tile, stream); });
  };
  // The staged X may carry an estimated scale: the first products that read it multiply by the
  // per-matrix correction (ratio for X, ratio_sq for X X^T; 1 after an exact staging). A
  // restart rewrites X exactly scaled.
  bool x_staged = true;
  // the current X and the buffer a restart writes the next one into
  uint16_t* x_cur = w.X;
  uint16_t* x_nxt = w.X2;
  // R = alpha X X^T
  auto gram_of_x = [&](uint16_t* R, float alpha) -> int {
    NtArgs s{};
    s.alpha_dev = x_staged ? w.ratio_sq : nullptr;
    s.elt = ELT_F16;
    s.A = x_cur; s.lda = n_pad; s.sA = xs;
    s.B = x_cur; s.ldb = n_pad; s.sB = xs;
    s.M = m_pad; s.N = m_pad; s.K = n_pad; s.L = batch; s.k_loop = kn;
    s.mt = s.nt = m_pad / tile; s.tiles_per_mat = tri_tiles(m_pad, tile); s.tri = 1;
    s.sym_exact = 1; s.diag_skip = kDiagSkipGram;
    s.live_rows = s.live_cols = km < m_pad ? km : 0;
    s.mode = EPI_SYM; s.alpha = alpha;
    s.D = R; s.ldd = m_pad; s.sD = as;
    return timed(PC_SYRK, syrk_flops, 0.0, stream, who, [&] { return launch_nt(s, tile, stream); });
  };
  // X <- Q X (an NS restart), or the final U = Q X / KX with the Muon update in the epilogue
  auto qx = [&](const uint16_t* Q, bool last) -> int {
    NtArgs g{};
    g.alpha_dev = x_staged ? w.ratio : nullptr;
    g.elt = ELT_F16;
    g.A = Q; g.lda = m_pad; g.sA = as;
    g.B = x_cur; g.ldb = n_pad; g.sB = xs; g.b_kmajor = 1;
    g.M = m_pad; g.N = n_pad; g.K = m_pad; g.L = batch; g.k_loop = km;
    g.live_rows = km < m_pad ? km : 0;
    g.live_cols = kn < n_pad ? kn : 0;
    g.mt = m_pad / tile; g.nt = n_pad / tile; g.tiles_per_mat = g.mt * g.nt; g.tri = 0;
    g.beta = 0.f;
    if (!last) {
      g.alpha = 1.f;
      g.mode = EPI_NS;
      g.D = x_nxt; g.ldd = n_pad; g.sD = xs;   // X is the B operand: the new X goes elsewhere
      if (timed(PC_GEMM, gemm_flops, 0.0, stream, who, [&] { return launch_nt(g, tile, stream); }))
        return 1;
      uint16_t* t = x_cur; x_cur = x_nxt; x_nxt = t;
      x_staged = false;
      return 0;
    }
    g.alpha = 1.f / kNsKx;
    g.mode = EPI_FINAL;
    g.out_ptrs = out_ptrs; g.out_dtype = out_dtype;
    g.w_ptrs = w_ptrs; g.w_dtype = w_dtype; g.decay = decay; g.lrs = lrs;
    g.pub_ptrs = pub_ptrs; g.pub_dtype = pub_dtype;
    g.m_real = m; g.n_real = n; g.transposed = tall ? 1 : 0; g.n_flip = n_flip;
    return timed(PC_FINAL, gemm_flops, final_bytes, stream, who,
                 [&] { return launch_nt(g, tile, stream); });
  };
  // Q <- P Q = Z Q + a Q as a full product (Q is a product of polynomials that no longer
  // commute once rounded; its factor order must match R's). Z is symmetric, so the update runs
  // transposed, Q^T <- Q^T Z + a Q^T: Q^T is its A operand and its addend (the K loop takes the
  // addend's slices last), and the output is Q^T -- except for the last update before the Q X
  // that consumes Q, which writes only its transposed output, the row form Q that Q X reads.
  // A Q that is still P itself (after a start or restart) is symmetric and serves as either
  // form. Two slots, used in turn.
  uint16_t* qslot[2] = {w.Q0, w.Q1};
  uint16_t* qbuf[2] = {w.Q0, w.Q1};          // the row form of a slot's Q, once it has one
  auto q_update = [&](const uint16_t* Zm, int from, float a_, bool last) -> int {
    const int to = 1 - from;
    NtArgs g{};
    g.elt = ELT_F16;
    g.M = m_pad; g.N = m_pad; g.K = m_pad; g.L = batch; g.k_loop = km;
    g.live_rows = g.live_cols = km < m_pad ? km : 0;
    g.mt = g.nt = m_pad / tile; g.tiles_per_mat = g.mt * g.nt; g.tri = 0;
    g.mode = EPI_NS; g.alpha = 1.f; g.beta = a_;
    g.lda = g.ldb = g.ldc = g.ldd = g.lddt = m_pad;
    g.sA = g.sB = g.sC = g.sD = g.sDT = as;
    g.A = qslot[from]; g.B = Zm; g.C = qslot[from];
    g.c_in = C_IS_A;                           // the addend is the A panel's last slices
    if (last) g.DT = qslot[to];                // Q, the row form
    else g.D = qslot[to];                      // Q^T
    qbuf[to] = qslot[to];
    return timed(PC_POLY, full_sq_flops, 0.0, stream, who,
                 [&] { return launch_nt(g, tile, stream); });
  };
  // iterations from it up to the next restart (or T): the Q updates the segment has left
  auto updates_left = [&](int it) {
    int end = it + 1;
    while (end < T && !is_restart(end)) ++end;
    return end - it;
  };
  int kr = 1;
  while (kr * 2 <= m && kr < 4096) kr *= 2;
  uint16_t* R = w.Am;
  uint16_t* Z = w.Pm;
  uint16_t* W = w.Wm;
  int qs = -1;               // slot of the current Q, -1: none since the last (re)start
  float rs = (float)kr;      // the stored R is rs * (X X^T of the normalised X)
  if (gram_of_x(R, rs / (kNsKx * kNsKx))) return 1;
  for (int it = 0; it < T; ++it) {
    if (it != 0 && is_restart(it) && qs >= 0) {
      if (qx(qbuf[qs], false)) return 1;
      rs = 1.f;
      if (gram_of_x(R, 1.f / (kNsKx * kNsKx))) return 1;
      qs = -1;
    }
    const float ca = coeffs[3 * it], cb = coeffs[3 * it + 1], cc = coeffs[3 * it + 2];
    const bool evolve = it + 1 < T && !is_restart(it + 1);
    const float zr2 = cc / (rs * rs), zr1 = cb / rs;
    if (qs < 0 && !evolve) {
      // Q = Z + a I in one product (Z itself is not needed); symmetric, its own transpose
      if (sq(R, R, R, qslot[0], zr2, zr1, ca, true)) return 1;
      qbuf[0] = qslot[0];
      qs = 0;
      continue;
    }
    if (qs < 0) {
      // Z = c R^2 + b R, and Q = Z + a I written by the same epilogue
      if (sq(R, R, R, Z, zr2, zr1, 0.f, true, qslot[0], ca)) return 1;
      qbuf[0] = qslot[0];
      qs = 0;
    } else {
      if (sq(R, R, R, Z, zr2, zr1, 0.f, true)) return 1;   // Z = c R^2 + b R
      if (q_update(Z, qs, ca, updates_left(it) == 1)) return 1;   // Q <- Z Q + a Q
      qs = 1 - qs;
    }
    if (evolve) {
      if (sq(Z, R, R, W, 1.f, ca, 0.f, true)) return 1;               // rs * (P R)
      if (sq(W, Z, W, R, 1.f / rs, ca / rs, 0.f, true)) return 1;     // P R P
      rs = 1.f;
    }
  }
  return qx(qbuf[qs], true);
}

// The whole Newton-Schulz + optional update sequence of one group; see dmuon_muon_step_group.
// phases: PH_STAGE (momentum, norm, NS operand staging into the workspace), PH_APPLY (the NS
// products and the fused update / output from a staged workspace), or both.
enum { PH_STAGE = 1, PH_APPLY = 2 };
int run_group(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs, float* const* est_ptrs,
              void* const* w_ptrs, int w_dtype, void* const* pub_ptrs, int pub_dtype, void* const* out_ptrs,
              int out_dtype, int rows, int cols, int batch, int n_t,
              float mu, int nesterov, int first_step, float decay, float lrs, const float* coeffs,
              int T, int backend, const int* restarts, int n_restarts, float eps, void* workspace,
              int64_t workspace_bytes, int tile_req, hipStream_t stream, const char* who,
              int phases = PH_STAGE | PH_APPLY) {
  const bool do_stage = phases & PH_STAGE, do_apply = phases & PH_APPLY;
  if (do_stage) {
    if (!g_ptrs) return fail("%s: g_ptrs is NULL", who);
    if (g_dtype != DMUON_DTYPE_F32 && g_dtype != DMUON_DTYPE_BF16)
      return fail("%s: unsupported gradient dtype code %d", who, g_dtype);
  }
  if (do_apply) {
    if (w_ptrs && w_dtype != DMUON_DTYPE_F32 && w_dtype != DMUON_DTYPE_BF16)
      return fail("%s: unsupported weight dtype code %d", who, w_dtype);
    if (out_ptrs && out_dtype != DMUON_DTYPE_F32 && out_dtype != DMUON_DTYPE_BF16)
      return fail("%s: unsupported output dtype code %d", who, out_dtype);
    if (pub_ptrs && !w_ptrs) return fail("%s: pub_ptrs needs w_ptrs (it copies the new W)", who);
    if (pub_ptrs && pub_dtype != DMUON_DTYPE_F32 && pub_dtype != DMUON_DTYPE_BF16)
      return fail("%s: unsupported publish dtype code %d", who, pub_dtype);
    if (!coeffs || T <= 0)
      return fail("%s: need at least one (a, b, c) coefficient triple", who);
    if (n_restarts < 0 || (n_restarts > 0 && !restarts))
      return fail("%s: restart list NULL or of negative length", who);
  }
  if (backend != DMUON_NS_DIRECT && backend != DMUON_NS_GRAM)
    return fail("%s: unknown NS backend %d", who, backend);
  if (n_t < 0 || n_t > batch)
    return fail("%s: n_transposed=%d outside [0, batch=%d]", who, n_t, batch);
  const int gram = backend == DMUON_NS_GRAM;
  if (!workspace || !aligned16(workspace)) return fail("%s: workspace NULL or misaligned", who);
  int tile, m_pad, n_pad;
  int64_t need;
  if (plan(rows, cols, batch, tile_req, 0, gram, &tile, &m_pad, &n_pad, &need)) return 1;
  if (workspace_bytes < need)
    return fail("%s: workspace of %lld bytes is smaller than the %lld bytes planned", who,
                (long long)workspace_bytes, (long long)need);
  const bool tall = rows > cols;
  const int m = tall ? cols : rows, n = tall ? rows : cols;
  const int Rp = tall ? n_pad : m_pad, Cp = tall ? m_pad : n_pad;
  Workspace w = carve(static_cast<char*>(workspace), m_pad, n_pad, Rp, Cp, batch, gram);
  const long long xs = (long long)m_pad * n_pad, as = (long long)m_pad * m_pad;

  (void)Rp; (void)Cp;
  // The group's matrices share the m x n NS shape: [0, batch - n_t) are rows x cols and the last
  // n_t are cols x rows (their transposes). Each orientation is staged by its own launch into
  // its slice of the workspace; everything after the staging sees one m x n batch, and the final
  // epilogue writes each matrix back in its own orientation. (Square shapes have one
  // orientation: the n_t part is staged and written like the rest.)
  const int n_flip = rows == cols ? 0 : n_t;
  auto pre_args = [&](int part) {
    const int l0 = part == 0 ? 0 : batch - n_t;
    const int r_ = part == 0 ? rows : cols, c_ = part == 0 ? cols : rows;
    const bool tall_ = r_ > c_;
    PreArgs q{};
    q.g_ptrs = g_ptrs ? g_ptrs + l0 : nullptr;
    q.g_dtype = g_dtype;
    q.buf_ptrs = buf_ptrs ? buf_ptrs + l0 : nullptr;
    q.est_ptrs = est_ptrs ? est_ptrs + l0 : nullptr;
    q.Y = w.X + l0 * xs;
    q.ldy = tall_ ? m_pad : n_pad;
    q.sY = xs;
    q.YT = w.X + l0 * xs;
    q.ldyt = tall_ ? n_pad : m_pad;
    q.sYT = xs;
    q.partials = w.partials + (long long)l0 * w.nparts;
    q.rows = r_;
    q.cols = c_;
    q.Rp = tall_ ? n_pad : m_pad;
    q.Cp = tall_ ? m_pad : n_pad;
    q.L = part == 0 ? batch - n_t : n_t;
    q.mu = mu;
    q.first_step = first_step;
    q.nesterov = nesterov;
    q.kx = kNsKx;
    q.scale = w.scale + l0;
    // the NS products read X k-major, so only X is staged: by the direct write for a wide
    // orientation, by the transposed one for a tall orientation
    q.skip_y = tall_ ? 1 : 0;
    q.skip_yt = tall_ ? 0 : 1;
    return q;
  };
  const double Ld = batch, md = m, nd = n, elems = (double)rows * cols * batch;
  const double gbytes = g_dtype == DMUON_DTYPE_F32 ? 4.0 : 2.0;
  if (do_stage) {
  // algorithmic bytes (what one ideal pass moves): gradient read, fp32 momentum read (not on
  // the first step) and write, one 2-byte copy of the normalised ns_in. The second pass's
  // re-read of the gradient and the new momentum (fp16 cannot hold an un-normalised gradient,
  // so the copy waits for the norm) is overhead, not counted.
  // With est_ptrs (a per-matrix scale kept from the previous step) the first pass also writes
  // the fp16 copy as fp16(kx * est * ns_in); the norm finalize then keeps that copy when
  // r = scale / est is within [1/4, 4] (the first products multiply by r or r^2, and every copy
  // entry stays below kx / r <= 2^14) and otherwise flags the matrix for the second pass,
  // which then stages exactly as without an estimate.
  const bool est = est_ptrs != nullptr;
  const double mom_bytes = buf_ptrs ? (first_step ? 4.0 : 8.0) : 0.0;
  for (int part = 0; part < 2; ++part) {
    PreArgs p = pre_args(part);
    if (p.L == 0) continue;
    p.stage = est ? PRE_EST : PRE_NORM;
    const double pre_bytes = elems * p.L / batch * (gbytes + mom_bytes + (est ? 2.0 : 0.0));
    if (timed(PC_PRE, 0.0, pre_bytes, stream, who, [&] { return launch_pre(p, stream); }))
      return 1;
  }
  if (timed(PC_NORM, 0.0, (double)batch * w.nparts * 4, stream, who, [&] {
        return launch_norm_finalize_est(w.partials, w.nparts, batch, eps, w.scale, w.scale_sq,
                                        est_ptrs, w.ratio, w.ratio_sq, w.restage, stream);
      }))
    return 1;
  for (int part = 0; part < 2; ++part) {
    PreArgs p = pre_args(part);
    if (p.L == 0) continue;
    p.stage = PRE_F16;
    p.restage = est ? w.restage + (part == 0 ? 0 : batch - n_t) : nullptr;
    const double st_bytes = est ? 0.0 : elems * p.L / batch * 2.0;
    if (timed(PC_PRE, 0.0, st_bytes, stream, who, [&] { return launch_pre(p, stream); }))
      return 1;
  }
  }  // do_stage
  if (!do_apply) return 0;
  const double syrk_flops = Ld * md * (md + 1) * nd, poly_flops = Ld * md * (md + 1) * md;
  const double gemm_flops = 2.0 * Ld * md * md * nd;
  const double wbytes = w_ptrs ? 2.0 * elems * (w_dtype == DMUON_DTYPE_F32 ? 4.0 : 2.0) : 0.0;
  const double obytes = out_ptrs ? elems * (out_dtype == DMUON_DTYPE_F32 ? 4.0 : 2.0) : 0.0;
  const double pbytes = pub_ptrs ? elems * (pub_dtype == DMUON_DTYPE_F32 ? 4.0 : 2.0) : 0.0;

  if (gram)
    return run_gram(w, m, n, m_pad, n_pad, tile, batch, tall, n_flip, coeffs, T, restarts,
                    n_restarts,
                    w_ptrs, w_dtype, pub_ptrs, pub_dtype, out_ptrs, out_dtype, decay, lrs,
                    syrk_flops, poly_flops, gemm_flops, wbytes + obytes + pbytes, stream, who);
  // Direct NS on the same fp16 operands as the Gram form: X carries the power-of-two scale
  // kNsKx throughout; the first A (eigenvalues ~1/m) carries kr until its polynomial.
  int kr = 1;
  while (kr * 2 <= m && kr < 4096) kr *= 2;
  const int km = (int)round_up(m, 64), kn = (int)round_up(n, 64);   // K loops (zero past m, n)
  // the current X and the buffer the next one is written to
  uint16_t* x_cur = w.X;
  uint16_t* x_nxt = w.X2;
  for (int it = 0; it < T; ++it) {
    const float ca = coeffs[3 * it], cb = coeffs[3 * it + 1], cc = coeffs[3 * it + 2];
    const float rs = it == 0 ? (float)kr : 1.f;   // the stored A is rs * (X X^T)
    // A = X X^T of the normalised X (the stored X is kNsKx * X)
    NtArgs s{};
    s.elt = ELT_F16;
    s.A = x_cur; s.lda = n_pad; s.sA = xs;
    s.B = x_cur; s.ldb = n_pad; s.sB = xs;
    s.M = m_pad; s.N = m_pad; s.K = n_pad; s.L = batch; s.k_loop = kn;
    s.mt = s.nt = m_pad / tile; s.tiles_per_mat = tri_tiles(m_pad, tile); s.tri = 1;
    s.sym_exact = 1; s.diag_skip = kDiagSkipGram;
    s.live_rows = s.live_cols = km < m_pad ? km : 0;
    s.mode = EPI_SYM; s.alpha = rs / (kNsKx * kNsKx); s.beta = 0.f; s.diag = 0.f;
    s.alpha_dev = it == 0 ? w.ratio_sq : nullptr;   // the staged X's scale correction
    s.D = w.Am; s.ldd = m_pad; s.sD = as;
    if (timed(PC_SYRK, syrk_flops, 0.0, stream, who, [&] { return launch_nt(s, tile, stream); }))
      return 1;
    // P = c A A^T + b A
    NtArgs q{};
    q.elt = ELT_F16;
    q.A = w.Am; q.lda = m_pad; q.sA = as;
    q.B = w.Am; q.ldb = m_pad; q.sB = as;
    q.M = m_pad; q.N = m_pad; q.K = m_pad; q.L = batch; q.k_loop = km;
    q.mt = q.nt = m_pad / tile; q.tiles_per_mat = s.tiles_per_mat; q.tri = 1;
    q.sym_exact = 1; q.diag_skip = kDiagSkipPoly;
    q.live_rows = q.live_cols = km < m_pad ? km : 0;
    q.mode = EPI_SYM; q.alpha = cc / (rs * rs); q.beta = cb / rs; q.diag = 0.f;
    q.C = w.Am; q.ldc = m_pad; q.sC = as;
    q.c_in = C_IS_A;
    q.D = w.Pm; q.ldd = m_pad; q.sD = as;
    if (timed(PC_POLY, poly_flops, 0.0, stream, who, [&] { return launch_nt(q, tile, stream); }))
      return 1;
    // X' = P X + a X (scale kNsKx kept); the final step writes U = X' / kNsKx
    NtArgs g{};
    g.elt = ELT_F16;
    g.A = w.Pm; g.lda = m_pad; g.sA = as;
    g.B = x_cur; g.ldb = n_pad; g.sB = xs; g.b_kmajor = 1;
    g.M = m_pad; g.N = n_pad; g.K = m_pad; g.L = batch; g.k_loop = km;
    g.live_rows = km < m_pad ? km : 0;
    g.live_cols = kn < n_pad ? kn : 0;
    g.mt = m_pad / tile; g.nt = n_pad / tile; g.tiles_per_mat = g.mt * g.nt; g.tri = 0;
    g.alpha = it + 1 < T ? 1.f : 1.f / kNsKx; g.beta = ca;
    g.alpha_dev = it == 0 ? w.ratio : nullptr;
    g.C = x_cur; g.ldc = n_pad; g.sC = xs;
    if (it + 1 < T) {
      g.mode = EPI_NS;
      g.D = x_nxt; g.ldd = n_pad; g.sD = xs;   // X is the B operand: the new X goes elsewhere
      if (timed(PC_GEMM, gemm_flops, 0.0, stream, who, [&] { return launch_nt(g, tile, stream); }))
        return 1;
      uint16_t* t = x_cur; x_cur = x_nxt; x_nxt = t;
    } else {
      g.mode = EPI_FINAL;
      g.out_ptrs = out_ptrs; g.out_dtype = out_dtype;
      g.w_ptrs = w_ptrs; g.w_dtype = w_dtype; g.decay = decay; g.lrs = lrs;
      g.pub_ptrs = pub_ptrs; g.pub_dtype = pub_dtype;
      g.m_real = m; g.n_real = n; g.transposed = tall ? 1 : 0; g.n_flip = n_flip;
      if (timed(PC_FINAL, gemm_flops, wbytes + obytes + pbytes, stream, who,
                [&] { return launch_nt(g, tile, stream); }))
        return 1;
    }
  }
  return 0;
}

// ---- scratch of dmuon_muon_step_group_noalloc (the array itself is at file scope above) --------
constexpr int64_t kScratchBytes = DMUON_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of the current GPU's copy of `scratch`, resolved once per device. The
// first resolution may load the library's code object, so it is not itself allocation-free:
// dmuon_noalloc_init does it at set-up. With `capture_stream_checked`, a first resolution while
// `stream` is being captured is refused instead (it would run inside the capture).
int scratch_of_current_device(const char* who, void** out, bool capture_stream_checked = false,
                              hipStream_t stream = nullptr) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail("%s: no current HIP device (%s)", who, hipGetErrorString(ge));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (capture_stream_checked) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return fail("%s: first use on device %d while its stream is being captured: call "
                    "dmuon_noalloc_init() (or the entry point once, eagerly) on this device "
                    "before capturing", who, dev);
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", who, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

struct NoEvents {
  NoEvents() { g_no_events = true; }
  ~NoEvents() { g_no_events = false; }
};

}  // namespace

extern "C" {

const char* dmuon_last_error(void) { return g_last_error.c_str(); }

int dmuon_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  const char* who = "dmuon_stream_copy";
  if (bytes == 0) return 0;
  if (!src || !dst || bytes < 0) return fail("%s: NULL buffer or negative size", who);
  if (!aligned16(src) || !aligned16(dst) || bytes % 16)
    return fail("%s: buffers must be 16-byte aligned and the size a multiple of 16 (got %lld)",
                who, (long long)bytes);
  const uintptr_t s = reinterpret_cast<uintptr_t>(src), d = reinterpret_cast<uintptr_t>(dst);
  if (s < d + (uintptr_t)bytes && d < s + (uintptr_t)bytes)
    return fail("%s: source and destination overlap", who);
  return check_launch(launch_stream_copy(src, dst, bytes / 16, static_cast<hipStream_t>(stream)),
                      who);
}

int dmuon_profile_enable(int on) {
  g_prof.on = on != 0;
  return 0;
}

int dmuon_profile_collect(double* ms, int64_t* launches, double* flops, double* bytes,
                          int n_classes) {
  if (n_classes < PC_COUNT || !ms || !launches || !flops || !bytes)
    return fail("dmuon_profile_collect: need arrays of at least %d classes", (int)PC_COUNT);
  for (int c = 0; c < n_classes; ++c) {
    ms[c] = 0.0;
    launches[c] = 0;
    flops[c] = 0.0;
    bytes[c] = 0.0;
  }
  int rc = 0;
  for (const ProfRec& r : g_prof.recs) {
    float t = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&t, r.a, r.b) != hipSuccess)
      rc = fail("dmuon_profile_collect: event query failed");
    ms[r.cls] += t;
    launches[r.cls] += 1;
    flops[r.cls] += r.flops;
    bytes[r.cls] += r.bytes;
    g_prof.pool.push_back(r.a);
    g_prof.pool.push_back(r.b);
  }
  g_prof.recs.clear();
  return rc;
}

int dmuon_abi_version(void) { return DMUON_ABI_VERSION; }

}  // extern "C"

namespace {

// 16-bit operand type of the product entry points: DMUON_DTYPE_BF16 or DMUON_DTYPE_F16
int elt_of(const char* who, int dtype, int* elt) {
  if (dtype == DMUON_DTYPE_BF16) { *elt = ELT_BF16; return 0; }
  if (dtype == DMUON_DTYPE_F16) { *elt = ELT_F16; return 0; }
  return fail("%s: operand dtype code %d is not a 16-bit type (bf16 %d, fp16 %d)", who, dtype,
              DMUON_DTYPE_BF16, DMUON_DTYPE_F16);
}

// The SYRK seam (syrk_or_cublas) for any M and K. The NT kernel reads whole tiles (M a
// multiple of the tile, K of the 64-wide slice) from 16-byte aligned rows; a call that does
// not meet that runs on zero-padded copies in the caller's workspace -- A [L][Mp][Kp], B (when
// it is another matrix), C [L][Mp][Mp] and D [L][Mp][Mp] -- and the M x M corner of the padded
// result is copied into D. Zero rows and columns of A and B leave the corner unchanged.
struct SyrkPlan {
  int tile, Mp, Kp;
  bool direct;                 // the caller's operands are used in place
  bool b_copy;
  int64_t offB, offC, offD, bytes;
};

int syrk_plan(const char* who, const void* A, int64_t lda, int64_t strideA, const void* B,
              int64_t ldb, int64_t strideB, const void* C, int64_t ldc, int64_t strideC,
              const void* D, int64_t ldd, int64_t strideD, int M, int K, int batch, int tile_req,
              SyrkPlan* pl) {
  if (tile_req != 0 && tile_req != 128 && tile_req != 256)
    return fail("%s: tile must be 0 (automatic), 128 or 256, got %d", who, tile_req);
  if (M < 0 || K < 0 || batch < 0) return fail("%s: bad sizes M=%d K=%d batch=%d", who, M, K, batch);
  if (!A || !D) return fail("%s: A and D must be non-NULL", who);
  if (lda < K || ldb < K || ldd < M || (C && ldc < M))
    return fail("%s: leading dimension smaller than the row length", who);
  if (batch > 1 && (strideA < 0 || strideB < 0 || strideD < 0 || (C && strideC < 0)))
    return fail("%s: batch strides must be non-negative", who);
  if (D == A || D == B || (C && D == C)) return fail("%s: D must not alias A, B or C", who);
  // C is an M x M matrix; an operand is M x K. The two can be one matrix only when K == M
  // (the polynomial Z = c R R^T + b R); otherwise the epilogue would read an M x M addend
  // over an M x K operand's rows.
  if (C && (C == A || C == B) && K != M)
    return fail("%s: C aliases %s but K=%d != M=%d (an M x M addend cannot be an M x K operand)",
                who, C == A ? "A" : "B", K, M);
  int t = tile_req;
  if (t == 0) {
    t = auto_tile(M, K > 0 ? K : 1, batch, 256);
    if (t == 256 && round_up(M, 256) != round_up(M, 128)) t = 128;   // no padded copy for 256
  }
  pl->tile = t;
  pl->Mp = (int)round_up(M, t);
  pl->Kp = (int)round_up(K > 0 ? K : 1, 64);
  const bool b_same = B == A && ldb == lda && strideB == strideA;
  pl->direct = M % t == 0 && K % 64 == 0 && K > 0 && aligned16(A) && aligned16(B) &&
               aligned16(D) && (!C || aligned16(C)) && ld_ok(lda) && ld_ok(ldb) && ld_ok(ldd) &&
               (!C || ld_ok(ldc)) && stride_ok(strideA, batch) && stride_ok(strideB, batch) &&
               stride_ok(strideD, batch) && (!C || stride_ok(strideC, batch));
  pl->b_copy = !b_same;
  const int64_t L = batch, xa = L * pl->Mp * (int64_t)pl->Kp * 2, xd = L * pl->Mp * (int64_t)pl->Mp * 2;
  int64_t off = align256(xa);
  pl->offB = pl->b_copy ? off : 0;
  if (pl->b_copy) off += align256(xa);
  pl->offC = C ? off : 0;
  if (C) off += align256(xd);
  pl->offD = off;
  off += align256(xd);
  pl->bytes = pl->direct ? 0 : off;
  return 0;
}

int syrk_impl(const char* who, int elt, const void* A, int64_t lda, int64_t strideA,
              const void* B, int64_t ldb, int64_t strideB, const void* C, int64_t ldc,
              int64_t strideC, void* D, int64_t ldd, int64_t strideD, int M, int K, int batch,
              float alpha, float beta, float diag_add, const float* alpha_dev, int tile_req,
              void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if (batch == 0 || M == 0) return 0;
  if (!B) { B = A; ldb = lda; strideB = strideA; }
  SyrkPlan pl;
  if (syrk_plan(who, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, D, ldd, strideD, M, K,
                batch, tile_req, &pl))
    return 1;
  NtArgs s{};
  s.elt = elt;
  s.M = pl.Mp; s.N = pl.Mp; s.K = pl.Kp; s.L = batch;
  s.mt = s.nt = pl.Mp / pl.tile; s.tiles_per_mat = tri_tiles(pl.Mp, pl.tile); s.tri = 1;
  s.mode = EPI_SYM; s.alpha = alpha; s.beta = C ? beta : 0.f; s.diag = diag_add;
  s.alpha_dev = alpha_dev;
  if (pl.direct) {
    s.A = static_cast<const uint16_t*>(A); s.lda = lda; s.sA = strideA;
    s.B = static_cast<const uint16_t*>(B); s.ldb = ldb; s.sB = strideB;
    s.C = static_cast<const uint16_t*>(C); s.ldc = ldc; s.sC = strideC;
    if (C && C == A && ldc == lda && (batch <= 1 || strideC == strideA) && K == M) s.c_in = C_IS_A;
    s.D = static_cast<uint16_t*>(D); s.ldd = ldd; s.sD = strideD;
    return check_launch(launch_nt(s, pl.tile, stream), who);
  }
  if (!workspace)
    return fail("%s: M=%d, K=%d or the operand layout needs the padded path (M a multiple of "
                "the tile %d, K of 64, 16-byte aligned rows otherwise), which needs a workspace "
                "of %lld bytes (dmuon_syrk_workspace_size)", who, M, K, pl.tile,
                (long long)pl.bytes);
  if (!aligned16(workspace) || workspace_bytes < pl.bytes)
    return fail("%s: workspace misaligned or smaller than the %lld bytes of the padded path", who,
                (long long)pl.bytes);
  char* ws = static_cast<char*>(workspace);
  const long long sa = (long long)pl.Mp * pl.Kp, sd = (long long)pl.Mp * pl.Mp;
  uint16_t* Ap = reinterpret_cast<uint16_t*>(ws);
  uint16_t* Bp = pl.b_copy ? reinterpret_cast<uint16_t*>(ws + pl.offB) : Ap;
  uint16_t* Cp = C ? reinterpret_cast<uint16_t*>(ws + pl.offC) : nullptr;
  uint16_t* Dp = reinterpret_cast<uint16_t*>(ws + pl.offD);
  if (check_launch(launch_pad_copy(static_cast<const uint16_t*>(A), lda, strideA, Ap, pl.Kp, sa,
                                   M, K, pl.Mp, pl.Kp, batch, stream), who))
    return 1;
  if (pl.b_copy &&
      check_launch(launch_pad_copy(static_cast<const uint16_t*>(B), ldb, strideB, Bp, pl.Kp, sa,
                                   M, K, pl.Mp, pl.Kp, batch, stream), who))
    return 1;
  // C == A (K == M): the padded C is the padded copy of A itself, and its tile is the A panel's
  // last slices (NtArgs::c_in)
  const bool c_from_a = C && C == A && ldc == lda && (batch <= 1 || strideC == strideA) &&
                        K == M && pl.Kp == pl.Mp;
  if (C && !c_from_a &&
      check_launch(launch_pad_copy(static_cast<const uint16_t*>(C), ldc, strideC, Cp, pl.Mp, sd,
                                   M, M, pl.Mp, pl.Mp, batch, stream), who))
    return 1;
  s.A = Ap; s.lda = pl.Kp; s.sA = sa;
  s.B = Bp; s.ldb = pl.Kp; s.sB = sa;
  s.C = Cp; s.ldc = pl.Mp; s.sC = sd;
  if (c_from_a) { s.C = Ap; s.ldc = pl.Kp; s.sC = sa; s.c_in = C_IS_A; }
  s.D = Dp; s.ldd = pl.Mp; s.sD = sd;
  if (check_launch(launch_nt(s, pl.tile, stream), who)) return 1;
  return check_launch(launch_pad_copy(Dp, pl.Mp, sd, static_cast<uint16_t*>(D), ldd, strideD, M,
                                      M, M, M, batch, stream), who);
}

}  // namespace

extern "C" {

int dmuon_syrk_workspace_size(int dtype, const void* A, int64_t lda, int64_t strideA,
                              const void* B, int64_t ldb, int64_t strideB, const void* C,
                              int64_t ldc, int64_t strideC, const void* D, int64_t ldd,
                              int64_t strideD, int M, int K, int batch, int tile,
                              int64_t* workspace_bytes) {
  const char* who = "dmuon_syrk_workspace_size";
  int elt;
  if (!workspace_bytes) return fail("%s: NULL output", who);
  *workspace_bytes = 0;
  if (elt_of(who, dtype, &elt)) return 1;
  if (batch == 0 || M == 0) return 0;
  if (!B) { B = A; ldb = lda; strideB = strideA; }
  SyrkPlan pl;
  if (syrk_plan(who, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, D, ldd, strideD, M, K,
                batch, tile, &pl))
    return 1;
  *workspace_bytes = pl.bytes;
  return 0;
}

int dmuon_syrk(int dtype, const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
               int64_t strideB, const void* C, int64_t ldc, int64_t strideC, void* D, int64_t ldd,
               int64_t strideD, int M, int K, int batch, float alpha, float beta, float diag_add,
               const float* alpha_dev, int tile, void* workspace, int64_t workspace_bytes,
               void* stream) {
  const char* who = "dmuon_syrk";
  int elt;
  if (elt_of(who, dtype, &elt)) return 1;
  return syrk_impl(who, elt, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, D, ldd, strideD,
                   M, K, batch, alpha, beta, diag_add, alpha_dev, tile, workspace,
                   workspace_bytes, static_cast<hipStream_t>(stream));
}

int dmuon_syrk_bf16(const void* A, int64_t lda, int64_t strideA, const void* B, int64_t ldb,
                    int64_t strideB, const void* C, int64_t ldc, int64_t strideC, void* D,
                    int64_t ldd, int64_t strideD, int M, int K, int batch, float alpha, float beta,
                    float diag_add, const float* alpha_dev, int tile, void* stream) {
  const char* who = "dmuon_syrk_bf16";
  if (batch == 0 || M == 0) return 0;
  if (tile != 128 && tile != 256) return fail("%s: tile must be 128 or 256, got %d", who, tile);
  if (M > 0 && M % tile) return fail("%s: M=%d is not a multiple of the tile %d", who, M, tile);
  if (K > 0 && K % 64) return fail("%s: K=%d is not a multiple of 64", who, K);
  if (!aligned16(A) || (B && !aligned16(B)) || !aligned16(D) || (C && !aligned16(C)))
    return fail("%s: operands must be 16-byte aligned", who);
  return syrk_impl(who, ELT_BF16, A, lda, strideA, B, ldb, strideB, C, ldc, strideC, D, ldd,
                   strideD, M, K, batch, alpha, beta, diag_add, alpha_dev, tile, nullptr, 0,
                   static_cast<hipStream_t>(stream));
}

static int gemm_common_checks(const char* who, const void* P, int64_t ldp, int64_t strideP,
                              const void* XT, int64_t ldxt, int64_t strideXT, const void* X,
                              int64_t ldx, int64_t strideX, int M, int N, int batch, int tile) {
  if (tile != 128 && tile != 256) return fail("%s: tile must be 128 or 256, got %d", who, tile);
  if (M <= 0 || N <= 0 || batch < 0) return fail("%s: bad sizes M=%d N=%d batch=%d", who, M, N, batch);
  if (M % tile || N % tile) return fail("%s: M=%d and N=%d must be multiples of the tile %d", who, M, N, tile);
  if (!P || (!XT && !X)) return fail("%s: P and one of XT / X must be non-NULL", who);
  if (!aligned16(P) || (XT && !aligned16(XT)) || (X && !aligned16(X)))
    return fail("%s: operands must be 16-byte aligned", who);
  if (!ld_ok(ldp) || ldp < M || (XT && (!ld_ok(ldxt) || ldxt < M)) || (X && (!ld_ok(ldx) || ldx < N)))
    return fail("%s: bad leading dimensions", who);
  if (!stride_ok(strideP, batch) || (XT && !stride_ok(strideXT, batch)) ||
      (X && !stride_ok(strideX, batch)))
    return fail("%s: batch strides must be non-negative multiples of 8", who);
  // XT == NULL: the product reads X itself as its k-major B operand (one 32-bit buffer range
  // per matrix)
  if (!XT && (int64_t)M * ldx * 2 >= (1LL << 31))
    return fail("%s: X read in place needs M * ldx * 2 < 2^31 bytes (pass XT instead)", who);
  return 0;
}

// B operand of the NS-GEMM exports: X^T when given, else X read k-major
static void gemm_b_operand(NtArgs& g, const void* XT, int64_t ldxt, int64_t strideXT,
                           const void* X, int64_t ldx, int64_t strideX) {
  if (XT) {
    g.B = static_cast<const uint16_t*>(XT); g.ldb = ldxt; g.sB = strideXT;
  } else {
    g.B = static_cast<const uint16_t*>(X); g.ldb = ldx; g.sB = strideX; g.b_kmajor = 1;
  }
}

static int ns_gemm_impl(const char* who, int elt, const void* P, int64_t ldp, int64_t strideP, const void* XT, int64_t ldxt,
                       int64_t strideXT, const void* X, int64_t ldx, int64_t strideX, void* Xout,
                       int64_t ldxo, int64_t strideXo, void* XTout, int64_t ldxto,
                       int64_t strideXTo, int M, int N, int batch, float alpha, float beta,
                       const float* alpha_dev, int tile, void* stream) {
  if (batch == 0) return 0;
  if (gemm_common_checks(who, P, ldp, strideP, XT, ldxt, strideXT, X, ldx, strideX, M, N, batch, tile))
    return 1;
  if (!Xout || !aligned16(Xout) || !ld_ok(ldxo) || ldxo < N || !stride_ok(strideXo, batch))
    return fail("%s: bad Xout", who);
  if (XTout && (!aligned16(XTout) || !ld_ok(ldxto) || ldxto < M || !stride_ok(strideXTo, batch)))
    return fail("%s: bad XTout", who);
  if (XT && XTout == XT) return fail("%s: XTout must not alias XT", who);
  if (Xout == P || (XT && Xout == XT)) return fail("%s: Xout must not alias P or XT", who);
  if (!XT && Xout == X) return fail("%s: Xout must not alias X when X is the B operand", who);
  NtArgs g{};
  g.elt = elt;
  g.A = static_cast<const uint16_t*>(P); g.lda = ldp; g.sA = strideP;
  gemm_b_operand(g, XT, ldxt, strideXT, X, ldx, strideX);
  g.M = M; g.N = N; g.K = M; g.L = batch;
  g.mt = M / tile; g.nt = N / tile; g.tiles_per_mat = g.mt * g.nt; g.tri = 0;
  g.mode = EPI_NS; g.alpha = alpha; g.beta = X ? beta : 0.f; g.alpha_dev = alpha_dev;
  g.C = static_cast<const uint16_t*>(X); g.ldc = ldx; g.sC = strideX;
  g.D = static_cast<uint16_t*>(Xout); g.ldd = ldxo; g.sD = strideXo;
  g.DT = static_cast<uint16_t*>(XTout); g.lddt = ldxto; g.sDT = strideXTo;
  return check_launch(launch_nt(g, tile, static_cast<hipStream_t>(stream)), who);
}

static int ns_gemm_final_impl(const char* who, int elt, const void* P, int64_t ldp, int64_t strideP, const void* XT,
                             int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx,
                             int64_t strideX, int M, int N, int batch, float alpha, float beta,
                             const float* alpha_dev, int m_real, int n_real, int transposed,
                             void* const* out_ptrs, int out_dtype, void* const* w_ptrs,
                             int w_dtype, void* const* pub_ptrs, int pub_dtype, float decay,
                             float lrs, int tile, void* stream) {
  if (batch == 0) return 0;
  if (gemm_common_checks(who, P, ldp, strideP, XT, ldxt, strideXT, X, ldx, strideX, M, N, batch, tile))
    return 1;
  if (m_real <= 0 || n_real <= 0 || m_real > M || n_real > N)
    return fail("%s: real extent %dx%d outside the padded %dx%d", who, m_real, n_real, M, N);
  if (!out_ptrs && !w_ptrs) return fail("%s: nothing to write (out_ptrs and w_ptrs NULL)", who);
  if (out_ptrs && out_dtype != DMUON_DTYPE_F32 && out_dtype != DMUON_DTYPE_BF16)
    return fail("%s: unsupported output dtype %d", who, out_dtype);
  if (w_ptrs && w_dtype != DMUON_DTYPE_F32 && w_dtype != DMUON_DTYPE_BF16)
    return fail("%s: unsupported weight dtype %d", who, w_dtype);
  if (pub_ptrs && !w_ptrs) return fail("%s: pub_ptrs needs w_ptrs (it copies the new W)", who);
  if (pub_ptrs && pub_dtype != DMUON_DTYPE_F32 && pub_dtype != DMUON_DTYPE_BF16)
    return fail("%s: unsupported publish dtype %d", who, pub_dtype);
  NtArgs g{};
  g.elt = elt;
  g.A = static_cast<const uint16_t*>(P); g.lda = ldp; g.sA = strideP;
  gemm_b_operand(g, XT, ldxt, strideXT, X, ldx, strideX);
  g.M = M; g.N = N; g.K = M; g.L = batch;
  g.mt = M / tile; g.nt = N / tile; g.tiles_per_mat = g.mt * g.nt; g.tri = 0;
  g.mode = EPI_FINAL; g.alpha = alpha; g.beta = X ? beta : 0.f; g.alpha_dev = alpha_dev;
  g.C = static_cast<const uint16_t*>(X); g.ldc = ldx; g.sC = strideX;
  g.out_ptrs = out_ptrs; g.out_dtype = out_dtype;
  g.w_ptrs = w_ptrs; g.w_dtype = w_dtype; g.decay = decay; g.lrs = lrs;
  g.pub_ptrs = pub_ptrs; g.pub_dtype = pub_dtype;
  g.m_real = m_real; g.n_real = n_real; g.transposed = transposed ? 1 : 0;
  return check_launch(launch_nt(g, tile, static_cast<hipStream_t>(stream)), who);
}

int dmuon_ns_gemm(int dtype, const void* P, int64_t ldp, int64_t strideP, const void* XT,
                  int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx, int64_t strideX,
                  void* Xout, int64_t ldxo, int64_t strideXo, void* XTout, int64_t ldxto,
                  int64_t strideXTo, int M, int N, int batch, float alpha, float beta,
                  const float* alpha_dev, int tile, void* stream) {
  int elt;
  if (elt_of("dmuon_ns_gemm", dtype, &elt)) return 1;
  return ns_gemm_impl("dmuon_ns_gemm", elt, P, ldp, strideP, XT, ldxt, strideXT, X, ldx, strideX,
                      Xout, ldxo, strideXo, XTout, ldxto, strideXTo, M, N, batch, alpha, beta,
                      alpha_dev, tile, stream);
}

int dmuon_ns_gemm_bf16(const void* P, int64_t ldp, int64_t strideP, const void* XT, int64_t ldxt,
                       int64_t strideXT, const void* X, int64_t ldx, int64_t strideX, void* Xout,
                       int64_t ldxo, int64_t strideXo, void* XTout, int64_t ldxto,
                       int64_t strideXTo, int M, int N, int batch, float alpha, float beta,
                       const float* alpha_dev, int tile, void* stream) {
  return ns_gemm_impl("dmuon_ns_gemm_bf16", ELT_BF16, P, ldp, strideP, XT, ldxt, strideXT, X, ldx,
                      strideX, Xout, ldxo, strideXo, XTout, ldxto, strideXTo, M, N, batch, alpha,
                      beta, alpha_dev, tile, stream);
}

int dmuon_ns_gemm_final(int dtype, const void* P, int64_t ldp, int64_t strideP, const void* XT,
                        int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx,
                        int64_t strideX, int M, int N, int batch, float alpha, float beta,
                        const float* alpha_dev, int m_real, int n_real, int transposed,
                        void* const* out_ptrs, int out_dtype, void* const* w_ptrs, int w_dtype,
                        void* const* pub_ptrs, int pub_dtype, float decay, float lrs, int tile,
                        void* stream) {
  int elt;
  if (elt_of("dmuon_ns_gemm_final", dtype, &elt)) return 1;
  return ns_gemm_final_impl("dmuon_ns_gemm_final", elt, P, ldp, strideP, XT, ldxt, strideXT, X,
                            ldx, strideX, M, N, batch, alpha, beta, alpha_dev, m_real, n_real,
                            transposed, out_ptrs, out_dtype, w_ptrs, w_dtype, pub_ptrs, pub_dtype,
                            decay, lrs, tile, stream);
}

int dmuon_ns_gemm_final_bf16(const void* P, int64_t ldp, int64_t strideP, const void* XT,
                             int64_t ldxt, int64_t strideXT, const void* X, int64_t ldx,
                             int64_t strideX, int M, int N, int batch, float alpha, float beta,
                             const float* alpha_dev, int m_real, int n_real, int transposed,
                             void* const* out_ptrs, int out_dtype, void* const* w_ptrs,
                             int w_dtype, void* const* pub_ptrs, int pub_dtype, float decay,
                             float lrs, int tile, void* stream) {
  return ns_gemm_final_impl("dmuon_ns_gemm_final_bf16", ELT_BF16, P, ldp, strideP, XT, ldxt,
                            strideXT, X, ldx, strideX, M, N, batch, alpha, beta, alpha_dev, m_real,
                            n_real, transposed, out_ptrs, out_dtype, w_ptrs, w_dtype, pub_ptrs,
                            pub_dtype, decay, lrs, tile, stream);
}

int dmuon_muon_pre_partials(int Rp, int Cp) { return pre_blocks_per_mat(Rp, Cp); }

int dmuon_muon_pre(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs, void* Y, int64_t ldy,
                   int64_t strideY, void* YT, int64_t ldyt, int64_t strideYT, float* partials,
                   int rows, int cols, int Rp, int Cp, int batch, float mu, int first_step,
                   int nesterov, void* stream) {
  const char* who = "dmuon_muon_pre";
  if (batch == 0) return 0;
  if (!g_ptrs || (!Y && !YT) || !partials) return fail("%s: NULL argument", who);
  if (g_dtype != DMUON_DTYPE_F32 && g_dtype != DMUON_DTYPE_BF16)
    return fail("%s: unsupported gradient dtype %d", who, g_dtype);
  if (rows <= 0 || cols <= 0 || batch < 0) return fail("%s: bad sizes", who);
  if (Rp % 64 || Cp % 64 || Rp < rows || Cp < cols)
    return fail("%s: padded extent %dx%d must be multiples of 64 covering %dx%d", who, Rp, Cp, rows, cols);
  if ((Y && (!aligned16(Y) || !ld_ok(ldy) || ldy < Cp || !stride_ok(strideY, batch))) ||
      (YT && (!aligned16(YT) || !ld_ok(ldyt) || ldyt < Rp || !stride_ok(strideYT, batch))))
    return fail("%s: bad Y/YT layout", who);
  PreArgs p{};
  p.g_ptrs = g_ptrs; p.g_dtype = g_dtype; p.buf_ptrs = buf_ptrs;
  p.Y = static_cast<uint16_t*>(Y); p.ldy = ldy; p.sY = strideY;
  p.YT = static_cast<uint16_t*>(YT); p.ldyt = ldyt; p.sYT = strideYT;
  p.skip_y = Y ? 0 : 1;
  p.skip_yt = YT ? 0 : 1;
  p.partials = partials;
  p.rows = rows; p.cols = cols; p.Rp = Rp; p.Cp = Cp; p.L = batch;
  p.mu = mu; p.first_step = first_step; p.nesterov = nesterov;
  return check_launch(launch_pre(p, static_cast<hipStream_t>(stream)), who);
}

int dmuon_norm_finalize(const float* partials, int nparts, int batch, float eps, float* scale,
                        float* scale_sq, void* stream) {
  const char* who = "dmuon_norm_finalize";
  if (batch == 0) return 0;
  if (!partials || !scale || !scale_sq || nparts <= 0 || batch < 0) return fail("%s: bad arguments", who);
  return check_launch(launch_norm_finalize(partials, nparts, batch, eps, scale, scale_sq,
                                           static_cast<hipStream_t>(stream)),
                      who);
}

int dmuon_muon_update(void* const* w_ptrs, int w_dtype, const void* const* u_ptrs, int u_dtype,
                      int64_t numel, int batch, float decay, float lrs, void* stream) {
  const char* who = "dmuon_muon_update";
  if (batch == 0 || numel == 0) return 0;
  if (!w_ptrs || !u_ptrs || numel < 0 || batch < 0) return fail("%s: bad arguments", who);
  if ((w_dtype != DMUON_DTYPE_F32 && w_dtype != DMUON_DTYPE_BF16) ||
      (u_dtype != DMUON_DTYPE_F32 && u_dtype != DMUON_DTYPE_BF16))
    return fail("%s: unsupported dtype", who);
  UpdateArgs u{};
  u.w_ptrs = w_ptrs; u.w_dtype = w_dtype; u.u_ptrs = u_ptrs; u.u_dtype = u_dtype;
  u.numel = numel; u.L = batch; u.decay = decay; u.lrs = lrs;
  return check_launch(launch_update(u, static_cast<hipStream_t>(stream)), who);
}

int dmuon_adamw_multi(const int64_t* p_ptrs, const int64_t* g_ptrs, const int64_t* m_ptrs,
                      const int64_t* v_ptrs, const int64_t* pub_ptrs, const int64_t* offsets,
                      int n, int64_t total, int p_dtype, int g_dtype, int pub_dtype, int apply_wd,
                      float wd_scale, float beta1, float alpha1, float beta2, float alpha2,
                      float bc2_sqrt, float eps, float neg_step, void* stream) {
  const char* who = "dmuon_adamw_multi";
  if (n == 0 || total == 0) return 0;
  if (n < 0 || total < 0) return fail("%s: negative tensor count or size", who);
  if (!p_ptrs || !g_ptrs || !m_ptrs || !v_ptrs || !offsets)
    return fail("%s: pointer arrays must be non-NULL", who);
  if ((p_dtype != DMUON_DTYPE_F32 && p_dtype != DMUON_DTYPE_BF16) ||
      (g_dtype != DMUON_DTYPE_F32 && g_dtype != DMUON_DTYPE_BF16))
    return fail("%s: unsupported dtype (p %d, g %d)", who, p_dtype, g_dtype);
  if (pub_ptrs && pub_dtype != DMUON_DTYPE_F32 && pub_dtype != DMUON_DTYPE_BF16)
    return fail("%s: unsupported publish dtype %d", who, pub_dtype);
  if (!(bc2_sqrt > 0.f)) return fail("%s: bias correction must be positive", who);
  AdamWArgs a{};
  a.p_ptrs = p_ptrs; a.g_ptrs = g_ptrs; a.m_ptrs = m_ptrs; a.v_ptrs = v_ptrs;
  a.pub_ptrs = pub_ptrs; a.pub_dtype = pub_dtype;
  a.offsets = offsets; a.n = n; a.total = total;
  a.p_dtype = p_dtype; a.g_dtype = g_dtype; a.apply_wd = apply_wd != 0;
  a.wd_scale = wd_scale; a.beta1 = beta1; a.alpha1 = alpha1; a.beta2 = beta2; a.alpha2 = alpha2;
  a.bc2_sqrt = bc2_sqrt; a.eps = eps; a.neg_step = neg_step;
  const int pb = p_dtype == DMUON_DTYPE_F32 ? 4 : 2, gb = g_dtype == DMUON_DTYPE_F32 ? 4 : 2;
  const double qb = pub_ptrs ? (pub_dtype == DMUON_DTYPE_F32 ? 4 : 2) : 0;
  const double bytes = (double)total * (6.0 * pb + gb + qb);   // read p,g,m,v; write p,m,v(,q)
  hipStream_t st = static_cast<hipStream_t>(stream);
  return timed(PC_ADAMW, 0.0, bytes, st, who, [&] { return launch_adamw(a, st); });
}

static int clip_common(const int64_t* ptrs, const int64_t* numels, const int32_t* dtypes,
                       const int32_t* segments, const int32_t* job_tensor_ids,
                       const int64_t* job_offsets, int64_t n_jobs, int64_t chunk_size,
                       const char* who, ClipArgs* a) {
  if (chunk_size <= 0) return fail("%s: chunk_size must be positive", who);
  if (n_jobs < 0 || n_jobs > 0x7fffffff) return fail("%s: job count out of range", who);
  if (n_jobs > 0 && (!ptrs || !numels || !dtypes || !segments || !job_tensor_ids || !job_offsets))
    return fail("%s: metadata arrays must be non-NULL", who);
  a->ptrs = ptrs; a->numels = numels; a->dtypes = dtypes; a->segments = segments;
  a->job_tensor_ids = job_tensor_ids; a->job_offsets = job_offsets;
  a->n_jobs = n_jobs; a->chunk = chunk_size;
  return 0;
}

int dmuon_segmented_l2_norm_sq(const int64_t* ptrs, const int64_t* numels, const int32_t* dtypes,
                               const int32_t* segments, const int32_t* job_tensor_ids,
                               const int64_t* job_offsets, int64_t n_jobs, int64_t chunk_size,
                               float* local_sq, void* stream) {
  const char* who = "dmuon_segmented_l2_norm_sq";
  ClipArgs a{};
  if (clip_common(ptrs, numels, dtypes, segments, job_tensor_ids, job_offsets, n_jobs, chunk_size,
                  who, &a))
    return 1;
  if (n_jobs == 0) return 0;
  if (!local_sq) return fail("%s: local_sq must be non-NULL", who);
  a.local_sq = local_sq;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return timed(PC_CLIP, 0.0, 0.0, st, who, [&] { return launch_clip_sumsq(a, st); });
}

int dmuon_segmented_scale(const int64_t* ptrs, const int64_t* numels, const int32_t* dtypes,
                          const int32_t* segments, const int32_t* job_tensor_ids,
                          const int64_t* job_offsets, int64_t n_jobs, int64_t chunk_size,
                          const float* coefs, void* stream) {
  const char* who = "dmuon_segmented_scale";
  ClipArgs a{};
  if (clip_common(ptrs, numels, dtypes, segments, job_tensor_ids, job_offsets, n_jobs, chunk_size,
                  who, &a))
    return 1;
  if (n_jobs == 0) return 0;
  if (!coefs) return fail("%s: coefs must be non-NULL", who);
  a.coefs = coefs;
  hipStream_t st = static_cast<hipStream_t>(stream);
  return timed(PC_CLIP, 0.0, 0.0, st, who, [&] { return launch_clip_scale(a, st); });
}

int dmuon_ns_plan(int rows, int cols, int batch, int tile_req, int num_cus, int backend,
                  int* tile, int* m_pad, int* n_pad, int64_t* workspace_bytes) {
  if (!tile || !m_pad || !n_pad || !workspace_bytes) return fail("dmuon_ns_plan: NULL output");
  if (backend != DMUON_NS_DIRECT && backend != DMUON_NS_GRAM)
    return fail("dmuon_ns_plan: unknown NS backend %d", backend);
  return plan(rows, cols, batch, tile_req, num_cus, backend == DMUON_NS_GRAM, tile, m_pad, n_pad,
              workspace_bytes);
}

int dmuon_muon_step_group(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                          float* const* est_ptrs, void* const* w_ptrs, int w_dtype,
                          void* const* pub_ptrs, int pub_dtype, int rows, int cols, int batch,
                          int n_transposed, double lr, double mu, double wd, int nesterov,
                          int first_step,
                          const float* coeffs, int T, int backend, const int* restarts,
                          int n_restarts, float eps, void* workspace, int64_t workspace_bytes,
                          int tile, void* stream) {
  const char* who = "dmuon_muon_step_group";
  if (batch == 0) return 0;
  if (!buf_ptrs || !w_ptrs) return fail("%s: buf_ptrs and w_ptrs must be non-NULL", who);
  // host scalars in double, rounded once to fp32, as torch does with Python-float arguments
  const double scale = 0.2 * sqrt((double)(rows > cols ? rows : cols));
  const float decay = wd > 0.0 ? (float)(1.0 - lr * wd) : 1.f;
  const float lrs = (float)(lr * scale);
  return run_group(g_ptrs, g_dtype, buf_ptrs, est_ptrs, w_ptrs, w_dtype, pub_ptrs, pub_dtype,
                   nullptr, 0, rows, cols, batch, n_transposed, (float)mu, nesterov, first_step,
                   decay, lrs, coeffs, T, backend, restarts, n_restarts, eps, workspace, workspace_bytes, tile,
                   static_cast<hipStream_t>(stream), who);
}

int dmuon_muon_step_group_noalloc(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                                  float* const* est_ptrs, void* const* w_ptrs, int w_dtype,
                                  void* const* pub_ptrs, int pub_dtype, int rows, int cols,
                                  int batch, int n_transposed, double lr, double mu, double wd,
                                  int nesterov,
                                  int first_step, const float* coeffs, int T, int backend,
                                  const int* restarts, int n_restarts, float eps, int tile,
                                  void* stream) {
  const char* who = "dmuon_muon_step_group_noalloc";
  if (batch == 0) return 0;
  if (!buf_ptrs || !w_ptrs) return fail("%s: buf_ptrs and w_ptrs must be non-NULL", who);
  if (backend != DMUON_NS_DIRECT && backend != DMUON_NS_GRAM)
    return fail("%s: unknown NS backend %d", who, backend);
  int t, mp, np_;
  int64_t need;
  if (plan(rows, cols, batch, tile, 0, backend == DMUON_NS_GRAM, &t, &mp, &np_, &need)) return 1;
  if (need > kScratchBytes)
    return fail("%s: this group needs %lld bytes of scratch, more than the %lld bytes the "
                "entry point holds per GPU; split the group or use dmuon_muon_step_group with "
                "a workspace", who, (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (scratch_of_current_device(who, &ws, true, static_cast<hipStream_t>(stream))) return 1;
  NoEvents no_events;
  const double scale = 0.2 * sqrt((double)(rows > cols ? rows : cols));
  const float decay = wd > 0.0 ? (float)(1.0 - lr * wd) : 1.f;
  const float lrs = (float)(lr * scale);
  return run_group(g_ptrs, g_dtype, buf_ptrs, est_ptrs, w_ptrs, w_dtype, pub_ptrs, pub_dtype,
                   nullptr, 0, rows, cols, batch, n_transposed, (float)mu, nesterov, first_step,
                   decay, lrs, coeffs, T, backend, restarts, n_restarts, eps, ws, kScratchBytes, tile,
                   static_cast<hipStream_t>(stream), who);
}

int dmuon_noalloc_init(void** scratch_out, int64_t* scratch_bytes) {
  void* p = nullptr;
  if (scratch_of_current_device("dmuon_noalloc_init", &p)) return 1;
  if (scratch_out) *scratch_out = p;
  if (scratch_bytes) *scratch_bytes = kScratchBytes;
  return 0;
}

int dmuon_newton_schulz_group(void* const* g_ptrs, int g_dtype, void* const* out_ptrs,
                              int out_dtype, int rows, int cols, int batch, int n_transposed,
                              const float* coeffs,
                              int T, int backend, const int* restarts, int n_restarts, float eps,
                              void* workspace, int64_t workspace_bytes, int tile, void* stream) {
  const char* who = "dmuon_newton_schulz_group";
  if (batch == 0) return 0;
  if (!out_ptrs) return fail("%s: out_ptrs must be non-NULL", who);
  return run_group(g_ptrs, g_dtype, nullptr, nullptr, nullptr, 0, nullptr, 0, out_ptrs, out_dtype,
                   rows, cols, batch, n_transposed, 0.f, 0, 1, 1.f, 0.f, coeffs, T, backend,
                   restarts, n_restarts, eps, workspace, workspace_bytes, tile,
                   static_cast<hipStream_t>(stream), who);
}

int dmuon_muon_stage_group(void* const* g_ptrs, int g_dtype, float* const* buf_ptrs,
                           float* const* est_ptrs, int rows, int cols, int batch,
                           int n_transposed, double mu, int nesterov, int first_step,
                           int backend, float eps, void* workspace, int64_t workspace_bytes,
                           int tile, void* stream) {
  const char* who = "dmuon_muon_stage_group";
  if (batch == 0) return 0;
  if (!buf_ptrs) return fail("%s: buf_ptrs must be non-NULL", who);
  return run_group(g_ptrs, g_dtype, buf_ptrs, est_ptrs, nullptr, 0, nullptr, 0, nullptr, 0, rows,
                   cols, batch, n_transposed, (float)mu, nesterov, first_step, 1.f, 0.f, nullptr,
                   0, backend,
                   nullptr, 0, eps, workspace, workspace_bytes, tile,
                   static_cast<hipStream_t>(stream), who, PH_STAGE);
}

int dmuon_muon_apply_group(void* const* w_ptrs, int w_dtype, void* const* pub_ptrs,
                           int pub_dtype, int rows, int cols, int batch, int n_transposed,
                           double lr, double wd,
                           const float* coeffs, int T, int backend, const int* restarts,
                           int n_restarts, void* workspace, int64_t workspace_bytes, int tile,
                           void* stream) {
  const char* who = "dmuon_muon_apply_group";
  if (batch == 0) return 0;
  if (!w_ptrs) return fail("%s: w_ptrs must be non-NULL", who);
  const double scale = 0.2 * sqrt((double)(rows > cols ? rows : cols));
  const float decay = wd > 0.0 ? (float)(1.0 - lr * wd) : 1.f;
  const float lrs = (float)(lr * scale);
  return run_group(nullptr, 0, nullptr, nullptr, w_ptrs, w_dtype, pub_ptrs, pub_dtype, nullptr, 0,
                   rows, cols, batch, n_transposed, 0.f, 0, 0, decay, lrs, coeffs, T, backend,
                   restarts, n_restarts, 0.f, workspace, workspace_bytes, tile, static_cast<hipStream_t>(stream), who,
                   PH_APPLY);
}

}  // extern "C"

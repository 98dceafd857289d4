// NT-form bf16 / fp16 MFMA product family for the Newton-Schulz iteration on gfx950 (CDNA4).
//
//   acc[i][j] = sum_k A[i][k] * B[j][k]          (both operands K-contiguous, row-major)
//
// Three uses inside one NS iteration on X (m x n, m <= n):
//   SYRK   A = X X^T             A=B=X,   upper-triangle tiles, mirror written   (EPI_SYM)
//   POLY   P = c*A A^T + b*A     A=B=A,   upper-triangle tiles, C=A              (EPI_SYM)
//   GEMM   X' = a*X + P X        A=P, B=X^T (the transposed copy kept alongside X)
//          writes X' and X'^T (EPI_NS), or on the last iteration applies the Muon
//          weight update in the original orientation (EPI_FINAL)
//
// Two tile machines on v_mfma_f32_16x16x32 (fp32 accumulate), K staged through LDS in 64-wide
// slices by direct global->LDS DMA (buffer_load_dwordx4 ... lds: each wave instruction fills
// 1 KiB of LDS, no staging registers) into a two-slot ring, 16-byte chunks under an XOR swizzle
// (chunk ^ f(row)) so that every 16-lane pass of a fragment read covers all 64 banks:
//   256x256 tiles (nt_pp_kernel): 8 waves of 128x64, two per SIMD, in a ping-pong schedule --
//     one wave of a SIMD issues its MFMAs while the other reads its next fragments and moves
//     the operands, so barrier and memory waits overlap MFMA work;
//   128x128 tiles (nt_mfma_kernel): 4 waves of 64x64, two blocks per CU, for batches too small
//     to fill the machine with 256-tiles; fragments double-buffered per substep, one barrier
//     per slice. Per launch (launch_nt), a 128-tile product that leaves CUs idle runs on 64x64
//     tiles (4 waves, eight-slot ring) or on 8 waves with a four-slot ring, one block per CU,
//     and one with more than two 128-tiles per CU may take 256-tiles: such small launches wait
//     on load latency, not bandwidth. Tile size, waves and ring depth change where operands
//     wait, not the arithmetic, so every variant gives the same bits.
#include "dmuon_amd_internal.h"

#include <atomic>
#include <type_traits>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

namespace dmuon {
namespace {


__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Operand / intermediate element type of one kernel instance: E = ELT_BF16 or ELT_F16. The
// product operands, the addend C and the outputs D / D^T are 16-bit words of that type; the
// accumulators are fp32 either way (round to nearest even on the way out).
template <int E>
__device__ __forceinline__ uint16_t to_elt(float f) {
  if constexpr (E == ELT_F16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  else return f2bf(f);
}
template <int E>
__device__ __forceinline__ float from_elt(uint16_t h) {
  if constexpr (E == ELT_F16) return static_cast<float>(__builtin_bit_cast(_Float16, h));
  else return bf2f(h);
}
// Two values rounded (nearest even) to E and packed, low half first: one packed convert
// instruction on gfx950 instead of two converts and a pack.
template <int E>
__device__ __forceinline__ unsigned pack2_elt(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  if constexpr (E == ELT_F16) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{lo, hi}, f16x2_t));
  } else {
    typedef __bf16 b16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{lo, hi}, b16x2_t));
  }
}
// v_mfma_f32_16x16x32: a lane holds row (l % 16) of both operands at k-chunk l / 16, and four
// consecutive output columns of one row. It gives the same bits as the 32x32x16 form (measured:
// the products accumulate in the same order and round identically), and on MI355X it sustains
// a higher clock under the board's power limit at equal MFMA work (sustained MFMA-only loops:
// 1.90 vs 1.65-1.69 PFLOP/s; with 0.5 KB of fragment reads per 32 KFLOP: 1.70 vs 1.53).
template <int E>
__device__ __forceinline__ f32x4_t mfma_16x16x32(bf16x8_t b, bf16x8_t a, f32x4_t c) {
  if constexpr (E == ELT_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, b),
                                                  __builtin_bit_cast(f16x8_t, a), c, 0, 0, 0);
  else return __builtin_amdgcn_mfma_f32_16x16x32_bf16(b, a, c, 0, 0, 0);
}

// k-major operand (stored [K][N], N contiguous): a slice of BK k-rows sits in LDS row by row,
// 16-byte chunk c of row r at slot c ^ kswz(r). ds_read_b64_tr_b16 gives lane i of each 16-lane
// group element i % 4 of the 8 bytes addressed by lane 4j + i / 4 of that group (j = 0..3), so
// when the 16 lanes of group g address rows 8g + s / 4 (s = lane % 16) at values 4 (s % 4) ..
// of a 16-value block, lane i receives the 4 consecutive k of value i -- half of the 16x16x32
// operand; a second read 4 rows further gives the other half. The swizzle spreads the 16 rows
// of one read over all 64 banks (two passes for its 512 bytes).
typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int kswz(int r) { return 2 * ((r & 3) | (((r >> 3) & 1) << 2)); }
__device__ __forceinline__ bf16x8_t read_kmajor(const char* p, int row_bytes) {
  typedef __attribute__((address_space(3))) s16x4_t* lds_s4_t;
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(p));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(p + 4 * row_bytes));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
// The ping-pong kernel keeps a k-major B tile as four column blocks of 64 values, BK rows of
// 128 bytes each; rows r and r + 1 share a 256-byte bank line, so the swizzle of a read's 16
// rows (two passes) comes from row bits 1 and 3.
__device__ __forceinline__ int kswz64(int r) { return 2 * (((r >> 1) & 1) | (((r >> 3) & 1) << 1)); }
__device__ __forceinline__ int kmajor64_lane_off(int lane, int n0) {
  const int s16 = lane & 15, g = lane >> 4;
  const int h = 2 * (((s16 >> 3) & 1) | ((g & 1) << 1));   // kswz64 of every row this lane reads
  const int chunk = ((n0 / 8) ^ h) | ((s16 & 3) >> 1);
  return (8 * g + (s16 >> 2)) * 128 + chunk * 16 + (s16 & 1) * 8;
}
// byte offset, within a k-major slice of `row_bytes`-wide rows, of what lane (s = lane % 16,
// g = lane / 16) addresses for the 16-value block starting at value n0 (a multiple of 16)
__device__ __forceinline__ int kmajor_lane_off(int lane, int n0, int row_bytes) {
  const int s16 = lane & 15, g = lane >> 4;
  const int h = 2 * ((s16 >> 2) | ((g & 1) << 2));          // kswz of every row this lane reads
  const int chunk = ((n0 / 8) ^ h) | ((s16 & 3) >> 1);
  return (8 * g + (s16 >> 2)) * row_bytes + chunk * 16 + (s16 & 1) * 8;
}

// A wave's accumulators as the epilogue walks them: per 32-row slab x of the wave tile, NQ groups
// of four values -- group q of a lane holds slab row row(q), columns col(q) .. col(q) + 3. Indices
// are compile-time after unrolling, so the registers are addressed statically.
template <int BI, int BJ>            // BI x BJ blocks of 16x16 (v_mfma_f32_16x16x32)
struct Acc16 {
  static constexpr int SLABS = BI / 2, NQ = 2 * BJ;
  f32x4_t (&acc)[BI][BJ];
  int lane;
  __device__ __forceinline__ int row(int q) const { return 16 * (q / BJ) + (lane & 15); }
  __device__ __forceinline__ int col(int q) const { return 16 * (q % BJ) + 4 * (lane >> 4); }
  __device__ __forceinline__ float val(int x, int q, int e) const { return acc[2 * x + q / BJ][q % BJ][e]; }
};

// Maps the hardware block id (blocks are dealt round-robin over the 8 XCDs) to a logical tile.
// The logical tiles go in windows of 8 x kXcdWindow, one run of kXcdWindow consecutive tiles
// per XCD: with a window of one tile per CU (gfx950: 8 XCDs x 32 CUs), the blocks resident at
// any time cover one contiguous stretch of the tile order, so all XCDs work on the same few
// matrices and the operand panels one XCD's L2 misses bring into the shared Infinity Cache serve
// the others (c5 step 299.0 -> 291.9 ms, NT 50.0 -> 51.3% of peak, same box), while each XCD's
// own run keeps the neighbouring tiles that share panels in its L2. (Whole contiguous ranges per
// XCD, every XCD on its own matrices, and windows of 8, 16, 24, 48 or 64 tiles per XCD were
// slower.) The last partial window falls back to contiguous ranges of its remainder.
__host__ __device__ __forceinline__ int xcd_remap_contig(int b, int nb) {
  const int q = nb >> 3, r = nb & 7;
  const int x = b & 7, idx = b >> 3;
  const int base = (x < r) ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  return base + idx;
}
constexpr int kXcdWindow = 32;
__host__ __device__ __forceinline__ int xcd_remap(int b, int nb) {
  constexpr int W = kXcdWindow, WW = 8 * kXcdWindow;
  const int x = b & 7, idx = b >> 3;
  const int full = nb / WW;
  if (idx < full * W) return (idx / W) * WW + x * W + idx % W;
  return full * WW + xcd_remap_contig(b - full * WW, nb - full * WW);
}

template <int BM_, int BN_, int BK_, int S_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, S = S_, WM = WM_, WN = WN_;
  static constexpr int NW = WM * WN;              // waves per block
  static constexpr int NT = 64 * NW;              // threads per block
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave sub-tile
  static constexpr int TI = WTM / 32;             // MFMA blocks along i per wave
  static constexpr int TJ = WTN / 32;             // MFMA blocks along j per wave
  static constexpr int ROWB = BK * 2;             // bytes of one tile row in LDS
  static constexpr int CPR = BK / 8;              // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROWB;         // rows filled by one DMA wave instruction
  static constexpr int A_INST = BM / RPI / NW;    // DMA instructions per wave per slice
  static constexpr int B_INST = BN / RPI / NW;
  static constexpr int LPT = A_INST + B_INST;     // outstanding loads a slice adds per wave
  static constexpr int RPL = 256 / ROWB;          // rows per 256-byte LDS bank line (64 banks)
  static constexpr int A_BYTES = BM * ROWB;
  static constexpr int STAGE = (BM + BN) * ROWB;
  // epilogue staging per wave: one 32-row slab row-major at pitch EPN (WTN values + 16 B: rows
  // stay 16-byte aligned for the 16-byte reads of the stores), two slabs transposed at pitch EPT
  // (64 values + 16 B: the four lane groups of a scatter hit different banks), and the fp32 slab
  // of the final step (32 rows of WTN + 4 floats)
  static constexpr int EPN = WTN * 2 + 16;
  static constexpr int EPT = 64 * 2 + 16;
  static constexpr int EPF = 32 * (WTN + 4) * 4;
  static constexpr int EPI_MAX2 = 32 * EPN + WTN * EPT;
  static constexpr int EPI_REGION_RAW = (EPI_MAX2 > EPF ? EPI_MAX2 : EPF);
  static constexpr int EPI_REGION = (EPI_REGION_RAW + 15) / 16 * 16;
  static constexpr int LDS_BYTES = (S * STAGE > NW * EPI_REGION ? S * STAGE : NW * EPI_REGION);
  static_assert(BM % (NW * RPI) == 0 && BN % (NW * RPI) == 0, "tile rows vs DMA rows");
  static_assert(S * LPT <= 63 && S <= 10, "vmcnt range (the prologue has S slices in flight)");
  // LDS slot of 16-byte chunk kc of row r. A ds_read_b128 serves 16 lanes (256 B, all 64
  // banks) per pass; a fragment read has those 16 lanes on 16 consecutive rows at one chunk,
  // so rows sharing a bank line (r % RPL) must take distinct slots along r / RPL.
  static __device__ __forceinline__ int slot(int kc, int r) { return kc ^ ((r / RPL) & (CPR - 1)); }
};

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left alone (gfx9 encoding: vmcnt[3:0] + vmcnt[5:4] at
// bits 15:14, expcnt bits 6:4 = 7, lgkmcnt bits 11:8 = 15).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// Workgroup barrier without the memory fence of __syncthreads (which would also wait for every
// in-flight LDS DMA); the empty asm statements keep the compiler from moving LDS accesses
// across it.
__device__ __forceinline__ void bare_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// A barrier that is also a scheduling fence: the compiler treats s_barrier as ordering memory
// accesses only, and would otherwise move arithmetic (the MFMAs of a ping-pong phase) across it.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <class T>
__device__ __forceinline__ void wait_slices() {
  // wait until slice 0 of the ring has landed: at most S - 1 newer slices (T::LPT loads each)
  // still in flight
  wait_vmcnt<(T::S - 1) * T::LPT>();
}

// End-of-slice meeting point: wait until at most N loads of this wave are in flight (its share
// of the next slice has landed) and all of its LDS reads have returned (its fragments of the
// current slot are in registers), then s_barrier. gfx9 s_waitcnt encoding: vmcnt[3:0] +
// vmcnt[5:4] at bits 15:14, expcnt bits 6:4 = 7 (untouched), lgkmcnt bits 11:8 = 0.
template <int N>
__device__ __forceinline__ void slice_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// sched_group_barrier sequence of one substep: M MFMAs, each followed by up to K = ceil((R+D)/M)
// memory instructions, DS reads (R) first, then DMA (D, VMEM reads). The builtin needs literal
// arguments, hence the compile-time recursion.
template <int I, int M, int R, int D>
__device__ __forceinline__ void sched_front() {
  if constexpr (I < M) {
    constexpr int N = R + D, K = (N + M - 1) / M;
    constexpr int lo = K * I < N ? K * I : N, hi = K * (I + 1) < N ? K * (I + 1) : N;
    constexpr int rlo = lo < R ? lo : R, rhi = hi < R ? hi : R;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if constexpr (rhi > rlo) __builtin_amdgcn_sched_group_barrier(0x100, rhi - rlo, 0);
    if constexpr (hi - lo > rhi - rlo)
      __builtin_amdgcn_sched_group_barrier(0x020, (hi - lo) - (rhi - rlo), 0);
    sched_front<I + 1, M, R, D>();
  }
}
template <int N, int M, int R>
__device__ __forceinline__ void sched_substeps() {
  if constexpr (N > 0) {
    sched_front<0, M, R, 0>();
    sched_substeps<N - 1, M, R>();
  }
}

// Waves per SIMD: a 128x128 wave tile holds 256 accumulator registers, so its block runs one
// wave per SIMD with the whole 512-entry register file; smaller wave tiles run two blocks per
// CU, unless the block's LDS (more than half of the CU's 160 KiB) leaves room for one block per
// CU only. A block of more than four waves puts NW / 4 of them on each SIMD.
template <int BM, int BN, int BK, int S, int WM, int WN>
struct Occupancy {
  static constexpr int BPC =
      (BM / WM) * (BN / WN) >= 128 * 128 || Tile<BM, BN, BK, S, WM, WN>::LDS_BYTES > 80 * 1024
          ? 1 : 2;
  static constexpr int WPE = BPC * ((WM * WN + 3) / 4);
};

// First K slice of the tile's loop (see NtArgs::c_in): the slices that hold the tile's addend
// values -- columns j0.. of A (C is A) or rows i0.. of B (C is B), read in the 256-aligned block
// that contains them -- come last (a block that ends past the loop's KT slices starts it at 0).
__device__ __forceinline__ int first_slice(const NtArgs& a, int i0, int j0, int BK, int KT) {
  if (a.c_in == C_NONE) return 0;
  const int blk = (a.c_in == C_IS_A ? j0 : i0) / 256 + 1;
  return min(blk * 256 / BK, KT) % KT;
}

// Logical tile of this block: matrix l of the batch, tile row bi, tile column bj.
struct TilePos {
  int l, bi, bj;
};

// tile rows per group of the walks (with the XCD windows, 4 or 16 rows for the triangle walk
// and 4 or 16 for the rectangular one measured 0.3-0.9% slower per c5 step)
constexpr int kTileGroupTri = 8, kTileGroupRect = 8;
__device__ __forceinline__ TilePos decode_tile(const NtArgs& a, int hb, int nblocks) {
  const int lb = xcd_remap(hb, nblocks);
  const int l = lb / a.tiles_per_mat;
  int t = lb - l * a.tiles_per_mat;
  int bi, bj;
  if (a.tri) {
    // upper triangle in groups of 8 tile-rows, each walked column-major: first the group's
    // own triangular diagonal block (column c holds rows 0..c), then full 8-row columns, so
    // that the tiles resident on one XCD at a time form compact blocks sharing panels in L2
    int g0 = 0, gs = 0;
    for (;;) {
      gs = min(kTileGroupTri, a.mt - g0);
      const int cnt = gs * (gs + 1) / 2 + gs * (a.mt - g0 - gs);
      if (t < cnt) break;
      t -= cnt;
      g0 += gs;
    }
    const int ntri = gs * (gs + 1) / 2;
    if (t < ntri) {
      int c = 0;
      while (t > c) { t -= c + 1; ++c; }
      bi = g0 + t;
      bj = g0 + c;
    } else {
      t -= ntri;
      bi = g0 + t % gs;
      bj = g0 + gs + t / gs;
    }
  } else {
    // groups of 8 tile-rows walked column-major so neighbouring blocks share B panels
    const int group = kTileGroupRect;
    const int per_group = group * a.nt;
    const int g = t / per_group;
    const int first = g * group;
    const int gsize = min(a.mt - first, group);
    const int r = t - g * per_group;
    bi = first + r % gsize;
    bj = r / gsize;
  }
  return TilePos{l, bi, bj};
}

// Epilogue of a finished tile: the accumulators of this wave (rows iw.., columns jw.. of
// matrix l) through the MODE-specific staging and stores. Uses the per-wave LDS area
// smem + wave * EPI_REGION; the caller guarantees no operand slice is still in use there.
template <class T, int MODE, int E, class Acc>
__device__ __forceinline__ void nt_epilogue(const NtArgs& a, char* smem, const Acc& acc, int l,
                                            int bi, int bj, int i0, int j0, int lane, int wave,
                                            int wi, int wj) {
  constexpr int NQ = Acc::NQ;
  static_assert(Acc::SLABS * 32 == T::WTM && NQ * 4 * 64 == 32 * T::WTN, "accumulator layout");
  const int iw = i0 + wi * T::WTM, jw = j0 + wj * T::WTN;
  const uint16_t* Cb = a.C ? a.C + (long long)l * a.sC : nullptr;
  // addend C (X for the NS step, A for the polynomial), one 32-row slab at a time, read row by
  // row in whole 128-byte lines per instruction (WTN / 4 lanes per row, 4 values each): group q
  // of slab x is row iw + 32x + CRI q + lane / CLR, columns jw + 4 (lane % CLR) .. +3. The
  // epilogues pass it through the wave's LDS slab to the accumulator layout: loading it in that
  // layout directly touches 16 lines per instruction for 32 bytes each, which made the addend
  // read cost twice as long per tile (measured on a 34-wave triangle product: ~190 us per
  // launch against ~90)
  constexpr int CLR = T::WTN / 4, CRI = 64 / CLR;
  static_assert(CRI * NQ == 32, "coalesced addend groups cover the slab");
  auto load_c_rows = [&](int x, u32x2_t* dst) {
    const uint16_t* crow =
        Cb + (long long)(iw + 32 * x + lane / CLR) * a.ldc + jw + 4 * (lane % CLR);
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      dst[q] = *reinterpret_cast<const u32x2_t*>(crow + (long long)(CRI * q) * a.ldc);
  };
  float s = a.alpha;
  if (a.alpha_dev) s *= a.alpha_dev[l];

  if constexpr (MODE == EPI_SYM || MODE == EPI_NS) {
    // Each 32-row slab of the wave tile goes through a small per-wave LDS staging area row-major
    // for D, and pairs of slabs transposed for D^T (NS step) or the mirrored block (SYRK), so
    // that the global stores are whole 128-byte row segments (8 B x 16 lanes for a D row,
    // 16 B x 8 lanes for a 64-value D^T row) instead of scattered 2-byte stores.
    static_assert(Acc::SLABS % 2 == 0, "transposed rows pair the slabs");
    // EPI_NS may write D^T alone (D == nullptr): the last Q update of a Gram segment, which
    // runs transposed and produces the row form the Q X product reads
    const bool row_out = MODE == EPI_SYM || a.D != nullptr;
    uint16_t* Db = row_out ? a.D + (long long)l * a.sD : nullptr;
    uint16_t* DTb = nullptr;
    long long ldt = 0;
    // diagonal tile of a result that must be exactly symmetric: each value computed for (i, j)
    // with i <= j is stored at (i, j) by the row path and at (j, i) by the mirror path, and the
    // values computed below the diagonal are dropped (a product of two different symmetric
    // factors is symmetric only to rounding otherwise); both paths mask element-wise only in
    // the chunks that straddle the diagonal
    const bool diag = MODE == EPI_SYM && a.sym_exact && a.tri && bi == bj;
    if constexpr (MODE == EPI_SYM) {
      // mirror into the lower triangle
      if (a.tri && (bi != bj || a.sym_exact)) { DTb = Db; ldt = a.ldd; }
    } else {
      if (a.DT) { DTb = a.DT + (long long)l * a.sDT; ldt = a.lddt; }
    }
    char* reg = smem + wave * T::EPI_REGION;
    char* regt = reg + 32 * T::EPN;               // [WTN][64] transposed pair of slabs
    // optional second output of a triangle product: D2 = D + diag2 * I (same layout as D; the
    // diagonal only lives in the straddling chunks of diagonal tiles' row path)
    uint16_t* D2b = nullptr;
    if constexpr (MODE == EPI_SYM) {
      if (a.D2) D2b = a.D2 + (long long)l * a.sD;
    }
    u32x2_t cbuf[2][NQ];
    if (Cb) load_c_rows(0, cbuf[0]);
#pragma unroll
    for (int x = 0; x < Acc::SLABS; ++x) {
      if (Cb) {
        // slab x's addend rows into the wave's slab area, read back in accumulator layout (one
        // wave's LDS accesses complete in order, so neither needs a barrier; the previous
        // slab's reads of this area were issued before)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          *reinterpret_cast<u32x2_t*>(reg + (CRI * q + lane / CLR) * T::EPN +
                                      8 * (lane % CLR)) = cbuf[x & 1][q];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          cbuf[x & 1][q] = *reinterpret_cast<const u32x2_t*>(reg + acc.row(q) * T::EPN +
                                                               acc.col(q) * 2);
      }
      if (Cb && x + 1 < Acc::SLABS) load_c_rows(x + 1, cbuf[(x + 1) & 1]);
      // r = s v + beta c (SYM; + diag where i == j) or s (v + beta c) (NS), rounded to E. The
      // tests that do not depend on the element -- an addend at all, a slab that meets the
      // diagonal -- are taken once per slab; without C the addend term is the constant
      // beta * 0, so every element takes the same operations as with C.
      u32x2_t o2[NQ];
      const bool slab_diag = MODE == EPI_SYM && iw + 32 * x < jw + T::WTN && jw < iw + 32 * x + 32;
      const float bz = a.beta * 0.f;
      float r[NQ][4];
      if (Cb) {
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          const u32x2_t c2 = cbuf[x & 1][q];
          const float cv[4] = {from_elt<E>(c2.x & 0xffff), from_elt<E>(c2.x >> 16),
                               from_elt<E>(c2.y & 0xffff), from_elt<E>(c2.y >> 16)};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc.val(x, q, e);
            if constexpr (MODE == EPI_SYM) r[q][e] = s * v + a.beta * cv[e];
            else r[q][e] = s * (v + a.beta * cv[e]);
          }
        }
      } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc.val(x, q, e);
            if constexpr (MODE == EPI_SYM) r[q][e] = s * v + bz;
            else r[q][e] = s * (v + bz);
          }
      }
      if (slab_diag) {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (iw + 32 * x + acc.row(q) == jw + acc.col(q) + e) r[q][e] += a.diag;
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        o2[q].x = pack2_elt<E>(r[q][0], r[q][1]);
        o2[q].y = pack2_elt<E>(r[q][2], r[q][3]);
        if (row_out)
          *reinterpret_cast<u32x2_t*>(reg + acc.row(q) * T::EPN + acc.col(q) * 2) = o2[q];
      }
      if (row_out) {
        // the slab as whole 16-byte row chunks (8 lanes per 64-value row), all of its LDS reads
        // ahead of the stores
        static_assert(T::EPN % 16 == 0, "16-byte slab rows");
        constexpr int CPRW = T::WTN / 8;          // 16-byte chunks per slab row
        constexpr int RPIT = 64 / CPRW;           // slab rows per wave instruction
        constexpr int NR = 32 / RPIT;
        const int cr = lane / CPRW, cc = lane % CPRW;
        const long long doff = (long long)(iw + 32 * x + cr) * a.ldd + jw + 8 * cc;
        u32x4_t dv[NR];
#pragma unroll
        for (int k = 0; k < NR; ++k)
          dv[k] = *reinterpret_cast<const u32x4_t*>(reg + (k * RPIT + cr) * T::EPN + 16 * cc);
        if (!diag) {
          // non-temporal: the outputs of a launch exceed L2 and the next product streams them
          // back from HBM / Infinity Cache anyway (measured 0.9% on the c5 step)
#pragma unroll
          for (int k = 0; k < NR; ++k)
            __builtin_nontemporal_store(
                dv[k], reinterpret_cast<u32x4_t*>(Db + doff + (long long)k * RPIT * a.ldd));
          if (D2b) {
#pragma unroll
            for (int k = 0; k < NR; ++k)
              __builtin_nontemporal_store(
                  dv[k], reinterpret_cast<u32x4_t*>(D2b + doff + (long long)k * RPIT * a.ldd));
          }
        } else {
#pragma unroll
          for (int k = 0; k < NR; ++k) {
            const u32x4_t v = dv[k];
            const long long o = doff + (long long)k * RPIT * a.ldd;
            // diagonal tile: row i keeps columns j >= i (chunk j0 .. j0+7)
            const int di = iw + 32 * x + k * RPIT + cr, dj = jw + 8 * cc;
            if (dj > di) {
              __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(Db + o));
              if (D2b) __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(D2b + o));
            } else if (dj + 7 >= di) {
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                if (dj + e < di) continue;
                const unsigned word = v[e >> 1];
                const uint16_t h = (uint16_t)((e & 1) ? (word >> 16) : (word & 0xffff));
                Db[o + e] = h;
                if (D2b) D2b[o + e] = dj + e == di ? to_elt<E>(from_elt<E>(h) + a.diag2) : h;
              }
            }
          }
        }
      }
      if (DTb) {
        // slab x into columns 32 (x & 1) .. + 31 of the transposed pair; each lane scatters its
        // 4 consecutive j
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          uint16_t* col = reinterpret_cast<uint16_t*>(regt + acc.col(q) * T::EPT) +
                          32 * (x & 1) + acc.row(q);
          const u32x2_t p = o2[q];
          col[0] = (uint16_t)(p.x & 0xffff);
          col[T::EPT / 2] = (uint16_t)(p.x >> 16);
          col[T::EPT] = (uint16_t)(p.y & 0xffff);
          col[3 * T::EPT / 2] = (uint16_t)(p.y >> 16);
        }
      }
      if (DTb && (x & 1)) {
        // the pair (slabs x - 1, x): D^T rows j of 64 values i = iw + 32 (x - 1) .. + 63; the
        // 16-byte chunks of a D^T row are 8 lanes, so a store writes 8 whole 128-byte row
        // segments (a transposing read of a row-major pair would give 16 lanes one row each and
        // 64-byte segments: measured 1-4% slower)
        const int cr = lane >> 3, cc = lane & 7;  // 8 lanes x 16 B per 64-value row
        const int ip = iw + 32 * (x - 1);
        const long long toff = (long long)(jw + cr) * ldt + ip + 8 * cc;
        uint16_t* dst = DTb + toff;
#pragma unroll
        for (int r0 = 0; r0 < T::WTN; r0 += 8) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(regt + (r0 + cr) * T::EPT + 16 * cc);
          // diagonal tile: output row j keeps columns i < j (chunk i0 .. i0+7)
          const int dj = jw + r0 + cr, di = ip + 8 * cc;
          if (!diag || di + 7 < dj) {
            __builtin_nontemporal_store(v,
                                        reinterpret_cast<u32x4_t*>(dst + (long long)r0 * ldt));
            if (D2b)
              __builtin_nontemporal_store(
                  v, reinterpret_cast<u32x4_t*>(D2b + toff + (long long)r0 * ldt));
          } else if (di < dj) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              if (di + e >= dj) continue;
              const unsigned word = v[e >> 1];
              const uint16_t h = (uint16_t)((e & 1) ? (word >> 16) : (word & 0xffff));
              dst[(long long)r0 * ldt + e] = h;
              if (D2b) D2b[toff + (long long)r0 * ldt + e] = h;
            }
          }
        }
      }
    }
  } else {
    // EPI_FINAL: U = s*(acc + beta*C) for the real m_real x n_real corner, stored/applied in
    // the original orientation (transposed: original[j][i]). Each 32-row slab of a wave's
    // tile goes through LDS (fp32) so the weight read-modify-write is coalesced in either
    // orientation and the register-resident accumulators are only indexed statically.
    constexpr int kLd = T::WTN + 4;
    float* slab = reinterpret_cast<float*>(smem + wave * T::EPI_REGION);
    void* outp = a.out_ptrs ? a.out_ptrs[l] : nullptr;
    void* wp = a.w_ptrs ? a.w_ptrs[l] : nullptr;
    void* pp = (wp && a.pub_ptrs) ? a.pub_ptrs[l] : nullptr;   // forward copy of the new W
    // the last n_flip matrices of the batch are stored in the other orientation
    const bool tr = (a.transposed != 0) != (l >= a.L - a.n_flip);
    const long long pitch = tr ? a.m_real : a.n_real;
    // 16-byte vectors need 16-byte aligned bases (torch allocations are; views may not be)
    const bool valign = ((reinterpret_cast<uintptr_t>(wp) | reinterpret_cast<uintptr_t>(outp) |
                          reinterpret_cast<uintptr_t>(pp)) & 15) == 0;
#pragma unroll
    for (int x = 0; x < Acc::SLABS; ++x) {
      u32x2_t cfin[NQ];
      if (Cb) {
        // the addend's rows as whole lines, through the slab area into the accumulator layout
        // (all of them read back before the fp32 values below overwrite the area)
        load_c_rows(x, cfin);
        char* reg = smem + wave * T::EPI_REGION;
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          *reinterpret_cast<u32x2_t*>(reg + (CRI * q + lane / CLR) * T::EPN +
                                      8 * (lane % CLR)) = cfin[q];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          cfin[q] = *reinterpret_cast<const u32x2_t*>(reg + acc.row(q) * T::EPN + acc.col(q) * 2);
      }
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        float cv[4] = {0.f, 0.f, 0.f, 0.f};
        if (Cb) {
          const u32x2_t c2 = cfin[q];
          cv[0] = from_elt<E>(c2.x & 0xffff); cv[1] = from_elt<E>(c2.x >> 16);
          cv[2] = from_elt<E>(c2.y & 0xffff); cv[3] = from_elt<E>(c2.y >> 16);
        }
        float4 u4;
        u4.x = s * (acc.val(x, q, 0) + a.beta * cv[0]);
        u4.y = s * (acc.val(x, q, 1) + a.beta * cv[1]);
        u4.z = s * (acc.val(x, q, 2) + a.beta * cv[2]);
        u4.w = s * (acc.val(x, q, 3) + a.beta * cv[3]);
        *reinterpret_cast<float4*>(slab + acc.row(q) * kLd + acc.col(q)) = u4;
      }
      const int ibase = iw + 32 * x;
      // Read-modify-write of the slab in 8-element vectors (16 B of bf16 / 32 B of fp32):
      // normal orientation: vector = 8 consecutive j of one row i (8 lanes per 64-column row);
      // transposed: vector = 8 consecutive i of one original row j (4 lanes per 32-row column).
      // All weight loads of the slab are issued before any store. Vectors that cross the real
      // extent, or rows whose pitch breaks 16-byte alignment, take the per-element path.
      constexpr int NV = 32 * T::WTN / 8 / 64;
      const bool vpitch = (pitch & 7) == 0 && valign;
      long long voff[NV];
      bool vfull[NV];
      int vr[NV], vc[NV];
      u32x4_t wraw[NV][2];
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int idx = v * 64 + lane;
        if (!tr) {
          vr[v] = idx / (T::WTN / 8);
          vc[v] = (idx % (T::WTN / 8)) * 8;
          const int i = ibase + vr[v], j = jw + vc[v];
          voff[v] = (long long)i * pitch + j;
          vfull[v] = vpitch && i < a.m_real && j + 7 < a.n_real;
        } else {
          vc[v] = idx / 4;
          vr[v] = (idx % 4) * 8;
          const int i = ibase + vr[v], j = jw + vc[v];
          voff[v] = (long long)j * pitch + i;
          vfull[v] = vpitch && j < a.n_real && i + 7 < a.m_real;
        }
        if (wp && vfull[v]) {
          if (a.w_dtype == DT_F32) {
            const u32x4_t* q = reinterpret_cast<const u32x4_t*>(static_cast<const float*>(wp) + voff[v]);
            wraw[v][0] = q[0];
            wraw[v][1] = q[1];
          } else {
            wraw[v][0] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(wp) + voff[v]);
          }
        }
      }
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        float u[8];
#pragma unroll
        for (int t = 0; t < 8; ++t)
          u[t] = tr ? slab[(vr[v] + t) * kLd + vc[v]] : slab[vr[v] * kLd + vc[v] + t];
        if (vfull[v]) {
          if (outp) {
            if (a.out_dtype == DT_F32) {
              u32x4_t* q = reinterpret_cast<u32x4_t*>(static_cast<float*>(outp) + voff[v]);
              q[0] = u32x4_t{__float_as_uint(u[0]), __float_as_uint(u[1]), __float_as_uint(u[2]),
                             __float_as_uint(u[3])};
              q[1] = u32x4_t{__float_as_uint(u[4]), __float_as_uint(u[5]), __float_as_uint(u[6]),
                             __float_as_uint(u[7])};
            } else {
              u32x4_t o;
              o.x = (unsigned)f2bf(u[0]) | ((unsigned)f2bf(u[1]) << 16);
              o.y = (unsigned)f2bf(u[2]) | ((unsigned)f2bf(u[3]) << 16);
              o.z = (unsigned)f2bf(u[4]) | ((unsigned)f2bf(u[5]) << 16);
              o.w = (unsigned)f2bf(u[6]) | ((unsigned)f2bf(u[7]) << 16);
              *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(outp) + voff[v]) = o;
            }
          }
          if (wp) {
            float wn[8];   // the updated weights
            if (a.w_dtype == DT_F32) {
              float w[8];
#pragma unroll
              for (int t = 0; t < 4; ++t) {
                w[t] = __uint_as_float(wraw[v][0][t]);
                w[t + 4] = __uint_as_float(wraw[v][1][t]);
              }
              unsigned r[8];
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                float wv = w[t];
                if (a.decay != 1.f) wv = __fmul_rn(wv, a.decay);
                wn[t] = __builtin_fmaf(-a.lrs, u[t], wv);
                r[t] = __float_as_uint(wn[t]);
              }
              u32x4_t* q = reinterpret_cast<u32x4_t*>(static_cast<float*>(wp) + voff[v]);
              q[0] = u32x4_t{r[0], r[1], r[2], r[3]};
              q[1] = u32x4_t{r[4], r[5], r[6], r[7]};
            } else {
              unsigned r[8];
#pragma unroll
              for (int t = 0; t < 8; ++t) {
                const unsigned word = wraw[v][0][t >> 1];
                float wv = bf2f((t & 1) ? (word >> 16) : (word & 0xffff));
                if (a.decay != 1.f) wv = bf2f(f2bf(__fmul_rn(wv, a.decay)));
                r[t] = f2bf(__builtin_fmaf(-a.lrs, u[t], wv));
                wn[t] = bf2f(r[t]);
              }
              *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(wp) + voff[v]) =
                  u32x4_t{r[0] | (r[1] << 16), r[2] | (r[3] << 16), r[4] | (r[5] << 16),
                          r[6] | (r[7] << 16)};
            }
            if (pp) {
              // publish: the forward copy in its own dtype, same layout as W
              if (a.pub_dtype == DT_BF16) {
                *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(pp) + voff[v]) =
                    u32x4_t{(unsigned)f2bf(wn[0]) | ((unsigned)f2bf(wn[1]) << 16),
                            (unsigned)f2bf(wn[2]) | ((unsigned)f2bf(wn[3]) << 16),
                            (unsigned)f2bf(wn[4]) | ((unsigned)f2bf(wn[5]) << 16),
                            (unsigned)f2bf(wn[6]) | ((unsigned)f2bf(wn[7]) << 16)};
              } else {
                u32x4_t* q = reinterpret_cast<u32x4_t*>(static_cast<float*>(pp) + voff[v]);
                q[0] = u32x4_t{__float_as_uint(wn[0]), __float_as_uint(wn[1]),
                               __float_as_uint(wn[2]), __float_as_uint(wn[3])};
                q[1] = u32x4_t{__float_as_uint(wn[4]), __float_as_uint(wn[5]),
                               __float_as_uint(wn[6]), __float_as_uint(wn[7])};
              }
            }
          }
        } else {
          // ragged edges and unaligned bases, one element at a time (kept rolled, re-reading U
          // from the slab, so the unrolled slab loop around it stays small)
#pragma unroll 1
          for (int t = 0; t < 8; ++t) {
            const int i = ibase + vr[v] + (tr ? t : 0);
            const int j = jw + vc[v] + (tr ? 0 : t);
            if (i >= a.m_real || j >= a.n_real) continue;
            const long long off = tr ? (long long)j * pitch + i : (long long)i * pitch + j;
            const float ut = tr ? slab[(vr[v] + t) * kLd + vc[v]]
                                          : slab[vr[v] * kLd + vc[v] + t];
            if (outp) {
              if (a.out_dtype == DT_F32) static_cast<float*>(outp)[off] = ut;
              else static_cast<uint16_t*>(outp)[off] = f2bf(ut);
            }
            if (wp) {
              float wn;
              if (a.w_dtype == DT_F32) {
                float wv = static_cast<const float*>(wp)[off];
                if (a.decay != 1.f) wv = __fmul_rn(wv, a.decay);
                wn = __builtin_fmaf(-a.lrs, ut, wv);
                static_cast<float*>(wp)[off] = wn;
              } else {
                float wv = bf2f(static_cast<const uint16_t*>(wp)[off]);
                if (a.decay != 1.f) wv = bf2f(f2bf(__fmul_rn(wv, a.decay)));
                const uint16_t h = f2bf(__builtin_fmaf(-a.lrs, ut, wv));
                static_cast<uint16_t*>(wp)[off] = h;
                wn = bf2f(h);
              }
              if (pp) {
                if (a.pub_dtype == DT_BF16) static_cast<uint16_t*>(pp)[off] = f2bf(wn);
                else static_cast<float*>(pp)[off] = wn;
              }
            }
          }
        }
      }
    }
  }
}

template <int BM, int BN, int BK, int S, int WM, int WN, int MODE, int E, bool BKM>
__global__ __launch_bounds__(64 * WM * WN)
__attribute__((amdgpu_waves_per_eu(Occupancy<BM, BN, BK, S, WM, WN>::WPE,
                                   Occupancy<BM, BN, BK, S, WM, WN>::WPE)))
void nt_mfma_kernel(const NtArgs a) {
  using T = Tile<BM, BN, BK, S, WM, WN>;
  __shared__ __attribute__((aligned(16))) char smem[T::LDS_BYTES];
  static_assert(T::LDS_BYTES <= 160 * 1024, "LDS budget");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform by construction; held in an SGPR, the DMA's LDS addresses (M0) are scalar
  // work instead of a VALU computation + v_readfirstlane per DMA instruction (measured 1-2%)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wi = wave / WN, wj = wave % WN;

  // ---- tile decode -------------------------------------------------------------------
  // the decode is the same for every lane; readfirstlane states it, so the buffer descriptors
  // and offsets built from it stay scalar whatever the compiler's uniformity analysis proves
  const TilePos tp = decode_tile(a, blockIdx.x, gridDim.x);
  const int l = __builtin_amdgcn_readfirstlane(tp.l);
  const int bi = __builtin_amdgcn_readfirstlane(tp.bi), bj = __builtin_amdgcn_readfirstlane(tp.bj);
  const int i0 = bi * BM, j0 = bj * BN;

  const uint16_t* __restrict__ Ab = a.A + (long long)l * a.sA + (long long)i0 * a.lda;
  const uint16_t* __restrict__ Bb =
      a.B + (long long)l * a.sB + (BKM ? (long long)j0 : (long long)j0 * a.ldb);
  constexpr int KROWB = BN * 2;                   // k-major B: bytes of one k-row of the tile
  constexpr int KCPR = BN / 8, KRPK = 1024 / KROWB;

  // ---- global -> LDS DMA ring --------------------------------------------------------
  // DMA instruction q of wave w fills rows R0 = (NW q + w) * RPI .. R0 + RPI - 1 of a tile: lane l
  // writes LDS slot l % CPR of row R0 + l / CPR, so it fetches the global chunk that the
  // swizzle places in that slot (slot() is an involution in its chunk argument).
  const int lrow = lane / T::CPR, lsl = lane % T::CPR;
  // byte offsets from the tile's first row (fixed-size arrays: a template-dependent array
  // bound here makes clang drop the kernel's host launch stub)
  static_assert(T::A_INST <= 8 && T::B_INST <= 8, "DMA instructions per slice");
  unsigned offa[8], offb[8];
#pragma unroll
  for (int q = 0; q < T::A_INST; ++q) {
    const int r = (T::NW * q + wave) * T::RPI + lrow;
    offa[q] = (unsigned)(r * a.lda + T::slot(lsl, r) * 8) * 2u;
  }
#pragma unroll
  for (int q = 0; q < T::B_INST; ++q) {
    if constexpr (BKM) {
      // k-major: instruction q fills k-rows (NW q + w) KRPK.. of the slice; lane l writes slot
      // l % KCPR of its row, i.e. fetches the chunk the swizzle places there (64-wide tiles:
      // 128-byte k-rows, the ping-pong kernel's block layout)
      const int kr = (T::NW * q + wave) * KRPK + lane / KCPR, sl = lane % KCPR;
      const int sw = BN == 64 ? kswz64(kr) : kswz(kr);
      offb[q] = (unsigned)(kr * a.ldb + 8 * (sl ^ sw)) * 2u;
    } else {
      const int r = (T::NW * q + wave) * T::RPI + lrow;
      offb[q] = (unsigned)(r * a.ldb + T::slot(lsl, r) * 8) * 2u;
    }
  }
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  // The loads are MUBUF buffer loads into LDS (buffer_load_dwordx4 ... lds): one resource per
  // operand panel of this tile (SGPR base, range = the panel's rows), 32-bit lane offsets, the
  // slice offset in soffset. Cheaper to issue than 64-bit-address global loads (measured 1-3%
  // on the full kernel) and range-checked by the hardware: an offset past the panel reads 0.
  // Word 3 0x00020000: 32-bit data format, as gfx9 raw buffers use.
  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Ab), (short)0, (int)((long long)BM * a.lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Bb), (short)0,
      (int)((long long)(BKM ? a.K : BN) * a.ldb * 2), 0x00020000);
  const unsigned kstepB = BKM ? (unsigned)a.ldb : 1u;   // B slice offset: k-rows or k values
  // slice sl_ of A and B into ring slot slot_ (this wave's share)
#define DMUON_ISSUE(slice_, slot_)                                                             \
  do {                                                                                         \
    char* st_ = smem + (slot_) * T::STAGE + wave * 1024;                                       \
    const unsigned so_ = (unsigned)((slice_) * BK * 2);                                        \
    const unsigned sob_ = so_ * kstepB;                                                        \
    _Pragma("unroll") for (int q = 0; q < T::A_INST; ++q)                                      \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsA, (lds_ptr_t)(st_ + q * 1024 * T::NW), 16, \
                                                 offa[q], so_, 0, 0);                          \
    _Pragma("unroll") for (int q = 0; q < T::B_INST; ++q)                                      \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                              \
            rsB, (lds_ptr_t)(st_ + T::A_BYTES + q * 1024 * T::NW), 16, offb[q], sob_, 0, 0);   \
  } while (0)

  // the wave sub-tile as BI x BJ blocks of 16x16 (v_mfma_f32_16x16x32)
  constexpr int BI = T::WTM / 16, BJ = T::WTN / 16;
  f32x4_t acc[BI][BJ];
#pragma unroll
  for (int x = 0; x < BI; ++x)
#pragma unroll
    for (int y = 0; y < BJ; ++y) acc[x][y] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int KT = (a.k_loop > 0 ? a.k_loop : a.K) / BK;
  const int kt0 = __builtin_amdgcn_readfirstlane(first_slice(a, i0, j0, BK, KT));
  auto rot = [&](int t) { return t + kt0 >= KT ? t + kt0 - KT : t + kt0; };
  constexpr int KS = BK / 32;                     // MFMA substeps per slice
  static_assert(KS % 2 == 0, "fragment double buffer alternates per substep");
  const int arow0 = wi * T::WTM + (lane & 15);
  const int brow0 = wj * T::WTN + (lane & 15);
  const int kq = lane >> 4;
  int kboff[BJ];                                  // k-major B: this lane's read offsets
#pragma unroll
  for (int y = 0; y < BJ; ++y)
    kboff[y] = !BKM ? 0
               : BN == 64 ? kmajor64_lane_off(lane, wj * T::WTN + 16 * y)
                          : kmajor_lane_off(lane, wj * T::WTN + 16 * y, KROWB);

  // lane l reads row (l % 16) of each 16-row block at the 16-byte chunk 4 ks + l / 16
  auto load_frags = [&](const char* sa, const char* sb, int ks, bf16x8_t* af, bf16x8_t* bfr) {
    const int kc = ks * 4 + kq;
#pragma unroll
    for (int x = 0; x < BI; ++x) {
      const int row = arow0 + x * 16;
      af[x] = *reinterpret_cast<const bf16x8_t*>(sa + row * T::ROWB + (T::slot(kc, row) << 4));
    }
#pragma unroll
    for (int y = 0; y < BJ; ++y) {
      if constexpr (BKM) {
        bfr[y] = read_kmajor(sb + kboff[y] + ks * 32 * KROWB, KROWB);
      } else {
        const int row = brow0 + y * 16;
        bfr[y] = *reinterpret_cast<const bf16x8_t*>(sb + row * T::ROWB + (T::slot(kc, row) << 4));
      }
    }
  };
  constexpr int NF = BI + (BKM ? 2 : 1) * BJ, NM = BI * BJ;
  bf16x8_t af[2][BI], bfr[2][BJ];

  // Ring schedule: slot s % S holds slice s; the prologue fills all S slots. Iteration kt
  // consumes slice kt. Substeps 0 .. KS-2 each read the next substep's fragments under their
  // own MFMAs. Before the last substep the wave waits for its share of slice kt+1 and for its
  // own reads of slice kt, then meets the others at the barrier: past it slice kt+1 is complete
  // and slot kt % S is free, so the DMA of slice kt+S and the reads of slice kt+1's first
  // fragments both run under the last substep's MFMAs and no wave starts a slice with an empty
  // pipeline. Past the end the DMA re-fetches the last slice into the free slot (never read),
  // which keeps the number of loads per iteration, and so the vmcnt targets, uniform.
#pragma unroll
  for (int s0 = 0; s0 < S; ++s0) DMUON_ISSUE(rot(min(s0, KT - 1)), s0);
  wait_slices<T>();
  bare_barrier();
  load_frags(smem, smem + T::A_BYTES, 0, af[0], bfr[0]);

  for (int kt = 0; kt < KT; ++kt) {
    const char* sa = smem + (kt % S) * T::STAGE;
    const char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      // raised issue priority through the substeps before the barrier, back to normal for the
      // wait, the barrier and the DMA issue: a wave still in its MFMA run goes ahead of its
      // SIMD partner that has reached the slice's end (measured 1-2%)
      __builtin_amdgcn_s_setprio(1);
      load_frags(sa, sb, ks + 1, af[(ks + 1) & 1], bfr[(ks + 1) & 1]);
#pragma unroll
      for (int x = 0; x < BI; ++x)
#pragma unroll
        for (int y = 0; y < BJ; ++y)
          // MFMA rows <- j (B operand), MFMA cols <- i (A operand): each lane then holds
          // four consecutive j of one i, i.e. 8-byte row-major stores of D.
          acc[x][y] = mfma_16x16x32<E>(bfr[ks & 1][y], af[ks & 1][x], acc[x][y]);
    }
    sched_substeps<KS - 1, NM, NF>();
    __builtin_amdgcn_s_setprio(0);
    slice_barrier<(S - 2) * T::LPT>();
    {
      // reads first in program order: the DMA writes LDS, so later reads could not be
      // scheduled ahead of it
      const char* na = smem + ((kt + 1) % S) * T::STAGE;
      load_frags(na, na + T::A_BYTES, 0, af[0], bfr[0]);
    }
    DMUON_ISSUE(rot(min(kt + S, KT - 1)), kt % S);
#pragma unroll
    for (int x = 0; x < BI; ++x)
#pragma unroll
      for (int y = 0; y < BJ; ++y)
        acc[x][y] = mfma_16x16x32<E>(bfr[1][y], af[1][x], acc[x][y]);
    sched_front<0, NM, NF, T::LPT>();
  }
#undef DMUON_ISSUE
  wait_vmcnt<0>();
  bare_barrier();

  nt_epilogue<T, MODE, E>(a, smem, Acc16<BI, BJ>{acc, lane}, l, bi, bj, i0, j0, lane, wave, wi,
                          wj);
}

// Ping-pong schedule of the 256x256 tile with 8 waves of 128x64 (wave w and w + 4 share a SIMD).
// Group 0 (waves 0-3) owns tile rows 0-127, group 1 (waves 4-7) rows 128-255; the groups run one
// phase apart, every phase ending at a workgroup barrier:
//   group 0:  |0 M0 |1 C0 |2 M1 |3 C1 |4 ... M(KT-1) |2KT-1 C(KT-1) |2KT epilogue
//   group 1:  |0    |1 M0 |2 C0 |3 M1 |4 ...         |2KT-1 M(KT-1) |2KT C(KT-1), epilogue
// M(k) reads all of the wave's fragments of K slice k from LDS into registers; C(k) issues its
// 16x16x32 MFMAs on them. While one wave of a SIMD runs its MFMAs back to back, its partner does the LDS
// reads, so the MFMA pipe never waits on a fragment read or a barrier. The operand DMA is issued
// only in memory phases, half by each group, so no MFMA burst has DMA issue in its way: group 0's
// M(k) starts slice k + 1's A rows into the slot slice k - 1 used (its last readers, group 1's
// M(k - 1), ended at the barrier that opened this phase) and waits for them at the end of C(k);
// group 1's M(k) refills each wave's own B block with slice k + 2 and waits for slice k + 1's B
// before the barrier that opens group 0's M(k + 1). (Measured against all refill DMA issued by
// group 1, part of it in its compute phase: 5-10% faster, bit-identical.)
// One 256 x 256 tile of the ping-pong schedule, this wave's part of it. LIM: the wave computes
// the 16x16 blocks (x, y) of its 128 x 64 sub-tile with x - y <= LIM -- all of them (LIM = 7),
// or, on a diagonal tile of an exactly symmetric triangle product (whose values below the
// diagonal the epilogue drops), those on or above the diagonal (see nt_pp_kernel); LIM = -8:
// none (no fragment reads, no MFMAs, no epilogue). Each LIM is its own straight-line copy of the
// whole schedule: a runtime choice inside the loop made the compiler spill ~1000 VGPRs.
template <int BK, int S, int MODE, int E, bool BKM, int LIM>
__device__ __forceinline__ void pp_tile(const NtArgs& a, char* smem, int l, int bi, int bj) {
  using T = Tile<256, 256, BK, S, 2, 4>;
  constexpr int KS = BK / 32;                        // 16x16x32 MFMA substeps per slice
  // Wave v of either group moves, per slice, three parts of a ring slot (RPI rows per
  // instruction): A rows v*32 .. +31 and 128 + v*32 .. +31 (group 0 in the loop, group 1 in the
  // prologue) and the B block v (rows / values v*64 .. +63; group 1).
  static_assert(S == 2, "the refill split between the groups assumes a two-slot ring");
  constexpr int NAL = 32 / T::RPI, NB = 64 / T::RPI;
  constexpr int LPT1 = 2 * NAL + NB;                 // per group-1 wave per prologue slice
  static_assert(NB <= 8 && (S - 1) * LPT1 <= 63, "DMA instruction counts");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2, v = wave & 3, wi = grp;
  // Column block of the wave's 128 x 64 sub-tile: group 1's wave v takes block v (the B block it
  // also moves, so it refills only a block whose last reader in this phase pair is itself), group
  // 0's takes block 3 - v. The two waves that share a SIMD (v and v + 4) thus cover blocks 3 - v
  // and v. Every assignment gives the same bits; this one evens out the SIMDs' MFMA counts on
  // diagonal tiles.
  const int wj = grp == 0 ? 3 - v : v;

  const int i0 = bi * 256, j0 = bj * 256;
  const uint16_t* __restrict__ Ab = a.A + (long long)l * a.sA + (long long)i0 * a.lda;
  const uint16_t* __restrict__ Bb =
      a.B + (long long)l * a.sB + (BKM ? (long long)j0 : (long long)j0 * a.ldb);
  // k-major B: four column blocks of 64 values (one per wave column), each BK k-rows of 128
  // bytes; chunk c of row r at slot c ^ kswz64(r)
  constexpr int KBLK = BK * 128;

  // lane l of a DMA instruction writes LDS slot l % CPR of row l / CPR of its RPI-row group: it
  // fetches the global chunk the swizzle places there
  const int lrow = lane / T::CPR, lsl = lane % T::CPR;
  // The swizzle of a row (and of a k-major row) repeats every 16 rows, so instructions q and
  // q + 2 of a part differ by 16 rows: two per-lane offsets per operand, the rest of the
  // distance (16 rows per q / 2, and 128 rows for A's upper half) in the scalar offset. That
  // keeps 12 VGPRs free for the whole kernel.
  static_assert(T::RPI == 8 && T::RPL * T::CPR == 16, "swizzle period of 16 rows");
  unsigned offa2[2], offb2[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = v * 32 + q * T::RPI + lrow;
    offa2[q] = (unsigned)(r * a.lda + T::slot(lsl, r) * 8) * 2u;
    if constexpr (BKM) {
      const int kr = q * 8 + (lane >> 3), sl = lane & 7;
      offb2[q] = (unsigned)(kr * a.ldb + v * 64 + 8 * (sl ^ kswz64(kr))) * 2u;
    } else {
      const int rb = v * 64 + q * T::RPI + lrow;
      offb2[q] = (unsigned)(rb * a.ldb + T::slot(lsl, rb) * 8) * 2u;
    }
  }
  const unsigned a16 = 16u * (unsigned)a.lda * 2u, b16 = 16u * (unsigned)a.ldb * 2u;
  const unsigned ahi = 128u * (unsigned)a.lda * 2u;
  typedef __attribute__((address_space(3))) void* lds_ptr_t;
  const __amdgpu_buffer_rsrc_t rsA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Ab), (short)0, (int)((long long)256 * a.lda * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(Bb), (short)0,
      (int)((long long)(BKM ? a.K : 256) * a.ldb * 2), 0x00020000);
  const unsigned kstepB = BKM ? (unsigned)a.ldb : 1u;   // B slice offset: k-rows or k values
  char* const a_lo = smem + v * 32 * T::ROWB;
  char* const a_hi = smem + (128 + v * 32) * T::ROWB;
  char* const b_own = smem + T::A_BYTES + v * 64 * T::ROWB;
  static_assert(64 * T::ROWB == KBLK, "B block of a wave column");
#define DMUON_PP_PART(rs_, base_, off_, step_, n_, soff_, slot_)                               \
  do {                                                                                         \
    _Pragma("unroll") for (int q = 0; q < (n_); ++q)                                           \
        __builtin_amdgcn_raw_ptr_buffer_load_lds(                                              \
            rs_, (lds_ptr_t)((base_) + (slot_) * T::STAGE + q * 1024), 16, off_[q & 1],        \
            (soff_) + (unsigned)(q >> 1) * (step_), 0, 0);                                     \
  } while (0)
#define DMUON_PP_ALO(slice_, slot_) \
  DMUON_PP_PART(rsA, a_lo, offa2, a16, NAL, (unsigned)((slice_) * BK * 2), slot_)
#define DMUON_PP_AHI(slice_, slot_) \
  DMUON_PP_PART(rsA, a_hi, offa2, a16, NAL, (unsigned)((slice_) * BK * 2) + ahi, slot_)
#define DMUON_PP_B(slice_, slot_) \
  DMUON_PP_PART(rsB, b_own, offb2, b16, NB, (unsigned)((slice_) * BK * 2) * kstepB, slot_)

  // the wave's 128x64 sub-tile as 8 x 4 blocks of 16x16
  f32x4_t acc[8][4];
#pragma unroll
  for (int x = 0; x < 8; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // fragment of a 16-row block at substep ks: lane l reads row (l % 16) at 16-byte chunk
  // 4 ks + l / 16 (every 16-lane pass of a ds_read_b128: 16 rows at one chunk, all 64 banks)
  const int arow0 = wi * 128 + (lane & 15);
  const int brow0 = wj * 64 + (lane & 15);
  const int kq = lane >> 4;
  int kboff[4];                                      // k-major B: this lane's read offsets
#pragma unroll
  for (int y = 0; y < 4; ++y) kboff[y] = BKM ? wj * KBLK + kmajor64_lane_off(lane, 16 * y) : 0;
  bf16x8_t af[KS][8], bfr[KS][4];
  // the fragments of slot `slot` that the blocks x - y <= LIM use: A block x for x <= LIM + 3,
  // B block y for y >= -LIM
  auto mem_phase = [&](int slot) {
    const char* sa = smem + slot * T::STAGE;
    const char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int kc = ks * 4 + kq;
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        if (x > LIM + 3) continue;
        const int row = arow0 + x * 16;
        af[ks][x] = *reinterpret_cast<const bf16x8_t*>(sa + row * T::ROWB + (T::slot(kc, row) << 4));
      }
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        if (y < -LIM) continue;
        if constexpr (BKM) {
          bfr[ks][y] = read_kmajor(sb + kboff[y] + ks * 32 * 128, 128);
        } else {
          const int row = brow0 + y * 16;
          bfr[ks][y] = *reinterpret_cast<const bf16x8_t*>(sb + row * T::ROWB + (T::slot(kc, row) << 4));
        }
      }
    }
  };
  auto compute_phase = [&]() {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int x = 0; x < 8; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
          if (x - y <= LIM) acc[x][y] = mfma_16x16x32<E>(bfr[ks][y], af[ks][x], acc[x][y]);
  };

  const int KT = (a.k_loop > 0 ? a.k_loop : a.K) / BK;
  const int kt0 = __builtin_amdgcn_readfirstlane(first_slice(a, i0, j0, BK, KT));
  auto rot = [&](int t) { return t + kt0 >= KT ? t + kt0 - KT : t + kt0; };
  if (grp == 1) {
    // slices 0 .. S-1 (past the end: the last slice again, into a slot never read)
#pragma unroll
    for (int s0 = 0; s0 < S; ++s0) {
      DMUON_PP_ALO(rot(min(s0, KT - 1)), s0);
      DMUON_PP_B(rot(min(s0, KT - 1)), s0);
      DMUON_PP_AHI(rot(min(s0, KT - 1)), s0);
    }
    wait_vmcnt<(S - 1) * LPT1>();                     // slice 0 has landed
  }
  phase_barrier();                                    // |0
  if (grp == 1) phase_barrier();                      // |1: group 1 starts one phase behind
  // RA: group 0 moves slice kt + 1's A rows into slot (kt + 1) % 2 = (kt - 1) % 2 (kt >= 1: slice 1
  // came with the prologue); RB: group 1 refills its B block of slot kt % 2 with slice kt + 2
  // after its own reads of it (group 0 read it in the previous phase). Nothing is moved past the
  // last slice, and every DMA has landed when the loop ends, before the epilogue reuses the LDS.
  // The four iteration kinds are separate instances, so no body branches around its DMA
  // (measured: a runtime refill test inside one loop costs 3-11%).
  auto iteration = [&](int kt, auto ra_c, auto rb_c, auto last_c) {
    constexpr bool RA = decltype(ra_c)::value, RB = decltype(rb_c)::value;
    constexpr bool LAST = decltype(last_c)::value;
    mem_phase(kt % S);
    if (RA && grp == 0) {
      DMUON_PP_ALO(rot(kt + 1), (kt + 1) % S);
      DMUON_PP_AHI(rot(kt + 1), (kt + 1) % S);
    }
    // this wave's fragments are in registers
    __builtin_amdgcn_s_waitcnt(0xC07F);              // lgkmcnt(0), vmcnt / expcnt untouched
    if (grp == 1) {
      if (RB) {
        DMUON_PP_B(rot(kt + 2), kt % S);
        wait_vmcnt<NB>();                            // all of slice kt + 1 has landed
      } else {
        wait_vmcnt<0>();
      }
    }
    phase_barrier();
    compute_phase();
    if (RA && grp == 0) wait_vmcnt<0>();             // slice kt + 1's A rows have landed
    // Last slice: group 1 stops at the barrier before its MFMAs (|2KT), which is also the one
    // after group 0's; no wave reads the ring after it, so group 0's epilogue overlaps group 1's
    // last MFMA phase. Both groups pass 2KT + 1 barriers.
    if (!(LAST && grp == 1)) phase_barrier();
  };
  const std::false_type no{};
  const std::true_type yes{};
  if (KT >= 3) {
    iteration(0, no, yes, no);
    int kt = 1;
    for (; kt + 2 < KT; ++kt) iteration(kt, yes, yes, no);
    iteration(kt, yes, no, no);                      // kt = KT - 2
    iteration(kt + 1, no, no, yes);
  } else {
    for (int kt = 0; kt + 1 < KT; ++kt) iteration(kt, no, no, no);
    iteration(KT - 1, no, no, yes);
  }
#undef DMUON_PP_PART
#undef DMUON_PP_ALO
#undef DMUON_PP_AHI
#undef DMUON_PP_B
  wait_vmcnt<0>();
  // a diagonal-tile wave whose values all lie below the diagonal has nothing to store
  if constexpr (LIM >= -3)
    nt_epilogue<T, MODE, E>(a, smem, Acc16<8, 4>{acc, lane}, l, bi, bj, i0, j0, lane, wave, wi,
                            wj);
}

template <int BK, int S, int MODE, int E, bool BKM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void nt_pp_kernel(const NtArgs a) {
  using T = Tile<256, 256, BK, S, 2, 4>;
  __shared__ __attribute__((aligned(16))) char smem[T::LDS_BYTES];
  static_assert(T::LDS_BYTES <= 160 * 1024, "LDS budget");
  // the decode is the same for every lane; readfirstlane states it, so the buffer descriptors
  // and offsets built from it stay scalar whatever the compiler's uniformity analysis proves
  const TilePos tp = decode_tile(a, blockIdx.x, gridDim.x);
  const int l = __builtin_amdgcn_readfirstlane(tp.l);
  const int bi = __builtin_amdgcn_readfirstlane(tp.bi), bj = __builtin_amdgcn_readfirstlane(tp.bj);
  // Which copy of the schedule this wave runs (one call site each: pp_tile is inlined wherever
  // it is called). 0: every block; on a diagonal tile of an exactly symmetric product, block
  // (x, y) of a wave (tile rows 128 wi + 16 x, columns 64 wj + 16 y) lies strictly below the
  // diagonal when 8 wi + x > 4 wj + y and its values are dropped: with c = 4 wj - 8 wi a wave
  // keeps the blocks with x - y <= c -- all (c >= 7: copy 0), none (c <= -4: 1), x <= y
  // (c = 0: 2) or x <= y + 4 (c = 4: 3). With group 0 in reversed column order (pp_tile) that
  // is 32 + 0, 32 + 0, 26 + 10 and 10 + 26 of the 64 MFMAs per slice on the four SIMDs (10, 26,
  // 42 and 58 in natural order). s_barrier counts waves, not program counters, and every copy
  // passes the same barriers.
  // NtArgs::diag_skip chooses how much of that is used: DIAG_SKIP_WAVES only copies 0 and 1.
  // NtArgs::live_rows / live_cols: a wave whose rows or columns all lie in the unread padding
  // takes copy 1 too, in every mode.
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int grp = wave >> 2, v = wave & 3;
  int copy = (a.live_rows > 0 && bi * 256 + 128 * grp >= a.live_rows) ||
                     (a.live_cols > 0 && bj * 256 + 64 * (grp == 0 ? 3 - v : v) >= a.live_cols)
                 ? 1 : 0;
  if constexpr (MODE == EPI_SYM) {
    if (copy == 0 && a.sym_exact && a.tri && bi == bj && a.diag_skip != DIAG_SKIP_NONE) {
      const int c = 4 * (grp == 0 ? 3 - v : v) - 8 * grp;
      copy = c <= -4 ? 1 : (c >= 7 || a.diag_skip != DIAG_SKIP_BLOCKS) ? 0 : c == 0 ? 2 : 3;
    }
  }
  if (copy == 1) {
    pp_tile<BK, S, MODE, E, BKM, -8>(a, smem, l, bi, bj);
  } else if constexpr (MODE == EPI_SYM) {
    if (copy == 2) pp_tile<BK, S, MODE, E, BKM, 0>(a, smem, l, bi, bj);
    else if (copy == 3) pp_tile<BK, S, MODE, E, BKM, 4>(a, smem, l, bi, bj);
    else pp_tile<BK, S, MODE, E, BKM, 7>(a, smem, l, bi, bj);
  } else {
    pp_tile<BK, S, MODE, E, BKM, 7>(a, smem, l, bi, bj);
  }
}

// Compute units of the current device, queried once per device (0 if the query fails).
int current_device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int v = cus[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace

// 64x64 tiles of small launches: ring slots and waves (64 x 64 / kT64WN each). With four
// waves each issues half the DMA of two, so the per-wave count of loads in flight (vmcnt, at
// most 63) allows an eighth slot: seven slices in flight instead of six, twice the SIMDs issuing
// MFMAs (measured c1 0.186 -> 0.162 ms, c3 1024 x 16384 0.405 -> 0.364 ms; ten slots slower).
constexpr int kT64S = 8, kT64WN = 4;
// 128x128 tiles of launches with at most one tile per CU: ring slots and waves (2 x kT128WN);
// eight waves, two per SIMD, so one wave's fragment reads run under its partner's MFMAs
// (2048 x 8192: 0.677 -> 0.616 ms per step against four waves; five slots slower).
constexpr int kT128S = 4, kT128WN = 4;

int nt_block_tile(int b, int nb) { return xcd_remap(b, nb); }

hipError_t launch_nt(const NtArgs& a, int tile, hipStream_t stream) {
  const long long nb = (long long)a.tiles_per_mat * a.L;
  if (nb <= 0) return hipSuccess;
  // the K loops run whole 64-wide slices, at least one
  if (a.K <= 0 || a.K % 64 != 0) return hipErrorInvalidValue;
  // the second output relies on the exactly symmetric diagonal-tile path for its diagonal
  if (a.D2 && !(a.mode == EPI_SYM && a.tri && a.sym_exact)) return hipErrorInvalidValue;
  // an output to write: D for a symmetric product, D or D^T for an NS step
  if ((a.mode == EPI_SYM && !a.D) || (a.mode == EPI_NS && !a.D && !a.DT))
    return hipErrorInvalidValue;
  // k-major B: whole-panel buffer range and slice offsets in 32 bits, rows of whole tiles
  if (a.b_kmajor && ((long long)a.K * a.ldb * 2 >= (1LL << 31) || a.ldb < a.N))
    return hipErrorInvalidValue;
  // An addend named as one of the operands (the K-loop rotation's C_IS_A / C_IS_B) is read by
  // the epilogue as an M x N matrix at ldc: that is the operand itself only for a square
  // product (K == M == N) with the operand's own layout. Anything else would read the addend
  // past the operand's rows (a 4096 x 64 panel read as 4096 x 4096), so it is refused.
  if (a.c_in == C_IS_A &&
      !(a.C == a.A && a.K == a.M && a.M == a.N && a.ldc == a.lda && (a.L <= 1 || a.sC == a.sA)))
    return hipErrorInvalidValue;
  if (a.c_in == C_IS_B &&
      !(a.C == a.B && a.K == a.M && a.M == a.N && a.ldc == a.ldb && (a.L <= 1 || a.sC == a.sB)))
    return hipErrorInvalidValue;
  if (a.c_in != C_NONE && a.c_in != C_IS_A && a.c_in != C_IS_B) return hipErrorInvalidValue;
  if (a.k_loop < 0 || a.k_loop > a.K || a.k_loop % 64 != 0) return hipErrorInvalidValue;
  if (a.live_rows < 0 || a.live_rows % 64 != 0 || a.live_cols < 0 || a.live_cols % 64 != 0 ||
      (a.tri && a.live_rows != a.live_cols))
    return hipErrorInvalidValue;
  dim3 grid((unsigned)nb);
#define DMUON_NT3(TILE, BK, S, WM, WN, E, KM)                                                  \
  do {                                                                                         \
    dim3 block(64 * WM * WN);                                                                  \
    if (a.mode == EPI_SYM)                                                                     \
      hipLaunchKernelGGL((nt_mfma_kernel<TILE, TILE, BK, S, WM, WN, EPI_SYM, E, KM>), grid,    \
                         block, 0, stream, a);                                                 \
    else if (a.mode == EPI_NS)                                                                 \
      hipLaunchKernelGGL((nt_mfma_kernel<TILE, TILE, BK, S, WM, WN, EPI_NS, E, KM>), grid,     \
                         block, 0, stream, a);                                                 \
    else                                                                                       \
      hipLaunchKernelGGL((nt_mfma_kernel<TILE, TILE, BK, S, WM, WN, EPI_FINAL, E, KM>), grid,  \
                         block, 0, stream, a);                                                 \
  } while (0)
#define DMUON_NT(TILE, BK, S, WM, WN, E)                                                       \
  do {                                                                                         \
    if (a.b_kmajor) DMUON_NT3(TILE, BK, S, WM, WN, E, true);                                   \
    else DMUON_NT3(TILE, BK, S, WM, WN, E, false);                                             \
  } while (0)
#define DMUON_PP3(E, KM)                                                                       \
  do {                                                                                         \
    dim3 block(512);                                                                           \
    if (a.mode == EPI_SYM)                                                                     \
      hipLaunchKernelGGL((nt_pp_kernel<64, 2, EPI_SYM, E, KM>), grid, block, 0, stream, a);    \
    else if (a.mode == EPI_NS)                                                                 \
      hipLaunchKernelGGL((nt_pp_kernel<64, 2, EPI_NS, E, KM>), grid, block, 0, stream, a);     \
    else                                                                                       \
      hipLaunchKernelGGL((nt_pp_kernel<64, 2, EPI_FINAL, E, KM>), grid, block, 0, stream, a);  \
  } while (0)
#define DMUON_PP(E)                                                                            \
  do {                                                                                         \
    if (a.b_kmajor) DMUON_PP3(E, true);                                                        \
    else DMUON_PP3(E, false);                                                                  \
  } while (0)
  // 256-tiles: the ping-pong kernel, 8 waves, 64-wide K slices in a two-slot ring; 128-tiles:
  // 4 waves, two blocks per CU, or, when every tile has a CU to itself, one block per CU with a
  // four-slot ring (128 KiB). Measured and not kept: 32-wide slices in a four-slot ring for the
  // ping-pong kernel (7-12% slower: twice the phases and barriers), the in-phase 8-wave schedule
  // it replaced (3-11% slower on the c5 product shapes), 256-tiles of 4 waves with 128x128 per
  // wave, and 32x32x16 MFMAs (identical results; 5-15% slower under the board power limit).
  const int cus = current_device_cus();
  if (tile == 128 && a.M % 256 == 0 && a.N % 256 == 0 && cus > 0) {
    // A launch of more than two 128-tiles per CU whose result also splits into 256-tiles runs
    // on the ping-pong kernel when that takes fewer units of work per CU, by the cost model of
    // the planner (a wave of 256-tiles: 4 units; a wave of two 128-tiles per CU: 2.7). With
    // both sides multiples of 256 the two kernels give the same bits, so only the time changes
    // (e.g. Q X of one 1024 x 16384 matrix: 256 tiles in one wave instead of 1024 in two).
    const int mt2 = a.M / 256, nt2 = a.N / 256;
    const long long n256 = (long long)(a.tri ? mt2 * (mt2 + 1) / 2 : mt2 * nt2) * a.L;
    const double c256 = 4.0 * (double)((n256 + cus - 1) / cus);
    const double c128 = 2.7 * (double)((nb + 2LL * cus - 1) / (2LL * cus));
    if (nb > 2LL * cus && c256 < c128) {
      NtArgs s = a;
      s.mt = mt2;
      s.nt = nt2;
      s.tiles_per_mat = (int)(n256 / a.L);
      return launch_nt(s, 256, stream);
    }
  }
  if (tile == 128) {
    // The same products on 64x64 tiles (4 waves of 64x16, an eight-slot ring of 16 KiB slots,
    // one block per CU) when those still fit one wave of blocks on the device: four times the
    // CUs on a launch that waits on load latency. Every value keeps its K order -- the slice
    // rotation depends only on the 256-aligned block of the tile's columns -- so the bits match
    // the 128-tile kernel's. A k-major B is one 64-value block of 128-byte k-rows per slice.
    NtArgs s = a;
    s.mt = 2 * a.mt;
    s.nt = 2 * a.nt;
    s.tiles_per_mat = a.tri ? s.mt * (s.mt + 1) / 2 : s.mt * s.nt;
    const long long nb64 = (long long)s.tiles_per_mat * a.L;
    if (nb64 <= cus) {
      dim3 g64((unsigned)nb64), b64(64 * kT64WN);
#define DMUON_NT64K(E, KM)                                                                     \
  do {                                                                                         \
    if (s.mode == EPI_SYM)                                                                     \
      hipLaunchKernelGGL((nt_mfma_kernel<64, 64, 64, kT64S, 1, kT64WN, EPI_SYM, E, KM>), g64, b64, 0,    \
                         stream, s);                                                           \
    else if (s.mode == EPI_NS)                                                                 \
      hipLaunchKernelGGL((nt_mfma_kernel<64, 64, 64, kT64S, 1, kT64WN, EPI_NS, E, KM>), g64, b64, 0,     \
                         stream, s);                                                           \
    else                                                                                       \
      hipLaunchKernelGGL((nt_mfma_kernel<64, 64, 64, kT64S, 1, kT64WN, EPI_FINAL, E, KM>), g64, b64, 0,  \
                         stream, s);                                                           \
  } while (0)
#define DMUON_NT64(E)                                                                          \
  do {                                                                                         \
    if (s.b_kmajor) DMUON_NT64K(E, true);                                                      \
    else DMUON_NT64K(E, false);                                                                \
  } while (0)
      if (a.elt == ELT_F16) DMUON_NT64(ELT_F16);
      else DMUON_NT64(ELT_BF16);
#undef DMUON_NT64
#undef DMUON_NT64K
      return hipGetLastError();
    }
  }
  const bool deep = tile != 256 && nb <= cus;
  if (a.elt == ELT_F16) {
    if (tile == 256) DMUON_PP(ELT_F16);
    else if (deep) DMUON_NT(128, 64, kT128S, 2, kT128WN, ELT_F16);
    else DMUON_NT(128, 64, 2, 2, 2, ELT_F16);
  } else {
    if (tile == 256) DMUON_PP(ELT_BF16);
    else if (deep) DMUON_NT(128, 64, kT128S, 2, kT128WN, ELT_BF16);
    else DMUON_NT(128, 64, 2, 2, 2, ELT_BF16);
  }
#undef DMUON_NT
#undef DMUON_NT3
#undef DMUON_PP
#undef DMUON_PP3
  return hipGetLastError();
}

}  // namespace dmuon

// NT-form bf16 MFMA product family for the Newton-Schulz iteration on gfx950 (CDNA4).
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
// Tile machine: 256 threads = 4 waves (2x2); each wave owns a (BM/2)x(BN/2) sub-tile made of
// 32x32 MFMA blocks (v_mfma_f32_32x32x16_bf16, fp32 accumulate). K is staged through LDS in
// BK=64 slices, double-buffered, register-staged global loads, 16-byte chunks stored with an
// XOR swizzle (chunk ^ (row & 7)) so both the stores and the fragment reads are bank-conflict
// free without padding.
#include "dmuon_amd_internal.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

namespace dmuon {
namespace {

constexpr int kThreads = 256;
constexpr int kBK = 64;

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Maps the hardware block id so that each XCD (blocks are dealt round-robin over 8 XCDs)
// works on a contiguous range of logical tiles, which then share operands in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int nb) {
  const int q = nb >> 3, r = nb & 7;
  const int x = b & 7, idx = b >> 3;
  const int base = (x < r) ? x * (q + 1) : r * (q + 1) + (x - r) * q;
  return base + idx;
}

template <int BM, int BN>
struct Tile {
  static constexpr int TI = BM / 2 / 32;              // MFMA blocks along i per wave
  static constexpr int TJ = BN / 2 / 32;              // MFMA blocks along j per wave
  static constexpr int A_CH = BM * kBK / 8 / kThreads;  // 16-byte chunks per thread per slice
  static constexpr int B_CH = BN * kBK / 8 / kThreads;
  static constexpr int A_BYTES = BM * kBK * 2;
  static constexpr int STAGE = (BM + BN) * kBK * 2;
};

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 2)))
void nt_mfma_kernel(const NtArgs a) {
  using T = Tile<BM, BN>;
  __shared__ __attribute__((aligned(16))) char smem[2 * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wi = wave >> 1, wj = wave & 1;

  // ---- tile decode -------------------------------------------------------------------
  const int nblocks = gridDim.x;
  const int lb = xcd_remap(blockIdx.x, nblocks);
  const int l = lb / a.tiles_per_mat;
  int t = lb - l * a.tiles_per_mat;
  int bi, bj;
  if (a.tri) {
    bi = 0;
    while (t >= a.mt - bi) { t -= a.mt - bi; ++bi; }
    bj = bi + t;
  } else {
    // groups of 8 tile-rows walked column-major so neighbouring blocks share B panels
    const int group = 8;
    const int per_group = group * a.nt;
    const int g = t / per_group;
    const int first = g * group;
    const int gsize = min(a.mt - first, group);
    const int r = t - g * per_group;
    bi = first + r % gsize;
    bj = r / gsize;
  }
  const int i0 = bi * BM, j0 = bj * BN;

  const uint16_t* __restrict__ Ab = a.A + (long long)l * a.sA + (long long)i0 * a.lda;
  const uint16_t* __restrict__ Bb = a.B + (long long)l * a.sB + (long long)j0 * a.ldb;

  // ---- global -> register staging (per thread: fixed row/chunk, slices advance along K) ---
  const int crow = tid >> 3, ckc = tid & 7;
  const uint16_t* __restrict__ ga = Ab + (long long)crow * a.lda + ckc * 8;
  const uint16_t* __restrict__ gb = Bb + (long long)crow * a.ldb + ckc * 8;
  const long long astep = 32LL * a.lda, bstep = 32LL * a.ldb;  // 256 threads cover 32 rows
  // rows crow + 32q share (row & 7), so the swizzled LDS offset is one per thread
  const int soff = crow * 128 + ((ckc ^ (crow & 7)) << 4);
  u32x4_t ra[T::A_CH], rb[T::B_CH];
  f32x16_t acc[T::TI][T::TJ];
#pragma unroll
  for (int x = 0; x < T::TI; ++x)
#pragma unroll
    for (int y = 0; y < T::TJ; ++y)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[x][y][v] = 0.f;

  const int KT = a.K / kBK;
  {
      const int k0_ = 0;
#pragma unroll
      for (int q = 0; q < T::A_CH; ++q) ra[q] = *reinterpret_cast<const u32x4_t*>(ga + q * astep + k0_);
#pragma unroll
      for (int q = 0; q < T::B_CH; ++q) rb[q] = *reinterpret_cast<const u32x4_t*>(gb + q * bstep + k0_);
    }
  {
      char* sa_ = smem + (0) * T::STAGE;
#pragma unroll
      for (int q = 0; q < T::A_CH; ++q) *reinterpret_cast<u32x4_t*>(sa_ + soff + q * 4096) = ra[q];
#pragma unroll
      for (int q = 0; q < T::B_CH; ++q)
        *reinterpret_cast<u32x4_t*>(sa_ + T::A_BYTES + soff + q * 4096) = rb[q];
    }
  __syncthreads();

  const int arow0 = wi * (BM / 2) + (lane & 31);
  const int brow0 = wj * (BN / 2) + (lane & 31);
  const int khalf = lane >> 5;

  for (int kt = 0; kt < KT; ++kt) {
    const bool more = (kt + 1) < KT;
    if (more) {
      const int k0_ = (kt + 1) * kBK;
#pragma unroll
      for (int q = 0; q < T::A_CH; ++q) ra[q] = *reinterpret_cast<const u32x4_t*>(ga + q * astep + k0_);
#pragma unroll
      for (int q = 0; q < T::B_CH; ++q) rb[q] = *reinterpret_cast<const u32x4_t*>(gb + q * bstep + k0_);
    }
    const char* sa = smem + (kt & 1) * T::STAGE;
    const char* sb = sa + T::A_BYTES;
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      const int kc = ks * 2 + khalf;
      bf16x8_t af[T::TI], bfr[T::TJ];
#pragma unroll
      for (int x = 0; x < T::TI; ++x) {
        const int row = arow0 + x * 32;
        af[x] = *reinterpret_cast<const bf16x8_t*>(sa + row * 128 + ((kc ^ (row & 7)) << 4));
      }
#pragma unroll
      for (int y = 0; y < T::TJ; ++y) {
        const int row = brow0 + y * 32;
        bfr[y] = *reinterpret_cast<const bf16x8_t*>(sb + row * 128 + ((kc ^ (row & 7)) << 4));
      }
#pragma unroll
      for (int x = 0; x < T::TI; ++x)
#pragma unroll
        for (int y = 0; y < T::TJ; ++y)
          // MFMA rows <- j (B operand), MFMA cols <- i (A operand): each lane then holds
          // four consecutive j of one i, i.e. 8-byte row-major stores of D.
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[y], af[x], acc[x][y], 0, 0, 0);
    }
    if (more) {
      char* sa_ = smem + ((kt + 1) & 1) * T::STAGE;
#pragma unroll
      for (int q = 0; q < T::A_CH; ++q) *reinterpret_cast<u32x4_t*>(sa_ + soff + q * 4096) = ra[q];
#pragma unroll
      for (int q = 0; q < T::B_CH; ++q)
        *reinterpret_cast<u32x4_t*>(sa_ + T::A_BYTES + soff + q * 4096) = rb[q];
    }
    __syncthreads();
  }

  // ---- epilogue -----------------------------------------------------------------------
  // element (x, y, g, e) of the wave tile, with li = lane & 31, lh = lane >> 5:
  //   i = iw + 32x + li,   j = jw + 32y + 8g + 4lh + e      (acc[x][y][4g + e])
  // Addresses split into a wave-uniform part (scalar registers) and one per-lane offset.
  const int li = lane & 31, lh = lane >> 5;
  const int iw = i0 + wi * (BM / 2), jw = j0 + wj * (BN / 2);
  float s = a.alpha;
  if (a.alpha_dev) s *= a.alpha_dev[l];

  if constexpr (MODE == EPI_SYM || MODE == EPI_NS) {
    const uint16_t* Cb = a.C ? a.C + (long long)l * a.sC : nullptr;
    uint16_t* Db = a.D + (long long)l * a.sD;
    uint16_t* DTb = nullptr;
    long long ldt = 0;
    if constexpr (MODE == EPI_SYM) {
      if (a.tri && bi != bj) { DTb = Db; ldt = a.ldd; }   // mirror into the lower triangle
    } else {
      if (a.DT) { DTb = a.DT + (long long)l * a.sDT; ldt = a.lddt; }
    }
    const unsigned lo_d = (unsigned)(li * a.ldd + 4 * lh);
    const unsigned lo_c = (unsigned)(li * a.ldc + 4 * lh);
    const unsigned lo_t = (unsigned)(4 * lh * ldt + li);
#pragma unroll
    for (int x = 0; x < T::TI; ++x) {
      uint16_t* drow = Db + (long long)(iw + 32 * x) * a.ldd + jw;
      const uint16_t* crow = Cb ? Cb + (long long)(iw + 32 * x) * a.ldc + jw : nullptr;
#pragma unroll
      for (int y = 0; y < T::TJ; ++y) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int jo = 32 * y + 8 * g;
          float cv[4] = {0.f, 0.f, 0.f, 0.f};
          if (crow) {
            const u32x2_t c2 = *reinterpret_cast<const u32x2_t*>(crow + lo_c + jo);
            cv[0] = bf2f(c2.x & 0xffff); cv[1] = bf2f(c2.x >> 16);
            cv[2] = bf2f(c2.y & 0xffff); cv[3] = bf2f(c2.y >> 16);
          }
          uint16_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc[x][y][4 * g + e];
            float r;
            if constexpr (MODE == EPI_SYM) {
              r = s * v + a.beta * cv[e];
              if (iw + 32 * x + li == jw + jo + 4 * lh + e) r += a.diag;
            } else {
              r = s * (v + a.beta * cv[e]);
            }
            o[e] = f2bf(r);
          }
          u32x2_t packed;
          packed.x = (unsigned)o[0] | ((unsigned)o[1] << 16);
          packed.y = (unsigned)o[2] | ((unsigned)o[3] << 16);
          *reinterpret_cast<u32x2_t*>(drow + lo_d + jo) = packed;
          if (DTb) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              uint16_t* tcol = DTb + (long long)(jw + jo + e) * ldt + iw + 32 * x;
              tcol[lo_t] = o[e];
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
    constexpr int kLd = BN / 2 + 4;
    float* slab = reinterpret_cast<float*>(smem) + wave * 32 * kLd;
    const uint16_t* Cb = a.C ? a.C + (long long)l * a.sC : nullptr;
    void* outp = a.out_ptrs ? a.out_ptrs[l] : nullptr;
    void* wp = a.w_ptrs ? a.w_ptrs[l] : nullptr;
    const long long pitch = a.transposed ? a.m_real : a.n_real;
    const unsigned lo_c = (unsigned)(li * a.ldc + 4 * lh);
#pragma unroll
    for (int x = 0; x < T::TI; ++x) {
      const uint16_t* crow = Cb ? Cb + (long long)(iw + 32 * x) * a.ldc + jw : nullptr;
#pragma unroll
      for (int y = 0; y < T::TJ; ++y) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int jo = 32 * y + 8 * g;
          float cv[4] = {0.f, 0.f, 0.f, 0.f};
          if (crow) {
            const u32x2_t c2 = *reinterpret_cast<const u32x2_t*>(crow + lo_c + jo);
            cv[0] = bf2f(c2.x & 0xffff); cv[1] = bf2f(c2.x >> 16);
            cv[2] = bf2f(c2.y & 0xffff); cv[3] = bf2f(c2.y >> 16);
          }
          float4 u4;
          u4.x = s * (acc[x][y][4 * g + 0] + a.beta * cv[0]);
          u4.y = s * (acc[x][y][4 * g + 1] + a.beta * cv[1]);
          u4.z = s * (acc[x][y][4 * g + 2] + a.beta * cv[2]);
          u4.w = s * (acc[x][y][4 * g + 3] + a.beta * cv[3]);
          *reinterpret_cast<float4*>(slab + li * kLd + jo + 4 * lh) = u4;
        }
      }
      __syncthreads();
      const int ibase = iw + 32 * x;
      for (int p = lane; p < 32 * (BN / 2); p += 64) {
        // normal: consecutive lanes walk j; transposed: consecutive lanes walk i
        const int r = a.transposed ? (p & 31) : p / (BN / 2);
        const int c = a.transposed ? (p >> 5) : p % (BN / 2);
        const int i = ibase + r, j = jw + c;
        if (i >= a.m_real || j >= a.n_real) continue;
        const float u = slab[r * kLd + c];
        const long long off = a.transposed ? (long long)j * pitch + i : (long long)i * pitch + j;
        if (outp) {
          if (a.out_dtype == DT_F32) static_cast<float*>(outp)[off] = u;
          else static_cast<uint16_t*>(outp)[off] = f2bf(u);
        }
        if (wp) {
          if (a.w_dtype == DT_F32) {
            float* w = static_cast<float*>(wp) + off;
            float wv = *w;
            if (a.decay != 1.f) wv = __fmul_rn(wv, a.decay);
            *w = __fadd_rn(wv, -a.lrs * u);
          } else {
            uint16_t* w = static_cast<uint16_t*>(wp) + off;
            float wv = bf2f(*w);
            if (a.decay != 1.f) wv = bf2f(f2bf(__fmul_rn(wv, a.decay)));
            *w = f2bf(__fadd_rn(wv, -a.lrs * u));
          }
        }
      }
      __syncthreads();
    }
  }
}

}  // namespace

hipError_t launch_nt(const NtArgs& a, int tile, hipStream_t stream) {
  const long long nb = (long long)a.tiles_per_mat * a.L;
  if (nb <= 0) return hipSuccess;
  dim3 grid((unsigned)nb), block(kThreads);
#define DMUON_LAUNCH(T, M) hipLaunchKernelGGL((nt_mfma_kernel<T, T, M>), grid, block, 0, stream, a)
  if (tile == 256) {
    if (a.mode == EPI_SYM) DMUON_LAUNCH(256, EPI_SYM);
    else if (a.mode == EPI_NS) DMUON_LAUNCH(256, EPI_NS);
    else DMUON_LAUNCH(256, EPI_FINAL);
  } else {
    if (a.mode == EPI_SYM) DMUON_LAUNCH(128, EPI_SYM);
    else if (a.mode == EPI_NS) DMUON_LAUNCH(128, EPI_NS);
    else DMUON_LAUNCH(128, EPI_FINAL);
  }
#undef DMUON_LAUNCH
  return hipGetLastError();
}

}  // namespace dmuon

// Bandwidth-bound kernels of the Muon step on gfx950.
//
//  pre      buf <- mu*buf + g (first step: buf <- g); ns_in = g + mu*buf (Nesterov) or buf;
//           writes a 16-bit copy of ns_in into a zero-padded NS operand -- in the gradient's
//           own layout (Y) and/or transposed through LDS (YT); the callers' skip flags choose,
//           and the Muon step writes only the m x n orientation the products read -- plus
//           partial sums of ns_in^2 for the Frobenius norm. Unpadded matrices with one copy run
//           on kernels whose wave instructions each move one contiguous run (a wide matrix as a
//           flat array, a tall one in 64 x 256 tiles); padded ones, or both copies, on 64x64
//           tiles.
//           PRE_EST (the Muon step's default) is one pass, 2 (g) + 4 + 4 (buf) + 2 (copy) B/elt:
//           the copy is fp16(kx * est * ns_in) with the parameter's kept scale est, used when
//           the new norm confirms it. Otherwise two passes: PRE_NORM (momentum + partials), then,
//           once the norm is known, PRE_F16 recomputes ns_in and writes fp16(kx * ns_in / norm)
//           (fp16 cannot hold an un-normalised gradient safely): 2+4+4, then 2+4+2 B/elt.
//           PRE_BF16 writes bf16(ns_in) (the stand-alone staging entry point).
//  finalize scale = 1/(||ns_in||_F + eps) per matrix, fixed-order (deterministic) reduction.
//  update   W <- W*(1 - lr*wd) - lr*scale*U   for callers holding a materialised U.
#include <algorithm>
#include <type_traits>

#include "dmuon_amd_internal.h"

namespace dmuon {
namespace {

constexpr int kTile = 64;
constexpr int kPad = 8;  // u16 of padding per LDS row (keeps 16-byte alignment)

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ float load_any(const void* p, int dtype, long long idx) {
  return dtype == DT_F32 ? static_cast<const float*>(p)[idx]
                         : bf2f(static_cast<const uint16_t*>(p)[idx]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_copy_t __attribute__((ext_vector_type(4)));
// The gradient and the momentum buffer are streamed once per pass: non-temporal loads (and the
// buffer's non-temporal store) keep them from displacing cache lines the NS kernels reuse
// (measured 26.6 -> 24.8 ms per c5 step over both passes). The 64x64-tile kernel stores the NS
// operands X, X^T normally; the contiguous-run kernels store X non-temporal (+3% on their own,
// the products reading X only after the whole batch is staged).
// The pointers come from device pointer tables, so the compiler cannot tell they are global
// memory and would emit flat accesses (which also count against lgkmcnt); cast to the global
// address space.
template <class V>
__device__ __forceinline__ V ldg_nt(const V* p) {
  return __builtin_nontemporal_load((const __attribute__((address_space(1))) V*)p);
}
template <class V>
__device__ __forceinline__ void stg_nt(V* p, V v) {
  __builtin_nontemporal_store(v, (__attribute__((address_space(1))) V*)p);
}

// One 64x64 tile (rows r0.., columns c0..) of matrix l; returns this thread's share of the
// tile's sum of squares of ns_in. The caller synchronises before tileT is used again.
template <int ST>
__device__ __forceinline__ float pre_tile(const PreArgs& a, int l, int r0, int c0,
                                          uint16_t (*tileT)[kTile + kPad]) {
  const int tid = threadIdx.x;
  const int tc = tid & 15, tr = tid >> 4;

  const void* g = a.g_ptrs[l];
  float* buf = a.buf_ptrs ? a.buf_ptrs[l] : nullptr;  // null: plain NS input, no momentum
  uint16_t* Y = a.Y + (long long)l * a.sY;
  uint16_t* YT = a.YT + (long long)l * a.sYT;
  const float mu = a.mu;
  const bool vec = (a.cols & 3) == 0;
  // PRE_F16 reads the buffer PRE_NORM left (the new momentum) and only recomputes ns_in
  const bool read_buf = buf && (ST == PRE_F16 || !a.first_step);
  float sc = 1.f;
  if constexpr (ST == PRE_F16) sc = a.scale[l] * a.kx;
  if constexpr (ST == PRE_EST) sc = *a.est_ptrs[l] * a.kx;
  // PRE_EST without a usable estimate: momentum and partials only (the copy is staged later)
  const bool copy = ST != PRE_NORM && (ST != PRE_EST || sc > 0.f);

  // All loads of the thread's four rows are issued before any of them is used (raw words in
  // registers, converted afterwards): interior tiles take one block-uniform vector path.
  float gv[4][4], bv[4][4];
  const int col0 = c0 + 4 * tc;
  if (vec && r0 + kTile <= a.rows && c0 + kTile <= a.cols) {
    const long long base0 = (long long)(r0 + tr) * a.cols + col0, rs = 16LL * a.cols;
    if (a.g_dtype == DT_F32) {
      f32x4_t t[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        t[q] = ldg_nt(reinterpret_cast<const f32x4_t*>(static_cast<const float*>(g) + base0 +
                                                       q * rs));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        gv[q][0] = t[q].x; gv[q][1] = t[q].y; gv[q][2] = t[q].z; gv[q][3] = t[q].w;
      }
    } else {
      u32x2_t t[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        t[q] = ldg_nt(reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(g) + base0 +
                                                       q * rs));
      f32x4_t b[4];
      if (read_buf) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          b[q] = ldg_nt(reinterpret_cast<const f32x4_t*>(buf + base0 + q * rs));
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        gv[q][0] = bf2f(t[q].x & 0xffff); gv[q][1] = bf2f(t[q].x >> 16);
        gv[q][2] = bf2f(t[q].y & 0xffff); gv[q][3] = bf2f(t[q].y >> 16);
        bv[q][0] = read_buf ? b[q].x : 0.f; bv[q][1] = read_buf ? b[q].y : 0.f;
        bv[q][2] = read_buf ? b[q].z : 0.f; bv[q][3] = read_buf ? b[q].w : 0.f;
      }
    }
    if (a.g_dtype == DT_F32) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4_t b = {0.f, 0.f, 0.f, 0.f};
        if (read_buf) b = ldg_nt(reinterpret_cast<const f32x4_t*>(buf + base0 + q * rs));
        bv[q][0] = b.x; bv[q][1] = b.y; bv[q][2] = b.z; bv[q][3] = b.w;
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int row = r0 + tr + 16 * q;
      const long long base = (long long)row * a.cols + col0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gv[q][e] = bv[q][e] = 0.f;
        if (row < a.rows && col0 + e < a.cols) {
          gv[q][e] = load_any(g, a.g_dtype, base + e);
          if (read_buf) bv[q][e] = buf[base + e];
        }
      }
    }
  }

  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int rl = tr + 16 * q;
    const int row = r0 + rl;
    const int col = c0 + 4 * tc;
    bool in[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) in[e] = (row < a.rows) && (col + e < a.cols);
    const long long base = (long long)row * a.cols + col;
    float nb[4], ns[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // buf.mul_(mu).add_(g): two roundings, as the reference does them
      if (buf) {
        if constexpr (ST == PRE_F16) nb[e] = bv[q][e];
        else nb[e] = a.first_step ? gv[q][e] : __fadd_rn(__fmul_rn(bv[q][e], mu), gv[q][e]);
        // grad.add(buf, alpha=mu): one op, one rounding (a fused multiply-add)
        ns[e] = a.nesterov ? __builtin_fmaf(mu, nb[e], gv[q][e]) : nb[e];
      } else {
        nb[e] = gv[q][e];
        ns[e] = gv[q][e];
      }
      if (!in[e]) ns[e] = 0.f;
      ss += ns[e] * ns[e];
    }
    if (ST != PRE_F16 && buf) {   // PRE_BF16, PRE_NORM, PRE_EST write the new momentum
      if (vec && in[3]) {
        f32x4_t t; t.x = nb[0]; t.y = nb[1]; t.z = nb[2]; t.w = nb[3];
        stg_nt(reinterpret_cast<f32x4_t*>(buf + base), t);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (in[e]) buf[base + e] = nb[e];
      }
    }
    if (!copy) continue;
    uint16_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = ST == PRE_BF16 ? f2bf(ns[e]) : f2h(__fmul_rn(ns[e], sc));
    if (row < a.Rp && !a.skip_y) {
      uint2 p;
      p.x = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
      p.y = (uint32_t)o[2] | ((uint32_t)o[3] << 16);
      *reinterpret_cast<uint2*>(Y + (long long)row * a.ldy + col) = p;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) tileT[4 * tc + e][rl] = o[e];
  }
  if (copy && !a.skip_yt) {   // block-uniform
    __syncthreads();
    // transposed write: row cl of YT gets 64 consecutive source rows (128 B)
    const int cl = tid >> 2, seg = tid & 3;
    const int col = c0 + cl;
    if (col < a.Cp) {
      const uint4* src = reinterpret_cast<const uint4*>(&tileT[cl][16 * seg]);
      uint4* dst = reinterpret_cast<uint4*>(YT + (long long)col * a.ldyt + r0 + 16 * seg);
      dst[0] = src[0];
      dst[1] = src[1];
    }
  }
  return ss;
}

// Partial sums of ns_in^2: one per 1024 elements' unit of work of whichever staging kernel ran
// (a wave of a 64x64 tile, a 1024-element block of a wide matrix, four rows of a tall one's 64 x
// 256 tile), (Rp / 32) * (Cp / 32) per matrix, summed in a fixed order by the norm finalize.
template <int ST>
__global__ __launch_bounds__(256) void muon_pre_kernel(const PreArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tileT[kTile][kTile + kPad];
  const int tid = threadIdx.x;
  float ss = pre_tile<ST>(a, blockIdx.z, blockIdx.y * kTile, blockIdx.x * kTile, tileT);
  if constexpr (ST == PRE_F16) return;
  ss = wave_sum(ss);
  if ((tid & 63) == 0) {
    const long long blk = (long long)blockIdx.z * gridDim.x * gridDim.y +
                          blockIdx.y * gridDim.x + blockIdx.x;
    a.partials[blk * 4 + (tid >> 6)] = ss;
  }
}

// The per-element arithmetic of every staging kernel (the reference's order of roundings):
// buf.mul_(mu).add_(g) (two roundings; the first step takes g), then grad.add(buf, alpha=mu)
// (one fused rounding) for Nesterov. PRE_F16 recomputes ns_in from the momentum already written.
template <int ST>
__device__ __forceinline__ void pre_elem(const PreArgs& a, bool has_buf, float g, float b,
                                         float& nb, float& ns) {
  if (has_buf) {
    if constexpr (ST == PRE_F16) nb = b;
    else nb = a.first_step ? g : __fadd_rn(__fmul_rn(b, a.mu), g);
    ns = a.nesterov ? __builtin_fmaf(a.mu, nb, g) : nb;
  } else {
    nb = g;
    ns = g;
  }
}

template <int ST>
__device__ __forceinline__ uint16_t pre_out(float ns, float sc) {
  return ST == PRE_BF16 ? f2bf(ns) : f2h(__fmul_rn(ns, sc));
}

// Raw words of four consecutive gradient values (GF: fp32, else bf16) at flat index i, one
// vector load; unpacked by pre_unpack once every load of a batch has been issued.
template <bool GF>
using GradWords = typename std::conditional<GF, f32x4_t, u32x2_t>::type;
template <bool GF>
__device__ __forceinline__ GradWords<GF> pre_load_g(const void* g, long long i) {
  if constexpr (GF)
    return ldg_nt(reinterpret_cast<const f32x4_t*>(static_cast<const float*>(g) + i));
  else
    return ldg_nt(reinterpret_cast<const u32x2_t*>(static_cast<const uint16_t*>(g) + i));
}
template <bool GF>
__device__ __forceinline__ void pre_unpack(const GradWords<GF>& t, const f32x4_t& b,
                                           float (&gv)[4], float (&bv)[4]) {
  if constexpr (GF) {
    gv[0] = t.x; gv[1] = t.y; gv[2] = t.z; gv[3] = t.w;
  } else {
    gv[0] = bf2f(t.x & 0xffff); gv[1] = bf2f(t.x >> 16);
    gv[2] = bf2f(t.y & 0xffff); gv[3] = bf2f(t.y >> 16);
  }
  bv[0] = b.x; bv[1] = b.y; bv[2] = b.z; bv[3] = b.w;
}

// Copy scale of this launch for matrix l (1 for PRE_BF16 / PRE_NORM), and whether it writes one
// (PRE_EST without a usable estimate writes momentum and partials only).
template <int ST>
__device__ __forceinline__ float pre_scale(const PreArgs& a, int l, bool& copy) {
  float sc = 1.f;
  if constexpr (ST == PRE_F16) sc = a.scale[l] * a.kx;
  if constexpr (ST == PRE_EST) sc = *a.est_ptrs[l] * a.kx;
  copy = ST != PRE_NORM && (ST != PRE_EST || sc > 0.f);
  return sc;
}

// Wide orientation without padding (Rp == rows, Cp == cols, Y in the gradient's own layout, no
// transposed copy): the matrix is one flat array, four consecutive elements per thread and 1024
// per block over a grid of the whole matrix, so every wave instruction moves one contiguous run
// (1 KiB of momentum, 512 B of gradient and copy). Measured on a 64 x 4096^2 batch: 79% of 8 TB/s
// against 67% for the 64x64 tiles (whose wave instructions cover four 256-byte row pieces), and
// 58-70% for 8 elements per thread or several pieces per block. The copy is stored non-temporal:
// the products read it only after the whole batch is staged.
template <int ST, bool GF>
__global__ __launch_bounds__(256) void muon_pre_wide_kernel(const PreArgs a) {
  const int l = blockIdx.y;
  const long long i = (long long)blockIdx.x * 1024 + 4 * threadIdx.x;
  const void* g = a.g_ptrs[l];
  float* buf = a.buf_ptrs ? a.buf_ptrs[l] : nullptr;
  const bool read_buf = buf && (ST == PRE_F16 || !a.first_step);
  bool copy;
  const float sc = pre_scale<ST>(a, l, copy);
  const GradWords<GF> gw = pre_load_g<GF>(g, i);
  const f32x4_t bw = read_buf ? ldg_nt(reinterpret_cast<const f32x4_t*>(buf + i))
                              : f32x4_t{0.f, 0.f, 0.f, 0.f};
  float gv[4], bv[4], nb[4], ns[4];
  pre_unpack<GF>(gw, bw, gv, bv);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    pre_elem<ST>(a, buf != nullptr, gv[e], bv[e], nb[e], ns[e]);
    ss += ns[e] * ns[e];
  }
  if (ST != PRE_F16 && buf)
    stg_nt(reinterpret_cast<f32x4_t*>(buf + i), f32x4_t{nb[0], nb[1], nb[2], nb[3]});
  if (copy) {
    u32x2_t p;
    p.x = (uint32_t)pre_out<ST>(ns[0], sc) | ((uint32_t)pre_out<ST>(ns[1], sc) << 16);
    p.y = (uint32_t)pre_out<ST>(ns[2], sc) | ((uint32_t)pre_out<ST>(ns[3], sc) << 16);
    stg_nt(reinterpret_cast<u32x2_t*>(a.Y + (long long)l * a.sY + i), p);
  }
  if constexpr (ST == PRE_F16) return;
  __shared__ float red[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0)
    a.partials[(long long)l * gridDim.x + blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

// Tall orientation without padding (rows % 64 == 0, cols % 256 == 0; only the transposed copy
// YT, the NS operand X = ns_in^T): 64 x 256 tiles of the gradient, wave w taking rows w, w + 4,
// ... with four consecutive columns per lane (each wave instruction one contiguous row run, as
// in the wide kernel), eight rows' loads in flight; the copy goes through LDS and leaves as X rows
// of 64 values (128-byte runs). Measured on a 32 x 14336x4096 batch: 76% of 8 TB/s against 65%
// for the 64x64 tiles (128 x 256 tiles: 74%, four rows in flight: 75%).
template <int ST, bool GF>
__global__ __launch_bounds__(256) void muon_pre_tall_kernel(const PreArgs a) {
  constexpr int TR = 64, TC = 256, RB = 8;
  __shared__ __attribute__((aligned(16))) uint16_t tt[TC][TR + kPad];
  const int l = blockIdx.z;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const long long r0 = (long long)blockIdx.y * TR, c0 = (long long)blockIdx.x * TC;
  const int c = 4 * lane;
  const void* g = a.g_ptrs[l];
  float* buf = a.buf_ptrs ? a.buf_ptrs[l] : nullptr;
  const bool read_buf = buf && (ST == PRE_F16 || !a.first_step);
  bool copy;
  const float sc = pre_scale<ST>(a, l, copy);
  float ss[TR / 16] = {0.f, 0.f, 0.f, 0.f};   // one per four rows of this wave
#pragma unroll
  for (int rb = 0; rb < TR / 4; rb += RB) {
    // every load of the batch issued before any is used
    GradWords<GF> gw[RB];
    f32x4_t bw[RB];
#pragma unroll
    for (int q = 0; q < RB; ++q)
      gw[q] = pre_load_g<GF>(g, (r0 + w + 4 * (rb + q)) * a.cols + c0 + c);
    if (read_buf) {
#pragma unroll
      for (int q = 0; q < RB; ++q)
        bw[q] = ldg_nt(reinterpret_cast<const f32x4_t*>(buf + (r0 + w + 4 * (rb + q)) * a.cols +
                                                        c0 + c));
    } else {
#pragma unroll
      for (int q = 0; q < RB; ++q) bw[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int q = 0; q < RB; ++q) {
      const int rl = w + 4 * (rb + q);
      float gv[4], bv[4], nb[4], ns[4];
      pre_unpack<GF>(gw[q], bw[q], gv, bv);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pre_elem<ST>(a, buf != nullptr, gv[e], bv[e], nb[e], ns[e]);
        ss[(rb + q) / 4] += ns[e] * ns[e];
      }
      if (ST != PRE_F16 && buf)
        stg_nt(reinterpret_cast<f32x4_t*>(buf + (r0 + rl) * a.cols + c0 + c),
               f32x4_t{nb[0], nb[1], nb[2], nb[3]});
      if (copy) {
#pragma unroll
        for (int e = 0; e < 4; ++e) tt[c + e][rl] = pre_out<ST>(ns[e], sc);
      }
    }
  }
  if (copy) {   // block-uniform
    __syncthreads();
    // X rows c0 + cr, 64 values (eight 16-byte pieces) each, 32 rows per pass
    uint16_t* X = a.YT + (long long)l * a.sYT;
#pragma unroll
    for (int pass = 0; pass < TC / 32; ++pass) {
      const int cr = pass * 32 + (threadIdx.x >> 3), pc = threadIdx.x & 7;
      const u32x4_copy_t v = *reinterpret_cast<const u32x4_copy_t*>(&tt[cr][pc * 8]);
      stg_nt(reinterpret_cast<u32x4_copy_t*>(X + (c0 + cr) * a.ldyt + r0 + pc * 8), v);
    }
  }
  if constexpr (ST == PRE_F16) return;
  const long long blk = (long long)l * gridDim.x * gridDim.y + blockIdx.y * gridDim.x + blockIdx.x;
#pragma unroll
  for (int j = 0; j < TR / 16; ++j) {
    const float s = wave_sum(ss[j]);
    if (lane == 0) a.partials[blk * 16 + w * 4 + j] = s;
  }
}

// The exact-scale copy for the matrices flagged in a.restage (a scale that moved by more than
// 4x, or none kept yet). Rarely any are, so the grid is small and strides over the tiles of
// the flagged matrices only; with nothing flagged each block reads L flags and exits.
__global__ __launch_bounds__(256) void muon_restage_kernel(const PreArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t tileT[kTile][kTile + kPad];
  const int tx = a.Cp / kTile, per = tx * (a.Rp / kTile);
  for (int l = 0; l < a.L; ++l) {
    if (!a.restage[l]) continue;   // block-uniform
    for (int t = blockIdx.x; t < per; t += gridDim.x) {
      __syncthreads();   // the previous tile's transposed read of tileT is done
      pre_tile<PRE_F16>(a, l, (t / tx) * kTile, (t % tx) * kTile, tileT);
    }
  }
}

// Sum of matrix l's partials in fp64, in a fixed order (the same bits on every call): thread t
// adds groups of four consecutive partials t, t + 1024, ..., then a tree over the 1024 threads.
// One block per matrix; 1024 threads with four loads per step keep ~57K partials of a
// 4096 x 14336 matrix from being a long chain of dependent load latencies. Result in red[0].
constexpr int kFinThreads = 1024;
__device__ __forceinline__ void sum_partials(const float* partials, int nparts, int l,
                                             double* red) {
  const float* p = partials + (long long)l * nparts;
  const int t = threadIdx.x;
  double s = 0.0;
  if ((nparts & 3) == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0) {
    const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(p);
    for (int q = t; q < nparts / 4; q += kFinThreads) {
      const f32x4_t v = p4[q];
      s += ((double)v.x + (double)v.y) + ((double)v.z + (double)v.w);
    }
  } else {
    for (int q = t; q < nparts; q += kFinThreads) s += (double)p[q];
  }
  red[t] = s;
  __syncthreads();
  for (int w = kFinThreads / 2; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
}

__global__ __launch_bounds__(kFinThreads) void norm_finalize_kernel(const float* partials,
                                                                    int nparts, float eps,
                                                                    float* scale,
                                                                    float* scale_sq) {
  __shared__ double red[kFinThreads];
  const int l = blockIdx.x;
  sum_partials(partials, nparts, l, red);
  if (threadIdx.x == 0) {
    const float nrm = (float)sqrt(red[0]);
    const float sc = 1.0f / (nrm + eps);
    scale[l] = sc;
    scale_sq[l] = sc * sc;
  }
}

__global__ __launch_bounds__(256) void muon_update_kernel(const UpdateArgs a) {
  const int l = blockIdx.y;
  void* w = a.w_ptrs[l];
  const void* u = a.u_ptrs[l];
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.numel; i += stride) {
    const float uv = load_any(u, a.u_dtype, i);
    if (a.w_dtype == DT_F32) {
      float* wp = static_cast<float*>(w) + i;
      float wv = *wp;
      if (a.decay != 1.f) wv = __fmul_rn(wv, a.decay);
      *wp = __builtin_fmaf(-a.lrs, uv, wv);   // add_(U, alpha=-lrs): one rounding
    } else {
      uint16_t* wp = static_cast<uint16_t*>(w) + i;
      float wv = bf2f(*wp);
      if (a.decay != 1.f) wv = bf2f(f2bf(__fmul_rn(wv, a.decay)));
      *wp = f2bf(__builtin_fmaf(-a.lrs, uv, wv));
    }
  }
}

__global__ __launch_bounds__(kFinThreads) void norm_finalize_est_kernel(
    const float* partials, int nparts, float eps, float* scale, float* scale_sq,
    float* const* est_ptrs, float* ratio, float* ratio_sq, int* restage) {
  __shared__ double red[kFinThreads];
  const int l = blockIdx.x;
  sum_partials(partials, nparts, l, red);
  if (threadIdx.x == 0) {
    const float nrm = (float)sqrt(red[0]);
    const float sc = 1.0f / (nrm + eps);
    scale[l] = sc;
    scale_sq[l] = sc * sc;
    float r = 1.f;
    bool ok = false;
    if (est_ptrs) {
      const float est = *est_ptrs[l];
      if (est > 0.f) {
        r = sc / est;
        ok = r >= 0.25f && r <= 4.f;   // false for NaN / inf too
      }
      *est_ptrs[l] = sc;
    }
    if (!ok) r = 1.f;
    ratio[l] = r;
    ratio_sq[l] = r * r;
    restage[l] = ok ? 0 : 1;
  }
}

// dst[l][r][c] = src[l][r][c] for r < rows, c < cols, 0 elsewhere in the rows_out x cols_out
// extent: the zero-padded operand copies of an unaligned or ragged SYRK call, and the copy of
// its M x M corner back out. One block per output row; 16-bit elements of either type.
__global__ __launch_bounds__(256) void pad_copy_kernel(const uint16_t* src, long long lds,
                                                       long long ss, uint16_t* dst, long long ldd,
                                                       long long sd, int rows, int cols,
                                                       int rows_out, int cols_out) {
  const long long row = blockIdx.x;
  const int l = (int)(row / rows_out), r = (int)(row % rows_out);
  uint16_t* d = dst + (long long)l * sd + (long long)r * ldd;
  const uint16_t* s = src + (long long)l * ss + (long long)r * lds;
  const bool live = r < rows;
  for (int c = threadIdx.x; c < cols_out; c += 256) d[c] = (live && c < cols) ? s[c] : (uint16_t)0;
}

// dst = src in 16-byte chunks, one per thread over a grid of the whole array, non-temporal loads
// and stores: the streaming rate of this HBM for a read + write of distinct buffers (measured
// 82% of the 8 TB/s spec on MI355X; a grid-stride loop of the same loads tops out near 72%).
__global__ __launch_bounds__(256) void stream_copy_kernel(const u32x4_copy_t* __restrict__ src,
                                                          u32x4_copy_t* __restrict__ dst,
                                                          long long n16) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

hipError_t launch_stream_copy(const void* src, void* dst, long long n16, hipStream_t stream) {
  if (n16 <= 0) return hipSuccess;
  const long long blocks = (n16 + 255) / 256;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(stream_copy_kernel, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const u32x4_copy_t*>(src), static_cast<u32x4_copy_t*>(dst), n16);
  return hipGetLastError();
}

hipError_t launch_pad_copy(const uint16_t* src, long long lds, long long ss, uint16_t* dst,
                           long long ldd, long long sd, int rows, int cols, int rows_out,
                           int cols_out, int L, hipStream_t stream) {
  const long long nb = (long long)L * rows_out;
  if (nb <= 0 || cols_out <= 0) return hipSuccess;
  hipLaunchKernelGGL(pad_copy_kernel, dim3((unsigned)nb), dim3(256), 0, stream, src, lds, ss, dst,
                     ldd, sd, rows, cols, rows_out, cols_out);
  return hipGetLastError();
}

int pre_blocks_per_mat(int Rp, int Cp) { return (Rp / 32) * (Cp / 32); }

hipError_t launch_pre(const PreArgs& a, hipStream_t stream) {
  dim3 block(256);
  if (a.stage == PRE_F16 && a.restage) {
    const int tiles = (a.Rp / kTile) * (a.Cp / kTile);
    hipLaunchKernelGGL(muon_restage_kernel, dim3(std::min(tiles, 2048)), block, 0, stream, a);
    return hipGetLastError();
  }
  // Which copy the launch writes: Y (the gradient's layout), YT (transposed), both or none
  // (PRE_NORM writes none). Unpadded matrices with one copy take the contiguous-run kernels;
  // everything else (padding, both copies) the 64x64 tiles. All three write the same partials
  // layout size, (Rp / 32) * (Cp / 32) per matrix.
  const bool y = a.stage != PRE_NORM && !a.skip_y, yt = a.stage != PRE_NORM && !a.skip_yt;
  const bool unpadded = a.Rp == a.rows && a.Cp == a.cols;
  const bool wide = unpadded && !yt && (!y || a.ldy == a.cols);
  const bool tall = !wide && unpadded && !y && a.rows % 64 == 0 && a.cols % 256 == 0;
#define DMUON_PRE(KERNEL, GRID, ...)                                                           \
  do {                                                                                         \
    if (a.stage == PRE_NORM)                                                                   \
      hipLaunchKernelGGL((KERNEL<PRE_NORM __VA_ARGS__>), GRID, block, 0, stream, a);           \
    else if (a.stage == PRE_F16)                                                               \
      hipLaunchKernelGGL((KERNEL<PRE_F16 __VA_ARGS__>), GRID, block, 0, stream, a);            \
    else if (a.stage == PRE_EST)                                                               \
      hipLaunchKernelGGL((KERNEL<PRE_EST __VA_ARGS__>), GRID, block, 0, stream, a);            \
    else                                                                                       \
      hipLaunchKernelGGL((KERNEL<PRE_BF16 __VA_ARGS__>), GRID, block, 0, stream, a);           \
  } while (0)
  const bool gf = a.g_dtype == DT_F32;
  const dim3 gwide((unsigned)((long long)a.rows * a.cols / 1024), a.L);
  const dim3 gtall(a.cols / 256, a.rows / 64, a.L);
  if (wide && gf) DMUON_PRE(muon_pre_wide_kernel, gwide, , true);
  else if (wide) DMUON_PRE(muon_pre_wide_kernel, gwide, , false);
  else if (tall && gf) DMUON_PRE(muon_pre_tall_kernel, gtall, , true);
  else if (tall) DMUON_PRE(muon_pre_tall_kernel, gtall, , false);
  else DMUON_PRE(muon_pre_kernel, dim3(a.Cp / kTile, a.Rp / kTile, a.L));
#undef DMUON_PRE
  return hipGetLastError();
}

hipError_t launch_norm_finalize_est(const float* partials, int nparts, int L, float eps,
                                    float* scale, float* scale_sq, float* const* est_ptrs,
                                    float* ratio, float* ratio_sq, int* restage,
                                    hipStream_t stream) {
  hipLaunchKernelGGL(norm_finalize_est_kernel, dim3(L), dim3(kFinThreads), 0, stream, partials,
                     nparts, eps, scale, scale_sq, est_ptrs, ratio, ratio_sq, restage);
  return hipGetLastError();
}

hipError_t launch_norm_finalize(const float* partials, int nparts, int L, float eps, float* scale,
                                float* scale_sq, hipStream_t stream) {
  hipLaunchKernelGGL(norm_finalize_kernel, dim3(L), dim3(kFinThreads), 0, stream, partials,
                     nparts, eps, scale, scale_sq);
  return hipGetLastError();
}

hipError_t launch_update(const UpdateArgs& a, hipStream_t stream) {
  long long blocks = (a.numel + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(muon_update_kernel, dim3((unsigned)blocks, a.L), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace dmuon

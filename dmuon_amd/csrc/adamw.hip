// Fused multi-tensor decoupled AdamW on gfx950: one HBM pass over a bucket of tensors.
//
// Per element, in the storage dtype of the parameter (p, exp_avg m and exp_avg_sq v share it)
// with fp32 arithmetic, and rounded back to that dtype after every step exactly where the
// reference's torch._foreach sequence materialises a tensor (muon.py:1902-1916):
//
//   p = R(p * (1 - lr*wd))                     (only when wd > 0)
//   m = R(m * b1);  m = R(m + (1-b1) * g)
//   v = R(v * b2);  v = R(v + (1-b2) * (g*g))
//   d = R(sqrt(v)); d = R(d / sqrt(bc2)); d = R(d + eps)
//   p = R(p + (-lr/bc1) * (m / d))
//   q = round_to_q_dtype(p)                    (optional: the forward copy of a master p)
//
// Multiplies and adds are separate roundings (the library is built with -ffp-contract=off);
// sqrt and division are the correctly rounded ones. For fp32 storage R is the identity.
//
// Work split: the tensors are concatenated into one index space (offsets = prefix sums of
// their sizes); block b takes the contiguous range [4096 b, 4096 (b + 1)) of it, finds its
// first tensor by binary search and walks the tensors the range overlaps. Small ranges over a
// grid of the whole index space keep the addresses that the resident blocks touch close
// together; with a few long ranges per block (8192 blocks over 1.05 G elements) the same
// kernel moved 4.5 TB/s instead of 5.4 on MI355X. Inside a tensor, 8-element vectors (16-byte
// loads/stores of bf16, two of fp32) cover the aligned middle; ragged ends and tensors whose
// base pointers are not 16-byte aligned take the per-element path.
#include "dmuon_amd_internal.h"

namespace dmuon {
namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

template <int D>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (D == DT_BF16) return bf2f(f2bf(x));
  else return x;
}

template <int D>
__device__ __forceinline__ float ld1(const void* p, long long i) {
  if constexpr (D == DT_BF16) return bf2f(static_cast<const uint16_t*>(p)[i]);
  else return static_cast<const float*>(p)[i];
}
template <int D>
__device__ __forceinline__ void st1(void* p, long long i, float x) {
  if constexpr (D == DT_BF16) static_cast<uint16_t*>(p)[i] = f2bf(x);
  else static_cast<float*>(p)[i] = x;
}

// 8 consecutive elements starting at element i (i % 8 == 0, base 16-byte aligned). Every
// stream is read and written once per step, so all vector accesses are non-temporal: on MI355X
// the c5 AdamW bucket (1.05 G bf16 elements) took 2.59 ms this way against 2.75 with ordinary
// loads and stores (non-temporal loads or stores alone: 2.81 and 2.73 ms; the gradient's loads
// alone 2.69).
template <int D>
__device__ __forceinline__ void ld8(const void* p, long long i, float* x) {
  if constexpr (D == DT_BF16) {
    const u32x4_t w = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = bf2f(w[k] & 0xffff);
      x[2 * k + 1] = bf2f(w[k] >> 16);
    }
  } else {
    const u32x4_t* q = reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p) + i);
    const u32x4_t w0 = __builtin_nontemporal_load(q), w1 = __builtin_nontemporal_load(q + 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[k] = __uint_as_float(w0[k]);
      x[k + 4] = __uint_as_float(w1[k]);
    }
  }
}
template <int D>
__device__ __forceinline__ void st8(void* p, long long i, const float* x) {
  if constexpr (D == DT_BF16) {
    u32x4_t w;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = (unsigned)f2bf(x[2 * k]) | ((unsigned)f2bf(x[2 * k + 1]) << 16);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p) + i));
  } else {
    u32x4_t* q = reinterpret_cast<u32x4_t*>(static_cast<float*>(p) + i);
    __builtin_nontemporal_store(u32x4_t{__float_as_uint(x[0]), __float_as_uint(x[1]),
                                        __float_as_uint(x[2]), __float_as_uint(x[3])}, q);
    __builtin_nontemporal_store(u32x4_t{__float_as_uint(x[4]), __float_as_uint(x[5]),
                                        __float_as_uint(x[6]), __float_as_uint(x[7])}, q + 1);
  }
}

template <int D>
__device__ __forceinline__ void adamw_elt(float& p, float g, float& m, float& v,
                                          const AdamWArgs& a) {
  if (a.apply_wd) p = rnd<D>(p * a.wd_scale);
  m = rnd<D>(m * a.beta1);
  m = rnd<D>(m + a.alpha1 * g);
  v = rnd<D>(v * a.beta2);
  v = rnd<D>(v + a.alpha2 * (g * g));
  float d = rnd<D>(sqrtf(v));
  d = rnd<D>(d / a.bc2_sqrt);
  d = rnd<D>(d + a.eps);
  p = rnd<D>(p + a.neg_step * (m / d));
}

// Two elements at once, the same operations as adamw_elt: bf16 roundings of a pair share one
// v_cvt_pk_bf16_f32 (each half rounded to nearest even on its own, as f2bf does).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
template <int D>
__device__ __forceinline__ void rnd2(float& x, float& y) {
  if constexpr (D == DT_BF16) {
    const f32x2_t v = {x, y};
    const unsigned w = __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2_t));
    x = __uint_as_float(w << 16);
    y = __uint_as_float(w & 0xffff0000u);
  }
}
template <int D>
__device__ __forceinline__ void adamw_elt2(float* p, const float* g, float* m, float* v,
                                           const AdamWArgs& a) {
  if (a.apply_wd) {
    p[0] = p[0] * a.wd_scale; p[1] = p[1] * a.wd_scale; rnd2<D>(p[0], p[1]);
  }
  m[0] = m[0] * a.beta1; m[1] = m[1] * a.beta1; rnd2<D>(m[0], m[1]);
  m[0] = m[0] + a.alpha1 * g[0]; m[1] = m[1] + a.alpha1 * g[1]; rnd2<D>(m[0], m[1]);
  v[0] = v[0] * a.beta2; v[1] = v[1] * a.beta2; rnd2<D>(v[0], v[1]);
  v[0] = v[0] + a.alpha2 * (g[0] * g[0]); v[1] = v[1] + a.alpha2 * (g[1] * g[1]);
  rnd2<D>(v[0], v[1]);
  float d0 = sqrtf(v[0]), d1 = sqrtf(v[1]);
  rnd2<D>(d0, d1);
  d0 = d0 / a.bc2_sqrt; d1 = d1 / a.bc2_sqrt; rnd2<D>(d0, d1);
  d0 = d0 + a.eps; d1 = d1 + a.eps; rnd2<D>(d0, d1);
  p[0] = p[0] + a.neg_step * (m[0] / d0); p[1] = p[1] + a.neg_step * (m[1] / d1);
  rnd2<D>(p[0], p[1]);
}

template <int PD, int GD>
__global__ __launch_bounds__(256) void adamw_kernel(const AdamWArgs a) {
  const long long lo = (long long)blockIdx.x * a.per_block;
  if (lo >= a.total) return;
  const long long hi = min(lo + a.per_block, a.total);
  // last tensor whose start is <= lo
  int t = 0, r = a.n - 1;
  while (t < r) {
    const int mid = (t + r + 1) >> 1;
    if (a.offsets[mid] <= lo) t = mid; else r = mid - 1;
  }
  const int tid = threadIdx.x;
  for (; t < a.n && a.offsets[t] < hi; ++t) {
    const long long t0 = a.offsets[t];
    const long long s = max(lo, t0) - t0, e = min(hi, a.offsets[t + 1]) - t0;
    if (s >= e) continue;
    void* P = reinterpret_cast<void*>(a.p_ptrs[t]);
    const void* G = reinterpret_cast<const void*>(a.g_ptrs[t]);
    void* M = reinterpret_cast<void*>(a.m_ptrs[t]);
    void* V = reinterpret_cast<void*>(a.v_ptrs[t]);
    const int64_t pub_addr = a.pub_ptrs ? a.pub_ptrs[t] : 0;
    void* Q = reinterpret_cast<void*>(pub_addr);           // forward copy of p, or null
    const bool aligned =
        ((a.p_ptrs[t] | a.g_ptrs[t] | a.m_ptrs[t] | a.v_ptrs[t] | pub_addr) & 15) == 0;
    long long vs = e, ve = e;
    if (aligned) {
      vs = min((s + 7) & ~7LL, e);
      ve = max(e & ~7LL, vs);
    }
    for (long long i = vs + 8LL * tid; i < ve; i += 8LL * 256) {
      float p[8], g[8], m[8], v[8];
      ld8<PD>(P, i, p);
      ld8<GD>(G, i, g);
      ld8<PD>(M, i, m);
      ld8<PD>(V, i, v);
#pragma unroll
      for (int k = 0; k < 8; k += 2) adamw_elt2<PD>(p + k, g + k, m + k, v + k, a);
      st8<PD>(P, i, p);
      st8<PD>(M, i, m);
      st8<PD>(V, i, v);
      if (Q) {
        if (a.pub_dtype == DT_BF16) st8<DT_BF16>(Q, i, p);
        else st8<DT_F32>(Q, i, p);
      }
    }
    // ragged head [s, vs) and tail [ve, e) (the whole range when unaligned: vs = ve = e)
    const long long nh = vs - s, nt = e - ve;
    for (long long k = tid; k < nh + nt; k += 256) {
      const long long i = k < nh ? s + k : ve + (k - nh);
      float p = ld1<PD>(P, i), m = ld1<PD>(M, i), v = ld1<PD>(V, i);
      adamw_elt<PD>(p, ld1<GD>(G, i), m, v, a);
      st1<PD>(P, i, p);
      st1<PD>(M, i, m);
      st1<PD>(V, i, v);
      if (Q) {
        if (a.pub_dtype == DT_BF16) st1<DT_BF16>(Q, i, p);
        else st1<DT_F32>(Q, i, p);
      }
    }
  }
}

}  // namespace

hipError_t launch_adamw(AdamWArgs a, hipStream_t stream) {
  if (a.total <= 0 || a.n <= 0) return hipSuccess;
  // 4096 elements per block (a multiple of the 8-element vector), more when the grid would
  // exceed 2^31 blocks
  long long per = 4096;
  if ((a.total + per - 1) / per > 0x7fffffffLL) per = ((a.total + 0x7ffffffeLL) / 0x7fffffffLL + 7) & ~7LL;
  a.per_block = per;
  const long long blocks = (a.total + per - 1) / per;
  const dim3 grid((unsigned)blocks), block(256);
  if (a.p_dtype == DT_F32 && a.g_dtype == DT_F32)
    hipLaunchKernelGGL((adamw_kernel<DT_F32, DT_F32>), grid, block, 0, stream, a);
  else if (a.p_dtype == DT_F32)
    hipLaunchKernelGGL((adamw_kernel<DT_F32, DT_BF16>), grid, block, 0, stream, a);
  else if (a.g_dtype == DT_F32)
    hipLaunchKernelGGL((adamw_kernel<DT_BF16, DT_F32>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((adamw_kernel<DT_BF16, DT_BF16>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace dmuon

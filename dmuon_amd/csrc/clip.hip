// Segmented gradient clipping on gfx950: the two device operations of the reference's fast
// clip path (dmuon/csrc/fast_clip_kernel.cu:34-107), over the same job table.
//
//   sumsq  local_sq[segments[t]] += sum over the job's elements of float(x)^2
//   scale  x <- T(float(x) * coefs[segments[t]])          in place
//
// A job is (tensor t = job_tensor_ids[j], elements [job_offsets[j], +chunk_size) clipped to
// numels[t]). The norm pass runs one 256-thread block per job (one atomic add per job, as in
// the reference); the scale pass, which has no reduction, splits each job into pieces of
// ClipArgs::piece elements (8192), one block per piece, consecutive blocks on consecutive
// pieces: on MI355X that moved the c5 gradients at 5.9 TB/s instead of 5.2 with one block per
// 262144-element job (the addresses the resident blocks touch stay close together). Tensor dtypes use the reference's codes
// (0 fp32, 1 fp16, 2 bf16; fast_clip.py:31-35). Where the reference walks a job with one
// scalar load per thread and reduces through a shared-memory tree, here the aligned middle of
// the job is read in 16-byte vectors (4 fp32 / 8 half-precision values per lane; the norm pass
// keeps four non-temporal loads in flight per lane, the scale pass two vectors), the partial
// sums are reduced across the wave with cross-lane shuffles and across the four waves through
// a 16-byte LDS array, and one lane per block adds the block's sum into local_sq with a
// global float atomic (so, as in the reference, the order of those additions -- and hence the
// last bits of local_sq -- may differ from run to run).
#include "dmuon_amd_internal.h"

namespace dmuon {
namespace {

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

constexpr int CF32 = 0, CF16 = 1, CBF16 = 2;

template <int D>
__device__ __forceinline__ float to_f(uint32_t bits16) {
  if constexpr (D == CF16) return static_cast<float>(__builtin_bit_cast(_Float16, (uint16_t)bits16));
  else return __uint_as_float(bits16 << 16);
}
template <int D>
__device__ __forceinline__ uint32_t from_f(float f) {
  if constexpr (D == CF16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  else return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

template <int D>
__device__ __forceinline__ float load1(const void* p, long long i) {
  if constexpr (D == CF32) return static_cast<const float*>(p)[i];
  else return to_f<D>(static_cast<const uint16_t*>(p)[i]);
}
template <int D>
__device__ __forceinline__ void scale1(void* p, long long i, float c) {
  if constexpr (D == CF32) {
    float* q = static_cast<float*>(p) + i;
    *q = *q * c;
  } else {
    uint16_t* q = static_cast<uint16_t*>(p) + i;
    *q = (uint16_t)from_f<D>(to_f<D>(*q) * c);
  }
}

struct Job {
  int t;
  long long begin, end;
};
__device__ __forceinline__ Job job_of(const ClipArgs& a) {
  Job j;
  j.t = a.job_tensor_ids[blockIdx.x];
  j.begin = a.job_offsets[blockIdx.x];
  j.end = min(j.begin + a.chunk, (long long)a.numels[j.t]);
  return j;
}
// piece blockIdx.x % pieces of job blockIdx.x / pieces (empty past the end of its tensor)
__device__ __forceinline__ Job piece_of(const ClipArgs& a) {
  const long long pieces = (a.chunk + a.piece - 1) / a.piece;
  const long long b = blockIdx.x, job = b / pieces, k = b - job * pieces;
  Job j;
  j.t = a.job_tensor_ids[job];
  const long long end = min(a.job_offsets[job] + a.chunk, (long long)a.numels[j.t]);
  j.begin = min(a.job_offsets[job] + k * a.piece, end);
  j.end = min(j.begin + a.piece, end);
  return j;
}

// vector width in elements of a 16-byte access
template <int D>
constexpr int vw() { return D == CF32 ? 4 : 8; }

template <int D>
__device__ float job_sumsq(const void* p, long long begin, long long end) {
  constexpr int V = vw<D>();
  const bool aligned = (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  long long vs = end, ve = end;
  if (aligned && begin < end) {
    vs = min((begin + V - 1) / V * V, end);
    ve = max(end / V * V, vs);
  }
  // four 16-byte loads in flight per thread, four partial sums
  float s4[4] = {0.f, 0.f, 0.f, 0.f};
  long long i = vs + (long long)V * threadIdx.x;
  for (; i + 3LL * V * 256 < ve; i += 4LL * V * 256) {
    u32x4_t w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (D == CF32) w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p) + i + u * V * 256));
      else w[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i + u * V * 256));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if constexpr (D == CF32) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float x = __uint_as_float(w[u][k]);
          s4[u] += x * x;
        }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float x0 = to_f<D>(w[u][k] & 0xffff), x1 = to_f<D>(w[u][k] >> 16);
          s4[u] += x0 * x0;
          s4[u] += x1 * x1;
        }
      }
    }
  }
  float s = (s4[0] + s4[1]) + (s4[2] + s4[3]);
  for (; i < ve; i += (long long)V * 256) {
    if constexpr (D == CF32) {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p) + i);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x = __uint_as_float(w[k]);
        s += x * x;
      }
    } else {
      const u32x4_t w = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float x0 = to_f<D>(w[k] & 0xffff), x1 = to_f<D>(w[k] >> 16);
        s += x0 * x0;
        s += x1 * x1;
      }
    }
  }
  const long long nh = vs - begin, nt = end - ve;
  for (long long k = threadIdx.x; k < nh + nt; k += 256) {
    const float x = load1<D>(p, k < nh ? begin + k : ve + (k - nh));
    s += x * x;
  }
  return s;
}

template <int D>
__device__ void job_scale(void* p, long long begin, long long end, float c) {
  constexpr int V = vw<D>();
  const bool aligned = (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  long long vs = end, ve = end;
  if (aligned && begin < end) {
    vs = min((begin + V - 1) / V * V, end);
    ve = max(end / V * V, vs);
  }
  auto sc = [&](u32x4_t w) {
    if constexpr (D == CF32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = __float_as_uint(__uint_as_float(w[k]) * c);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        w[k] = from_f<D>(to_f<D>(w[k] & 0xffff) * c) | (from_f<D>(to_f<D>(w[k] >> 16) * c) << 16);
    }
    return w;
  };
  u32x4_t* base = D == CF32 ? reinterpret_cast<u32x4_t*>(static_cast<float*>(p))
                            : reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(p));
  long long i = vs + (long long)V * threadIdx.x;
  // four vectors in flight per thread; the gradient is streamed once (non-temporal both ways)
  for (; i + 3LL * V * 256 < ve; i += 4LL * V * 256) {
    u32x4_t w[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) w[u] = __builtin_nontemporal_load(base + i / V + u * 256);
#pragma unroll
    for (int u = 0; u < 4; ++u) __builtin_nontemporal_store(sc(w[u]), base + i / V + u * 256);
  }
  for (; i < ve; i += (long long)V * 256) {
    u32x4_t* q = base + i / V;
    *q = sc(*q);
  }
  const long long nh = vs - begin, nt = end - ve;
  for (long long k = threadIdx.x; k < nh + nt; k += 256)
    scale1<D>(p, k < nh ? begin + k : ve + (k - nh), c);
}

__global__ __launch_bounds__(256) void seg_sumsq_kernel(const ClipArgs a) {
  __shared__ float part[4];
  const Job j = job_of(a);
  const void* p = reinterpret_cast<const void*>(a.ptrs[j.t]);
  const int dt = a.dtypes[j.t];
  float s;
  if (dt == CF32) s = job_sumsq<CF32>(p, j.begin, j.end);
  else if (dt == CF16) s = job_sumsq<CF16>(p, j.begin, j.end);
  else s = job_sumsq<CBF16>(p, j.begin, j.end);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) part[wave] = s;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(a.local_sq + a.segments[j.t], (part[0] + part[1]) + (part[2] + part[3]));
}

__global__ __launch_bounds__(256) void seg_scale_kernel(const ClipArgs a) {
  const Job j = piece_of(a);
  if (j.begin >= j.end) return;
  void* p = reinterpret_cast<void*>(a.ptrs[j.t]);
  const int dt = a.dtypes[j.t];
  const float c = a.coefs[a.segments[j.t]];
  if (dt == CF32) job_scale<CF32>(p, j.begin, j.end, c);
  else if (dt == CF16) job_scale<CF16>(p, j.begin, j.end, c);
  else job_scale<CBF16>(p, j.begin, j.end, c);
}

}  // namespace

hipError_t launch_clip_sumsq(const ClipArgs& a, hipStream_t stream) {
  if (a.n_jobs <= 0) return hipSuccess;
  hipLaunchKernelGGL(seg_sumsq_kernel, dim3((unsigned)a.n_jobs), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_clip_scale(ClipArgs a, hipStream_t stream) {
  if (a.n_jobs <= 0) return hipSuccess;
  // 8192-element pieces; longer ones when the grid would exceed 2^31 blocks
  a.piece = 8192;
  long long pieces = (a.chunk + a.piece - 1) / a.piece;
  if (pieces > 0x7fffffffLL / a.n_jobs) {
    pieces = 0x7fffffffLL / a.n_jobs;
    a.piece = (a.chunk + pieces - 1) / pieces;
    pieces = (a.chunk + a.piece - 1) / a.piece;
  }
  hipLaunchKernelGGL(seg_scale_kernel, dim3((unsigned)(a.n_jobs * pieces)), dim3(256), 0, stream,
                     a);
  return hipGetLastError();
}

}  // namespace dmuon

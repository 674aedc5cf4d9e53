// Device-side helpers shared by the gfx950 kernels: vector types, activation
// functions with the reference's formulas, 64-lane wavefront reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace di {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Request one dword of every 64-byte line of a kernel's argument struct, and
// the launch's hidden arguments (gridDim) that follow it, at entry: all of
// them arrive in one scalar-cache round trip.  Left to itself the compiler
// loads the fields it needs in dependent batches, each a scalar-cache miss
// before the first memory access of the kernel.  The empty asm statement (an
// assembler comment) only keeps the loads.
template <typename T>
__device__ __forceinline__ void kernarg_warm(const T& a) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(&a);
  uint32_t t = gridDim.x;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); i += 16) t |= w[i];
  asm volatile("; kernel arguments in the scalar cache %0" ::"s"(t));
}

// SiLU x/(1+e^-x): UNARY_EXPRS.SiLU wgsl-ops.js:68, fused-resnet.js:162.  The
// quotient is x times the hardware reciprocal (1 ulp; 1 + e^-x >= 1, so no
// denormal, and an infinite e^-x still gives the limit 0): a correctly
// rounded division costs ~10 VALU instructions per value, most of the
// normalise-and-store phase of a GroupNorm apply.
__device__ __forceinline__ float silu_f(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// erf by Abramowitz & Stegun 7.1.26 (max abs error 1.5e-7), the approximation
// the reference's GELU and Erf kernels use (wgsl-ops.js:77-81).  t comes from
// the hardware reciprocal (1 ulp): the formula's own error is ~2 orders larger,
// and a correctly rounded division costs 8 more VALU instructions per value.
__device__ __forceinline__ float erf_as(float x) {
  float a = fabsf(x);
  float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
  float y = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t -
                     0.284496736f) * t + 0.254829592f) * t * __expf(-a * a);
  return x >= 0.0f ? y : -y;
}

// GELU x*0.5*(1+erf(x/sqrt2)): UNARY_EXPRS.GELU wgsl-ops.js:70.
__device__ __forceinline__ float gelu_erf_f(float x) {
  return x * 0.5f * (1.0f + erf_as(x * 0.70710678f));
}

// tanh-approximation GELU of the FFN bench (fused-block.js:68-75).
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float c = 0.044715f, s = 0.7978845608f;
  return 0.5f * x * (1.0f + tanhf(s * (x + c * x * x * x)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

// Statistics exchange between the kXchgSlices workgroups that share a
// GroupNorm group (k_norm.hip's NCHW GroupNorm, k_gemm.hip's fused split-K
// reducer).  A record of kXchgWords 64-bit words per group holds one (sum,
// sumsq) word pair per slice, then a 32-bit arrival counter.  Every launch
// adds exactly kXchgSlices to the counter of each record it uses and the
// owner's launches are stream-ordered, so o / kXchgSlices + 1 (o: a
// workgroup's fetch-add result) is an epoch that the workgroups of one
// launch share and no earlier launch used; a word {epoch, float bits} is
// written and read whole (relaxed agent-scope atomics), so no fence orders
// the words.  The context's exchange area: kXchgNchwRecs records for the
// NCHW GroupNorm, then kXchgRedRecs for the reducer, zeroed at creation.
constexpr uint32_t kXchgSlices = 8;  // divides 2^32: epochs stay aligned when o wraps
constexpr uint32_t kXchgWords = 32;  // 256 B per record
// regions: the NCHW GroupNorm's, then the reducer's with eight and with four
// slices per record (a record serves one slice count only, so its counter
// advances by that count at every launch)
constexpr uint32_t kXchgNchwRecs = 64, kXchgRedRecs = 512, kXchgRed4Recs = 512;
static_assert(2 * kXchgSlices + 1 <= kXchgWords && 2 * kXchgSlices <= 64, "record layout");

// The arrival fetch-add on record rec (one thread of the workgroup).
__device__ __forceinline__ uint32_t xchg_arrive(uint64_t* rec) {
  return __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(rec + 2 * kXchgSlices), 1u,
                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Publish slice s's (a, b) under epoch word ep (thread 0), then wave 0 polls
// the record's 2 NS words until all carry ep, at most `spin` polls, and
// leaves them in sv[2 NS] (LDS).  Returns, in wave 0, whether every slice
// arrived; the caller shares that through LDS.  No barrier.
template <uint32_t NS = kXchgSlices>
__device__ __forceinline__ bool xchg_publish_poll(uint64_t* rec, uint64_t ep, uint32_t s, float a,
                                                  float b, uint32_t spin, float* sv) {
  static_assert(NS <= kXchgSlices && (NS & (NS - 1)) == 0, "a power of two up to the record's");
  const uint32_t tid = threadIdx.x;
  if (tid == 0) {
    __hip_atomic_store(rec + 2 * s, ep | __float_as_uint(a), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(rec + 2 * s + 1, ep | __float_as_uint(b), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  bool all = false;
  if (tid < (uint32_t)kWave) {
    uint64_t word = ep;
    for (uint32_t it = 0; it < spin; it++) {
      if (tid < 2 * NS)
        word = __hip_atomic_load(rec + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      all = __all((word & 0xffffffff00000000ull) == ep);
      if (all) break;
      __builtin_amdgcn_s_sleep(2);
    }
    if (tid < 2 * NS) sv[tid] = __uint_as_float((uint32_t)word);
  }
  return all;
}

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  return (float)v;
}

template <typename T>
__device__ __forceinline__ T from_f(float v) {
  return (T)v;
}

// SplitMix64 finaliser. Element j of the SplitMix64 stream seeded with s is
// mix64(s + (j+1) * 0x9E3779B97F4A7C15), which makes the stream addressable
// by counter and therefore parallel.
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t j) {
  return mix64(seed + (j + 1) * 0x9E3779B97F4A7C15ull);
}

}  // namespace di

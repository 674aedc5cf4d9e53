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

// Euler Discrete scheduler kernels (reference scheduler.js) and their C-ABI
// entry points: the noise latent, scaleModelInput and the Euler update run on
// the device, so an N-step denoise leaves the GPU only for its result.
//
// The reference keeps its arrays in Float32Arrays and computes in JavaScript
// doubles, rounding once per stored element.  The kernels do the same: fp64
// arithmetic with contraction off (a JavaScript multiply-add rounds twice),
// one fp32 rounding at the store.  All are one-pass HBM streams.
#include "di_device.h"
#include "di_kernels.h"

namespace di {

namespace {

constexpr int kBlock = 256;

unsigned grid_for(uint64_t n) {
  uint64_t b = (n + kBlock - 1) / kBlock;
  if (b < 1) b = 1;
  if (b > 65535ull * 16) b = 65535ull * 16;  // grid-stride covers the rest
  return (unsigned)b;
}

// The LCG of sampleNoiseLatent (scheduler.js:122-126): s' = s * 1664525 +
// 1013904223 (mod 2^32).  Applying it k times is the affine map
// s -> A_k s + C_k, built by squaring, so every pair of draws is computed
// independently from the seed state.
struct Affine {
  uint32_t a, c;
};

__device__ __forceinline__ Affine lcg_jump(uint64_t k) {
  Affine r{1u, 0u}, p{1664525u, 1013904223u};
  while (k) {
    if (k & 1) r = Affine{p.a * r.a, p.a * r.c + p.c};
    p = Affine{p.a * p.a, p.a * p.c + p.c};
    k >>= 1;
  }
  return r;
}

// sampleNoiseLatent (scheduler.js:117-134): pair p uses draws 2p + 1 and
// 2p + 2 of the generator: u1 = max(s / 2^32, 1e-9), u2 = s' / 2^32,
// r = sqrt(-2 ln u1); out[2p] = r cos(2 pi u2) sigma, out[2p + 1] =
// r sin(2 pi u2) sigma (fp32 stores of double expressions).
__global__ void k_noise_latent(float* __restrict__ out, uint64_t n, uint32_t s0, double sigma) {
#pragma clang fp contract(off)
  const uint64_t pairs = (n + 1) / 2, stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t p = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < pairs; p += stride) {
    const Affine j = lcg_jump(2 * p + 1);
    const uint32_t s1 = j.a * s0 + j.c;
    const uint32_t s2 = 1664525u * s1 + 1013904223u;
    const double u1 = fmax((double)s1 / 4294967296.0, 1e-9);
    const double u2 = (double)s2 / 4294967296.0;
    const double r = sqrt(-2.0 * log(u1));
    const double ang = 2.0 * 3.141592653589793 * u2;
    out[2 * p] = (float)(r * cos(ang) * sigma);
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(r * sin(ang) * sigma);
  }
}

// scaleModelInput (scheduler.js:95-101): y = x * inv.
__global__ void k_euler_scale(const float* __restrict__ x, float* __restrict__ y, uint64_t n,
                              double inv) {
#pragma clang fp contract(off)
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (float)((double)x[i] * inv);
}

// step (scheduler.js:105-110): y = x + dt * pred; optionally the next step's
// scaleModelInput of the stored result.  y may alias x (same element only).
__global__ void k_euler_step(const float* x, const float* __restrict__ pred, float* y,
                             float* __restrict__ next_in, uint64_t n, double dt, double inv_next) {
#pragma clang fp contract(off)
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = (float)((double)x[i] + dt * (double)pred[i]);
    y[i] = v;
    if (next_in) next_in[i] = (float)((double)v * inv_next);
  }
}

}  // namespace
}  // namespace di

using namespace di;

extern "C" {

int32_t di_noise_latent(di_ctx* ctx, di_handle out, uint64_t n, int32_t seed, double sigma) {
  DI_CTX(ctx);
  DI_BUF(ctx, out, o, n * 4);
  if (n == 0) return DI_OK;
  // (seed | 0) || 1
  const uint32_t s0 = seed != 0 ? (uint32_t)seed : 1u;
  k_noise_latent<<<grid_for((n + 1) / 2), kBlock, 0, ctx->stream>>>((float*)o->ptr, n, s0, sigma);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_euler_scale(di_ctx* ctx, di_handle latent, di_handle out, uint64_t n, double inv) {
  DI_CTX(ctx);
  DI_BUF(ctx, latent, x, n * 4);
  DI_BUF(ctx, out, y, n * 4);
  if (n == 0) return DI_OK;
  k_euler_scale<<<grid_for(n), kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, n,
                                                         inv);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_euler_step(di_ctx* ctx, di_handle latent, di_handle pred, di_handle out,
                      di_handle next_in, uint64_t n, double dt, double inv_next) {
  DI_CTX(ctx);
  DI_BUF(ctx, latent, x, n * 4);
  DI_BUF(ctx, pred, p, n * 4);
  DI_BUF(ctx, out, y, n * 4);
  float* nx = nullptr;
  if (next_in) {
    DI_BUF(ctx, next_in, ni, n * 4);
    DI_REQUIRE(ni->ptr != x->ptr && ni->ptr != p->ptr && ni->ptr != y->ptr, DI_EINVAL,
               "di_euler_step: next_in must not alias latent, pred or out");
    nx = (float*)ni->ptr;
  }
  DI_REQUIRE(p->ptr != y->ptr, DI_EINVAL, "di_euler_step: out must not alias pred");
  if (n == 0) return DI_OK;
  k_euler_step<<<grid_for(n), kBlock, 0, ctx->stream>>>((const float*)x->ptr, (const float*)p->ptr,
                                                        (float*)y->ptr, nx, n, dt, inv_next);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"

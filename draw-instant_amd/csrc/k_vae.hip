// VAE decoder input kernel: the caller's latent scaling, post_quant_conv (a
// 1x1 conv over the latent channels) and the NCHW fp32 -> NHWC fp16 layout
// change with zero channel padding, in one pass over the latent.
#include "di_device.h"
#include "di_kernels.h"

namespace di {

namespace {

constexpr int kMaxLatent = 16;

// One thread per (image, pixel): y[b][p][c] = bias[c] + sum_ci w[c][ci] *
// scale * z[b][ci][p] for c < C, 0 for C <= c < cpad.
__global__ void k_vae_latent_in(const float* __restrict__ z, const float* __restrict__ w,
                                const float* __restrict__ bias, float scale, f16* __restrict__ y,
                                uint32_t B, uint32_t C, uint32_t HW, uint32_t cpad) {
  const uint64_t n = (uint64_t)B * HW;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t b = i / HW, p = i % HW;
    float v[kMaxLatent];
    for (uint32_t ci = 0; ci < C; ci++) v[ci] = scale * z[(b * C + ci) * HW + p];
    f16* yo = y + i * cpad;
    for (uint32_t c = 0; c < cpad; c++) {
      float a = 0.0f;
      if (c < C) {
        a = bias[c];
        for (uint32_t ci = 0; ci < C; ci++) a += w[c * C + ci] * v[ci];
      }
      yo[c] = (f16)a;
    }
  }
}

}  // namespace

void launch_vae_latent_in(hipStream_t s, const float* z, const float* w, const float* bias,
                          float scale, f16* y, uint32_t B, uint32_t C, uint32_t HW,
                          uint32_t cpad) {
  const uint64_t n = (uint64_t)B * HW;
  if (!n) return;
  uint64_t g = (n + 255) / 256;
  if (g > 65535ull * 8) g = 65535ull * 8;
  k_vae_latent_in<<<(unsigned)g, 256, 0, s>>>(z, w, bias, scale, y, B, C, HW, cpad);
}

}  // namespace di

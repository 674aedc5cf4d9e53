// Batched GEMV (k_tembed.hip): y[b][n] = act(sum_k x'[b][k] W[n][k] + bias[n])
// with x' = x, SiLU(x) or the timestep sinusoid of t[b].  fp32 vectors,
// fp16 or fp32 weights [N][ldw].
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace di {

enum GemvX { GEMV_X_PLAIN = 0, GEMV_X_SINUSOID = 1, GEMV_X_SILU = 2 };
enum GemvAct { GEMV_ACT_NONE = 0, GEMV_ACT_SILU = 1 };

struct GemvArgs {
  int x_mode = GEMV_X_PLAIN;
  const float* x = nullptr;  // [B][ldx]
  uint64_t ldx = 0;
  const float* t = nullptr;  // [B] timesteps (sinusoid mode)
  const void* w = nullptr;
  uint64_t ldw = 0;
  const float* bias = nullptr;
  int act = GEMV_ACT_NONE;
  float* y = nullptr;  // [B][ldy]
  uint64_t ldy = 0;
  uint32_t B = 1, N = 0, K = 0;
  uint32_t vec_ok = 1;
};

int gemv_supported(uint32_t B, uint32_t K);
void launch_gemv(const GemvArgs& g, int wdt, hipStream_t s);

}  // namespace di

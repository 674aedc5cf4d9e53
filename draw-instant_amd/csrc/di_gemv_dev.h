// Device side of the batched vector GEMV (k_tembed.hip), shared with the
// kernels that run a GEMV as a side job of their own launch: conv_in (the
// timestep sinusoid's first linear) and the NHWC GroupNorm apply (every
// ResNet's time_emb_proj), which saves those GEMVs a launch each.
#pragma once

#include "di_device.h"
#include "di_tembed.h"

namespace di {

template <typename W>
struct WVec;
template <>
struct WVec<f16> {
  static constexpr int V = 8;
  typedef f16x8 type;
};
template <>
struct WVec<float> {
  static constexpr int V = 4;
  typedef f32x4 type;
};

// x' of the GEMV (sinusoid when SIN, else SiLU or plain) into xs[b * K + k]
template <bool SIN>
__device__ __forceinline__ void gemv_stage_x(const GemvArgs& g, float* xs) {
  const uint32_t B = g.B, K = g.K;
  for (uint32_t i = threadIdx.x; i < B * K; i += 256) {
    const uint32_t b = i / K, k = i % K;
    float v;
    if constexpr (SIN) {
      const uint32_t half = K / 2;
      const uint32_t fi = k < half ? k : k - half;
      const double freq = exp(-9.210340371976184 * (double)fi / (double)half);
      const double arg = (double)g.t[b] * freq;
      v = (float)(k < half ? cos(arg) : sin(arg));
    } else {
      v = g.x[(uint64_t)b * g.ldx + k];
      if (g.x_mode == GEMV_X_SILU) v = silu_f(v);
    }
    xs[i] = v;
  }
}

// Vector path (K % V == 0, K <= 64 * V * NV, B <= BMAX) for one 256-thread
// block: wavefront w of block i owns rows (4 i + w) * RPW .. + RPW - 1; lane
// l holds vectors l, l + 64, .. of each row.  Rows past N load row N - 1 (in
// range) and store nothing.  xs: B * K floats of LDS.  Also run as a side
// job by kernels that take a GEMV into their own launch (launch_gemv_rows).
template <typename W, int NV, int RPW, int BMAX, bool SIN>
__device__ __forceinline__ void gemv_vec_block(const GemvArgs& g, float* xs, uint32_t block) {
  using WV = typename WVec<W>::type;
  constexpr int V = WVec<W>::V;
  const int lane = threadIdx.x & 63;
  const uint32_t n0 = (block * 4 + (threadIdx.x >> 6)) * RPW;
  const uint32_t K = g.K, B = g.B;
  WV wv[RPW][NV];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint32_t n = min(n0 + r, g.N - 1);
    const W* wr = (const W*)g.w + (uint64_t)n * g.ldw;
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const uint32_t k = (uint32_t)(lane + 64 * i) * V;
      wv[r][i] = k < K ? *(const WV*)(wr + k) : WV{};
    }
  }
  gemv_stage_x<SIN>(g, xs);
  __syncthreads();
  float acc[RPW][BMAX];
#pragma unroll
  for (int r = 0; r < RPW; r++)
#pragma unroll
    for (int b = 0; b < BMAX; b++) acc[r][b] = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const uint32_t k = (uint32_t)(lane + 64 * i) * V;
    if (k < K) {
#pragma unroll
      for (int b = 0; b < BMAX; b++) {
        if (b < (int)B) {
          float x[V];
#pragma unroll
          for (int j = 0; j < V; j++) x[j] = xs[b * K + k + j];
#pragma unroll
          for (int r = 0; r < RPW; r++)
#pragma unroll
            for (int j = 0; j < V; j++) acc[r][b] += (float)wv[r][i][j] * x[j];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint32_t n = n0 + r;
#pragma unroll
    for (int b = 0; b < BMAX; b++) {
      if (b < (int)B) {
        float s = wave_sum(acc[r][b]);
        if (lane == 0 && n < g.N) {
          s += g.bias ? g.bias[n] : 0.0f;
          if (g.act == GEMV_ACT_SILU) s = silu_f(s);
          g.y[(uint64_t)b * g.ldy + n] = s;
        }
      }
    }
  }
}

// Blocks of 256 threads a side-job GEMV needs (RPW rows per wavefront).
constexpr uint32_t gemv_side_blocks(uint32_t N, int rpw) { return (N + 4 * rpw - 1) / (4 * rpw); }

}  // namespace di

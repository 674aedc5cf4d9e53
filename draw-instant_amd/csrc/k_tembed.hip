// Timestep embedding and batched GEMV for gfx950, and di_tembed.
//
// The reference's fused kernel (WGSL_FUSED fused-tembed.js:73-130) runs the
// whole sinusoid -> Linear(320,1280) -> SiLU -> Linear(1280,1280) chain in
// ONE workgroup (0.11x of naive, README.md:108): a GEMV is weight-bandwidth
// bound and needs the whole chip.  Here each linear is a GEMV with one
// wavefront per output row (16-byte coalesced weight reads, shuffle
// reduction), hundreds of workgroups per launch; the input vector (the
// sinusoid of fused-tembed.js:39-42, computed in fp64, or SiLU of the
// previous output) is staged per workgroup in LDS.  The same kernel computes
// every ResNet's time_emb_proj(SiLU(temb)) of a U-Net step in one launch
// (20,160 rows of 1280 fp16 weights at SD2.1: 51.6 MB, HBM-bound).  In the
// vector path every lane issues all loads of its rows' weights before it
// stages the input vector, each wavefront covers RPW rows, and the staged
// vector takes B * K floats of LDS (not the B = 8 maximum), so enough
// weight bytes are in flight to stream HBM instead of waiting on one
// 16-byte load per lane at a time.
#include "di_device.h"
#include "di_kernels.h"
#include "di_gemv_dev.h"
#include "di_tembed.h"

namespace di {

namespace {

constexpr int kMaxK = 1280;
constexpr int kMaxB = 8;

template <typename W>
__global__ __launch_bounds__(256) void k_gemv(GemvArgs g) {
  __shared__ float xs[kMaxB * kMaxK];
  const uint32_t B = g.B, K = g.K;
  for (uint32_t i = threadIdx.x; i < B * K; i += 256) {
    uint32_t b = i / K, k = i % K;
    float v;
    if (g.x_mode == GEMV_X_SINUSOID) {
      // fused-tembed.js:36-42: freq_i = exp(-ln(1e4) i / half), [cos || sin]
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
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const uint32_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= g.N) return;
  const W* wr = (const W*)g.w + (uint64_t)n * g.ldw;
  constexpr int V = WVec<W>::V;
  float acc[kMaxB];
#pragma unroll
  for (int b = 0; b < kMaxB; b++) acc[b] = 0.0f;
  if (g.vec_ok) {
    for (uint32_t k = lane * V; k < K; k += 64 * V) {
      typename WVec<W>::type wv = *(const typename WVec<W>::type*)(wr + k);
#pragma unroll
      for (int b = 0; b < kMaxB; b++) {
        if (b < (int)B) {
#pragma unroll
          for (int j = 0; j < V; j++) acc[b] += (float)wv[j] * xs[b * K + k + j];
        }
      }
    }
  } else {
    for (uint32_t k = lane; k < K; k += 64) {
      float wv = (float)wr[k];
#pragma unroll
      for (int b = 0; b < kMaxB; b++)
        if (b < (int)B) acc[b] += wv * xs[b * K + k];
    }
  }
#pragma unroll
  for (int b = 0; b < kMaxB; b++) {
    if (b < (int)B) {
      float s = wave_sum(acc[b]);
      if (lane == 0) {
        s += g.bias ? g.bias[n] : 0.0f;
        if (g.act == GEMV_ACT_SILU) s = silu_f(s);
        g.y[(uint64_t)b * g.ldy + n] = s;
      }
    }
  }
}

template <typename W, int NV, int RPW, int BMAX, bool SIN>
__global__ __launch_bounds__(256) void k_gemv_vec(GemvArgs g) {
  extern __shared__ float xs[];  // [B][K]
  gemv_vec_block<W, NV, RPW, BMAX, SIN>(g, xs, blockIdx.x);
}

// Eight rows per wavefront for tall matrices at B <= 2 (the U-Net's stacked
// time_emb_proj: 630 workgroups, resident at once), else one (1280-row
// GEMVs keep 320 workgroups)
template <typename W, int NV>
void launch_gemv_vec(const GemvArgs& g, hipStream_t s) {
  const size_t lds = (size_t)g.B * g.K * sizeof(float);
  const bool sin = g.x_mode == GEMV_X_SINUSOID;
  if (g.B <= 2 && !sin && g.N >= 8192)
    k_gemv_vec<W, NV, 8, 2, false><<<(g.N + 31) / 32, 256, lds, s>>>(g);
  else if (!sin) k_gemv_vec<W, NV, 1, kMaxB, false><<<(g.N + 3) / 4, 256, lds, s>>>(g);
  else k_gemv_vec<W, NV, 1, kMaxB, true><<<(g.N + 3) / 4, 256, lds, s>>>(g);
}

}  // namespace

int gemv_supported(uint32_t B, uint32_t K) { return B >= 1 && B <= kMaxB && K >= 1 && K <= kMaxK; }

void launch_gemv(const GemvArgs& g, int wdt, hipStream_t s) {
  if (g.vec_ok && g.N > 0) {
    // K <= kMaxK = 1280: three 8-wide fp16 or five 4-wide fp32 vectors per lane
    if (wdt == DI_F16) launch_gemv_vec<f16, 3>(g, s);
    else launch_gemv_vec<float, 5>(g, s);
    return;
  }
  unsigned blocks = (g.N + 3) / 4;
  if (wdt == DI_F16) k_gemv<f16><<<blocks, 256, 0, s>>>(g);
  else k_gemv<float><<<blocks, 256, 0, s>>>(g);
}

}  // namespace di

using namespace di;

extern "C" {

int32_t di_tembed(di_ctx* ctx, di_handle T, di_handle W1, di_handle b1, di_handle W2, di_handle b2,
                  di_handle Y, uint32_t B, uint32_t emb_dim, uint32_t hid, int32_t wdt) {
  DI_CTX(ctx);
  DI_DTYPE(wdt);
  DI_REQUIRE(emb_dim % 2 == 0 && gemv_supported(B, emb_dim) && gemv_supported(B, hid),
             DI_EUNSUPPORTED, "di_tembed: B=%u emb_dim=%u hid=%u outside B<=8, dims<=1280, even emb",
             B, emb_dim, hid);
  const size_t es = dtype_size(wdt);
  DI_BUF(ctx, T, t, (uint64_t)B * 4);
  DI_BUF(ctx, W1, w1, (uint64_t)hid * emb_dim * es);
  DI_BUF(ctx, b1, bb1, (uint64_t)hid * 4);
  DI_BUF(ctx, W2, w2, (uint64_t)hid * hid * es);
  DI_BUF(ctx, b2, bb2, (uint64_t)hid * 4);
  DI_BUF(ctx, Y, y, (uint64_t)B * hid * 4);
  void* h = nullptr;
  uint64_t cap = 0;
  int rc = pool_alloc(ctx, (uint64_t)B * hid * 4, &h, &cap);
  if (rc) return rc;
  const uint32_t v = wdt == DI_F16 ? 8 : 4;
  GemvArgs g1;
  g1.x_mode = GEMV_X_SINUSOID;
  g1.t = (const float*)t->ptr;
  g1.w = w1->ptr;
  g1.ldw = emb_dim;
  g1.bias = (const float*)bb1->ptr;
  g1.act = GEMV_ACT_SILU;
  g1.y = (float*)h;
  g1.ldy = hid;
  g1.B = B;
  g1.N = hid;
  g1.K = emb_dim;
  g1.vec_ok = emb_dim % v == 0;
  launch_gemv(g1, wdt, ctx->stream);
  GemvArgs g2;
  g2.x = (const float*)h;
  g2.ldx = hid;
  g2.w = w2->ptr;
  g2.ldw = hid;
  g2.bias = (const float*)bb2->ptr;
  g2.y = (float*)y->ptr;
  g2.ldy = hid;
  g2.B = B;
  g2.N = hid;
  g2.K = hid;
  g2.vec_ok = hid % v == 0;
  launch_gemv(g2, wdt, ctx->stream);
  pool_release(ctx, h, cap);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"

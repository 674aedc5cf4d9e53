// Internal launch API of the gfx950 kernels.  Raw device pointers, explicit
// stream; used by the C-ABI wrappers and by the block / U-Net compositions.
// Every launcher validates nothing: callers check shapes first.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "di_device.h"
#include "di_internal.h"
#include "di_tembed.h"

namespace di {

// ---- element-wise / layout (k_eltwise.hip) ----
void launch_convert(hipStream_t s, const void* src, int sdt, void* dst, int ddt, uint64_t n);
// [N,C,H,W] layout/dtype change; C_dst >= C pads channels with zeros when the
// destination is NHWC (used to give conv_in an 8-aligned channel count).
void launch_layout(hipStream_t s, const void* src, int sdt, int slay, void* dst, int ddt,
                   int dlay, uint32_t N, uint32_t C, uint32_t H, uint32_t W,
                   uint32_t C_dst);
void launch_fill_normal(hipStream_t s, void* dst, int dt, uint64_t n, uint64_t seed,
                        float mean, float std);
void launch_fill_const(hipStream_t s, void* dst, int dt, uint64_t n, float v);
// y = a + b, n fp32 values.
void launch_add_f32(hipStream_t s, const float* a, const float* b, float* y, uint64_t n);
// Row softmax of [rows][inner] (in place allowed).
void launch_softmax(hipStream_t s, const void* x, void* y, uint32_t inner, uint32_t rows, int dt);
// fp16 per-batch matrix transpose: y[b][c][r] = x[b * sx + r * ldx + c] for
// r < rows, c < cols (strides below 2^32).
void launch_transpose_f16(hipStream_t s, const f16* x, uint32_t ldx, uint32_t sx, f16* y,
                          uint32_t batch, uint32_t rows, uint32_t cols);
// VAE decoder input: y[b][p][c] (NHWC fp16, cpad channels, zeros past C) =
// bias[c] + sum_ci w[c][ci] * scale * z[b][ci][p] (post_quant_conv, 1x1).
void launch_vae_latent_in(hipStream_t s, const float* z, const float* w, const float* bias,
                          float scale, f16* y, uint32_t B, uint32_t C, uint32_t HW,
                          uint32_t cpad);

// ---- normalisation (k_norm.hip) ----
// NCHW group norm: per-slice partial statistics, then fold + apply (two
// kernels; the partials go to the context workspace).
int launch_group_norm_nchw(Ctx* c, const void* x, const float* gamma, const float* beta,
                           void* y, uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW,
                           float eps, bool silu, int dt);
// NHWC fp16 group norm (two kernels: per-chunk partial stats; fold + apply).
// `ws` needs gn_nhwc_ws_floats() floats.
uint32_t gn_nhwc_chunks(uint32_t N, uint32_t HW);
uint64_t gn_nhwc_ws_floats(uint32_t N, uint32_t C, uint32_t G, uint32_t HW);
// Channel concat of two NHWC fp16 sources: channel c < c1 from p1 (pixel
// stride ld1), else channel c - c1 from p2 (pixel stride ld2); c1 % 8 == 0.
struct NhwcSrc {
  const f16* p1;
  const f16* p2;
  uint32_t c1;
  uint64_t ld1, ld2;
  __device__ __forceinline__ f16x8 load8(uint64_t pix, uint32_t c) const {
    return c < c1 ? *(const f16x8*)(p1 + pix * ld1 + c)
                  : *(const f16x8*)(p2 + pix * ld2 + (c - c1));
  }
};
// Producer statistics of an NHWC fp16 tensor (or channel concat of two):
// per 64-pixel chunk and channel, (sum, sum of squares) of the stored
// values; channels < c1 at s1[(chunk * ld1 + c) * 2], the rest at
// s2[(chunk * ld2 + c - c1) * 2].  Chunks count over all images (HW % 64 == 0).
struct GnStats {
  const float* s1;
  const float* s2;
  uint32_t c1;
  uint32_t ld1, ld2;
};
// GroupNorm apply from producer statistics (one kernel, no partial pass);
// returns false when the shape is not supported (the caller then runs
// launch_group_norm_nhwc).
// side: a GEMV run by extra workgroups of the same launch (B <= 2, fp16
// weights, K <= 1536, no sinusoid: gn_side_gemv_ok); if it does not qualify
// the caller launches it.
bool gn_side_gemv_ok(const GemvArgs& g);
bool launch_group_norm_nhwc_st(hipStream_t s, NhwcSrc x, const GnStats& st, const float* gamma,
                               const float* beta, void* y, uint32_t N, uint32_t C, uint32_t G,
                               uint32_t HW, float eps, bool silu, float* fold_ws = nullptr,
                               const GemvArgs* side = nullptr);
// Floats of fold_ws for an [N][HW][C] input (0: no pre-fold at this size).
// With fold_ws, statistics of large images are first summed to ~128 chunks
// per image, so the apply workgroups do not each re-read all HW / 64.
uint64_t gn_fold_ws_floats(uint32_t N, uint32_t C, uint32_t HW);
void launch_group_norm_nhwc(hipStream_t s, NhwcSrc x, const float* gamma, const float* beta,
                            void* y, uint32_t N, uint32_t C, uint32_t G, uint32_t HW,
                            float eps, bool silu, float* ws);
void launch_layer_norm(hipStream_t s, const void* x, const float* gamma,
                       const float* beta, void* y, uint32_t rows, uint32_t inner,
                       float eps, int dt);
// (sum, sum of squares) of each fp16 row into out[row * 2] (inner % 8 == 0).
void launch_row_stats(hipStream_t s, const f16* x, float* out, uint32_t rows, uint32_t inner);
// LayerNorm folded into the projection that consumes it: wf = w * gamma (per
// input column k, fp16), sum[n] = sum_k wf[n][k], cst[n] = sum_k beta[k]
// w[n][k] + bias[n] (bias optional).  w, wf: [N][K] fp16, K % 8 == 0.
void launch_ln_fold(hipStream_t s, const f16* w, const float* gamma, const float* beta,
                    const float* bias, f16* wf, float* sum, float* cst, uint32_t N, uint32_t K);

}  // namespace di

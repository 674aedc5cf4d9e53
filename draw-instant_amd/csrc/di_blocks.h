// Block compositions of the SD2.1 U-Net on the gfx950 kernels (blocks.cpp):
// ResnetBlock2D and Transformer2DModel (linear projection, one
// BasicTransformerBlock), on NHWC fp16 activations.
#pragma once

#include <cstdint>

#include "di_device.h"
#include "di_gemm.h"
#include "di_internal.h"
#include "di_kernels.h"

namespace di {

// Stream-ordered scratch allocation from the context pool; released (to the
// pool, not the driver) when the owner goes out of scope.  Safe because all
// work is on the context's single in-order stream.
// Request for the GroupNorm statistics of a GEMM's output (GemmArgs::stats
// layout): p is the destination; done reports whether the GEMM wrote them
// (it cannot on every path, e.g. K % 64 != 0).
struct StatsOut {
  float* p = nullptr;
  bool done = false;
};

// Request for a split-K conv's reducer to apply the GroupNorm (+SiLU) that
// is the output's only consumer (GnFuse); done reports whether it did (the
// plan may not split, or the shape may not fit the fused reducer), in which
// case the raw output and its statistics were written as usual.
struct GnFuseOut {
  GnFuse f;
  bool done = false;
};

// Request for a GEMM's row statistics (GemmArgs::rstats): p is the
// destination of `bytes` bytes ([rows][ceil(N/32)] float pairs suffice:
// tiles of 32 columns and more write it); nt and done are reported.  run()
// refuses a plan whose [rows][nt] pairs would not fit.
struct RowStatsOut {
  float* p = nullptr;
  uint64_t bytes = 0;
  uint32_t nt = 0;
  bool done = false;
};

// LayerNorm of a GEMM's A rows folded into its epilogue (GemmArgs::ln_*):
// the weights are W * gamma, the bias sum_k beta[k] W[n][k] + bias[n].
struct LnFold {
  const float* rows;  // row statistics of A (RowStatsOut layout)
  uint32_t nt;
  const float* s;  // [N] column sums of the scaled weights
  float eps;
};

struct Scratch {
  Ctx* c = nullptr;
  void* p = nullptr;
  uint64_t cap = 0;
  Scratch() = default;
  Scratch(const Scratch&) = delete;
  Scratch& operator=(const Scratch&) = delete;
  Scratch(Scratch&& o) noexcept : c(o.c), p(o.p), cap(o.cap) { o.p = nullptr; }
  Scratch& operator=(Scratch&& o) noexcept {
    if (this != &o) {
      release();
      c = o.c;
      p = o.p;
      cap = o.cap;
      o.p = nullptr;
    }
    return *this;
  }
  int alloc(Ctx* ctx, uint64_t bytes) {
    c = ctx;
    return pool_alloc(ctx, bytes, &p, &cap);
  }
  void release() {
    if (p) pool_release(c, p, cap);
    p = nullptr;
  }
  ~Scratch() { release(); }
  f16* h() const { return (f16*)p; }
  float* f() const { return (float*)p; }
};

struct ResnetW {
  const float *n1_g = nullptr, *n1_b = nullptr;
  const f16* c1_w = nullptr;  // OHWI [Cout][3][3][Cin]
  const float* c1_b = nullptr;
  const float *n2_g = nullptr, *n2_b = nullptr;
  const f16* c2_w = nullptr;  // OHWI [Cout][3][3][Cout]
  const float* c2_b = nullptr;
  const f16* sk_w = nullptr;  // 1x1 [Cout][Cin], null when Cin == Cout
  const float* sk_b = nullptr;
  // c2_b + sk_b (optional): lets conv2's split-K reducer sum the shortcut's
  // partials with its own, so the shortcut needs no reducer of its own
  const float* c2sk_b = nullptr;
};

struct ResnetShape {
  uint32_t B, H, W, Cin, Cout, groups;
  float eps;
};

// out[B][HW][Cout] = conv2(SiLU(GN2(conv1(SiLU(GN1(x))) + temb))) + skip(x).
// x is a channel concat of one or two NHWC sources.  temb: fp32 rows per
// image, temb[b * ld_temb + c] (already offset to this block), may be null.
// x_st: GroupNorm statistics of x from its producer (null: GN1 computes
// them); out_st: if non-null, asks for out's statistics ([B*HW/64][Cout]
// pairs, see GnStats; needs HW % 64 == 0) and reports whether they were
// written.  out_gn: if non-null, asks conv2's split-K reducer to apply the
// next block's GroupNorm to out as well (GnFuse with raw = 1) and reports
// whether it did; out's statistics are then written only where
// out_gn->f.stats is out_st's buffer.  x_gn: GN1(x) + SiLU already computed
// by x's producer (then x_st is not used).  gn1_side: an fp16-weight GEMV
// (producing temb) that GN1's apply launch runs as well where it can, and
// that is otherwise launched on its own before conv1.
int resnet_forward(Ctx* c, const ResnetW& w, const ResnetShape& s, NhwcSrc x,
                   const float* temb, uint32_t ld_temb, f16* out, const GnStats* x_st = nullptr,
                   StatsOut* out_st = nullptr, GnFuseOut* out_gn = nullptr,
                   const f16* x_gn = nullptr, const GemvArgs* gn1_side = nullptr);

struct TransformerW {
  const float *n_g = nullptr, *n_b = nullptr;       // GroupNorm
  const f16* pin_w = nullptr;                        // proj_in [C][C]
  const float* pin_b = nullptr;
  const float *ln1_g = nullptr, *ln1_b = nullptr;
  const f16* qkv_w = nullptr;  // [3C][C] = to_q ; to_k ; to_v (no bias)
  const f16* o1_w = nullptr;   // attn1.to_out.0 [C][C]
  const float* o1_b = nullptr;
  const float *ln2_g = nullptr, *ln2_b = nullptr;
  const f16* q2_w = nullptr;   // attn2.to_q [C][C]
  const f16* kv2_w = nullptr;  // [2C][cross] = to_k ; to_v
  // Optional: attn2 K / V already projected (rows [b*Sctx + s], K at columns
  // [0, C), V at [C, 2C), row stride kv_ld); kv2_w is then unused.
  const f16* kv_pre = nullptr;
  uint64_t kv_ld = 0;
  const f16* o2_w = nullptr;
  const float* o2_b = nullptr;
  const float *ln3_g = nullptr, *ln3_b = nullptr;
  const f16* ff1_w = nullptr;  // GEGLU proj [8C][C], rows in 32-groups [16 h | 16 gate]
  const float* ff1_b = nullptr;
  // Optional LayerNorms folded into their projections (qkv / q2 / ff1): when
  // *_s is set, *_w holds W * gamma (per input column, launch_ln_fold),
  // *_s[n] its row sums and *_c[n] = sum_k beta[k] W[n][k] + bias[n]; the
  // ln*_g / ln*_b and ff1_b fields are then unused.
  const float *qkv_s = nullptr, *qkv_c = nullptr;
  const float *q2_s = nullptr, *q2_c = nullptr;
  const float *ff1_s = nullptr, *ff1_c = nullptr;
  const f16* ff2_w = nullptr;  // [C][4C]
  const float* ff2_b = nullptr;
  const f16* pout_w = nullptr;  // proj_out [C][C]
  const float* pout_b = nullptr;
};

struct TransformerShape {
  uint32_t B, H, W, C, Sctx, cross, groups;
  float gn_eps, ln_eps;
};

// out = proj_out(block(proj_in(GN(x)))) + x; context fp16 [B][Sctx][cross].
// x_st / out_st: GroupNorm statistics of x and out, as for resnet_forward.
// x_gn: GN(x) already computed by x's producer (then x_st is not used).
int transformer_forward(Ctx* c, const TransformerW& w, const TransformerShape& s, const f16* x,
                        const f16* context, f16* out, const GnStats* x_st = nullptr,
                        StatsOut* out_st = nullptr, const f16* x_gn = nullptr);

// NHWC conv through the implicit-GEMM kernel (fp16 in, fp16 or NCHW fp32 out).
struct ConvCall {
  NhwcSrc x;
  uint32_t B, H, W, Cin, Cout, ks = 3, stride = 1, pad = 1, up = 1;
  const f16* w = nullptr;
  const float* bias = nullptr;
  const float* bias2 = nullptr;
  uint32_t rows_b2 = 0, ld_b2 = 0;
  const f16* res = nullptr;
  uint64_t ldr = 0;
  void* y = nullptr;
  uint64_t ldc = 0;
  int y_nchw_f32 = 0;
  StatsOut* stats = nullptr;  // GroupNorm statistics of y (GemmArgs::stats), optional
  GnFuseOut* gn = nullptr;    // GroupNorm of y applied by a split-K reducer, optional
  // shared split-K partial slots (GemmArgs::part_slot0 / part_slots /
  // part_only / part_cpg); only with a plan that splits
  uint32_t part_slot0 = 0, part_slots = 0, part_cpg = 0;
  int part_only = 0;
};
int conv_nhwc(Ctx* c, const ConvCall& cc);
// DI_GN_REDUCE_FUSE=0: no GroupNorm applied by a split-K reducer.
bool gn_reduce_fuse_off();
// The GEMM arguments conv_nhwc launches with, and their plan.
GemmArgs conv_args(const ConvCall& cc);
GemmPlan conv_plan(Ctx* c, const ConvCall& cc);

// Linear on token rows: y = act(x w^T + b) (+ res); fp16.  stats: optional
// GroupNorm statistics of y (GemmArgs::stats).
// rstats: optional row statistics of y; ln: optional LayerNorm of x's rows
// folded into the epilogue (w and b are then the folded weights and bias).
int linear_f16(Ctx* c, const f16* x, uint64_t ldx, uint32_t M, uint32_t K, const f16* w,
               uint32_t N, const float* b, int act, const f16* res, uint64_t ldr, f16* y,
               uint64_t ldy, StatsOut* stats = nullptr, RowStatsOut* rstats = nullptr,
               const LnFold* ln = nullptr);

// Floats of the GroupNorm statistics of a [rows][C] output (rows % 64 == 0).
inline uint64_t gn_stats_floats(uint64_t rows, uint32_t C) { return rows / 64 * C * 2; }

}  // namespace di

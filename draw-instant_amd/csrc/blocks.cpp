// ResnetBlock2D and Transformer2DModel compositions on the gfx950 kernels,
// and their C ABI (the fused-resnet.js / fused-block*.js block entry points).
//
// Fusion plan (per block, NHWC fp16 activations, fp32 accumulation):
//  ResNet      GN1+SiLU (1 pass) -> conv1 [+bias +temb broadcast in epilogue]
//              -> GN2+SiLU -> conv2 [+bias +skip residual in epilogue], the skip
//              being x itself or a 1x1 conv of x.  Up-block inputs are a channel
//              concat of two sources read in place by GN and the convs.
//  Transformer GN -> proj_in -> LN1 -> fused QKV GEMM -> flash self-attention
//              -> to_out [+bias +residual] -> LN2 -> to_q ; context K/V GEMM
//              -> flash cross-attention -> to_out [+residual] -> LN3 -> GEGLU
//              GEMM (h * GELU(gate) in the epilogue) -> ff out [+residual]
//              -> proj_out [+bias +block input residual].
// Versus the reference's executor this removes the materialised score
// matrices (320 MiB at 64x64), every standalone SiLU / add / transpose /
// slice pass, and the decomposed LayerNorm and GELU chains.
#include "di_attn.h"
#include "di_blocks.h"
#include "di_gemm.h"
#include "di_tembed.h"

namespace di {

namespace {

int run(Ctx* c, GemmArgs& g, int a_mode, StatsOut* st = nullptr, RowStatsOut* rst = nullptr,
        GnFuseOut* gn = nullptr) {
  const GemmPlan plan = gemm_plan(g, DI_F16, c->num_cus);
  const int tile = plan.tile;
  g.splits = plan.splits;
  g.stats = nullptr;
  g.rstats = nullptr;
  if (gn) {
    // the reducer's records of the context's statistics-exchange area
    gn->f.xchg = c->gn_xchg ? (uint64_t*)c->gn_xchg + (uint64_t)kXchgNchwRecs * kXchgWords
                            : nullptr;
    const char* e_spin = getenv("DI_GN_XCHG_SPIN");  // 0 forces the recomputing path
    gn->f.spin = e_spin ? (uint32_t)strtoul(e_spin, nullptr, 10) : 20000u;
    gn->done = splitk_gn_ok(g, gn->f);
  }
  if (st) st->done = false;
  if (gn && gn->done) {
    // the reducer writes GN(output) (and the raw output and its statistics
    // where the request asks: gn->f.raw / gn->f.stats)
    if (st) st->done = gn->f.stats != nullptr && gn->f.stats == st->p;
  } else if (st && st->p) {
    st->done = gemm_stats_ok(g, DI_F16, a_mode, B_NK, tile);
    if (st->done) g.stats = st->p;
  }
  if (rst && rst->p) {
    rst->done = gemm_rstats_ok(g, DI_F16, a_mode, B_NK, tile);
    if (rst->done) {
      const uint32_t nt = gemm_rstats_tiles(g, tile);
      const uint64_t need = (uint64_t)g.M * nt * 2 * sizeof(float);  // [M][nt] float2
      DI_REQUIRE(need <= rst->bytes, DI_EINVAL,
                 "row statistics of M=%u N=%u (tile %d, %u column tiles) need %llu bytes, "
                 "buffer holds %llu", g.M, g.N, tile, nt, (unsigned long long)need,
                 (unsigned long long)rst->bytes);
      g.rstats = rst->p;
      rst->nt = nt;
    }
  }
  DI_REQUIRE(!g.ln_rows || gemm_lnfold_ok(g, DI_F16, tile), DI_EUNSUPPORTED,
             "LayerNorm fold needs the vector epilogue (M=%u N=%u K=%u tile %d)", g.M, g.N, g.K,
             tile);
  if (g.splits > 1) {
    void* ws = nullptr;
    int rc = workspace(c, gemm_ws_bytes(g), &ws);
    if (rc) return rc;
    g.part = (float*)ws;
  }
  if (gn && gn->done) g.part_cpg = g.N / gn->f.groups;
  if (g.splits <= 1) {
    DI_REQUIRE(!g.part_only && !g.part_slots, DI_EINVAL,
               "shared partial slots need a plan that splits (M=%u N=%u K=%u)", g.M, g.N, g.K);
  }
  launch_gemm(g, DI_F16, a_mode, B_NK, tile, c->stream, gn && gn->done ? &gn->f : nullptr);
  return DI_OK;
}

// side / side_done: a GEMV for the apply launch to run as well (see
// launch_group_norm_nhwc_st); side_done reports whether it did.
int gn_nhwc(Ctx* c, NhwcSrc x, const float* g, const float* b, f16* y, uint32_t N, uint32_t C,
            uint32_t G, uint32_t HW, float eps, bool silu, const GnStats* st = nullptr,
            const GemvArgs* side = nullptr, bool* side_done = nullptr) {
  if (side_done) *side_done = false;
  if (st) {
    float* fold = nullptr;
    if (const uint64_t nf = gn_fold_ws_floats(N, C, HW)) {
      void* ws = nullptr;
      int rc = workspace(c, nf * sizeof(float), &ws);
      if (rc) return rc;
      fold = (float*)ws;
    }
    if (launch_group_norm_nhwc_st(c->stream, x, *st, g, b, y, N, C, G, HW, eps, silu, fold,
                                  side)) {
      if (side_done) *side_done = side && gn_side_gemv_ok(*side);
      return DI_OK;
    }
  }
  void* ws = nullptr;
  int rc = workspace(c, gn_nhwc_ws_floats(N, C, G, HW) * sizeof(float), &ws);
  if (rc) return rc;
  launch_group_norm_nhwc(c->stream, x, g, b, y, N, C, G, HW, eps, silu, (float*)ws);
  return DI_OK;
}

NhwcSrc single(const f16* p, uint32_t C) { return NhwcSrc{p, p, C, C, C}; }

// DI_SK_PARTIALS=0 keeps a ResNet's 1x1 shortcut as its own GEMM + reducer
// (comparison runs; read at every block call)
bool sk_partials_off() {
  const char* e = getenv("DI_SK_PARTIALS");
  return e && e[0] == '0';
}

}  // namespace

GemmArgs conv_args(const ConvCall& cc) {
  GemmArgs g;
  g.a = cc.x.p1;
  g.a2 = cc.x.p2;
  g.c1 = cc.x.c1;
  g.lda = cc.x.ld1;
  g.lda2 = cc.x.ld2;
  g.Cin = cc.Cin;
  g.H = cc.H;
  g.W = cc.W;
  g.ks = cc.ks;
  g.stride = cc.stride;
  g.pad = cc.pad;
  g.up = cc.up;
  const uint32_t Hi = cc.H * cc.up, Wi = cc.W * cc.up;
  g.Ho = (Hi + 2 * cc.pad - cc.ks) / cc.stride + 1;
  g.Wo = (Wi + 2 * cc.pad - cc.ks) / cc.stride + 1;
  g.M = cc.B * g.Ho * g.Wo;
  g.N = cc.Cout;
  g.K = cc.ks * cc.ks * cc.Cin;
  g.b = cc.w;
  g.ldb = g.K;
  const uint64_t pixels = (uint64_t)cc.B * cc.H * cc.W;
  g.a_bytes = gemm_extent(pixels * cc.x.ld1 * 2);
  g.a2_bytes = gemm_extent(pixels * cc.x.ld2 * 2);
  g.b_bytes = gemm_extent((uint64_t)g.N * g.K * 2);
  g.bias = cc.bias;
  g.bias2 = cc.bias2;
  g.rows_b2 = cc.rows_b2;
  g.ld_b2 = cc.ld_b2;
  g.res = cc.res;
  g.ldr = cc.ldr;
  g.c = cc.y;
  if (cc.y_nchw_f32) {
    g.c_f32 = 1;
    g.c_nchw = 1;
    g.c_hw = g.Ho * g.Wo;
  } else {
    g.ldc = cc.ldc ? cc.ldc : cc.Cout;
  }
  g.part_slot0 = cc.part_slot0;
  g.part_slots = cc.part_slots;
  g.part_cpg = cc.part_cpg;
  g.part_only = cc.part_only;
  return g;
}

GemmPlan conv_plan(Ctx* c, const ConvCall& cc) {
  return gemm_plan(conv_args(cc), DI_F16, c->num_cus);
}

// DI_GN_REDUCE_FUSE=0 keeps every GroupNorm as its own apply launch
// (comparison runs; read at every block call, so a test can switch it)
bool gn_reduce_fuse_off() {
  const char* e = getenv("DI_GN_REDUCE_FUSE");
  return e && e[0] == '0';
}

int conv_nhwc(Ctx* c, const ConvCall& cc) {
  GemmArgs g = conv_args(cc);
  return run(c, g, A_CONV_NHWC, cc.stats, nullptr, cc.gn);
}

int linear_f16(Ctx* c, const f16* x, uint64_t ldx, uint32_t M, uint32_t K, const f16* w,
               uint32_t N, const float* b, int act, const f16* res, uint64_t ldr, f16* y,
               uint64_t ldy, StatsOut* stats, RowStatsOut* rstats, const LnFold* ln) {
  GemmArgs g;
  g.a = x;
  g.lda = ldx;
  g.b = w;
  g.ldb = K;
  g.M = M;
  g.N = N;
  g.K = K;
  g.bias = b;
  g.act = act;
  g.res = res;
  g.ldr = ldr;
  g.c = y;
  g.ldc = ldy;
  g.a_vec_ok = (K % 8 == 0) && (ldx % 8 == 0);
  g.b_vec_ok = K % 8 == 0;
  g.a_bytes = gemm_extent((uint64_t)M * ldx * 2);
  g.b_bytes = gemm_extent((uint64_t)N * K * 2);
  if (ln) {
    g.ln_rows = ln->rows;
    g.ln_nt = ln->nt;
    g.ln_s = ln->s;
    g.ln_eps = ln->eps;
  }
  return run(c, g, A_DENSE, stats, rstats);
}

int resnet_forward(Ctx* c, const ResnetW& w, const ResnetShape& s, NhwcSrc x, const float* temb,
                   uint32_t ld_temb, f16* out, const GnStats* x_st, StatsOut* out_st,
                   GnFuseOut* out_gn, const f16* x_gn, const GemvArgs* gn1_side) {
  const uint32_t HW = s.H * s.W;
  const uint64_t rows = (uint64_t)s.B * HW;
  // conv1 hands GN2 the statistics of its output (no partial pass)
  const bool st2 = HW % 64 == 0;
  Scratch t1, t2, t3, sk, t2st;
  int rc = x_gn ? 0 : t1.alloc(c, rows * s.Cin * 2);
  if (!rc) rc = t2.alloc(c, rows * s.Cout * 2);
  if (!rc) rc = t3.alloc(c, rows * s.Cout * 2);
  if (!rc && st2) rc = t2st.alloc(c, gn_stats_floats(rows, s.Cout) * sizeof(float));
  if (rc) return rc;
  bool side_done = false;
  if (!x_gn) {
    rc = gn_nhwc(c, x, w.n1_g, w.n1_b, t1.h(), s.B, s.Cin, s.groups, HW, s.eps, true, x_st,
                 gn1_side, &side_done);
    if (rc) return rc;
    x_gn = t1.h();
  }
  if (gn1_side && !side_done) launch_gemv(*gn1_side, DI_F16, c->stream);  // before conv1 reads it
  ConvCall c1;
  c1.x = single(x_gn, s.Cin);
  c1.B = s.B;
  c1.H = s.H;
  c1.W = s.W;
  c1.Cin = s.Cin;
  c1.Cout = s.Cout;
  c1.w = w.c1_w;
  c1.bias = w.c1_b;
  c1.bias2 = temb;
  c1.rows_b2 = HW;
  c1.ld_b2 = ld_temb;
  c1.y = t2.h();
  StatsOut so2{st2 ? t2st.f() : nullptr};
  c1.stats = &so2;
  // GN2 + SiLU applied by conv1's split-K reducer where the plan splits
  GnFuseOut gn2;
  gn2.f.gamma = w.n2_g;
  gn2.f.beta = w.n2_b;
  gn2.f.y = t3.h();
  gn2.f.ldy = s.Cout;
  gn2.f.groups = s.groups;
  gn2.f.hw = HW;
  gn2.f.eps = s.eps;
  gn2.f.silu = 1;
  if (!gn_reduce_fuse_off()) c1.gn = &gn2;
  rc = conv_nhwc(c, c1);
  if (rc) return rc;
  if (!gn2.done) {
    const GnStats s2{t2st.f(), t2st.f(), s.Cout, s.Cout, s.Cout};
    rc = gn_nhwc(c, single(t2.h(), s.Cout), w.n2_g, w.n2_b, t3.h(), s.B, s.Cout, s.groups, HW,
                 s.eps, true, so2.done ? &s2 : nullptr);
    if (rc) return rc;
  }
  ConvCall c2;
  c2.x = single(t3.h(), s.Cout);
  c2.B = s.B;
  c2.H = s.H;
  c2.W = s.W;
  c2.Cin = s.Cout;
  c2.Cout = s.Cout;
  c2.w = w.c2_w;
  c2.bias = w.c2_b;
  c2.y = out;
  c2.stats = out_st;
  if (out_gn) out_gn->done = false;
  if (out_gn && !gn_reduce_fuse_off()) c2.gn = out_gn;
  if (w.sk_w) {
    ConvCall k1;
    k1.x = x;
    k1.B = s.B;
    k1.H = s.H;
    k1.W = s.W;
    k1.Cin = s.Cin;
    k1.Cout = s.Cout;
    k1.ks = 1;
    k1.pad = 0;
    k1.w = w.sk_w;
    k1.bias = w.sk_b;
    // Both split: the shortcut writes its partials into slots after
    // conv2's, launches no reducer, and conv2's reducer sums every slot
    // with the summed bias (conv2 + shortcut = one sum over both k ranges)
    const GemmPlan pk = conv_plan(c, k1), p2 = conv_plan(c, c2);
    if (w.c2sk_b && !sk_partials_off() && pk.splits > 1 && p2.splits > 1) {
      const uint32_t slots = pk.splits + p2.splits;
      c2.bias = w.c2sk_b;
      c2.part_slots = slots;
      if (c2.gn) {
        // the fused GroupNorm reducer reads the partials in column groups
        GemmArgs g2 = conv_args(c2);
        g2.splits = p2.splits;
        if (splitk_gn_ok(g2, c2.gn->f)) k1.part_cpg = s.Cout / c2.gn->f.groups;
      }
      k1.part_slot0 = p2.splits;
      k1.part_slots = slots;
      k1.part_only = 1;
      rc = conv_nhwc(c, k1);
      if (rc) return rc;
      return conv_nhwc(c, c2);
    }
    rc = sk.alloc(c, rows * s.Cout * 2);
    if (rc) return rc;
    k1.y = sk.h();
    rc = conv_nhwc(c, k1);
    if (rc) return rc;
    c2.res = sk.h();
    c2.ldr = s.Cout;
  } else {
    c2.res = x.p1;  // Cin == Cout: identity skip, single source
    c2.ldr = x.ld1;
  }
  return conv_nhwc(c, c2);
}

int transformer_forward(Ctx* c, const TransformerW& w, const TransformerShape& s, const f16* x,
                        const f16* context, f16* out, const GnStats* x_st, StatsOut* out_st,
                        const f16* x_gn) {
  const uint32_t HW = s.H * s.W, C = s.C;
  const uint64_t rows = (uint64_t)s.B * HW;
  Scratch t, h, n, qkv, a, q, kv, gg, rs;
  int rc = t.alloc(c, rows * C * 2);
  // row statistics of h from the GEMM that wrote it: the next LayerNorm runs
  // inside the consuming GEMM's A staging
  const uint64_t rs_bytes = rows * ((C + 31) / 32) * 2 * sizeof(float);
  if (!rc) rc = rs.alloc(c, rs_bytes);
  if (!rc) rc = h.alloc(c, rows * C * 2);
  if (!rc) rc = n.alloc(c, rows * C * 2);
  if (!rc) rc = qkv.alloc(c, rows * 3 * C * 2);
  if (!rc) rc = a.alloc(c, rows * C * 2);
  if (!rc && !w.kv_pre) rc = kv.alloc(c, (uint64_t)s.B * s.Sctx * 2 * C * 2);
  if (!rc) rc = gg.alloc(c, rows * 4 * C * 2);
  if (rc) return rc;
  const float scale_log2 = 0.125f * 1.4426950408889634f;  // 1/sqrt(64) * log2(e)
  // GN (eps 1e-6 in diffusers Transformer2DModel) -> proj_in
  if (!x_gn) {
    rc = gn_nhwc(c, single(x, C), w.n_g, w.n_b, t.h(), s.B, C, s.groups, HW, s.gn_eps, false, x_st);
    x_gn = t.h();
  }
  // a producer of h writes its row statistics when the next LayerNorm is folded
  RowStatsOut ro{rs.f(), rs_bytes};
  auto ro_for = [&](const float* fs) {
    ro.done = false;
    return fs ? &ro : nullptr;
  };
  if (!rc)
    rc = linear_f16(c, x_gn, C, rows, C, w.pin_w, C, w.pin_b, ACT_NONE, nullptr, 0, h.h(), C,
                    nullptr, ro_for(w.qkv_s));
  if (rc) return rc;
  // y = LayerNorm(h) @ W^T (+ bias / act).  With folded weights (fs set)
  // the LayerNorm is the GEMM epilogue's, from row statistics of h that its
  // producer wrote (or a statistics pass); else a LayerNorm kernel into n.
  auto ln_linear = [&](const float* lg, const float* lb, const f16* wt, const float* fs,
                       const float* fc, uint32_t N, const float* bias, int act, f16* y,
                       uint64_t ldy) {
    if (fs) {
      if (!ro.done) {
        launch_row_stats(c->stream, h.h(), rs.f(), rows, C);
        ro.nt = 1;
        ro.done = true;
      }
      const LnFold ln{rs.f(), ro.nt, fs, s.ln_eps};
      return linear_f16(c, h.h(), C, rows, C, wt, N, fc, act, nullptr, 0, y, ldy, nullptr,
                        nullptr, &ln);
    }
    launch_layer_norm(c->stream, h.h(), lg, lb, n.h(), rows, C, s.ln_eps, DI_F16);
    return linear_f16(c, n.h(), C, rows, C, wt, N, bias, act, nullptr, 0, y, ldy);
  };
  // self-attention
  rc = ln_linear(w.ln1_g, w.ln1_b, w.qkv_w, w.qkv_s, w.qkv_c, 3 * C, nullptr, ACT_NONE, qkv.h(),
                 3 * C);
  if (rc) return rc;
  AttnArgs sa;
  sa.q = qkv.h();
  sa.k = qkv.h() + C;
  sa.v = qkv.h() + 2 * C;
  sa.o = a.h();
  sa.ldq = sa.ldk = sa.ldv = 3 * C;
  sa.ldo = C;
  sa.hq = sa.hk = sa.hv = sa.ho = 64;
  sa.bq = sa.bk = sa.bv = (uint64_t)HW * 3 * C;
  sa.bo = (uint64_t)HW * C;
  sa.H = C / 64;
  sa.Sq = HW;
  sa.Skv = HW;
  sa.scale_log2 = scale_log2;
  rc = run_attention(c, sa, s.B);
  if (rc) return rc;
  rc = linear_f16(c, a.h(), C, rows, C, w.o1_w, C, w.o1_b, ACT_NONE, h.h(), C, h.h(), C, nullptr,
                  ro_for(w.q2_s));
  if (rc) return rc;
  // cross-attention
  rc = ln_linear(w.ln2_g, w.ln2_b, w.q2_w, w.q2_s, w.q2_c, C, nullptr, ACT_NONE, qkv.h(), C);
  const f16* kvp = w.kv_pre;
  const uint64_t kvld = w.kv_pre ? w.kv_ld : 2 * C;
  if (!rc && !kvp) {
    rc = linear_f16(c, context, s.cross, (uint64_t)s.B * s.Sctx, s.cross, w.kv2_w, 2 * C, nullptr,
                    ACT_NONE, nullptr, 0, kv.h(), 2 * C);
    kvp = kv.h();
  }
  if (rc) return rc;
  AttnArgs ca;
  ca.q = qkv.h();
  ca.k = kvp;
  ca.v = kvp + C;
  ca.o = a.h();
  ca.ldq = C;
  ca.ldk = ca.ldv = kvld;
  ca.ldo = C;
  ca.hq = ca.hk = ca.hv = ca.ho = 64;
  ca.bq = (uint64_t)HW * C;
  ca.bk = ca.bv = (uint64_t)s.Sctx * kvld;
  ca.bo = (uint64_t)HW * C;
  ca.H = C / 64;
  ca.Sq = HW;
  ca.Skv = s.Sctx;
  ca.scale_log2 = scale_log2;
  rc = run_attention(c, ca, s.B);
  if (rc) return rc;
  rc = linear_f16(c, a.h(), C, rows, C, w.o2_w, C, w.o2_b, ACT_NONE, h.h(), C, h.h(), C, nullptr,
                  ro_for(w.ff1_s));
  if (rc) return rc;
  // GEGLU feed-forward
  rc = ln_linear(w.ln3_g, w.ln3_b, w.ff1_w, w.ff1_s, w.ff1_c, 8 * C, w.ff1_b, ACT_GEGLU, gg.h(),
                 4 * C);
  if (!rc)
    rc = linear_f16(c, gg.h(), 4 * C, rows, 4 * C, w.ff2_w, C, w.ff2_b, ACT_NONE, h.h(), C, h.h(), C);
  if (rc) return rc;
  // proj_out + block input residual
  return linear_f16(c, h.h(), C, rows, C, w.pout_w, C, w.pout_b, ACT_NONE, x, C, out, C, out_st);
}

}  // namespace di

using namespace di;

namespace {

template <typename T>
int opt_ptr(di_ctx* ctx, di_handle h, uint64_t bytes, const T** out, bool required,
            const char* what) {
  *out = nullptr;
  if (h == 0) {
    DI_REQUIRE(!required, DI_EINVAL, "missing weight %s", what);
    return DI_OK;
  }
  Buffer* b = nullptr;
  int rc = lookup(ctx, h, &b);
  if (rc) return rc;
  DI_REQUIRE(b->bytes >= bytes, DI_EINVAL, "weight %s holds %llu bytes, needs %llu", what,
             (unsigned long long)b->bytes, (unsigned long long)bytes);
  *out = (const T*)b->ptr;
  return DI_OK;
}

#define DI_W(T, field, bytes, req)                                         \
  do {                                                                     \
    int _rc = opt_ptr<T>(ctx, W->field, (bytes), &wt.field##_p, req, #field); \
    if (_rc) return _rc;                                                   \
  } while (0)

}  // namespace

extern "C" {

int32_t di_resnet_block(di_ctx* ctx, const di_resnet_weights* W, di_handle X, di_handle temb,
                        di_handle Y, uint32_t B, uint32_t Cin, uint32_t Cout, uint32_t H,
                        uint32_t Wd, uint32_t temb_dim, uint32_t groups, float eps) {
  DI_CTX(ctx);
  DI_REQUIRE(W != nullptr, DI_EINVAL, "di_resnet_block: null weights");
  DI_REQUIRE(B && Cin && Cout && H && Wd && groups, DI_EINVAL, "di_resnet_block: zero dimension");
  DI_REQUIRE(Cin % groups == 0 && Cout % groups == 0, DI_EINVAL,
             "di_resnet_block: channels %u/%u not divisible by %u groups", Cin, Cout, groups);
  DI_REQUIRE(Cin % 8 == 0 && Cout % 8 == 0 && Cin <= 4096 && Cout <= 4096, DI_EUNSUPPORTED,
             "di_resnet_block: channels must be multiples of 8 and <= 4096");
  const uint64_t rows = (uint64_t)B * H * Wd;
  DI_BUF(ctx, X, x, rows * Cin * 2);
  DI_BUF(ctx, Y, y, rows * Cout * 2);
  struct {
    const float *norm1_gamma_p, *norm1_beta_p, *conv1_b_p, *temb_b_p, *norm2_gamma_p,
        *norm2_beta_p, *conv2_b_p, *skip_b_p;
    const f16 *conv1_w_p, *temb_w_p, *conv2_w_p, *skip_w_p;
  } wt;
  DI_W(float, norm1_gamma, Cin * 4, true);
  DI_W(float, norm1_beta, Cin * 4, true);
  DI_W(f16, conv1_w, (uint64_t)Cout * 9 * Cin * 2, true);
  DI_W(float, conv1_b, Cout * 4, true);
  DI_W(float, norm2_gamma, Cout * 4, true);
  DI_W(float, norm2_beta, Cout * 4, true);
  DI_W(f16, conv2_w, (uint64_t)Cout * 9 * Cout * 2, true);
  DI_W(float, conv2_b, Cout * 4, true);
  DI_W(f16, skip_w, (uint64_t)Cout * Cin * 2, Cin != Cout);
  DI_W(float, skip_b, Cout * 4, Cin != Cout);
  DI_W(f16, temb_w, (uint64_t)Cout * temb_dim * 2, temb != 0);
  DI_W(float, temb_b, Cout * 4, temb != 0);
  ResnetW rw;
  rw.n1_g = wt.norm1_gamma_p;
  rw.n1_b = wt.norm1_beta_p;
  rw.c1_w = wt.conv1_w_p;
  rw.c1_b = wt.conv1_b_p;
  rw.n2_g = wt.norm2_gamma_p;
  rw.n2_b = wt.norm2_beta_p;
  rw.c2_w = wt.conv2_w_p;
  rw.c2_b = wt.conv2_b_p;
  rw.sk_w = Cin != Cout ? wt.skip_w_p : nullptr;
  rw.sk_b = Cin != Cout ? wt.skip_b_p : nullptr;
  ResnetShape s{B, H, Wd, Cin, Cout, groups, eps};
  Scratch tproj;
  const float* tp = nullptr;
  if (temb) {
    DI_REQUIRE(gemv_supported(B, temb_dim), DI_EUNSUPPORTED,
               "di_resnet_block: temb B=%u dim=%u outside B<=8, dim<=1280", B, temb_dim);
    DI_BUF(ctx, temb, tb, (uint64_t)B * temb_dim * 4);
    int rc = tproj.alloc(ctx, (uint64_t)B * Cout * 4);
    if (rc) return rc;
    GemvArgs gv;
    gv.x_mode = GEMV_X_SILU;  // time_emb_proj(SiLU(temb))
    gv.x = (const float*)tb->ptr;
    gv.ldx = temb_dim;
    gv.w = wt.temb_w_p;
    gv.ldw = temb_dim;
    gv.bias = wt.temb_b_p;
    gv.y = tproj.f();
    gv.ldy = Cout;
    gv.B = B;
    gv.N = Cout;
    gv.K = temb_dim;
    gv.vec_ok = temb_dim % 8 == 0;
    launch_gemv(gv, DI_F16, ctx->stream);
    tp = tproj.f();
  }
  int rc = resnet_forward(ctx, rw, s, NhwcSrc{(const f16*)x->ptr, (const f16*)x->ptr, Cin, Cin, Cin},
                          tp, Cout, (f16*)y->ptr);
  if (rc) return rc;
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_transformer_block(di_ctx* ctx, const di_transformer_weights* W, di_handle X,
                             di_handle context, di_handle Y, uint32_t B, uint32_t C, uint32_t H,
                             uint32_t Wd, uint32_t Sctx, uint32_t cross_dim, uint32_t groups,
                             float gn_eps, float ln_eps) {
  DI_CTX(ctx);
  DI_REQUIRE(W != nullptr, DI_EINVAL, "di_transformer_block: null weights");
  DI_REQUIRE(B && C && H && Wd && Sctx && cross_dim && groups, DI_EINVAL,
             "di_transformer_block: zero dimension");
  DI_REQUIRE(C % 64 == 0 && C % groups == 0 && C <= 4096, DI_EUNSUPPORTED,
             "di_transformer_block: C=%u must be a multiple of 64 (head dim) and of groups", C);
  DI_REQUIRE(cross_dim % 8 == 0, DI_EUNSUPPORTED, "di_transformer_block: cross_dim %% 8 != 0");
  const uint64_t rows = (uint64_t)B * H * Wd;
  DI_BUF(ctx, X, x, rows * C * 2);
  DI_BUF(ctx, Y, y, rows * C * 2);
  DI_BUF(ctx, context, cx, (uint64_t)B * Sctx * cross_dim * 2);
  DI_REQUIRE(x->ptr != y->ptr, DI_EINVAL, "di_transformer_block: Y may not alias X");
  struct {
    const float *norm_gamma_p, *norm_beta_p, *proj_in_b_p, *ln1_gamma_p, *ln1_beta_p,
        *attn1_out_b_p, *ln2_gamma_p, *ln2_beta_p, *attn2_out_b_p, *ln3_gamma_p, *ln3_beta_p,
        *ff_in_b_p, *ff_out_b_p, *proj_out_b_p;
    const f16 *proj_in_w_p, *attn1_qkv_w_p, *attn1_out_w_p, *attn2_q_w_p, *attn2_kv_w_p,
        *attn2_out_w_p, *ff_in_w_p, *ff_out_w_p, *proj_out_w_p;
  } wt;
  const uint64_t cc = (uint64_t)C * C * 2;
  DI_W(float, norm_gamma, C * 4, true);
  DI_W(float, norm_beta, C * 4, true);
  DI_W(f16, proj_in_w, cc, true);
  DI_W(float, proj_in_b, C * 4, true);
  DI_W(float, ln1_gamma, C * 4, true);
  DI_W(float, ln1_beta, C * 4, true);
  DI_W(f16, attn1_qkv_w, 3 * cc, true);
  DI_W(f16, attn1_out_w, cc, true);
  DI_W(float, attn1_out_b, C * 4, true);
  DI_W(float, ln2_gamma, C * 4, true);
  DI_W(float, ln2_beta, C * 4, true);
  DI_W(f16, attn2_q_w, cc, true);
  DI_W(f16, attn2_kv_w, (uint64_t)2 * C * cross_dim * 2, true);
  DI_W(f16, attn2_out_w, cc, true);
  DI_W(float, attn2_out_b, C * 4, true);
  DI_W(float, ln3_gamma, C * 4, true);
  DI_W(float, ln3_beta, C * 4, true);
  DI_W(f16, ff_in_w, 8 * cc, true);
  DI_W(float, ff_in_b, 8 * C * 4, true);
  DI_W(f16, ff_out_w, 4 * cc, true);
  DI_W(float, ff_out_b, C * 4, true);
  DI_W(f16, proj_out_w, cc, true);
  DI_W(float, proj_out_b, C * 4, true);
  TransformerW tw;
  tw.n_g = wt.norm_gamma_p;
  tw.n_b = wt.norm_beta_p;
  tw.pin_w = wt.proj_in_w_p;
  tw.pin_b = wt.proj_in_b_p;
  tw.ln1_g = wt.ln1_gamma_p;
  tw.ln1_b = wt.ln1_beta_p;
  tw.qkv_w = wt.attn1_qkv_w_p;
  tw.o1_w = wt.attn1_out_w_p;
  tw.o1_b = wt.attn1_out_b_p;
  tw.ln2_g = wt.ln2_gamma_p;
  tw.ln2_b = wt.ln2_beta_p;
  tw.q2_w = wt.attn2_q_w_p;
  tw.kv2_w = wt.attn2_kv_w_p;
  tw.o2_w = wt.attn2_out_w_p;
  tw.o2_b = wt.attn2_out_b_p;
  tw.ln3_g = wt.ln3_gamma_p;
  tw.ln3_b = wt.ln3_beta_p;
  tw.ff1_w = wt.ff_in_w_p;
  tw.ff1_b = wt.ff_in_b_p;
  tw.ff2_w = wt.ff_out_w_p;
  tw.ff2_b = wt.ff_out_b_p;
  tw.pout_w = wt.proj_out_w_p;
  tw.pout_b = wt.proj_out_b_p;
  TransformerShape s{B, H, Wd, C, Sctx, cross_dim, groups, gn_eps, ln_eps};
  int rc = transformer_forward(ctx, tw, s, (const f16*)x->ptr, (const f16*)cx->ptr, (f16*)y->ptr);
  if (rc) return rc;
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_ffn(di_ctx* ctx, di_handle X, di_handle W1, di_handle b1, di_handle W2, di_handle b2,
               di_handle Y, uint32_t rows, uint32_t D, uint32_t F, int32_t act, int32_t dt) {
  DI_CTX(ctx);
  DI_REQUIRE(act == DI_ACT_GELU || act == DI_ACT_GELU_TANH || act == DI_ACT_GEGLU, DI_EINVAL,
             "di_ffn: act must be GELU, GELU_TANH or GEGLU");
  const uint32_t n1 = act == DI_ACT_GEGLU ? 2 * F : F;
  di_handle H = 0;
  int rc = di_alloc(ctx, (uint64_t)rows * F * dtype_size(dt), &H);
  if (rc) return rc;
  rc = di_linear(ctx, X, W1, b1, 0, H, rows, n1, D, act, dt);
  if (!rc) rc = di_linear(ctx, H, W2, b2, X, Y, rows, D, F, DI_ACT_NONE, dt);
  int rc2 = di_free(ctx, H);
  return rc ? rc : rc2;
}

}  // extern "C"

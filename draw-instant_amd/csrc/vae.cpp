// SD's VAE decoder (AutoencoderKL post_quant_conv + Decoder) as one native
// object on the gfx950 kernels: the model vae-wgsl.js runs through the
// executor op by op (vae_decoder/model.onnx, 525 nodes, vae-wgsl.js:28-140),
// here ~130 fused kernels on NHWC fp16 activations with fp32 accumulation.
//
//   latent fp32 NCHW * scale -> post_quant_conv (1x1) -> NHWC fp16 (one pass)
//   conv_in -> mid (ResNet, attention, ResNet)
//   4 up blocks of layers_per_block + 1 ResNets, the first three followed by
//   a nearest-x2 upsample fused into its conv3x3's input addressing
//   GroupNorm + SiLU -> conv_out (fp32 NCHW store)
//
// ResNets are the U-Net's (resnet_forward: GN+SiLU, implicit-GEMM convs with
// bias and residual in the epilogue, the GroupNorm statistics of each conv
// output written by its epilogue) without a time embedding.  The mid-block
// attention is one head over all C channels (d = 512, past the flash
// kernel's 64): GroupNorm -> one [3C][C] QKV GEMM with bias -> S = Q K^T /
// sqrt(C) as an MFMA GEMM -> row softmax -> O = P V (V transposed once so
// the GEMM takes the buffer-load path) -> to_out with bias and the residual
// in its epilogue.
//
// Parameters follow diffusers' names; layouts as the U-Net's (convs OHWI
// fp16, conv_in's input channels padded to 8, to_q / to_k / to_v stacked).
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "di_blocks.h"
#include "di_gemm.h"

namespace di {

namespace {

enum VArena { VA_W16 = 0, VA_F32 = 1, VA_COUNT = 2 };

struct VParam {
  std::string name;
  std::vector<uint32_t> shape;
  int arena;
  uint64_t offset, numel;
  float mean, std;
  int layout;
};

struct VRes {
  uint32_t cin, cout;
  int n1g, n1b, c1w, c1b, n2g, n2b, c2w, c2b, skw = -1, skb = -1;
};

struct VAttn {
  uint32_t c;
  int ng, nb, qkv_w, qkv_b, ow, ob;
};

}  // namespace

struct Vae {
  di_vae_config cfg;
  std::vector<VParam> params;
  uint64_t arena_elems[VA_COUNT] = {};
  void* arena[VA_COUNT] = {};
  uint64_t arena_cap[VA_COUNT] = {};
  int pq_w, pq_b, cin_w, cin_b, nog, nob, cow, cob;
  VRes mid_res[2];
  VAttn mid_attn;
  std::vector<std::vector<VRes>> up;
  std::vector<int> up_w, up_b;  // upsampler convs (-1 on the last level)
  std::vector<std::pair<void*, uint64_t>> graph_scratch;
  // the context workspace the captured graph's kernels address (pinned)
  void* graph_ws = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  uint64_t graph_key[6] = {0};

  int add(const std::string& name, std::vector<uint32_t> shape, int a, float mean, float std,
          int layout) {
    VParam p;
    p.name = name;
    p.shape = shape;
    p.arena = a;
    p.numel = 1;
    for (uint32_t d : shape) p.numel *= d;
    const uint64_t align = a == VA_F32 ? 4 : 8;  // 16-byte aligned tensors
    arena_elems[a] = (arena_elems[a] + align - 1) / align * align;
    p.offset = arena_elems[a];
    arena_elems[a] += p.numel;
    p.mean = mean;
    p.std = std;
    p.layout = layout;
    params.push_back(p);
    return (int)params.size() - 1;
  }
  f16* h(int i) const { return (f16*)arena[VA_W16] + params[i].offset; }
  float* f(int i) const { return (float*)arena[VA_F32] + params[i].offset; }
};

namespace {

float kaiming(uint32_t fan_in) { return sqrtf(2.0f / (float)fan_in); }

void vnorm(Vae& v, const std::string& p, uint32_t c, int* g, int* b) {
  *g = v.add(p + ".weight", {c}, VA_F32, 1.0f, 0.02f, DI_PARAM_VECTOR);
  *b = v.add(p + ".bias", {c}, VA_F32, 0.0f, 0.02f, DI_PARAM_VECTOR);
}

void vconv(Vae& v, const std::string& p, uint32_t cout, uint32_t cin, uint32_t k, int* w, int* b,
           uint32_t cin_phys = 0) {
  if (!cin_phys) cin_phys = cin;
  *w = v.add(p + ".weight", {cout, k, k, cin_phys}, VA_W16, 0.0f, kaiming(cin * k * k),
             DI_PARAM_CONV_OHWI);
  *b = v.add(p + ".bias", {cout}, VA_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
}

VRes vres(Vae& v, const std::string& p, uint32_t cin, uint32_t cout) {
  VRes r;
  r.cin = cin;
  r.cout = cout;
  vnorm(v, p + ".norm1", cin, &r.n1g, &r.n1b);
  vconv(v, p + ".conv1", cout, cin, 3, &r.c1w, &r.c1b);
  vnorm(v, p + ".norm2", cout, &r.n2g, &r.n2b);
  vconv(v, p + ".conv2", cout, cout, 3, &r.c2w, &r.c2b);
  if (cin != cout) vconv(v, p + ".conv_shortcut", cout, cin, 1, &r.skw, &r.skb);
  return r;
}

void build_vae(Vae& v) {
  const di_vae_config& c = v.cfg;
  const uint32_t L = c.latent_channels;
  v.pq_w = v.add("post_quant_conv.weight", {L, L}, VA_F32, 0.0f, kaiming(L), DI_PARAM_LINEAR);
  v.pq_b = v.add("post_quant_conv.bias", {L}, VA_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  uint32_t rev[4];
  for (int i = 0; i < 4; i++) rev[i] = c.block_channels[3 - i];
  vconv(v, "decoder.conv_in", rev[0], L, 3, &v.cin_w, &v.cin_b, (L + 7) / 8 * 8);
  const std::string mid = "decoder.mid_block";
  v.mid_res[0] = vres(v, mid + ".resnets.0", rev[0], rev[0]);
  VAttn& a = v.mid_attn;
  a.c = rev[0];
  const std::string ap = mid + ".attentions.0";
  vnorm(v, ap + ".group_norm", a.c, &a.ng, &a.nb);
  a.qkv_w = v.add(ap + ".to_qkv.weight", {3 * a.c, a.c}, VA_W16, 0.0f, sqrtf(1.0f / a.c),
                  DI_PARAM_LINEAR_STACKED);
  a.qkv_b = v.add(ap + ".to_qkv.bias", {3 * a.c}, VA_F32, 0.0f, 0.01f, DI_PARAM_LINEAR_STACKED);
  a.ow = v.add(ap + ".to_out.0.weight", {a.c, a.c}, VA_W16, 0.0f, sqrtf(1.0f / a.c),
               DI_PARAM_LINEAR);
  a.ob = v.add(ap + ".to_out.0.bias", {a.c}, VA_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  v.mid_res[1] = vres(v, mid + ".resnets.1", rev[0], rev[0]);
  uint32_t prev = rev[0];
  for (int i = 0; i < 4; i++) {
    const std::string p = "decoder.up_blocks." + std::to_string(i);
    std::vector<VRes> rs;
    for (uint32_t j = 0; j <= c.layers_per_block; j++) {
      rs.push_back(vres(v, p + ".resnets." + std::to_string(j), j == 0 ? prev : rev[i], rev[i]));
    }
    v.up.push_back(rs);
    int w = -1, b = -1;
    if (i < 3) vconv(v, p + ".upsamplers.0.conv", rev[i], rev[i], 3, &w, &b);
    v.up_w.push_back(w);
    v.up_b.push_back(b);
    prev = rev[i];
  }
  vnorm(v, "decoder.conv_norm_out", rev[3], &v.nog, &v.nob);
  vconv(v, "decoder.conv_out", c.out_channels, rev[3], 3, &v.cow, &v.cob);
}

ResnetW vres_w(const Vae& v, const VRes& r) {
  ResnetW w;
  w.n1_g = v.f(r.n1g);
  w.n1_b = v.f(r.n1b);
  w.c1_w = v.h(r.c1w);
  w.c1_b = v.f(r.c1b);
  w.n2_g = v.f(r.n2g);
  w.n2_b = v.f(r.n2b);
  w.c2_w = v.h(r.c2w);
  w.c2_b = v.f(r.c2b);
  if (r.skw >= 0) {
    w.sk_w = v.h(r.skw);
    w.sk_b = v.f(r.skb);
  }
  return w;
}

NhwcSrc one(const f16* p, uint32_t ch) { return NhwcSrc{p, p, ch, ch, ch}; }

// Batched fp16 GEMM C[b] = alpha * A[b] B[b]^T on the MFMA kernel (B_NK).
int gemm16_nk(Ctx* c, const f16* a, uint64_t lda, uint64_t sa, const f16* b, uint64_t ldb,
              uint64_t sb, f16* y, uint64_t ldc, uint64_t sc, uint32_t M, uint32_t N, uint32_t K,
              uint32_t batch, float alpha) {
  GemmArgs g;
  g.a = a;
  g.lda = lda;
  g.sa = sa;
  g.b = b;
  g.ldb = ldb;
  g.sb = sb;
  g.c = y;
  g.ldc = ldc;
  g.sc = sc;
  g.M = M;
  g.N = N;
  g.K = K;
  g.batch = batch;
  g.alpha = alpha;
  g.a_vec_ok = K % 8 == 0 && lda % 8 == 0;
  g.b_vec_ok = K % 8 == 0 && ldb % 8 == 0;
  g.a_bytes = gemm_extent(((uint64_t)(M - 1) * lda + K) * 2);
  g.b_bytes = gemm_extent(((uint64_t)(N - 1) * ldb + K) * 2);
  const GemmPlan plan = gemm_plan(g, DI_F16, c->num_cus);
  g.splits = plan.splits;
  if (g.splits > 1) {
    void* ws = nullptr;
    int rc = workspace(c, gemm_ws_bytes(g), &ws);
    if (rc) return rc;
    g.part = (float*)ws;
  }
  launch_gemm(g, DI_F16, A_DENSE, B_NK, plan.tile, c->stream);
  return DI_OK;
}

int vae_decode_step(Ctx* c, Vae& v, const float* z, float* img, uint32_t B, uint32_t H,
                    uint32_t W, float scale) {
  const di_vae_config& cf = v.cfg;
  const uint32_t G = cf.groups;
  const uint32_t L = cf.latent_channels, lp = (L + 7) / 8 * 8;

  // an activation and (HW % 64 == 0) the GroupNorm statistics its producer wrote
  struct Act {
    Scratch buf, st;
    uint32_t c = 0;
    StatsOut so;
    bool has_st = false;
  };
  auto act_alloc = [&](Act& a, uint32_t hh, uint32_t ww, uint32_t ch) {
    const uint64_t rows = (uint64_t)B * hh * ww;
    a.c = ch;
    a.has_st = false;
    int r = a.buf.alloc(c, rows * ch * 2);
    if (!r && (hh * ww) % 64 == 0) r = a.st.alloc(c, gn_stats_floats(rows, ch) * sizeof(float));
    a.so = StatsOut{a.st.f(), false};
    return r;
  };
  auto st_out = [](Act& a) { return a.so.p ? &a.so : (StatsOut*)nullptr; };
  auto st_done = [](Act& a) { a.has_st = a.so.done; };
  auto st_of = [](const Act& a) { return GnStats{a.st.f(), a.st.f(), a.c, a.c, a.c}; };
  auto gn = [&](const Act& x, const float* g, const float* b, f16* y, uint32_t hw, bool silu) {
    const GnStats xs = st_of(x);
    if (x.has_st) {
      float* fold = nullptr;
      if (const uint64_t nf = gn_fold_ws_floats(B, x.c, hw)) {
        void* fw = nullptr;
        int r = workspace(c, nf * sizeof(float), &fw);
        if (r) return r;
        fold = (float*)fw;
      }
      if (launch_group_norm_nhwc_st(c->stream, one(x.buf.h(), x.c), xs, g, b, y, B, x.c, G, hw,
                                    cf.eps, silu, fold))
        return (int)DI_OK;
    }
    void* ws = nullptr;
    int r = workspace(c, gn_nhwc_ws_floats(B, x.c, G, hw) * sizeof(float), &ws);
    if (r) return r;
    launch_group_norm_nhwc(c->stream, one(x.buf.h(), x.c), g, b, y, B, x.c, G, hw, cf.eps, silu,
                           (float*)ws);
    return (int)DI_OK;
  };
  auto resnet = [&](const VRes& r, Act& x, uint32_t hh, uint32_t ww, Act& y) {
    const ResnetShape s{B, hh, ww, r.cin, r.cout, G, cf.eps};
    const GnStats xs = st_of(x);
    int rc = act_alloc(y, hh, ww, r.cout);
    if (!rc)
      rc = resnet_forward(c, vres_w(v, r), s, one(x.buf.h(), x.c), nullptr, 0, y.buf.h(),
                          x.has_st ? &xs : nullptr, st_out(y));
    st_done(y);
    return rc;
  };

  // latent -> post_quant_conv -> NHWC fp16 (channels padded to 8)
  Scratch z16;
  int rc = z16.alloc(c, (uint64_t)B * H * W * lp * 2);
  if (rc) return rc;
  launch_vae_latent_in(c->stream, z, v.f(v.pq_w), v.f(v.pq_b), scale, z16.h(), B, L, H * W, lp);
  uint32_t hh = H, ww = W, ch = cf.block_channels[3];
  Act h;
  rc = act_alloc(h, hh, ww, ch);
  if (rc) return rc;
  {
    ConvCall cc;
    cc.x = one(z16.h(), lp);
    cc.B = B;
    cc.H = hh;
    cc.W = ww;
    cc.Cin = lp;
    cc.Cout = ch;
    cc.w = v.h(v.cin_w);
    cc.bias = v.f(v.cin_b);
    cc.y = h.buf.h();
    cc.stats = st_out(h);
    rc = conv_nhwc(c, cc);
    if (rc) return rc;
    st_done(h);
  }
  z16.release();
  // mid block
  {
    Act m1;
    rc = resnet(v.mid_res[0], h, hh, ww, m1);
    if (rc) return rc;
    h = std::move(m1);
  }
  {
    const VAttn& a = v.mid_attn;
    const uint32_t C = a.c, HW = hh * ww;
    const uint64_t rows = (uint64_t)B * HW;
    Scratch xn, qkv, S, vt, o;
    rc = xn.alloc(c, rows * C * 2);
    if (!rc) rc = qkv.alloc(c, rows * 3 * C * 2);
    if (!rc) rc = S.alloc(c, (uint64_t)B * HW * HW * 2);
    if (!rc) rc = vt.alloc(c, rows * C * 2);
    if (!rc) rc = o.alloc(c, rows * C * 2);
    if (!rc) rc = gn(h, v.f(a.ng), v.f(a.nb), xn.h(), HW, false);
    if (!rc)
      rc = linear_f16(c, xn.h(), C, (uint32_t)rows, C, v.h(a.qkv_w), 3 * C, v.f(a.qkv_b), ACT_NONE,
                      nullptr, 0, qkv.h(), 3 * C);
    if (rc) return rc;
    // S[b] = Q[b] K[b]^T / sqrt(C): Q at columns [0, C), K at [C, 2C)
    rc = gemm16_nk(c, qkv.h(), 3 * C, (uint64_t)HW * 3 * C, qkv.h() + C, 3 * C,
                   (uint64_t)HW * 3 * C, S.h(), HW, (uint64_t)HW * HW, HW, HW, C, B,
                   1.0f / sqrtf((float)C));
    if (rc) return rc;
    launch_softmax(c->stream, S.h(), S.h(), HW, B * HW, DI_F16);
    // V^T[b] = [C][HW] so P V runs as P (V^T)^T on the buffer-load kernel
    launch_transpose_f16(c->stream, qkv.h() + 2 * C, 3 * C, HW * 3 * C, vt.h(), B, HW, C);
    rc = gemm16_nk(c, S.h(), HW, (uint64_t)HW * HW, vt.h(), HW, (uint64_t)C * HW, o.h(), C,
                   (uint64_t)HW * C, HW, C, HW, B, 1.0f);
    if (rc) return rc;
    S.release();
    Act y;
    rc = act_alloc(y, hh, ww, C);
    if (!rc)
      rc = linear_f16(c, o.h(), C, (uint32_t)rows, C, v.h(a.ow), C, v.f(a.ob), ACT_NONE, h.buf.h(),
                      C, y.buf.h(), C, st_out(y));
    if (rc) return rc;
    st_done(y);
    h = std::move(y);
  }
  {
    Act m3;
    rc = resnet(v.mid_res[1], h, hh, ww, m3);
    if (rc) return rc;
    h = std::move(m3);
  }
  // up blocks
  for (size_t i = 0; i < v.up.size(); i++) {
    for (const VRes& r : v.up[i]) {
      Act nxt;
      rc = resnet(r, h, hh, ww, nxt);
      if (rc) return rc;
      h = std::move(nxt);
      ch = r.cout;
    }
    if (v.up_w[i] >= 0) {
      Act us;
      rc = act_alloc(us, hh * 2, ww * 2, ch);
      if (rc) return rc;
      ConvCall cc;
      cc.x = one(h.buf.h(), ch);
      cc.B = B;
      cc.H = hh;
      cc.W = ww;
      cc.Cin = ch;
      cc.Cout = ch;
      cc.up = 2;
      cc.w = v.h(v.up_w[i]);
      cc.bias = v.f(v.up_b[i]);
      cc.y = us.buf.h();
      cc.stats = st_out(us);
      rc = conv_nhwc(c, cc);
      if (rc) return rc;
      st_done(us);
      h = std::move(us);
      hh *= 2;
      ww *= 2;
    }
  }
  // conv_norm_out + SiLU -> conv_out (NCHW fp32)
  Scratch no;
  rc = no.alloc(c, (uint64_t)B * hh * ww * ch * 2);
  if (!rc) rc = gn(h, v.f(v.nog), v.f(v.nob), no.h(), hh * ww, true);
  if (rc) return rc;
  h.buf.release();
  h.st.release();
  ConvCall co;
  co.x = one(no.h(), ch);
  co.B = B;
  co.H = hh;
  co.W = ww;
  co.Cin = ch;
  co.Cout = cf.out_channels;
  co.w = v.h(v.cow);
  co.bias = v.f(v.cob);
  co.y = img;
  co.y_nchw_f32 = 1;
  return conv_nhwc(c, co);
}

void vae_default_config(di_vae_config* c) {
  memset(c, 0, sizeof(*c));
  c->latent_channels = 4;
  c->out_channels = 3;
  c->block_channels[0] = 128;
  c->block_channels[1] = 256;
  c->block_channels[2] = 512;
  c->block_channels[3] = 512;
  c->layers_per_block = 2;
  c->groups = 32;
  c->eps = 1e-6f;
}

}  // namespace
}  // namespace di

using namespace di;

struct di_vae : di::Vae {};

static void vae_drop_graph(di_ctx* ctx, di_vae* v) {
  if (v->graph_exec) (void)hipGraphExecDestroy(v->graph_exec);
  if (v->graph) (void)hipGraphDestroy(v->graph);
  v->graph_exec = nullptr;
  v->graph = nullptr;
  for (auto& pc : v->graph_scratch) pool_release(ctx, pc.first, pc.second);
  v->graph_scratch.clear();
  workspace_unpin(ctx, v->graph_ws);
  v->graph_ws = nullptr;
}

extern "C" {

int32_t di_vae_default_config(di_vae_config* cfg) {
  DI_REQUIRE(cfg != nullptr, DI_EINVAL, "di_vae_default_config: null config");
  vae_default_config(cfg);
  return DI_OK;
}

int32_t di_vae_create(di_ctx* ctx, const di_vae_config* cfg, uint64_t seed, di_vae** out) {
  DI_CTX(ctx);
  DI_REQUIRE(out != nullptr, DI_EINVAL, "di_vae_create: null out pointer");
  *out = nullptr;
  di_vae_config c;
  if (cfg) c = *cfg;
  else vae_default_config(&c);
  DI_REQUIRE(c.groups >= 1 && c.layers_per_block >= 1 && c.layers_per_block <= 8, DI_EINVAL,
             "di_vae_create: bad groups / layers_per_block");
  for (int i = 0; i < 4; i++)
    DI_REQUIRE(c.block_channels[i] % 8 == 0 && c.block_channels[i] % c.groups == 0 &&
                   c.block_channels[i] >= 8 && c.block_channels[i] <= 2048,
               DI_EUNSUPPORTED,
               "di_vae_create: block channels must be multiples of 8 and of groups (got %u)",
               c.block_channels[i]);
  DI_REQUIRE(c.latent_channels >= 1 && c.latent_channels <= 16 && c.out_channels >= 1 &&
                 c.out_channels <= 64,
             DI_EUNSUPPORTED, "di_vae_create: latent channels in [1, 16], out channels in [1, 64]");
  auto* v = new di_vae();
  v->cfg = c;
  build_vae(*v);
  const size_t esz[VA_COUNT] = {2, 4};
  for (int a = 0; a < VA_COUNT; a++) {
    int rc = pool_alloc(ctx, std::max<uint64_t>(v->arena_elems[a] * esz[a], 256), &v->arena[a],
                        &v->arena_cap[a]);
    if (rc) {
      for (int b = 0; b < a; b++) pool_release(ctx, v->arena[b], v->arena_cap[b]);
      delete v;
      return rc;
    }
  }
  for (size_t i = 0; i < v->params.size(); i++) {
    const VParam& p = v->params[i];
    void* dst = (char*)v->arena[p.arena] + p.offset * esz[p.arena];
    launch_fill_normal(ctx->stream, dst, p.arena == VA_W16 ? DI_F16 : DI_F32, p.numel,
                       seed * 1000003ull + 7919ull + i, p.mean, p.std);
  }
  DI_LAUNCH_CHECK();
  *out = v;
  return DI_OK;
}

int32_t di_vae_destroy(di_ctx* ctx, di_vae* v) {
  DI_CTX(ctx);
  DI_REQUIRE(v != nullptr, DI_EINVAL, "di_vae_destroy: null vae");
  DI_HIP(hipStreamSynchronize(ctx->stream));
  vae_drop_graph(ctx, v);
  for (int a = 0; a < VA_COUNT; a++) pool_release(ctx, v->arena[a], v->arena_cap[a]);
  delete v;
  return DI_OK;
}

int32_t di_vae_num_params(di_ctx* ctx, di_vae* v, uint32_t* n_tensors, uint64_t* n_elements) {
  DI_CTX(ctx);
  DI_REQUIRE(v != nullptr, DI_EINVAL, "null vae");
  if (n_tensors) *n_tensors = (uint32_t)v->params.size();
  if (n_elements) {
    uint64_t s = 0;
    for (const auto& p : v->params) s += p.numel;
    *n_elements = s;
  }
  return DI_OK;
}

int32_t di_vae_param_info(di_ctx* ctx, di_vae* v, uint32_t i, char* name, uint32_t name_cap,
                          uint32_t* dims, uint32_t* ndims, int32_t* dtype, int32_t* layout) {
  DI_CTX(ctx);
  DI_REQUIRE(v != nullptr, DI_EINVAL, "null vae");
  DI_REQUIRE(i < v->params.size(), DI_EINVAL, "param index %u out of range", i);
  const VParam& p = v->params[i];
  if (name && name_cap) {
    strncpy(name, p.name.c_str(), name_cap - 1);
    name[name_cap - 1] = 0;
  }
  if (ndims) *ndims = (uint32_t)p.shape.size();
  if (dims)
    for (size_t d = 0; d < p.shape.size() && d < 8; d++) dims[d] = p.shape[d];
  if (dtype) *dtype = p.arena == VA_F32 ? DI_F32 : DI_F16;
  if (layout) *layout = p.layout;
  return DI_OK;
}

static int vae_param_xfer(di_ctx* ctx, di_vae* v, uint32_t i, void* host, uint64_t bytes,
                          bool down) {
  DI_CTX(ctx);
  DI_REQUIRE(v != nullptr, DI_EINVAL, "null vae");
  DI_REQUIRE(i < v->params.size(), DI_EINVAL, "param index %u out of range", i);
  const VParam& p = v->params[i];
  const size_t es = p.arena == VA_F32 ? 4 : 2;
  DI_REQUIRE(bytes == p.numel * es, DI_EINVAL, "param %s is %llu bytes, got %llu", p.name.c_str(),
             (unsigned long long)(p.numel * es), (unsigned long long)bytes);
  DI_REQUIRE(host != nullptr, DI_EINVAL, "null host pointer");
  void* dev = (char*)v->arena[p.arena] + p.offset * es;
  if (down) DI_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
  else DI_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream));
  DI_HIP(hipStreamSynchronize(ctx->stream));
  return DI_OK;
}

int32_t di_vae_param_download(di_ctx* ctx, di_vae* v, uint32_t i, void* dst, uint64_t bytes) {
  return vae_param_xfer(ctx, v, i, dst, bytes, true);
}

int32_t di_vae_param_upload(di_ctx* ctx, di_vae* v, uint32_t i, const void* src, uint64_t bytes) {
  return vae_param_xfer(ctx, v, i, (void*)src, bytes, false);
}

int32_t di_vae_decode(di_ctx* ctx, di_vae* v, di_handle latent, di_handle image, uint32_t B,
                      uint32_t H, uint32_t W, float scale, int32_t flags) {
  DI_CTX(ctx);
  DI_REQUIRE(v != nullptr, DI_EINVAL, "null vae");
  DI_REQUIRE(B >= 1 && B <= 8, DI_EUNSUPPORTED, "di_vae_decode: batch %u outside [1, 8]", B);
  DI_REQUIRE(H >= 1 && W >= 1 && H <= 256 && W <= 256, DI_EUNSUPPORTED,
             "di_vae_decode: latent %ux%u outside [1, 256]", H, W);
  DI_REQUIRE((uint64_t)H * W * H * W * 2 < (1ull << 31), DI_EUNSUPPORTED,
             "di_vae_decode: attention scores of a %ux%u latent exceed 2 GiB per image", H, W);
  DI_REQUIRE((flags & ~DI_VAE_GRAPH) == 0, DI_EINVAL, "di_vae_decode: unknown flags 0x%x", flags);
  const di_vae_config& c = v->cfg;
  DI_BUF(ctx, latent, z, (uint64_t)B * c.latent_channels * H * W * 4);
  DI_BUF(ctx, image, im, (uint64_t)B * c.out_channels * 64 * H * W * 4);
  if (!(flags & DI_VAE_GRAPH)) {
    int rc = vae_decode_step(ctx, *v, (const float*)z->ptr, (float*)im->ptr, B, H, W, scale);
    if (rc) return rc;
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  uint32_t sbits;
  memcpy(&sbits, &scale, 4);
  const uint64_t key[6] = {(uint64_t)z->ptr, (uint64_t)im->ptr, B, H, W, sbits};
  if (!v->graph_exec || memcmp(key, v->graph_key, sizeof(key)) != 0) {
    DI_HIP(hipStreamSynchronize(ctx->stream));
    vae_drop_graph(ctx, v);
    // warm-up outside capture sizes the workspace and fills the pool
    int rc = vae_decode_step(ctx, *v, (const float*)z->ptr, (float*)im->ptr, B, H, W, scale);
    if (rc) return rc;
    DI_HIP(hipStreamSynchronize(ctx->stream));
    DI_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->hold_releases = true;
    rc = vae_decode_step(ctx, *v, (const float*)z->ptr, (float*)im->ptr, B, H, W, scale);
    ctx->hold_releases = false;
    v->graph_scratch.swap(ctx->held);
    ctx->held.clear();
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    DI_REQUIRE(e == hipSuccess, DI_EHIP, "graph capture failed: %s", hipGetErrorString(e));
    v->graph = g;
    v->graph_ws = workspace_pin(ctx);
    if (graph_check_enabled()) {
      size_t kernels = 0;
      int crc = graph_check_nodes(g, &kernels);
      if (crc) return crc;
    }
    DI_HIP(hipGraphInstantiate(&v->graph_exec, g, nullptr, nullptr, 0));
    memcpy(v->graph_key, key, sizeof(key));
  }
  if (graph_check_enabled()) {
    const void* io[2] = {z->ptr, im->ptr};
    int crc = graph_check_live(ctx, v->graph_ws, v->graph_scratch, io, 2);
    if (crc) return crc;
  }
  DI_HIP(hipGraphLaunch(v->graph_exec, ctx->stream));
  return DI_OK;
}

}  // extern "C"

// SD2.1 UNet2DConditionModel (the SD-Turbo U-Net) as one native object on
// the gfx950 kernels: parameters in device arenas, one denoise step per
// di_unet_forward, optionally replayed from a captured HIP graph.
//
// Role of unetForwardWGSL (unet-wgsl.js:145-195): same three inputs (sample
// [B,4,H,W] fp32, timestep, encoder_hidden_states [B,77,1024] fp32) and one
// output (out_sample [B,4,H,W] fp32, unet.js:13-19).  The reference walks the
// ~5478-node ONNX graph op by op (and computes batch 0 only); here the step is
// ~400 fused kernels on NHWC fp16 activations with fp32 accumulation.
//
// Parameters follow diffusers' names and semantics.  Physical layouts differ
// where the kernels want them: convs OHWI fp16 (conv_in's input channels
// padded 4 -> 8), linears [out][in] fp16, attn1 to_q/to_k/to_v fused into one
// [3C][C] matrix, attn2 to_k/to_v into [2C][cross], the GEGLU proj rows
// grouped as 32-row blocks [16 hidden | 16 gate], every ResNet's
// time_emb_proj stacked into one [sum Cout][1280] matrix (one GEMV per step),
// every attn2 to_k/to_v pair stacked into one [sum 2C][1024] matrix (all
// transformers' context projections are one GEMM per step), biases and norm
// affines fp32.  di_unet_param_info describes each tensor.
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "di_blocks.h"
#include "di_gemm.h"
#include "di_tembed.h"

namespace di {

namespace {

// AR_TEMB16 / AR_TEMB32 / AR_KV16 hold stacked matrices (no gaps between
// tensors).  AR_LNW16 / AR_LN32 hold no parameters: they are derived from
// them (the LayerNorm-folded attn1 qkv / attn2 to_q / GEGLU proj weights and
// their column sums and constants, refreshed after any parameter upload).
enum Arena {
  AR_W16 = 0,
  AR_TEMB16 = 1,
  AR_F32 = 2,
  AR_TEMB32 = 3,
  AR_KV16 = 4,
  AR_LNW16 = 5,
  AR_LN32 = 6,
  AR_COUNT = 7
};

struct Param {
  std::string name;
  std::vector<uint32_t> shape;  // physical shape
  int arena;
  uint64_t offset;  // elements within the arena
  uint64_t numel;
  float mean, std;
  int layout;  // DI_PARAM_* layout tag
};

struct ResIdx {
  uint32_t cin, cout;
  int n1g, n1b, c1w, c1b, n2g, n2b, c2w, c2b, skw = -1, skb = -1, tw, tb;
  uint64_t temb_row;  // row offset inside the stacked time_emb_proj matrix
  // with a shortcut: conv2's bias + the shortcut's, derived in AR_LN32
  uint64_t fb_c2sk = 0;
};

struct TfIdx {
  uint32_t c;
  uint64_t kv_row;  // row offset inside the stacked attn2 to_kv matrix
  int ng, nb, piw, pib, l1g, l1b, qkv, o1w, o1b, l2g, l2b, q2, kv2, o2w, o2b, l3g, l3b, f1w, f1b,
      f2w, f2b, pow_, pob;
  // folded projections: weights in AR_LNW16, column sums / constants in AR_LN32
  uint64_t fw_qkv, fw_q2, fw_ff1;
  uint64_t fs_qkv, fc_qkv, fs_q2, fc_q2, fs_ff1, fc_ff1;
};

struct Level {
  std::vector<ResIdx> res;
  std::vector<TfIdx> tf;
  int sample_w = -1, sample_b = -1;  // downsampler / upsampler conv
};

}  // namespace

struct UNet {
  di_unet_config cfg;
  std::vector<Param> params;
  uint64_t arena_elems[AR_COUNT] = {};
  void* arena[AR_COUNT] = {};
  uint64_t arena_cap[AR_COUNT] = {};
  // scratch buffers baked into the captured graph (owned until it is dropped)
  std::vector<std::pair<void*, uint64_t>> graph_scratch;
  // the context workspace the captured graph's kernels address (pinned)
  void* graph_ws = nullptr;
  int conv_in_w, conv_in_b, t1w, t1b, t2w, t2b, nog, nob, cow, cob;
  std::vector<Level> down, up;
  ResIdx mid_res[2];
  TfIdx mid_tf;
  uint32_t temb_rows = 0;
  uint32_t kv_rows = 0;
  bool ln_folded = false;  // AR_LNW16 / AR_LN32 match the parameters
  // captured step
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  size_t graph_kernels = 0;  // kernel nodes of the captured graph (DI_GRAPH_CHECK)
  uint64_t graph_key[8] = {0};

  int add(const std::string& name, std::vector<uint32_t> shape, int arena, float mean, float std,
          int layout) {
    Param p;
    p.name = name;
    p.shape = shape;
    p.arena = arena;
    p.numel = 1;
    for (uint32_t d : shape) p.numel *= d;
    // keep every tensor 16-byte aligned inside its arena
    const uint64_t align = (arena == AR_F32 || arena == AR_TEMB32) ? 4 : 8;
    if (arena != AR_TEMB16 && arena != AR_TEMB32 && arena != AR_KV16)
      arena_elems[arena] = (arena_elems[arena] + align - 1) / align * align;
    p.offset = arena_elems[arena];
    arena_elems[arena] += p.numel;
    p.mean = mean;
    p.std = std;
    p.layout = layout;
    params.push_back(p);
    return (int)params.size() - 1;
  }
  f16* h(int i) const { return (f16*)arena[params[i].arena] + params[i].offset; }
  float* f(int i) const { return (float*)arena[params[i].arena] + params[i].offset; }
};

namespace {

float kaiming(uint32_t fan_in) { return sqrtf(2.0f / (float)fan_in); }
float xavier(uint32_t fan_in, uint32_t fan_out) { return sqrtf(2.0f / (float)(fan_in + fan_out)); }

void add_norm(UNet& u, const std::string& p, uint32_t c, int* g, int* b) {
  *g = u.add(p + ".weight", {c}, AR_F32, 1.0f, 0.02f, DI_PARAM_VECTOR);
  *b = u.add(p + ".bias", {c}, AR_F32, 0.0f, 0.02f, DI_PARAM_VECTOR);
}

void add_conv(UNet& u, const std::string& p, uint32_t cout, uint32_t cin, uint32_t k, int* w, int* b,
              uint32_t cin_phys = 0) {
  if (!cin_phys) cin_phys = cin;
  *w = u.add(p + ".weight", {cout, k, k, cin_phys}, AR_W16, 0.0f, kaiming(cin * k * k),
             DI_PARAM_CONV_OHWI);
  *b = u.add(p + ".bias", {cout}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
}

int add_linear_w(UNet& u, const std::string& p, uint32_t out, uint32_t in, int layout) {
  return u.add(p + ".weight", {out, in}, AR_W16, 0.0f, xavier(in, out), layout);
}

ResIdx add_resnet(UNet& u, const std::string& p, uint32_t cin, uint32_t cout) {
  ResIdx r;
  r.cin = cin;
  r.cout = cout;
  add_norm(u, p + ".norm1", cin, &r.n1g, &r.n1b);
  add_conv(u, p + ".conv1", cout, cin, 3, &r.c1w, &r.c1b);
  r.temb_row = u.temb_rows;
  r.tw = u.add(p + ".time_emb_proj.weight", {cout, u.cfg.time_dim}, AR_TEMB16, 0.0f,
               xavier(u.cfg.time_dim, cout), DI_PARAM_LINEAR);
  r.tb = u.add(p + ".time_emb_proj.bias", {cout}, AR_TEMB32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  u.temb_rows += cout;
  add_norm(u, p + ".norm2", cout, &r.n2g, &r.n2b);
  add_conv(u, p + ".conv2", cout, cout, 3, &r.c2w, &r.c2b);
  if (cin != cout) {
    add_conv(u, p + ".conv_shortcut", cout, cin, 1, &r.skw, &r.skb);
    r.fb_c2sk = (u.arena_elems[AR_LN32] + 3) / 4 * 4;
    u.arena_elems[AR_LN32] = r.fb_c2sk + cout;
  }
  return r;
}

TfIdx add_transformer(UNet& u, const std::string& p, uint32_t c) {
  TfIdx t;
  t.c = c;
  const uint32_t x = u.cfg.cross_dim;
  const std::string tb = p + ".transformer_blocks.0";
  add_norm(u, p + ".norm", c, &t.ng, &t.nb);
  t.piw = add_linear_w(u, p + ".proj_in", c, c, DI_PARAM_LINEAR);
  t.pib = u.add(p + ".proj_in.bias", {c}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  add_norm(u, tb + ".norm1", c, &t.l1g, &t.l1b);
  t.qkv = u.add(tb + ".attn1.to_qkv.weight", {3 * c, c}, AR_W16, 0.0f, xavier(c, c),
                DI_PARAM_LINEAR_STACKED);
  t.o1w = add_linear_w(u, tb + ".attn1.to_out.0", c, c, DI_PARAM_LINEAR);
  t.o1b = u.add(tb + ".attn1.to_out.0.bias", {c}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  add_norm(u, tb + ".norm2", c, &t.l2g, &t.l2b);
  t.q2 = add_linear_w(u, tb + ".attn2.to_q", c, c, DI_PARAM_LINEAR);
  t.kv_row = u.kv_rows;
  t.kv2 = u.add(tb + ".attn2.to_kv.weight", {2 * c, x}, AR_KV16, 0.0f, xavier(x, c),
                DI_PARAM_LINEAR_STACKED);
  u.kv_rows += 2 * c;
  t.o2w = add_linear_w(u, tb + ".attn2.to_out.0", c, c, DI_PARAM_LINEAR);
  t.o2b = u.add(tb + ".attn2.to_out.0.bias", {c}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  add_norm(u, tb + ".norm3", c, &t.l3g, &t.l3b);
  t.f1w = u.add(tb + ".ff.net.0.proj.weight", {8 * c, c}, AR_W16, 0.0f, xavier(c, 8 * c),
                DI_PARAM_GEGLU_ROWS);
  t.f1b = u.add(tb + ".ff.net.0.proj.bias", {8 * c}, AR_F32, 0.0f, 0.01f, DI_PARAM_GEGLU_ROWS);
  t.f2w = add_linear_w(u, tb + ".ff.net.2", c, 4 * c, DI_PARAM_LINEAR);
  t.f2b = u.add(tb + ".ff.net.2.bias", {c}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  t.pow_ = add_linear_w(u, p + ".proj_out", c, c, DI_PARAM_LINEAR);
  t.pob = u.add(p + ".proj_out.bias", {c}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  auto derived = [&](int arena, uint64_t n) {
    const uint64_t align = arena == AR_LN32 ? 4 : 8;
    const uint64_t o = (u.arena_elems[arena] + align - 1) / align * align;
    u.arena_elems[arena] = o + n;
    return o;
  };
  t.fw_qkv = derived(AR_LNW16, 3ull * c * c);
  t.fw_q2 = derived(AR_LNW16, (uint64_t)c * c);
  t.fw_ff1 = derived(AR_LNW16, 8ull * c * c);
  t.fs_qkv = derived(AR_LN32, 3 * c);
  t.fc_qkv = derived(AR_LN32, 3 * c);
  t.fs_q2 = derived(AR_LN32, c);
  t.fc_q2 = derived(AR_LN32, c);
  t.fs_ff1 = derived(AR_LN32, 8 * c);
  t.fc_ff1 = derived(AR_LN32, 8 * c);
  return t;
}

void build_params(UNet& u) {
  const di_unet_config& c = u.cfg;
  const uint32_t L = c.layers_per_block;
  add_conv(u, "conv_in", c.block_channels[0], c.in_channels, 3, &u.conv_in_w, &u.conv_in_b,
           (c.in_channels + 7) / 8 * 8);
  u.t1w = add_linear_w(u, "time_embedding.linear_1", c.time_dim, c.block_channels[0], DI_PARAM_LINEAR);
  u.t1b = u.add("time_embedding.linear_1.bias", {c.time_dim}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  u.t2w = add_linear_w(u, "time_embedding.linear_2", c.time_dim, c.time_dim, DI_PARAM_LINEAR);
  u.t2b = u.add("time_embedding.linear_2.bias", {c.time_dim}, AR_F32, 0.0f, 0.01f, DI_PARAM_VECTOR);
  uint32_t ch = c.block_channels[0];
  u.down.resize(4);
  for (int i = 0; i < 4; i++) {
    const uint32_t out = c.block_channels[i];
    const std::string p = "down_blocks." + std::to_string(i);
    for (uint32_t j = 0; j < L; j++) {
      u.down[i].res.push_back(add_resnet(u, p + ".resnets." + std::to_string(j), j == 0 ? ch : out, out));
      if (c.cross_attn[i])
        u.down[i].tf.push_back(add_transformer(u, p + ".attentions." + std::to_string(j), out));
    }
    ch = out;
    if (i < 3) add_conv(u, p + ".downsamplers.0.conv", out, out, 3, &u.down[i].sample_w, &u.down[i].sample_b);
  }
  const uint32_t top = c.block_channels[3];
  u.mid_res[0] = add_resnet(u, "mid_block.resnets.0", top, top);
  u.mid_tf = add_transformer(u, "mid_block.attentions.0", top);
  u.mid_res[1] = add_resnet(u, "mid_block.resnets.1", top, top);
  u.up.resize(4);
  uint32_t prev = top;
  for (int i = 0; i < 4; i++) {
    const uint32_t out = c.block_channels[3 - i];
    const uint32_t in = c.block_channels[i >= 2 ? 0 : 2 - i];  // reversed[min(i + 1, 3)]
    const std::string p = "up_blocks." + std::to_string(i);
    for (uint32_t j = 0; j <= L; j++) {
      const uint32_t skip = j == L ? in : out;
      const uint32_t rin = (j == 0 ? prev : out) + skip;
      u.up[i].res.push_back(add_resnet(u, p + ".resnets." + std::to_string(j), rin, out));
      if (c.cross_attn[3 - i])
        u.up[i].tf.push_back(add_transformer(u, p + ".attentions." + std::to_string(j), out));
    }
    prev = out;
    if (i < 3) add_conv(u, p + ".upsamplers.0.conv", out, out, 3, &u.up[i].sample_w, &u.up[i].sample_b);
  }
  add_norm(u, "conv_norm_out", c.block_channels[0], &u.nog, &u.nob);
  add_conv(u, "conv_out", c.out_channels, c.block_channels[0], 3, &u.cow, &u.cob);
}

ResnetW res_w(const UNet& u, const ResIdx& r) {
  ResnetW w;
  w.n1_g = u.f(r.n1g);
  w.n1_b = u.f(r.n1b);
  w.c1_w = u.h(r.c1w);
  w.c1_b = u.f(r.c1b);
  w.n2_g = u.f(r.n2g);
  w.n2_b = u.f(r.n2b);
  w.c2_w = u.h(r.c2w);
  w.c2_b = u.f(r.c2b);
  if (r.skw >= 0) {
    w.sk_w = u.h(r.skw);
    w.sk_b = u.f(r.skb);
    if (u.ln_folded) w.c2sk_b = (const float*)u.arena[AR_LN32] + r.fb_c2sk;
  }
  return w;
}

TransformerW tf_w(const UNet& u, const TfIdx& t) {
  TransformerW w;
  w.n_g = u.f(t.ng);
  w.n_b = u.f(t.nb);
  w.pin_w = u.h(t.piw);
  w.pin_b = u.f(t.pib);
  w.ln1_g = u.f(t.l1g);
  w.ln1_b = u.f(t.l1b);
  w.qkv_w = u.h(t.qkv);
  w.o1_w = u.h(t.o1w);
  w.o1_b = u.f(t.o1b);
  w.ln2_g = u.f(t.l2g);
  w.ln2_b = u.f(t.l2b);
  w.q2_w = u.h(t.q2);
  w.kv2_w = u.h(t.kv2);
  w.o2_w = u.h(t.o2w);
  w.o2_b = u.f(t.o2b);
  w.ln3_g = u.f(t.l3g);
  w.ln3_b = u.f(t.l3b);
  w.ff1_w = u.h(t.f1w);
  w.ff1_b = u.f(t.f1b);
  w.ff2_w = u.h(t.f2w);
  w.ff2_b = u.f(t.f2b);
  w.pout_w = u.h(t.pow_);
  w.pout_b = u.f(t.pob);
  // the three LayerNorms run in the epilogues of their projections
  f16* fw = (f16*)u.arena[AR_LNW16];
  float* ff = (float*)u.arena[AR_LN32];
  w.qkv_w = fw + t.fw_qkv;
  w.qkv_s = ff + t.fs_qkv;
  w.qkv_c = ff + t.fc_qkv;
  w.q2_w = fw + t.fw_q2;
  w.q2_s = ff + t.fs_q2;
  w.q2_c = ff + t.fc_q2;
  w.ff1_w = fw + t.fw_ff1;
  w.ff1_s = ff + t.fs_ff1;
  w.ff1_c = ff + t.fc_ff1;
  return w;
}

// Derives every transformer's folded projections and the summed conv2 +
// shortcut biases of the ResNets from the parameters.
void fold_layer_norms(hipStream_t s, UNet& u) {
  f16* fw = (f16*)u.arena[AR_LNW16];
  float* ff = (float*)u.arena[AR_LN32];
  auto one = [&](const TfIdx& t) {
    const uint32_t c = t.c;
    launch_ln_fold(s, u.h(t.qkv), u.f(t.l1g), u.f(t.l1b), nullptr, fw + t.fw_qkv, ff + t.fs_qkv,
                   ff + t.fc_qkv, 3 * c, c);
    launch_ln_fold(s, u.h(t.q2), u.f(t.l2g), u.f(t.l2b), nullptr, fw + t.fw_q2, ff + t.fs_q2,
                   ff + t.fc_q2, c, c);
    launch_ln_fold(s, u.h(t.f1w), u.f(t.l3g), u.f(t.l3b), u.f(t.f1b), fw + t.fw_ff1,
                   ff + t.fs_ff1, ff + t.fc_ff1, 8 * c, c);
  };
  for (const Level& l : u.down)
    for (const TfIdx& t : l.tf) one(t);
  one(u.mid_tf);
  for (const Level& l : u.up)
    for (const TfIdx& t : l.tf) one(t);
  // summed conv2 + shortcut biases of the ResNets with a shortcut
  auto res = [&](const ResIdx& r) {
    if (r.skw >= 0) launch_add_f32(s, u.f(r.c2b), u.f(r.skb), ff + r.fb_c2sk, r.cout);
  };
  for (const Level& l : u.down)
    for (const ResIdx& r : l.res) res(r);
  for (const ResIdx& r : u.mid_res) res(r);
  for (const Level& l : u.up)
    for (const ResIdx& r : l.res) res(r);
}

// One denoise step (enqueue only).
int unet_step(Ctx* c, UNet& u, const float* sample, const float* tsteps, const float* context,
              float* out, uint32_t B, uint32_t H, uint32_t W, uint32_t Sctx) {
  const di_unet_config& cf = u.cfg;
  const uint32_t G = cf.groups;
  const uint32_t cin_p = (cf.in_channels + 7) / 8 * 8;
  // inputs: sample NCHW fp32 -> NHWC fp16 (channels padded), context -> fp16
  // conv_in reads the NCHW latent itself where its direct kernel applies
  // (DI_CONV_IN_DIRECT=0 selects the layout pass + implicit GEMM, for A/B runs)
  const char* env_ci = getenv("DI_CONV_IN_DIRECT");
  const bool ci_direct = (!env_ci || atoi(env_ci) != 0) &&
                         conv_in_direct_ok(cf.in_channels, cf.block_channels[0], H, W);
  Scratch x16, ctx16, th, temb, tproj;
  int rc = ci_direct ? 0 : x16.alloc(c, (uint64_t)B * H * W * cin_p * 2);
  if (!rc) rc = ctx16.alloc(c, (uint64_t)B * Sctx * cf.cross_dim * 2);
  if (!rc) rc = th.alloc(c, (uint64_t)B * cf.time_dim * 4);
  if (!rc) rc = temb.alloc(c, (uint64_t)B * cf.time_dim * 4);
  if (!rc) rc = tproj.alloc(c, (uint64_t)B * u.temb_rows * 4);
  if (rc) return rc;
  if (!ci_direct)
    launch_layout(c->stream, sample, DI_F32, DI_NCHW, x16.p, DI_F16, DI_NHWC, B, cf.in_channels,
                  H, W, cin_p);
  // the context's fp32 -> fp16 conversion rides in conv_in's launch where
  // the direct conv_in runs (then the K / V GEMM below follows conv_in)
  const uint64_t ctx_n = (uint64_t)B * Sctx * cf.cross_dim;
  const bool ctx_in_conv_in = ci_direct && conv_in_convert_ok(context, ctx16.p, ctx_n);
  if (!ctx_in_conv_in) launch_convert(c->stream, context, DI_F32, ctx16.p, DI_F16, ctx_n);
  // every transformer's attn2 K / V of the context: one GEMM over the
  // stacked [kv_rows][cross] weights -> kvall [B*Sctx][kv_rows]
  Scratch kvall;
  if (u.kv_rows) rc = kvall.alloc(c, (uint64_t)B * Sctx * u.kv_rows * 2);
  if (rc) return rc;
  auto kv_gemm = [&]() {
    if (!u.kv_rows) return (int)DI_OK;
    return linear_f16(c, ctx16.h(), cf.cross_dim, B * Sctx, cf.cross_dim,
                      (const f16*)u.arena[AR_KV16], u.kv_rows, nullptr, ACT_NONE, nullptr, 0,
                      kvall.h(), u.kv_rows);
  };
  if (!ctx_in_conv_in) rc = kv_gemm();
  if (rc) return rc;
  // time embedding: sinusoid -> linear_1 + SiLU -> linear_2 -> every
  // ResNet's time_emb_proj(SiLU(temb)) in one GEMV
  GemvArgs g1;
  g1.x_mode = GEMV_X_SINUSOID;
  g1.t = tsteps;
  g1.w = u.h(u.t1w);
  g1.ldw = cf.block_channels[0];
  g1.bias = u.f(u.t1b);
  g1.act = GEMV_ACT_SILU;
  g1.y = th.f();
  g1.ldy = cf.time_dim;
  g1.B = B;
  g1.N = cf.time_dim;
  g1.K = cf.block_channels[0];
  // the first GEMV rides in conv_in's launch where the direct conv_in runs;
  // the other two follow conv_in then
  const bool g1_side = ctx_in_conv_in && conv_in_gemv_ok(g1);
  GemvArgs g2;
  g2.x = th.f();
  g2.ldx = cf.time_dim;
  g2.w = u.h(u.t2w);
  g2.ldw = cf.time_dim;
  g2.bias = u.f(u.t2b);
  g2.y = temb.f();
  g2.ldy = cf.time_dim;
  g2.B = B;
  g2.N = cf.time_dim;
  g2.K = cf.time_dim;
  GemvArgs g3;
  g3.x_mode = GEMV_X_SILU;
  g3.x = temb.f();
  g3.ldx = cf.time_dim;
  g3.w = u.arena[AR_TEMB16];
  g3.ldw = cf.time_dim;
  g3.bias = (const float*)u.arena[AR_TEMB32];
  g3.y = tproj.f();
  g3.ldy = u.temb_rows;
  g3.B = B;
  g3.N = u.temb_rows;
  g3.K = cf.time_dim;
  if (!g1_side) {
    launch_gemv(g1, DI_F16, c->stream);
    launch_gemv(g2, DI_F16, c->stream);
    launch_gemv(g3, DI_F16, c->stream);
  }

  // An activation and, when its level allows (HW % 64 == 0), the GroupNorm
  // statistics its producer wrote (every GN input here is the output of a
  // GEMM epilogue, so no GN runs a separate statistics pass).
  struct Act {
    Scratch buf, st;
    uint32_t c = 0;
    StatsOut so;   // request / report of the producer's statistics
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
  // statistics request for a's producer; has_st follows once it has run
  auto st_out = [](Act& a) { return a.so.p ? &a.so : (StatsOut*)nullptr; };
  auto st_done = [](Act& a) { a.has_st = a.so.done; };
  auto st_of = [](const Act& a) { return GnStats{a.st.f(), a.st.f(), a.c, a.c, a.c}; };
  // the time_emb_proj GEMV (g3) still to run before the first conv1 reads
  // tproj: the first ResNet's GN1 launch takes it (or launches it)
  const GemvArgs* g3_pending = nullptr;
  auto resnet = [&](const ResIdx& r, NhwcSrc x, const GnStats* xs, uint32_t hh, uint32_t ww,
                    Act& y, GnFuseOut* og = nullptr, const f16* xg = nullptr) {
    ResnetShape s{B, hh, ww, r.cin, r.cout, G, cf.resnet_eps};
    const GemvArgs* side = g3_pending;
    g3_pending = nullptr;
    const int r2 = resnet_forward(c, res_w(u, r), s, x, tproj.f() + r.temb_row, u.temb_rows,
                                  y.buf.h(), xs, st_out(y), og, xg, side);
    st_done(y);
    return r2;
  };
  // An output that is the next ResNet's input and a skip: that ResNet's
  // GN1 + SiLU requested from the producer's split-K reducer, which then
  // also stores the raw output and its statistics (for the up path's
  // concatenated GroupNorm), into gbuf; o.done reports whether it ran
  auto res_gn = [&](const ResIdx& r, uint32_t hh, uint32_t ww, Act& y, Scratch& gbuf,
                    GnFuseOut& o) {
    const int r2 = gbuf.alloc(c, (uint64_t)B * hh * ww * r.cin * 2);
    o.f.gamma = u.f(r.n1g);
    o.f.beta = u.f(r.n1b);
    o.f.y = gbuf.h();
    o.f.ldy = r.cin;
    o.f.groups = G;
    o.f.hw = hh * ww;
    o.f.eps = cf.resnet_eps;
    o.f.silu = 1;
    o.f.raw = 1;
    o.f.stats = y.st.f();
    return r2;
  };
  auto transformer = [&](const TfIdx& t, const Act& x, uint32_t hh, uint32_t ww, Act& y,
                         const f16* xg = nullptr) {
    TransformerShape s{B, hh, ww, t.c, Sctx, cf.cross_dim, G, cf.transformer_gn_eps, cf.ln_eps};
    TransformerW w = tf_w(u, t);
    w.kv_pre = kvall.h() + t.kv_row;
    w.kv_ld = u.kv_rows;
    const GnStats xs = st_of(x);
    const int r2 = transformer_forward(c, w, s, x.buf.h(), ctx16.h(), y.buf.h(),
                                       x.has_st ? &xs : nullptr, st_out(y), xg);
    st_done(y);
    return r2;
  };
  // A ResNet output that enters a transformer: the transformer's GroupNorm
  // requested from the ResNet's conv2 reducer (GnFuse, raw output kept),
  // into gbuf; o.done reports whether it ran (else the transformer applies
  // it from the output's statistics)
  auto tf_gn = [&](const TfIdx& t, uint32_t hh, uint32_t ww, uint32_t ch, Scratch& gbuf,
                   GnFuseOut& o) {
    const int r2 = gbuf.alloc(c, (uint64_t)B * hh * ww * ch * 2);
    const TransformerW w = tf_w(u, t);
    o.f.gamma = w.n_g;
    o.f.beta = w.n_b;
    o.f.y = gbuf.h();
    o.f.ldy = ch;
    o.f.groups = G;
    o.f.hw = hh * ww;
    o.f.eps = cf.transformer_gn_eps;
    o.f.silu = 0;
    o.f.raw = 1;
    return r2;
  };
  auto one = [](const f16* p, uint32_t ch) { return NhwcSrc{p, p, ch, ch, ch}; };

  // conv_in
  std::vector<Act> skips;  // diffusers' down_block_res_samples
  uint32_t hh = H, ww = W;
  uint32_t ch = cf.block_channels[0];
  Act hcur;
  rc = act_alloc(hcur, hh, ww, ch);
  if (rc) return rc;
  if (ci_direct) {
    if (ctx_in_conv_in)
      launch_conv_in(c->stream, sample, u.h(u.conv_in_w), u.f(u.conv_in_b), hcur.buf.h(),
                     hcur.st.f(), B, ch, hh, ww, context, ctx16.h(), ctx_n,
                     g1_side ? &g1 : nullptr);
    else
      launch_conv_in(c->stream, sample, u.h(u.conv_in_w), u.f(u.conv_in_b), hcur.buf.h(),
                     hcur.st.f(), B, ch, hh, ww);
    hcur.so.done = hcur.st.f() != nullptr;
    st_done(hcur);
    if (ctx_in_conv_in) rc = kv_gemm();
    if (rc) return rc;
    if (g1_side) {
      launch_gemv(g2, DI_F16, c->stream);
      g3_pending = &g3;
    }
  } else {
    ConvCall cc;
    cc.x = one(x16.h(), cin_p);
    cc.B = B;
    cc.H = hh;
    cc.W = ww;
    cc.Cin = cin_p;
    cc.Cout = ch;
    cc.w = u.h(u.conv_in_w);
    cc.bias = u.f(u.conv_in_b);
    cc.y = hcur.buf.h();
    cc.stats = st_out(hcur);
    rc = conv_nhwc(c, cc);
    if (rc) return rc;
    st_done(hcur);
  }
  // down path: conv_in's output, every resnet(+transformer) output and every
  // downsampler output become skips; the current tensor is always the last one
  // GN1(hcur) + SiLU when hcur's producer applied it (gin_ok)
  Scratch gin;
  bool gin_ok = false;
  for (int i = 0; i < 4; i++) {
    Level& lv = u.down[i];
    for (size_t j = 0; j < lv.res.size(); j++) {
      const ResIdx& r = lv.res[j];
      Act nxt;
      const GnStats xs = st_of(hcur);
      Scratch gbuf;
      GnFuseOut og;
      const bool tf = !lv.tf.empty();
      // without a transformer the output is the next ResNet's input (the
      // level's next one, or after the last level's last the mid block's)
      const ResIdx* rn = tf ? nullptr
                         : j + 1 < lv.res.size()              ? &lv.res[j + 1]
                         : i == 3 && lv.sample_w < 0         ? &u.mid_res[0]
                                                               : nullptr;
      rc = act_alloc(nxt, hh, ww, r.cout);
      if (!rc && tf) rc = tf_gn(lv.tf[j], hh, ww, r.cout, gbuf, og);
      if (!rc && rn && nxt.st.f()) rc = res_gn(*rn, hh, ww, nxt, gbuf, og);  // (gated in the block)
      if (!rc)
        rc = resnet(r, one(hcur.buf.h(), ch), hcur.has_st ? &xs : nullptr, hh, ww, nxt,
                    tf || (rn && nxt.st.f()) ? &og : nullptr, gin_ok ? gin.h() : nullptr);
      if (rc) return rc;
      gin_ok = false;
      if (rn && og.done) {
        gin = std::move(gbuf);
        gin_ok = true;
      }
      if (tf) {
        Act t2;
        rc = act_alloc(t2, hh, ww, r.cout);
        if (!rc) rc = transformer(lv.tf[j], nxt, hh, ww, t2, og.done ? gbuf.h() : nullptr);
        if (rc) return rc;
        nxt = std::move(t2);
      }
      skips.push_back(std::move(hcur));
      hcur = std::move(nxt);
      ch = r.cout;
    }
    if (lv.sample_w >= 0) {
      Act ds;
      const uint32_t h2 = (hh - 1) / 2 + 1, w2 = (ww - 1) / 2 + 1;
      rc = act_alloc(ds, h2, w2, ch);
      if (rc) return rc;
      ConvCall cc;
      cc.x = one(hcur.buf.h(), ch);
      cc.B = B;
      cc.H = hh;
      cc.W = ww;
      cc.Cin = ch;
      cc.Cout = ch;
      cc.stride = 2;
      cc.w = u.h(lv.sample_w);
      cc.bias = u.f(lv.sample_b);
      cc.y = ds.buf.h();
      cc.stats = st_out(ds);
      // the next level's first ResNet's GN1 from the downsampler's reducer
      Scratch gbuf;
      GnFuseOut og;
      const ResIdx* rn = i + 1 < 4 && !u.down[i + 1].res.empty() ? &u.down[i + 1].res[0] : nullptr;
      if (rn && ds.st.f() && !gn_reduce_fuse_off()) {
        rc = res_gn(*rn, h2, w2, ds, gbuf, og);
        if (rc) return rc;
        cc.gn = &og;
      }
      rc = conv_nhwc(c, cc);
      if (rc) return rc;
      st_done(ds);
      gin_ok = false;
      if (rn && og.done) {
        gin = std::move(gbuf);
        gin_ok = true;
      }
      skips.push_back(std::move(hcur));
      hcur = std::move(ds);
      hh = h2;
      ww = w2;
    }
  }
  if (g3_pending) launch_gemv(*g3_pending, DI_F16, c->stream);  // (no down-path ResNet)
  g3_pending = nullptr;
  skips.push_back(std::move(hcur));
  // mid block on the last skip (which the first up resnet consumes again)
  Act m1, m2, m3;
  const Act& mid_in = skips.back();
  const GnStats ms = st_of(mid_in);
  Scratch mgbuf;
  GnFuseOut mog;
  rc = act_alloc(m1, hh, ww, ch);
  if (!rc) rc = tf_gn(u.mid_tf, hh, ww, ch, mgbuf, mog);
  if (!rc)
    rc = resnet(u.mid_res[0], one(mid_in.buf.h(), ch), mid_in.has_st ? &ms : nullptr, hh, ww, m1,
                &mog, gin_ok ? gin.h() : nullptr);
  gin_ok = false;
  gin.release();
  if (!rc) rc = act_alloc(m2, hh, ww, ch);
  if (!rc) rc = transformer(u.mid_tf, m1, hh, ww, m2, mog.done ? mgbuf.h() : nullptr);
  const GnStats m2s = st_of(m2);
  if (!rc) rc = act_alloc(m3, hh, ww, ch);
  if (!rc) rc = resnet(u.mid_res[1], one(m2.buf.h(), ch), m2.has_st ? &m2s : nullptr, hh, ww, m3);
  if (rc) return rc;
  m1.buf.release();
  m1.st.release();
  m2.buf.release();
  m2.st.release();
  hcur = std::move(m3);
  // up path: each resnet takes cat(current, last skip)
  for (int i = 0; i < 4; i++) {
    Level& lv = u.up[i];
    for (size_t j = 0; j < lv.res.size(); j++) {
      const ResIdx& r = lv.res[j];
      Act sk = std::move(skips.back());
      skips.pop_back();
      Act nxt;
      Scratch gbuf;
      GnFuseOut og;
      const bool tf = !lv.tf.empty();
      rc = act_alloc(nxt, hh, ww, r.cout);
      if (!rc && tf) rc = tf_gn(lv.tf[j], hh, ww, r.cout, gbuf, og);
      if (rc) return rc;
      NhwcSrc cat{hcur.buf.h(), sk.buf.h(), ch, ch, sk.c};
      const GnStats cs{hcur.st.f(), sk.st.f(), ch, ch, sk.c};
      rc = resnet(r, cat, hcur.has_st && sk.has_st ? &cs : nullptr, hh, ww, nxt,
                  tf ? &og : nullptr);
      if (rc) return rc;
      sk.buf.release();
      sk.st.release();
      ch = r.cout;
      if (tf) {
        Act t2;
        rc = act_alloc(t2, hh, ww, ch);
        if (!rc) rc = transformer(lv.tf[j], nxt, hh, ww, t2, og.done ? gbuf.h() : nullptr);
        if (rc) return rc;
        nxt = std::move(t2);
      }
      hcur = std::move(nxt);
    }
    if (lv.sample_w >= 0) {
      Act us;
      rc = act_alloc(us, hh * 2, ww * 2, ch);
      if (rc) return rc;
      ConvCall cc;
      cc.x = one(hcur.buf.h(), ch);
      cc.B = B;
      cc.H = hh;
      cc.W = ww;
      cc.Cin = ch;
      cc.Cout = ch;
      cc.up = 2;
      cc.w = u.h(lv.sample_w);
      cc.bias = u.f(lv.sample_b);
      cc.y = us.buf.h();
      cc.stats = st_out(us);
      rc = conv_nhwc(c, cc);
      if (rc) return rc;
      st_done(us);
      hcur = std::move(us);
      hh *= 2;
      ww *= 2;
    }
  }
  // conv_norm_out + SiLU -> conv_out (NCHW fp32 store)
  Scratch no;
  rc = no.alloc(c, (uint64_t)B * hh * ww * ch * 2);
  if (rc) return rc;
  {
    const GnStats hs = st_of(hcur);
    if (!hcur.has_st || !launch_group_norm_nhwc_st(c->stream, one(hcur.buf.h(), ch), hs, u.f(u.nog),
                                                   u.f(u.nob), no.h(), B, ch, G, hh * ww,
                                                   cf.resnet_eps, true)) {
      void* ws = nullptr;
      rc = workspace(c, gn_nhwc_ws_floats(B, ch, G, hh * ww) * sizeof(float), &ws);
      if (rc) return rc;
      launch_group_norm_nhwc(c->stream, one(hcur.buf.h(), ch), u.f(u.nog), u.f(u.nob), no.h(), B,
                             ch, G, hh * ww, cf.resnet_eps, true, (float*)ws);
    }
  }
  ConvCall co;
  co.x = one(no.h(), ch);
  co.B = B;
  co.H = hh;
  co.W = ww;
  co.Cin = ch;
  co.Cout = cf.out_channels;
  co.w = u.h(u.cow);
  co.bias = u.f(u.cob);
  co.y = out;
  co.y_nchw_f32 = 1;
  return conv_nhwc(c, co);
}

void default_config(di_unet_config* c) {
  memset(c, 0, sizeof(*c));
  c->in_channels = 4;
  c->out_channels = 4;
  c->block_channels[0] = 320;
  c->block_channels[1] = 640;
  c->block_channels[2] = 1280;
  c->block_channels[3] = 1280;
  c->cross_attn[0] = c->cross_attn[1] = c->cross_attn[2] = 1;
  c->cross_attn[3] = 0;
  c->layers_per_block = 2;
  c->cross_dim = 1024;
  c->time_dim = 1280;
  c->groups = 32;
  c->resnet_eps = 1e-5f;
  c->transformer_gn_eps = 1e-6f;
  c->ln_eps = 1e-5f;
}

}  // namespace
}  // namespace di

using namespace di;

struct di_unet : di::UNet {};

static void drop_graph(di_ctx* ctx, di_unet* u) {
  if (u->graph_exec) (void)hipGraphExecDestroy(u->graph_exec);
  if (u->graph) (void)hipGraphDestroy(u->graph);
  u->graph_exec = nullptr;
  u->graph = nullptr;
  for (auto& pc : u->graph_scratch) pool_release(ctx, pc.first, pc.second);
  u->graph_scratch.clear();
  workspace_unpin(ctx, u->graph_ws);
  u->graph_ws = nullptr;
}

extern "C" {

int32_t di_unet_default_config(di_unet_config* cfg) {
  DI_REQUIRE(cfg != nullptr, DI_EINVAL, "di_unet_default_config: null config");
  default_config(cfg);
  return DI_OK;
}

int32_t di_unet_create(di_ctx* ctx, const di_unet_config* cfg, uint64_t seed, di_unet** out) {
  DI_CTX(ctx);
  DI_REQUIRE(out != nullptr, DI_EINVAL, "di_unet_create: null out pointer");
  *out = nullptr;
  di_unet_config c;
  if (cfg) c = *cfg;
  else default_config(&c);
  for (int i = 0; i < 4; i++) {
    DI_REQUIRE(c.block_channels[i] % 64 == 0 && c.block_channels[i] % c.groups == 0 &&
                   c.block_channels[i] <= 1280,
               DI_EUNSUPPORTED,
               "di_unet_create: block channels must be multiples of 64 (head dim) and of groups, "
               "<= 1280 (got %u)",
               c.block_channels[i]);
  }
  DI_REQUIRE(c.in_channels >= 1 && c.in_channels <= 64 && c.out_channels >= 1, DI_EINVAL,
             "di_unet_create: bad in/out channels");
  DI_REQUIRE(c.layers_per_block >= 1 && c.groups >= 1 && c.cross_dim % 8 == 0 && c.time_dim % 8 == 0 &&
                 c.time_dim <= 1280 && c.block_channels[0] <= 1280,
             DI_EUNSUPPORTED, "di_unet_create: unsupported config");
  auto* u = new di_unet();
  u->cfg = c;
  build_params(*u);
  const size_t esz[AR_COUNT] = {2, 2, 4, 4, 2, 2, 4};
  for (int a = 0; a < AR_COUNT; a++) {
    int rc = pool_alloc(ctx, std::max<uint64_t>(u->arena_elems[a] * esz[a], 256), &u->arena[a],
                        &u->arena_cap[a]);
    if (rc) {
      for (int b = 0; b < a; b++) pool_release(ctx, u->arena[b], u->arena_cap[b]);
      delete u;
      return rc;
    }
  }
  for (size_t i = 0; i < u->params.size(); i++) {
    const Param& p = u->params[i];
    void* dst = (char*)u->arena[p.arena] + p.offset * esz[p.arena];
    launch_fill_normal(ctx->stream, dst, esz[p.arena] == 2 ? DI_F16 : DI_F32, p.numel,
                       seed * 1000003ull + i, p.mean, p.std);
  }
  DI_LAUNCH_CHECK();
  *out = u;
  return DI_OK;
}

int32_t di_unet_destroy(di_ctx* ctx, di_unet* u) {
  DI_CTX(ctx);
  DI_REQUIRE(u != nullptr, DI_EINVAL, "di_unet_destroy: null unet");
  DI_HIP(hipStreamSynchronize(ctx->stream));
  drop_graph(ctx, u);
  for (int a = 0; a < AR_COUNT; a++) pool_release(ctx, u->arena[a], u->arena_cap[a]);
  delete u;
  return DI_OK;
}

int32_t di_unet_num_params(di_ctx* ctx, di_unet* u, uint32_t* n_tensors, uint64_t* n_elements) {
  DI_CTX(ctx);
  DI_REQUIRE(u != nullptr, DI_EINVAL, "null unet");
  if (n_tensors) *n_tensors = (uint32_t)u->params.size();
  if (n_elements) {
    uint64_t s = 0;
    for (const auto& p : u->params) s += p.numel;
    *n_elements = s;
  }
  return DI_OK;
}

int32_t di_unet_param_info(di_ctx* ctx, di_unet* u, uint32_t i, char* name, uint32_t name_cap,
                           uint32_t* dims, uint32_t* ndims, int32_t* dtype, int32_t* layout) {
  DI_CTX(ctx);
  DI_REQUIRE(u != nullptr, DI_EINVAL, "null unet");
  DI_REQUIRE(i < u->params.size(), DI_EINVAL, "param index %u out of range", i);
  const Param& p = u->params[i];
  if (name && name_cap) {
    strncpy(name, p.name.c_str(), name_cap - 1);
    name[name_cap - 1] = 0;
  }
  if (ndims) *ndims = (uint32_t)p.shape.size();
  if (dims)
    for (size_t d = 0; d < p.shape.size() && d < 8; d++) dims[d] = p.shape[d];
  if (dtype) *dtype = (p.arena == AR_F32 || p.arena == AR_TEMB32) ? DI_F32 : DI_F16;
  if (layout) *layout = p.layout;
  return DI_OK;
}

static int param_xfer(di_ctx* ctx, di_unet* u, uint32_t i, void* host, uint64_t bytes, bool down) {
  DI_CTX(ctx);
  DI_REQUIRE(u != nullptr, DI_EINVAL, "null unet");
  DI_REQUIRE(i < u->params.size(), DI_EINVAL, "param index %u out of range", i);
  const Param& p = u->params[i];
  const size_t es = (p.arena == AR_F32 || p.arena == AR_TEMB32) ? 4 : 2;
  DI_REQUIRE(bytes == p.numel * es, DI_EINVAL, "param %s is %llu bytes, got %llu", p.name.c_str(),
             (unsigned long long)(p.numel * es), (unsigned long long)bytes);
  DI_REQUIRE(host != nullptr, DI_EINVAL, "null host pointer");
  void* dev = (char*)u->arena[p.arena] + p.offset * es;
  if (down) {
    DI_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
  } else {
    DI_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, ctx->stream));
    u->ln_folded = false;
  }
  DI_HIP(hipStreamSynchronize(ctx->stream));
  return DI_OK;
}

int32_t di_unet_param_download(di_ctx* ctx, di_unet* u, uint32_t i, void* dst, uint64_t bytes) {
  return param_xfer(ctx, u, i, dst, bytes, true);
}

int32_t di_unet_param_upload(di_ctx* ctx, di_unet* u, uint32_t i, const void* src, uint64_t bytes) {
  return param_xfer(ctx, u, i, (void*)src, bytes, false);
}

int32_t di_unet_forward(di_ctx* ctx, di_unet* u, di_handle sample, di_handle timesteps,
                        di_handle context, di_handle out, uint32_t B, uint32_t H, uint32_t W,
                        uint32_t Sctx, int32_t flags) {
  DI_CTX(ctx);
  DI_REQUIRE(u != nullptr, DI_EINVAL, "null unet");
  DI_REQUIRE(B >= 1 && B <= 8, DI_EUNSUPPORTED, "di_unet_forward: batch %u outside [1, 8]", B);
  DI_REQUIRE(H % 8 == 0 && W % 8 == 0 && H >= 8 && W >= 8, DI_EINVAL,
             "di_unet_forward: latent %ux%u must be a multiple of 8", H, W);
  DI_REQUIRE(Sctx >= 1, DI_EINVAL, "di_unet_forward: empty context");
  DI_REQUIRE((flags & ~DI_UNET_GRAPH) == 0, DI_EINVAL, "di_unet_forward: unknown flags 0x%x", flags);
  const di_unet_config& c = u->cfg;
  DI_BUF(ctx, sample, s, (uint64_t)B * c.in_channels * H * W * 4);
  DI_BUF(ctx, timesteps, t, (uint64_t)B * 4);
  DI_BUF(ctx, context, cx, (uint64_t)B * Sctx * c.cross_dim * 4);
  DI_BUF(ctx, out, o, (uint64_t)B * c.out_channels * H * W * 4);
  if (!u->ln_folded) {
    // stream-ordered before the step (a captured graph reads the same arenas)
    fold_layer_norms(ctx->stream, *u);
    DI_LAUNCH_CHECK();
    u->ln_folded = true;
  }
  if (!(flags & DI_UNET_GRAPH)) {
    int rc = unet_step(ctx, *u, (const float*)s->ptr, (const float*)t->ptr, (const float*)cx->ptr,
                       (float*)o->ptr, B, H, W, Sctx);
    if (rc) return rc;
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  // Graph mode: capture the step once per (buffers, shape) and replay it.
  const uint64_t key[8] = {(uint64_t)s->ptr, (uint64_t)t->ptr, (uint64_t)cx->ptr, (uint64_t)o->ptr,
                           B, H, W, Sctx};
  if (!u->graph_exec || memcmp(key, u->graph_key, sizeof(key)) != 0) {
    DI_HIP(hipStreamSynchronize(ctx->stream));
    drop_graph(ctx, u);
    // Warm-up run outside capture: sizes the workspace and fills the pool, so
    // the captured launches allocate nothing from the driver.
    int rc = unet_step(ctx, *u, (const float*)s->ptr, (const float*)t->ptr, (const float*)cx->ptr,
                       (float*)o->ptr, B, H, W, Sctx);
    if (rc) return rc;
    DI_HIP(hipStreamSynchronize(ctx->stream));
    // Scratch released during capture is kept out of the pool: the graph
    // writes it on every replay, so nothing else may be handed it.
    DI_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
    ctx->hold_releases = true;
    rc = unet_step(ctx, *u, (const float*)s->ptr, (const float*)t->ptr, (const float*)cx->ptr,
                   (float*)o->ptr, B, H, W, Sctx);
    ctx->hold_releases = false;
    u->graph_scratch.swap(ctx->held);
    ctx->held.clear();
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &g);
    if (rc) {
      if (g) (void)hipGraphDestroy(g);
      return rc;
    }
    DI_REQUIRE(e == hipSuccess, DI_EHIP, "graph capture failed: %s", hipGetErrorString(e));
    u->graph = g;
    u->graph_ws = workspace_pin(ctx);
    if (graph_check_enabled()) {
      int crc = graph_check_nodes(g, &u->graph_kernels);
      if (crc) return crc;
    }
    DI_HIP(hipGraphInstantiate(&u->graph_exec, g, nullptr, nullptr, 0));
    memcpy(u->graph_key, key, sizeof(key));
  }
  if (graph_check_enabled()) {
    const void* io[4] = {s->ptr, t->ptr, cx->ptr, o->ptr};
    int crc = graph_check_live(ctx, u->graph_ws, u->graph_scratch, io, 4);
    if (crc) return crc;
  }
  DI_HIP(hipGraphLaunch(u->graph_exec, ctx->stream));
  return DI_OK;
}

}  // extern "C"

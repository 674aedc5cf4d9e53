// C ABI of the contraction ops: matmul, gemm, linear, conv2d.  Validation
// here, arithmetic in k_gemm.hip.
#include "di_gemm.h"
#include "di_internal.h"
#include "di_kernels.h"

using namespace di;

namespace {

int run_gemm(di_ctx* ctx, GemmArgs& g, int elem, int a_mode, int b_mode, int tile = -1,
             int splits = -1) {
  const GemmPlan plan = gemm_plan(g, elem, ctx->num_cus);
  if (tile < 0) tile = plan.tile;
  g.splits = splits > 0 ? (uint32_t)splits : plan.splits;
  if (g.splits > 1) {
    void* ws = nullptr;
    int rc = workspace(ctx, gemm_ws_bytes(g), &ws);
    if (rc) return rc;
    g.part = (float*)ws;
  }
  launch_gemm(g, elem, a_mode, b_mode, tile, ctx->stream);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

// dtype of the activations / outputs and element size of B for the
// contractions that take DI_F32W16 (fp32 with fp16-resident weights).
struct Dts {
  int act;
  size_t es, esb;
  bool w16;
};
Dts contraction_dts(int dt) {
  const bool w16 = dt == DI_F32W16;
  const int act = w16 ? DI_F32 : dt;
  return Dts{act, dtype_size(act), w16 ? 2 : dtype_size(act), w16};
}
#define DI_DTYPE_W16(dt)                                                                    \
  DI_REQUIRE(::di::dtype_ok(dt) || (dt) == DI_F32W16, DI_EINVAL, "unsupported dtype %d", \
             (int)(dt))

// Optional fp32 per-channel parameter buffer (0 = absent).
int opt_f32(di_ctx* ctx, di_handle h, uint64_t n, const float** out) {
  *out = nullptr;
  if (h == 0) return DI_OK;
  Buffer* b = nullptr;
  int rc = lookup(ctx, h, &b);
  if (rc) return rc;
  DI_REQUIRE(b->bytes >= n * 4, DI_EINVAL, "fp32 parameter buffer holds %llu bytes, needs %llu",
             (unsigned long long)b->bytes, (unsigned long long)(n * 4));
  *out = (const float*)b->ptr;
  return DI_OK;
}

struct Tmp {
  di_ctx* c;
  void* p = nullptr;
  uint64_t cap = 0;
  explicit Tmp(di_ctx* ctx) : c(ctx) {}
  int alloc(uint64_t bytes) { return pool_alloc(c, bytes, &p, &cap); }
  ~Tmp() {
    if (p) pool_release(c, p, cap);
  }
};

}  // namespace

extern "C" {

int32_t di_matmul(di_ctx* ctx, di_handle A, di_handle B, di_handle Y, uint32_t M, uint32_t N,
                  uint32_t K, uint32_t batch, int32_t b_batched, int32_t dtype) {
  DI_CTX(ctx);
  DI_DTYPE_W16(dtype);
  DI_REQUIRE(M && N && K && batch, DI_EINVAL, "di_matmul: zero dimension (M=%u N=%u K=%u batch=%u)",
             M, N, K, batch);
  const Dts d = contraction_dts(dtype);
  const int dt = d.act;
  const size_t es = d.es;
  DI_BUF(ctx, A, a, (uint64_t)batch * M * K * es);
  DI_BUF(ctx, B, b, (uint64_t)(b_batched ? batch : 1) * K * N * d.esb);
  DI_BUF(ctx, Y, y, (uint64_t)batch * M * N * es);
  GemmArgs g;
  g.a = a->ptr;
  g.lda = K;
  g.sa = (uint64_t)M * K;
  g.b = b->ptr;
  g.ldb = N;
  g.sb = b_batched ? (uint64_t)K * N : 0;
  g.M = M;
  g.N = N;
  g.K = K;
  g.batch = batch;
  g.c = y->ptr;
  g.ldc = N;
  g.sc = (uint64_t)M * N;
  g.c_f32 = dt == DI_F32;
  const uint32_t kv = dt == DI_F32 ? 4 : 8;
  g.a_vec_ok = K % kv == 0;
  g.b_vec_ok = N % kv == 0;
  g.b_f16 = d.w16;
  return run_gemm(ctx, g, dt, A_DENSE, B_KN);
}

int32_t di_gemm(di_ctx* ctx, di_handle A, di_handle B, di_handle C, di_handle Y, uint32_t M,
                uint32_t N, uint32_t K, int32_t trans_b, int32_t dtype) {
  DI_CTX(ctx);
  DI_DTYPE_W16(dtype);
  DI_REQUIRE(M && N && K, DI_EINVAL, "di_gemm: zero dimension (M=%u N=%u K=%u)", M, N, K);
  const Dts d = contraction_dts(dtype);
  const int dt = d.act;
  const size_t es = d.es;
  DI_BUF(ctx, A, a, (uint64_t)M * K * es);
  DI_BUF(ctx, B, b, (uint64_t)K * N * d.esb);
  DI_BUF(ctx, Y, y, (uint64_t)M * N * es);
  const float* bias = nullptr;
  int rc = opt_f32(ctx, C, N, &bias);
  if (rc) return rc;
  GemmArgs g;
  g.a = a->ptr;
  g.lda = K;
  g.b = b->ptr;
  g.ldb = trans_b ? K : N;
  g.M = M;
  g.N = N;
  g.K = K;
  g.bias = bias;
  g.c = y->ptr;
  g.ldc = N;
  g.c_f32 = dt == DI_F32;
  const uint32_t kv = dt == DI_F32 ? 4 : 8;
  g.a_vec_ok = K % kv == 0;
  g.b_vec_ok = (trans_b ? K : N) % kv == 0;
  g.b_f16 = d.w16;
  g.a_bytes = gemm_extent((uint64_t)M * K * es);
  g.b_bytes = gemm_extent((uint64_t)K * N * d.esb);
  return run_gemm(ctx, g, dt, A_DENSE, trans_b ? B_NK : B_KN);
}

int32_t di_linear(di_ctx* ctx, di_handle X, di_handle W, di_handle bias, di_handle R, di_handle Y,
                  uint32_t M, uint32_t N, uint32_t K, int32_t act, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(M && N && K, DI_EINVAL, "di_linear: zero dimension (M=%u N=%u K=%u)", M, N, K);
  DI_REQUIRE(act >= ACT_NONE && act <= ACT_GELU_TANH, DI_EINVAL, "di_linear: unknown act %d", act);
  DI_REQUIRE(act != ACT_GEGLU || N % 32 == 0, DI_EINVAL,
             "di_linear: GEGLU needs N %% 32 == 0 (got %u)", N);
  const size_t es = dtype_size(dt);
  const uint32_t nout = act == ACT_GEGLU ? N / 2 : N;
  DI_BUF(ctx, X, x, (uint64_t)M * K * es);
  DI_BUF(ctx, W, w, (uint64_t)N * K * es);
  DI_BUF(ctx, Y, y, (uint64_t)M * nout * es);
  const float* b = nullptr;
  int rc = opt_f32(ctx, bias, N, &b);
  if (rc) return rc;
  GemmArgs g;
  if (R) {
    DI_BUF(ctx, R, r, (uint64_t)M * nout * es);
    g.res = r->ptr;
    g.ldr = nout;
    g.res_f32 = dt == DI_F32;
  }
  g.a = x->ptr;
  g.lda = K;
  g.b = w->ptr;
  g.ldb = K;
  g.M = M;
  g.N = N;
  g.K = K;
  g.bias = b;
  g.act = act;
  g.c = y->ptr;
  g.ldc = nout;
  g.c_f32 = dt == DI_F32;
  const uint32_t kv = dt == DI_F32 ? 4 : 8;
  g.a_vec_ok = g.b_vec_ok = K % kv == 0;
  g.a_bytes = gemm_extent((uint64_t)M * K * es);
  g.b_bytes = gemm_extent((uint64_t)N * K * es);
  return run_gemm(ctx, g, dt, A_DENSE, B_NK);
}

int32_t di_conv2d(di_ctx* ctx, di_handle X, di_handle Wt, di_handle bias, di_handle R, di_handle Y,
                  uint32_t N, uint32_t Cin, uint32_t Cout, uint32_t H, uint32_t W, uint32_t K,
                  uint32_t S, uint32_t pad, int32_t flags, int32_t dtype, int32_t layout) {
  DI_CTX(ctx);
  DI_DTYPE_W16(dtype);
  const Dts d = contraction_dts(dtype);
  const int dt = d.act;
  DI_REQUIRE(!d.w16 || layout == DI_NCHW, DI_EUNSUPPORTED,
             "di_conv2d: DI_F32W16 is for the NCHW fp32 path");
  DI_REQUIRE(N && Cin && Cout && H && W && K && S, DI_EINVAL, "di_conv2d: zero dimension");
  DI_REQUIRE((flags & ~(DI_CONV_F16_COMPUTE | DI_CONV_UPSAMPLE2X | DI_CONV_SILU)) == 0, DI_EINVAL,
             "di_conv2d: unknown flags 0x%x", flags);
  const uint32_t up = (flags & DI_CONV_UPSAMPLE2X) ? 2 : 1;
  const uint32_t Hi = H * up, Wi = W * up;
  DI_REQUIRE(Hi + 2 * pad >= K && Wi + 2 * pad >= K, DI_EINVAL,
             "di_conv2d: kernel %u larger than padded input %ux%u", K, Hi, Wi);
  const uint32_t Ho = (Hi + 2 * pad - K) / S + 1, Wo = (Wi + 2 * pad - K) / S + 1;
  const size_t es = dtype_size(dt);
  const uint64_t nx = (uint64_t)N * Cin * H * W, ny = (uint64_t)N * Cout * Ho * Wo;
  DI_BUF(ctx, X, x, nx * es);
  DI_BUF(ctx, Wt, w, (uint64_t)Cout * Cin * K * K * d.esb);
  DI_BUF(ctx, Y, y, ny * es);
  const float* b = nullptr;
  int rc = opt_f32(ctx, bias, Cout, &b);
  if (rc) return rc;
  const void* res = nullptr;
  if (R) {
    DI_BUF(ctx, R, r, ny * es);
    res = r->ptr;
  }
  GemmArgs g;
  g.H = H;
  g.W = W;
  g.Ho = Ho;
  g.Wo = Wo;
  g.ks = K;
  g.stride = S;
  g.pad = pad;
  g.up = up;
  g.M = N * Ho * Wo;
  g.N = Cout;
  g.bias = b;
  g.res = res;
  g.res_f32 = dt == DI_F32;
  if (flags & DI_CONV_SILU) g.act = ACT_SILU;  // silu(conv + bias) [+ R]

  if (layout == DI_NHWC) {
    DI_REQUIRE(dt == DI_F16, DI_EUNSUPPORTED, "di_conv2d: NHWC path is fp16 (OHWI weights)");
    DI_REQUIRE(Cin % 8 == 0, DI_EUNSUPPORTED, "di_conv2d: NHWC needs Cin %% 8 == 0 (got %u)", Cin);
    DI_REQUIRE(!(flags & DI_CONV_F16_COMPUTE), DI_EINVAL, "di_conv2d: F16_COMPUTE is for NCHW fp32");
    g.a = x->ptr;
    g.lda = Cin;
    g.Cin = Cin;
    g.K = Cin * K * K;
    g.b = w->ptr;
    g.ldb = g.K;
    g.c = y->ptr;
    g.ldc = Cout;
    g.ldr = Cout;
    g.a_bytes = gemm_extent(nx * 2);
    g.b_bytes = gemm_extent((uint64_t)Cout * g.K * 2);
    return run_gemm(ctx, g, DI_F16, A_CONV_NHWC, B_NK);
  }
  DI_REQUIRE(layout == DI_NCHW, DI_EINVAL, "di_conv2d: bad layout %d", layout);
  g.c = y->ptr;
  g.c_f32 = dt == DI_F32;
  g.c_nchw = 1;
  g.c_hw = Ho * Wo;
  if (!(flags & DI_CONV_F16_COMPUTE)) {
    // Reference k order (ci, ky, kx) straight on NCHW + OIHW, operand dtype.
    g.a = x->ptr;
    g.Cin = Cin;
    g.K = Cin * K * K;
    g.b = w->ptr;
    g.ldb = g.K;
    g.b_vec_ok = g.K % (dt == DI_F32 ? 4 : 8) == 0;
    g.b_f16 = d.w16;
    DI_REQUIRE(dt == DI_F32, DI_EUNSUPPORTED,
               "di_conv2d: NCHW fp16 needs DI_CONV_F16_COMPUTE or the NHWC layout");
    return run_gemm(ctx, g, DI_F32, A_CONV_NCHW, B_NK);
  }
  // fp16 MFMA on NCHW tensors: stage x as NHWC fp16 (channels padded to 8)
  // and the weights as OHWI fp16, then run the NHWC implicit GEMM with an
  // NCHW store.
  const uint32_t Cp = (Cin + 7) / 8 * 8;
  Tmp tx(ctx), tw(ctx);
  rc = tx.alloc((uint64_t)N * Cp * H * W * 2);
  if (rc) return rc;
  rc = tw.alloc((uint64_t)Cout * K * K * Cp * 2);
  if (rc) return rc;
  launch_layout(ctx->stream, x->ptr, dt, DI_NCHW, tx.p, DI_F16, DI_NHWC, N, Cin, H, W, Cp);
  launch_repack_oihw_ohwi(ctx->stream, w->ptr, d.w16 ? DI_F16 : dt, tw.p, Cout, Cin, K, Cp);
  DI_LAUNCH_CHECK();
  g.a = tx.p;
  g.lda = Cp;
  g.Cin = Cp;
  g.K = Cp * K * K;
  g.b = tw.p;
  g.ldb = g.K;
  g.a_bytes = gemm_extent((uint64_t)N * Cp * H * W * 2);
  g.b_bytes = gemm_extent((uint64_t)Cout * g.K * 2);
  return run_gemm(ctx, g, DI_F16, A_CONV_NHWC, B_NK);
}

}  // extern "C"

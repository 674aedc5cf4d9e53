/*
 * drawinstant.h — C ABI of libdrawinstant_hip.so, the MI355X (gfx950) kernel
 * library behind draw-instant's SD-Turbo U-Net op / fused-block layer.
 *
 * Conventions (all entry points):
 *   - every function returns int32 status, DI_OK (0) on success; on failure a
 *     thread-local message is available from di_last_error();
 *   - device memory is owned by the library and named by opaque u64 handles
 *     (replaces GPUBuffer, reference wgsl-executor.js:45-55);
 *   - one context = one device + one in-order HIP stream; ops enqueue and
 *     return immediately, only di_download / di_sync / di_timer_ms block;
 *   - shapes travel as scalar arguments (the reference packs them in uniform
 *     buffers, e.g. GnCfg wgsl-ops.js:395, ConvMmCfg wgsl-ops.js:585-598);
 *   - all validation (shape, dtype, null/freed handle, C%G, buffer sizes) runs
 *     before any launch, so it is testable without a GPU.
 *
 * Each declaration cites the reference interface it replaces (file:line in
 * abgnydn/draw-instant).
 */
#ifndef DRAWINSTANT_H
#define DRAWINSTANT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct di_ctx di_ctx;
typedef uint64_t di_handle;

/* ---- status codes ---- */
#define DI_OK 0
#define DI_EINVAL 1       /* bad argument / shape */
#define DI_ENOMEM 2       /* allocation failed or DI_ALLOC_LIMIT exceeded */
#define DI_EHIP 3         /* HIP runtime error (async faults surface here) */
#define DI_EUNSUPPORTED 4 /* valid request this build does not implement */
#define DI_EHANDLE 5      /* null, unknown or freed handle */

/* ---- dtypes (per tensor argument unless stated) ---- */
#define DI_F32 0
#define DI_F16 1
/* di_matmul / di_gemm / di_conv2d (NCHW) only: fp32 activations, outputs and
 * biases with the B operand (the weights) stored in fp16 and widened exactly
 * to fp32 as it loads, so results equal DI_F32 on the widened weights while
 * the weights keep half the bytes (the executor's fp16-resident weights). */
#define DI_F32W16 2

/* ---- activation layouts ---- */
#define DI_NCHW 0 /* reference layout (wgsl-executor.js Tensor dims) */
#define DI_NHWC 1 /* channels-last: the library's native U-Net layout */

/* ---- unary ops: UNARY_EXPRS wgsl-ops.js:58-72 (+ tanh GELU of fused-block.js:68-75) ---- */
#define DI_UN_SIGMOID 0
#define DI_UN_SQRT 1
#define DI_UN_NEG 2
#define DI_UN_ABS 3
#define DI_UN_SIN 4
#define DI_UN_COS 5
#define DI_UN_EXP 6
#define DI_UN_LOG 7
#define DI_UN_SILU 8
#define DI_UN_GELU 9       /* erf GELU, erf by Abramowitz-Stegun 7.1.26 */
#define DI_UN_ERF 10
#define DI_UN_GELU_TANH 11 /* tanh-approximation GELU */

/* ---- binary ops: BINARY_EXPRS wgsl-ops.js:130-134 ---- */
#define DI_BIN_ADD 0
#define DI_BIN_SUB 1
#define DI_BIN_MUL 2
#define DI_BIN_DIV 3
#define DI_BIN_POW 4 /* sign-aware pow */
#define DI_BIN_MAX 5
#define DI_BIN_MIN 6

/* ---- epilogue activations of the contraction ops ---- */
#define DI_ACT_NONE 0
#define DI_ACT_GELU 1  /* erf GELU */
#define DI_ACT_GEGLU 2 /* h * GELU(gate); weight rows interleaved in 16-row groups */
#define DI_ACT_SILU 3
#define DI_ACT_GELU_TANH 4 /* tanh GELU of the FFN bench, fused-block.js:68-75 */

/* ---- conv flags ---- */
#define DI_CONV_F16_COMPUTE 1 /* NCHW fp32 tensors through the fp16 MFMA path */
#define DI_CONV_UPSAMPLE2X 2  /* convolve the 2x nearest-upsampled input */
#define DI_CONV_SILU 4        /* epilogue silu(conv + bias) before the residual:
                                 WGSL_CONV silu(sum) + residual, fused-conv.js:50-100 */

/* ---- attention tensor layouts ---- */
#define DI_ATTN_BSHD 0 /* [B, S, H, d]: fused-attn.js:69-70 */
#define DI_ATTN_BHSD 1 /* [B, H, S, d]: fused-cross-attn.js:51-52 */

/* ---- norm flags ---- */
#define DI_NORM_SILU 1 /* apply x/(1+exp(-x)) after the affine (fused-resnet.js:162) */

/* ======================= lifecycle ======================= */

/* Replaces navigator.gpu.requestAdapter/requestDevice (unet-wgsl.js:63-72). */
int32_t di_create(int32_t device, di_ctx** out);
int32_t di_destroy(di_ctx* ctx);
/* Thread-local message of the last failing call on this thread. */
const char* di_last_error(void);
/* Replaces device.queue.onSubmittedWorkDone (bench-timing.js:28); surfaces
 * asynchronous kernel faults (role of getUNetGpuFault, unet-wgsl.js:172-175). */
int32_t di_sync(di_ctx* ctx);
/* Compute-unit count, current shader clock (kHz) and HBM bytes of the device. */
int32_t di_device_info(di_ctx* ctx, int32_t* num_cus, int32_t* clock_khz,
                       uint64_t* hbm_bytes);

/* ======================= memory ======================= */

/* BufferPool.acquire (wgsl-executor.js:71-80): 4 KiB-bucketed reuse. */
int32_t di_alloc(di_ctx* ctx, uint64_t bytes, di_handle* out);
/* BufferPool.release (wgsl-executor.js:84-90). Stream-ordered: safe to call
 * right after enqueueing the last op that reads the buffer. */
int32_t di_free(di_ctx* ctx, di_handle h);
int32_t di_buffer_size(di_ctx* ctx, di_handle h, uint64_t* bytes);
/* BufferPool live/peak/allocs counters (wgsl-executor.js:67-69). */
int32_t di_pool_stats(di_ctx* ctx, uint64_t* live, uint64_t* peak,
                      uint64_t* allocs, uint64_t* reserved_bytes);
/* Kernel workspace of the context (split-K partials, GroupNorm partial sums):
 * current size, how many workspace allocations captured graphs still hold,
 * and how many of those growth has already replaced (kept alive until their
 * graph is dropped).  No reference counterpart: WebGPU has no captured
 * command graphs; this makes the graph/workspace lifetime observable. */
int32_t di_workspace_stats(di_ctx* ctx, uint64_t* bytes, uint32_t* pinned,
                           uint32_t* retired);
/* createStorage / queue.writeBuffer (wgsl-ops.js:1172-1180). */
int32_t di_upload(di_ctx* ctx, di_handle h, uint64_t offset, const void* src,
                  uint64_t bytes);
/* readBack (wgsl-ops.js:1195-1210): synchronous, the only implicit sync. */
int32_t di_download(di_ctx* ctx, di_handle h, uint64_t offset, void* dst,
                    uint64_t bytes);
/* encoder.copyBufferToBuffer (wgsl-executor.js:1412-1423 output snapshot). */
int32_t di_copy(di_ctx* ctx, di_handle dst, uint64_t dst_offset, di_handle src,
                uint64_t src_offset, uint64_t bytes);
/* f32<->f16 element conversion, RNE (replaces f16BytesToF32 wgsl-unet.js:23-47
 * and f32ToF16 unet.js:108-135). */
int32_t di_convert(di_ctx* ctx, di_handle src, int32_t src_dtype, di_handle dst,
                   int32_t dst_dtype, uint64_t n);
/* Activation layout/dtype change for [N,C,H,W] tensors (NCHW<->NHWC, f32<->f16).
 * No reference counterpart: the reference is NCHW f32 only. */
int32_t di_layout_convert(di_ctx* ctx, di_handle src, int32_t src_dtype,
                          int32_t src_layout, di_handle dst, int32_t dst_dtype,
                          int32_t dst_layout, uint32_t N, uint32_t C, uint32_t H,
                          uint32_t W);
/* Seeded N(mean, std) fill on device (SplitMix64 counter hash + Box-Muller).
 * Replaces the benches' Math.random fills (e.g. fused-resnet.js:278-283). */
int32_t di_fill_normal(di_ctx* ctx, di_handle h, int32_t dtype, uint64_t n,
                       uint64_t seed, float mean, float std);

/* ======================= timing ======================= */

/* hipEvent pair per slot on the context stream; used with the reference's
 * slope method (measurePair bench-timing.js:49-97). */
int32_t di_timer_begin(di_ctx* ctx, int32_t slot);
int32_t di_timer_end(di_ctx* ctx, int32_t slot);
int32_t di_timer_ms(di_ctx* ctx, int32_t slot, float* ms);

/* ======================= executor element-wise ops ======================= */
/* All tensors share `dtype`; n / numel count elements. */

/* unary(device, op) dispatch (wgsl-ops.js:110-126) for OPS.Sigmoid/Sqrt/Erf/
 * Abs/Neg/Silu/Sin/Cos (wgsl-executor.js:694-706, :790-794, :508-516). */
int32_t di_unary(di_ctx* ctx, int32_t op, di_handle X, di_handle Y, uint64_t n,
                 int32_t dtype);
/* binary(device, op) same-shape dispatch (wgsl-ops.js:241-252). */
int32_t di_binary(di_ctx* ctx, int32_t op, di_handle A, di_handle B, di_handle Y,
                  uint64_t n, int32_t dtype);
/* binaryBcast (wgsl-ops.js:156-201): rank<=4, per-operand element strides
 * (0 on broadcast dims), as filled by wgsl-executor.js:644-667. */
int32_t di_binary_bcast(di_ctx* ctx, int32_t op, di_handle A, di_handle B,
                        di_handle Y, uint32_t rank, const uint32_t* out_dim,
                        const uint32_t* a_stride, const uint32_t* b_stride,
                        uint64_t numel, int32_t dtype);
/* affineBcast (wgsl-ops.js:206-237): Y = A*gamma + beta, gamma/beta sharing
 * one stride vector (OPS.AffineBcast wgsl-executor.js:753-785). */
int32_t di_affine_bcast(di_ctx* ctx, di_handle A, di_handle gamma, di_handle beta,
                        di_handle Y, uint32_t rank, const uint32_t* out_dim,
                        const uint32_t* a_stride, const uint32_t* bc_stride,
                        uint64_t numel, int32_t dtype);
/* softmax over the last axis (wgsl-ops.js:266-295, OPS.Softmax
 * wgsl-executor.js:1027-1037). One wavefront per row. */
int32_t di_softmax(di_ctx* ctx, di_handle X, di_handle Y, uint32_t inner,
                   uint32_t rows, int32_t dtype);
/* reduceMean over the last axis (wgsl-ops.js:958-983). */
int32_t di_reduce_mean(di_ctx* ctx, di_handle X, di_handle Y, uint32_t inner,
                       uint32_t rows, int32_t dtype);
/* resizeNearest (wgsl-ops.js:921-955, OPS.Resize wgsl-executor.js:1095-1114):
 * planes = N*C, floor index mapping. */
int32_t di_resize_nearest(di_ctx* ctx, di_handle X, di_handle Y, uint32_t planes,
                          uint32_t Hin, uint32_t Win, uint32_t Hout, uint32_t Wout,
                          int32_t dtype);
/* transpose (wgsl-ops.js:993-1044, OPS.Transpose wgsl-executor.js:410-441). */
int32_t di_transpose(di_ctx* ctx, di_handle X, di_handle Y, uint32_t rank,
                     const uint32_t* out_dim, const uint32_t* in_stride,
                     const uint32_t* perm, uint64_t numel, int32_t dtype);
/* slice, step 1 (wgsl-ops.js:1092-1134, OPS.Slice wgsl-executor.js:313-368). */
int32_t di_slice(di_ctx* ctx, di_handle X, di_handle Y, uint32_t rank,
                 const uint32_t* out_dim, const uint32_t* in_stride,
                 const uint32_t* start, uint64_t numel, int32_t dtype);
/* concatCopy (wgsl-ops.js:1142-1170, OPS.Concat wgsl-executor.js:444-488). */
int32_t di_concat_copy(di_ctx* ctx, di_handle X, di_handle Y, uint32_t stripe_in,
                       uint32_t stripe_out, uint32_t offset_out, uint64_t numel,
                       int32_t dtype);
/* powScalar (wgsl-ops.js:1050-1083, OPS.Pow wgsl-executor.js:519-539). */
int32_t di_pow_scalar(di_ctx* ctx, di_handle X, di_handle Y, uint64_t n,
                      float exponent, int32_t dtype);

/* ======================= normalisation ======================= */

/* GroupNorm over each (n, g) block of cpg*HW elements, then per-channel
 * gamma/beta (fp32, length G*cpg); optional fused SiLU.
 * Replaces groupNorm (wgsl-ops.js:390-469) as dispatched by OPS.GroupNorm
 * (wgsl-executor.js:715-746), and with DI_NORM_SILU the fused GN+SiLU kernel
 * WGSL_FUSED_GN_SILU (fused-resnet.js:121-166).  Statistics follow the
 * reference: var = E[x^2] - E[x]^2 clamped at 0, rstd = 1/sqrt(var + eps).
 * X, Y: dtype, layout NCHW or NHWC; Y may not alias X. */
int32_t di_group_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta,
                      di_handle Y, uint32_t N, uint32_t G, uint32_t cpg,
                      uint32_t HW, float eps, int32_t flags, int32_t dtype,
                      int32_t layout);
/* di_group_norm that allocates nothing: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results as di_group_norm; the partial sums live in a 1 MiB
 * static device array per GPU (held until the process ends) instead of the
 * context workspace.  That covers every NCHW call (at most 65535 groups) and
 * NHWC calls up to a batch of 4096 at G = 32 (512 at G = 256); larger
 * requests fail with DI_EUNSUPPORTED.  Nothing in the array needs clearing:
 * every partial is written before it is read within the call.  Every call on one GPU shares the array: calls that
 * overlap on one GPU (two streams or contexts at once) race. */
int32_t di_group_norm_noalloc(di_ctx* ctx, di_handle X, di_handle gamma,
                              di_handle beta, di_handle Y, uint32_t N,
                              uint32_t G, uint32_t cpg, uint32_t HW, float eps,
                              int32_t flags, int32_t dtype, int32_t layout);
/* The fused-resnet.js GN+SiLU entry point (== di_group_norm with DI_NORM_SILU). */
int32_t di_gn_silu(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta,
                   di_handle Y, uint32_t N, uint32_t C, uint32_t G, uint32_t HW,
                   float eps, int32_t dtype, int32_t layout);
/* InstanceNormalization (wgsl-ops.js:307-372, OPS.InstanceNormalization
 * wgsl-executor.js:1011-1025): GroupNorm with G = C. The reference hard-codes
 * eps 1e-5; here eps is an argument. NCHW. */
int32_t di_instance_norm(di_ctx* ctx, di_handle X, di_handle gamma,
                         di_handle beta, di_handle Y, uint32_t N, uint32_t C,
                         uint32_t HW, float eps, int32_t dtype);
/* Row LayerNorm over the last dim (layerNorm wgsl-ops.js:772-812, WGSL_LN
 * fused-block-full.js:62-122); gamma/beta fp32 of length inner. */
int32_t di_layer_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta,
                      di_handle Y, uint32_t rows, uint32_t inner, float eps,
                      int32_t dtype);

/* ======================= contractions (MFMA) ======================= */
/* Per-channel parameters (bias) are fp32 buffers; 0 = absent. */

/* matmul (wgsl-ops.js:477-569, OPS.MatMul wgsl-executor.js:1040-1054):
 * Y[b] = A[b] (M x K) . B (K x N), B batched (offset b*K*N) iff b_batched.
 * fp32 uses fp32 MFMA (exact fp32 products), fp16 the fp16 MFMA. */
int32_t di_matmul(di_ctx* ctx, di_handle A, di_handle B, di_handle Y, uint32_t M,
                  uint32_t N, uint32_t K, uint32_t batch, int32_t b_batched,
                  int32_t dtype);
/* gemm (wgsl-ops.js:821-910, OPS.Gemm wgsl-executor.js:1057-1065):
 * Y = A . B (+transB) + C[col]; C fp32 (0 = none). */
int32_t di_gemm(di_ctx* ctx, di_handle A, di_handle B, di_handle C, di_handle Y,
                uint32_t M, uint32_t N, uint32_t K, int32_t trans_b, int32_t dtype);
/* Linear in torch layout with the fused epilogue of fused-block.js WGSL_MATMUL
 * (:54-115: GELU / residual hooks): Y = act(X[M,K] . W[N,K]^T + bias) + R.
 * DI_ACT_GEGLU writes N/2 columns: out[:, 16t+j] = h * GELU(g) with h, g the
 * results of weight rows 32t+j and 32t+16+j. */
int32_t di_linear(di_ctx* ctx, di_handle X, di_handle W, di_handle bias, di_handle R,
                  di_handle Y, uint32_t M, uint32_t N, uint32_t K, int32_t act,
                  int32_t dtype);
/* Conv2d, square kernel K, stride S, symmetric pad (convMM wgsl-ops.js:584-711,
 * OPS.Conv wgsl-executor.js:1068-1092; batch N >= 1, the reference computes
 * batch 0 only).  Optional residual R (same shape as Y) added after the bias
 * (fused-resnet.js WGSL_CONV :173-208 residual epilogue).
 *   layout DI_NCHW: X NCHW, W OIHW, dtype fp32 (exact fp32 MFMA), or with
 *                   DI_CONV_F16_COMPUTE fp16-in / fp32-acc MFMA;
 *   layout DI_NHWC: X NHWC fp16, W OHWI fp16 ([Cout][K][K][Cin]), Cin % 8 == 0.
 * DI_CONV_UPSAMPLE2X convolves the 2x nearest upsample of X (H, W are X's).
 * DI_CONV_SILU applies SiLU to conv + bias; R (if any) is added after it. */
int32_t di_conv2d(di_ctx* ctx, di_handle X, di_handle W, di_handle bias, di_handle R,
                  di_handle Y, uint32_t N, uint32_t Cin, uint32_t Cout, uint32_t H,
                  uint32_t Wd, uint32_t K, uint32_t S, uint32_t pad, int32_t flags,
                  int32_t dtype, int32_t layout);

/* ======================= attention ======================= */
/* Flash attention, head dim d = 64, online softmax (no score matrix).  scale
 * <= 0 selects 1/sqrt(d).  fp16 tensors run directly; fp32 tensors are staged
 * through fp16 MFMA operands (fp32 accumulation and output). */

/* softmax(Q K^T * scale) V over S keys: WGSL_FUSED_ATTN (fused-attn.js:199-307,
 * runAttnBench :364-476) and the executor's MatMul -> Softmax -> MatMul chain. */
int32_t di_attn_self(di_ctx* ctx, di_handle Q, di_handle K, di_handle V, di_handle O,
                     uint32_t B, uint32_t H, uint32_t S, uint32_t d, int32_t layout,
                     float scale, int32_t dtype);
/* Cross attention over Skv keys (e.g. 77 text tokens): WGSL_FUSED
 * (fused-cross-attn.js:112-173, runCrossAttnBench :220-318). */
int32_t di_attn_cross(di_ctx* ctx, di_handle Q, di_handle K, di_handle V, di_handle O,
                      uint32_t B, uint32_t H, uint32_t Sq, uint32_t Skv, uint32_t d,
                      int32_t layout, float scale, int32_t dtype);

/* ======================= timestep embedding ======================= */

/* fused-tembed.js (WGSL_SINEMB :28-44, WGSL_FUSED :73-130, runTEmbedBench
 * :175-267): emb = [cos(t f) || sin(t f)], f_i = exp(-ln(1e4) i / (emb_dim/2)),
 * Y = W2 SiLU(W1 emb + b1) + b2.  T: fp32 [B] timesteps; W1 [hid][emb_dim],
 * W2 [hid][hid] of dtype wdtype; biases and Y fp32.  B <= 8, dims <= 1280. */
int32_t di_tembed(di_ctx* ctx, di_handle T, di_handle W1, di_handle b1, di_handle W2,
                  di_handle b2, di_handle Y, uint32_t B, uint32_t emb_dim, uint32_t hid,
                  int32_t wdtype);

/* ======================= fused blocks ======================= */
/* NHWC fp16 activations; conv weights OHWI fp16; linear weights [out][in]
 * fp16; biases, norm affines and temb fp32.  0 = absent optional weight. */

typedef struct {
  di_handle norm1_gamma, norm1_beta; /* [Cin] */
  di_handle conv1_w, conv1_b;        /* [Cout][3][3][Cin], [Cout] */
  di_handle temb_w, temb_b;          /* [Cout][temb_dim], [Cout] (temb given) */
  di_handle norm2_gamma, norm2_beta; /* [Cout] */
  di_handle conv2_w, conv2_b;        /* [Cout][3][3][Cout], [Cout] */
  di_handle skip_w, skip_b;          /* [Cout][Cin] 1x1, [Cout] (Cin != Cout) */
} di_resnet_weights;

/* ResnetBlock2D: y = conv2(SiLU(GN2(conv1(SiLU(GN1(x))) + temb_proj(SiLU(temb)))))
 * + skip(x).  runResNetBench (fused-resnet.js:267-420: GN+SiLU -> conv -> GN+SiLU
 * -> conv + residual) extended with the temb add and 1x1 skip its header says it
 * omits (fused-resnet.js:9-12).  temb: fp32 [B][temb_dim] or 0. */
int32_t di_resnet_block(di_ctx* ctx, const di_resnet_weights* w, di_handle X,
                        di_handle temb, di_handle Y, uint32_t B, uint32_t Cin,
                        uint32_t Cout, uint32_t H, uint32_t Wd, uint32_t temb_dim,
                        uint32_t groups, float eps);

typedef struct {
  di_handle norm_gamma, norm_beta;     /* GroupNorm [C] */
  di_handle proj_in_w, proj_in_b;      /* [C][C], [C] */
  di_handle ln1_gamma, ln1_beta;       /* [C] */
  di_handle attn1_qkv_w;               /* [3C][C] = to_q ; to_k ; to_v */
  di_handle attn1_out_w, attn1_out_b;  /* [C][C], [C] */
  di_handle ln2_gamma, ln2_beta;
  di_handle attn2_q_w;                 /* [C][C] */
  di_handle attn2_kv_w;                /* [2C][cross_dim] = to_k ; to_v */
  di_handle attn2_out_w, attn2_out_b;
  di_handle ln3_gamma, ln3_beta;
  di_handle ff_in_w, ff_in_b;          /* GEGLU [8C][C] rows as [16 h | 16 gate] groups, [8C] */
  di_handle ff_out_w, ff_out_b;        /* [C][4C], [C] */
  di_handle proj_out_w, proj_out_b;    /* [C][C], [C] */
} di_transformer_weights;

/* Transformer2DModel with linear projection and one BasicTransformerBlock
 * (GN -> proj_in -> LN+self-attn -> LN+cross-attn -> LN+GEGLU FFN -> proj_out
 * + residual), heads = C/64.  The SD block that runBlockBench
 * (fused-block-full.js:456-686) approximates with LN/attn/GELU-FFN only.
 * X, Y: [B][H*W][C] fp16; context: [B][Sctx][cross_dim] fp16. */
int32_t di_transformer_block(di_ctx* ctx, const di_transformer_weights* w, di_handle X,
                             di_handle context, di_handle Y, uint32_t B, uint32_t C,
                             uint32_t H, uint32_t Wd, uint32_t Sctx, uint32_t cross_dim,
                             uint32_t groups, float gn_eps, float ln_eps);

/* FFN of runFFNBench (fused-block.js:219-342): Y = act(X W1^T + b1) W2^T + b2 + X
 * with act DI_ACT_GELU_TANH (the bench's GELU), DI_ACT_GELU or DI_ACT_GEGLU
 * (W1 then [2F][D]).  W1 [F][D], W2 [D][F] torch layout. */
int32_t di_ffn(di_ctx* ctx, di_handle X, di_handle W1, di_handle b1, di_handle W2,
               di_handle b2, di_handle Y, uint32_t rows, uint32_t D, uint32_t F,
               int32_t act, int32_t dtype);

/* ======================= SD2.1 / SD-Turbo U-Net ======================= */

typedef struct {
  uint32_t in_channels, out_channels; /* 4, 4 */
  uint32_t block_channels[4];         /* 320, 640, 1280, 1280 (multiples of 64) */
  uint32_t cross_attn[4];             /* 1, 1, 1, 0: CrossAttn{Down,Up}Block2D levels */
  uint32_t layers_per_block;          /* 2 */
  uint32_t cross_dim;                 /* 1024 */
  uint32_t time_dim;                  /* 1280 */
  uint32_t groups;                    /* 32 */
  float resnet_eps;                   /* 1e-5 */
  float transformer_gn_eps;           /* 1e-6 */
  float ln_eps;                       /* 1e-5 */
} di_unet_config;

typedef struct di_unet di_unet;

/* physical layout tags of di_unet_param_info */
#define DI_PARAM_VECTOR 0         /* [n] */
#define DI_PARAM_LINEAR 1         /* [out][in] */
#define DI_PARAM_CONV_OHWI 2      /* [Cout][K][K][Cin] */
#define DI_PARAM_LINEAR_STACKED 3 /* [k*out][in]: k linears stacked by rows */
#define DI_PARAM_GEGLU_ROWS 4     /* rows (or entries) in 32-groups [16 hidden | 16 gate] */

#define DI_UNET_GRAPH 1 /* capture the step in a HIP graph once, replay after */

int32_t di_unet_default_config(di_unet_config* cfg);
/* Build the model with seeded random weights (no checkpoint is available
 * offline); cfg = NULL selects SD2.1.  Replaces loadUNetWGSL (unet-wgsl.js:40-114). */
int32_t di_unet_create(di_ctx* ctx, const di_unet_config* cfg, uint64_t seed, di_unet** out);
int32_t di_unet_destroy(di_ctx* ctx, di_unet* unet);
int32_t di_unet_num_params(di_ctx* ctx, di_unet* unet, uint32_t* n_tensors,
                           uint64_t* n_elements);
int32_t di_unet_param_info(di_ctx* ctx, di_unet* unet, uint32_t index, char* name,
                           uint32_t name_cap, uint32_t* dims, uint32_t* ndims,
                           int32_t* dtype, int32_t* layout);
int32_t di_unet_param_download(di_ctx* ctx, di_unet* unet, uint32_t index, void* dst,
                               uint64_t bytes);
/* Load one tensor (WeightCache upload role, wgsl-unet.js:55-97). */
int32_t di_unet_param_upload(di_ctx* ctx, di_unet* unet, uint32_t index, const void* src,
                             uint64_t bytes);
/* One denoise step: unetForwardWGSL (unet-wgsl.js:145-195).  sample, out: fp32
 * [B][4][H][W] (NCHW); timesteps: fp32 [B]; context: fp32 [B][Sctx][cross_dim].
 * Enqueues only; flags DI_UNET_GRAPH replays a captured graph. */
int32_t di_unet_forward(di_ctx* ctx, di_unet* unet, di_handle sample, di_handle timesteps,
                        di_handle context, di_handle out, uint32_t B, uint32_t H,
                        uint32_t W, uint32_t Sctx, int32_t flags);

/* ======================= VAE decoder ======================= */

/* SD's AutoencoderKL decode path (post_quant_conv + Decoder): the model
 * vae-wgsl.js runs through the executor (vae_decoder/model.onnx,
 * vae-wgsl.js:28-140), here as one native object on NHWC fp16 activations. */
typedef struct {
  uint32_t latent_channels;   /* 4 */
  uint32_t out_channels;      /* 3 */
  uint32_t block_channels[4]; /* 128, 256, 512, 512 (encoder order; the decoder runs them reversed) */
  uint32_t layers_per_block;  /* 2: each decoder up block has layers_per_block + 1 ResNets */
  uint32_t groups;            /* 32 */
  float eps;                  /* 1e-6 (every GroupNorm) */
} di_vae_config;

typedef struct di_vae di_vae;

#define DI_VAE_GRAPH 1 /* capture the decode in a HIP graph once, replay after */

int32_t di_vae_default_config(di_vae_config* cfg);
/* Build the decoder with seeded random weights; cfg = NULL selects SD's.
 * Replaces loadVAEWGSL (vae-wgsl.js:28-72). */
int32_t di_vae_create(di_ctx* ctx, const di_vae_config* cfg, uint64_t seed, di_vae** out);
int32_t di_vae_destroy(di_ctx* ctx, di_vae* vae);
int32_t di_vae_num_params(di_ctx* ctx, di_vae* vae, uint32_t* n_tensors, uint64_t* n_elements);
/* Same layout tags as di_unet_param_info (convs OHWI fp16, conv_in's input
 * channels padded to 8, attention to_q/to_k/to_v stacked [3C][C] with a [3C]
 * bias; post_quant_conv fp32 [C][C]). */
int32_t di_vae_param_info(di_ctx* ctx, di_vae* vae, uint32_t index, char* name,
                          uint32_t name_cap, uint32_t* dims, uint32_t* ndims, int32_t* dtype,
                          int32_t* layout);
int32_t di_vae_param_download(di_ctx* ctx, di_vae* vae, uint32_t index, void* dst,
                              uint64_t bytes);
int32_t di_vae_param_upload(di_ctx* ctx, di_vae* vae, uint32_t index, const void* src,
                            uint64_t bytes);
/* vaeDecodeWGSL (vae-wgsl.js:94-140): latent fp32 [B][4][H][W] times `scale`
 * (the caller's 1 / 0.18215) -> image fp32 [B][3][8H][8W] (NCHW).  Enqueues
 * only; DI_VAE_GRAPH replays a captured graph. */
int32_t di_vae_decode(di_ctx* ctx, di_vae* vae, di_handle latent, di_handle image,
                      uint32_t B, uint32_t H, uint32_t W, float scale, int32_t flags);

/* ======================= Euler Discrete scheduler ======================= */
/* The per-element halves of makeEulerScheduler / sampleNoiseLatent
 * (scheduler.js:77-134) on the device; the schedule constants (timesteps,
 * sigmas) stay host scalars, as in the reference.  fp32 tensors of n
 * elements; each element is a double expression rounded once to fp32, as the
 * reference's Float32Array stores are. */

/* sampleNoiseLatent (scheduler.js:117-134): seeded LCG (s * 1664525 +
 * 1013904223, from (seed | 0) || 1) + Box-Muller pairs, times sigma
 * (initNoiseSigma); n = B * 4 * H * W. */
int32_t di_noise_latent(di_ctx* ctx, di_handle out, uint64_t n, int32_t seed, double sigma);
/* scaleModelInput (scheduler.js:95-101): out = latent * inv, inv =
 * 1 / sqrt(sigma_i^2 + 1). */
int32_t di_euler_scale(di_ctx* ctx, di_handle latent, di_handle out, uint64_t n, double inv);
/* step (scheduler.js:105-110): out = latent + dt * pred, dt = sigma_{i+1} -
 * sigma_i; out may be latent.  next_in != 0 also writes the next step's
 * scaleModelInput of out with inv_next (fused: one pass per step). */
int32_t di_euler_step(di_ctx* ctx, di_handle latent, di_handle pred, di_handle out,
                      di_handle next_in, uint64_t n, double dt, double inv_next);

#ifdef __cplusplus
}
#endif

#endif /* DRAWINSTANT_H */

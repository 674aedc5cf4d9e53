/*
 * oracle.c — CPU restatement of the draw-instant WGSL kernels on the SD-Turbo
 * U-Net op / fused-block path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library (libdrawinstant_hip.so) and the "port" CPU baseline of bench.py; it
 * is never linked into, loaded by, or called from the product path.
 *
 * Conventions: fp32 tensors in and out, fp64 accumulation, the reference's
 * own formulas and index maths (each function cites the WGSL it restates).
 * Built a second time with -DOR_ACC=float (liboracle_f32.so): the same loops
 * accumulating in fp32, the reference kernels' own precision, which
 * bench.py times as the CPU baseline; the checker is always the fp64 build.
 * Layouts are the reference's: activations NCHW, conv weights OIHW, linear
 * weights as each reference kernel reads them.  Parallel over outer loops with
 * OpenMP; the thread count used is reported by or_threads().
 *
 * Parity pinning of every function is done by tests/test_oracle.py (closed-
 * form KATs from wgsl-ops-test.js, library routines, invariants).
 */
#include <tgmath.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* accumulation / intermediate type (see the header comment) */
#ifndef OR_ACC
#define OR_ACC double
#endif
typedef OR_ACC acc_t;

int or_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------- activations (wgsl-ops.js:58-81) ---------------- */

/* Abramowitz & Stegun 7.1.26, wgsl-ops.js:77-81 / wgsl-executor.js:687-691. */
static acc_t erf_as(acc_t x) {
  acc_t a = fabs(x);
  acc_t t = 1.0 / (1.0 + 0.3275911 * a);
  acc_t y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t -
                     0.284496736) * t + 0.254829592) * t * exp(-a * a);
  return x >= 0.0 ? y : -y;
}
static acc_t silu(acc_t x) { return x / (1.0 + exp(-x)); }                    /* :68 */
static acc_t gelu_erf(acc_t x) { return x * 0.5 * (1.0 + erf_as(x * 0.70710678)); } /* :70 */
/* fused-block.js:68-75 tanh approximation */
static acc_t gelu_tanh(acc_t x) {
  return 0.5 * x * (1.0 + tanh(0.7978845608 * (x + 0.044715 * x * x * x)));
}

/* op codes match include/drawinstant.h DI_UN_* */
static acc_t unary_op(int op, acc_t x) {
  switch (op) {
    case 0: return 1.0 / (1.0 + exp(-x));       /* Sigmoid */
    case 1: return sqrt(x > 0.0 ? x : 0.0);     /* Sqrt */
    case 2: return -x;                           /* Neg */
    case 3: return fabs(x);                      /* Abs */
    case 4: return sin(x);
    case 5: return cos(x);
    case 6: return exp(x);
    case 7: return log(x > 1e-12 ? x : 1e-12);   /* Log */
    case 8: return silu(x);
    case 9: return gelu_erf(x);
    case 10: return erf_as(x);
    case 11: return gelu_tanh(x);
  }
  return x;
}

void or_unary(int op, const float* x, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) y[i] = (float)unary_op(op, x[i]);
}

/* BINARY_EXPRS wgsl-ops.js:130-134, DI_BIN_* codes. */
static acc_t binary_op(int op, acc_t a, acc_t b) {
  switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    case 4: {
      acc_t r = pow(fabs(a), b);
      int neg = a < 0.0 && (b - floor(b)) == 0.0 && (((int)b) & 1) == 1;
      return neg ? -r : r;
    }
    case 5: return a > b ? a : b;
    case 6: return a < b ? a : b;
  }
  return a;
}

void or_binary(int op, const float* a, const float* b, float* y, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) y[i] = (float)binary_op(op, a[i], b[i]);
}

/* WGSL_BINARY_BCAST wgsl-ops.js:156-188: rank<=4 stride broadcast. */
void or_binary_bcast(int op, const float* a, const float* b, float* y, int rank,
                     const uint32_t* dim, const uint32_t* as, const uint32_t* bs,
                     int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    int64_t rem = i;
    uint32_t idx[4] = {0, 0, 0, 0};
    for (int d = rank - 1; d >= 1; d--) {
      idx[d] = (uint32_t)(rem % dim[d]);
      rem /= dim[d];
    }
    idx[0] = (uint32_t)rem;
    int64_t ao = 0, bo = 0;
    for (int d = 0; d < rank; d++) {
      ao += (int64_t)idx[d] * as[d];
      bo += (int64_t)idx[d] * bs[d];
    }
    y[i] = (float)binary_op(op, a[ao], b[bo]);
  }
}

/* powScalar wgsl-ops.js:1058-1071. */
void or_pow_scalar(const float* x, float* y, int64_t n, float e) {
  acc_t ei = floor(e);
  int is_int = fabs(e - ei) < 1e-6;
  for (int64_t i = 0; i < n; i++) {
    acc_t v = x[i];
    if (v < 0.0 && !is_int) y[i] = 0.0f;
    else {
      acc_t s = (v < 0.0 && (((int)ei) & 1) == 1) ? -1.0 : 1.0;
      y[i] = (float)(s * pow(fabs(v), e));
    }
  }
}

/* WGSL_SOFTMAX wgsl-ops.js:266-283 (max-subtract, exp, normalise). */
void or_softmax(const float* x, float* y, int64_t rows, int64_t inner) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * inner;
    acc_t m = -1e300, s = 0.0;
    for (int64_t j = 0; j < inner; j++) m = xr[j] > m ? xr[j] : m;
    for (int64_t j = 0; j < inner; j++) s += exp(xr[j] - m);
    for (int64_t j = 0; j < inner; j++) y[r * inner + j] = (float)(exp(xr[j] - m) / s);
  }
}

/* WGSL_REDUCE_MEAN wgsl-ops.js:958-972. */
void or_reduce_mean(const float* x, float* y, int64_t rows, int64_t inner) {
  for (int64_t r = 0; r < rows; r++) {
    acc_t s = 0.0;
    for (int64_t j = 0; j < inner; j++) s += x[r * inner + j];
    y[r] = (float)(s / (acc_t)inner);
  }
}

/* ---------------- normalisation ---------------- */

/* WGSL_GROUPNORM wgsl-ops.js:415-456 (+ SiLU epilogue of WGSL_FUSED_GN_SILU
 * fused-resnet.js:158-163).  NCHW; var = E[x^2]-E[x]^2 clamped at 0. */
void or_group_norm(const float* x, const float* gamma, const float* beta, float* y,
                   int64_t N, int64_t G, int64_t cpg, int64_t HW, float eps, int silu_on) {
  const int64_t L = cpg * HW;
#pragma omp parallel for schedule(static)
  for (int64_t ng = 0; ng < N * G; ng++) {
    const float* xg = x + ng * L;
    acc_t s = 0.0, q = 0.0;
    for (int64_t i = 0; i < L; i++) {
      s += xg[i];
      q += (acc_t)xg[i] * xg[i];
    }
    acc_t mean = s / (acc_t)L;
    acc_t var = q / (acc_t)L - mean * mean;
    if (var < 0.0) var = 0.0;
    acc_t rstd = 1.0 / sqrt(var + (acc_t)eps);
    int64_t g = ng % G;
    for (int64_t i = 0; i < L; i++) {
      int64_t c = g * cpg + i / HW;
      acc_t t = ((acc_t)xg[i] - mean) * rstd * gamma[c] + beta[c];
      y[ng * L + i] = (float)(silu_on ? silu(t) : t);
    }
  }
}

/* WGSL_LAYERNORM wgsl-ops.js:772-801 (eps as argument). */
void or_layer_norm(const float* x, const float* gamma, const float* beta, float* y,
                   int64_t rows, int64_t inner, float eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * inner;
    acc_t s = 0.0, q = 0.0;
    for (int64_t i = 0; i < inner; i++) {
      s += xr[i];
      q += (acc_t)xr[i] * xr[i];
    }
    acc_t mean = s / (acc_t)inner;
    acc_t var = q / (acc_t)inner - mean * mean;
    if (var < 0.0) var = 0.0;
    acc_t rstd = 1.0 / sqrt(var + (acc_t)eps);
    for (int64_t i = 0; i < inner; i++)
      y[r * inner + i] = (float)(((acc_t)xr[i] - mean) * rstd * gamma[i] + beta[i]);
  }
}

/* ---------------- contractions ---------------- */

/* WGSL_CONV_MM wgsl-ops.js:584-698: Y[n,oc,p] = bias[oc] + sum_k
 * W[oc, ci*K*K+ky*K+kx] * X[n, ci, oy*S+ky-PAD, ox*S+kx-PAD] (zero outside).
 * The reference computes batch 0 only (wgsl-executor.js:1082); this loops n. */
void or_conv2d(const float* x, const float* w, const float* bias, float* y, int64_t N,
               int64_t Cin, int64_t Cout, int64_t H, int64_t W, int64_t K, int64_t S,
               int64_t PAD) {
  const int64_t Ho = (H + 2 * PAD - K) / S + 1, Wo = (W + 2 * PAD - K) / S + 1;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t n = 0; n < N; n++) {
    for (int64_t oc = 0; oc < Cout; oc++) {
      acc_t* acc = (acc_t*)malloc(sizeof(acc_t) * Ho * Wo);
      for (int64_t p = 0; p < Ho * Wo; p++) acc[p] = bias ? bias[oc] : 0.0;
      for (int64_t ci = 0; ci < Cin; ci++) {
        const float* xc = x + (n * Cin + ci) * H * W;
        for (int64_t ky = 0; ky < K; ky++) {
          for (int64_t kx = 0; kx < K; kx++) {
            acc_t wv = w[((oc * Cin + ci) * K + ky) * K + kx];
            for (int64_t oy = 0; oy < Ho; oy++) {
              int64_t iy = oy * S + ky - PAD;
              if (iy < 0 || iy >= H) continue;
              acc_t* ar = acc + oy * Wo;
              const float* xr = xc + iy * W;
              for (int64_t ox = 0; ox < Wo; ox++) {
                int64_t ix = ox * S + kx - PAD;
                if (ix >= 0 && ix < W) ar[ox] += wv * xr[ix];
              }
            }
          }
        }
      }
      for (int64_t p = 0; p < Ho * Wo; p++) y[(n * Cout + oc) * Ho * Wo + p] = (float)acc[p];
      free(acc);
    }
  }
}

/* WGSL_MATMUL wgsl-ops.js:477-556: Y[b] = A[b] (MxK) . B (KxN), B batched
 * (offset b*K*N) iff b_batched (cfg.w), else shared. */
void or_matmul(const float* a, const float* b, float* y, int64_t M, int64_t N, int64_t K,
               int64_t batch, int b_batched) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t bz = 0; bz < batch; bz++) {
    for (int64_t r = 0; r < M; r++) {
      const float* ar = a + (bz * M + r) * K;
      const float* bb = b + (b_batched ? bz * K * N : 0);
      acc_t* acc = (acc_t*)calloc(N, sizeof(acc_t));
      for (int64_t k = 0; k < K; k++) {
        acc_t av = ar[k];
        const float* br = bb + k * N;
        for (int64_t c = 0; c < N; c++) acc[c] += av * br[c];
      }
      for (int64_t c = 0; c < N; c++) y[(bz * M + r) * N + c] = (float)acc[c];
      free(acc);
    }
  }
}

/* WGSL_GEMM wgsl-ops.js:821-897: Y = A . B (+transB) + C[col]. */
void or_gemm(const float* a, const float* b, const float* c, float* y, int64_t M, int64_t N,
             int64_t K, int trans_b) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < M; r++) {
    for (int64_t col = 0; col < N; col++) {
      acc_t s = 0.0;
      for (int64_t k = 0; k < K; k++)
        s += (acc_t)a[r * K + k] * (trans_b ? b[col * K + k] : b[k * N + col]);
      y[r * N + col] = (float)(s + (c ? c[col] : 0.0));
    }
  }
}

/* Linear layer in torch layout: Y[m, n] = sum_k X[m, k] W[n, k] + bias[n].
 * (Gemm with transB=1, wgsl-ops.js:875-877.) */
void or_linear(const float* x, const float* w, const float* bias, float* y, int64_t M,
               int64_t N, int64_t K) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < M; r++) {
    const float* xr = x + r * K;
    for (int64_t n = 0; n < N; n++) {
      const float* wr = w + n * K;
      acc_t s = 0.0;
      for (int64_t k = 0; k < K; k++) s += (acc_t)xr[k] * wr[k];
      y[r * N + n] = (float)(s + (bias ? bias[n] : 0.0));
    }
  }
}

/* Attention softmax(Q K^T * scale) V per (b, h, query row), the maths of
 * WGSL_FUSED_ATTN fused-attn.js:199-307 ([B,S,H,d] layout, strides given) and
 * WGSL_FUSED fused-cross-attn.js:112-173 ([B,H,S,d]).  Row/stride arguments
 * make both layouts (and strided token-major views) expressible:
 *   Q[b, h, i, :] at q + b*q_bs + h*q_hs + i*q_rs  (same for K, V, O). */
void or_attention(const float* q, const float* k, const float* v, float* o, int64_t B,
                  int64_t H, int64_t Sq, int64_t Skv, int64_t d, double scale,
                  int64_t q_bs, int64_t q_hs, int64_t q_rs, int64_t k_bs, int64_t k_hs,
                  int64_t k_rs, int64_t v_bs, int64_t v_hs, int64_t v_rs, int64_t o_bs,
                  int64_t o_hs, int64_t o_rs) {
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t bh = 0; bh < B * H; bh++) {
    for (int64_t i = 0; i < Sq; i++) {
      int64_t b = bh / H, h = bh % H;
      const float* qi = q + b * q_bs + h * q_hs + i * q_rs;
      acc_t* sc = (acc_t*)malloc(sizeof(acc_t) * Skv);
      acc_t m = -1e300;
      for (int64_t j = 0; j < Skv; j++) {
        const float* kj = k + b * k_bs + h * k_hs + j * k_rs;
        acc_t s = 0.0;
        for (int64_t t = 0; t < d; t++) s += (acc_t)qi[t] * kj[t];
        sc[j] = s * scale;
        if (sc[j] > m) m = sc[j];
      }
      acc_t z = 0.0;
      for (int64_t j = 0; j < Skv; j++) {
        sc[j] = exp(sc[j] - m);
        z += sc[j];
      }
      float* oi = o + b * o_bs + h * o_hs + i * o_rs;
      acc_t* acc = (acc_t*)calloc(d, sizeof(acc_t));
      for (int64_t j = 0; j < Skv; j++) {
        const float* vj = v + b * v_bs + h * v_hs + j * v_rs;
        for (int64_t t = 0; t < d; t++) acc[t] += sc[j] * vj[t];
      }
      for (int64_t t = 0; t < d; t++) oi[t] = (float)(acc[t] / z);
      free(acc);
      free(sc);
    }
  }
}

/* Timestep embedding, fused-tembed.js:28-44 and :73-130:
 *   freq_i = exp(-ln(1e4) * i / half), emb = [cos(t f) || sin(t f)],
 *   h = SiLU(W1 emb + b1), y = W2 h + b2 with W as [out, in]. */
void or_tembed(float t, const float* w1, const float* b1, const float* w2, const float* b2,
               float* y, int64_t emb_dim, int64_t hid) {
  int64_t half = emb_dim / 2;
  acc_t* e = (acc_t*)malloc(sizeof(acc_t) * emb_dim);
  acc_t* h = (acc_t*)malloc(sizeof(acc_t) * hid);
  for (int64_t i = 0; i < emb_dim; i++) {
    int64_t fi = i < half ? i : i - half;
    acc_t freq = exp(-log(10000.0) * (acc_t)fi / (acc_t)half);
    acc_t arg = (acc_t)t * freq;
    e[i] = i < half ? cos(arg) : sin(arg);
  }
  for (int64_t o = 0; o < hid; o++) {
    acc_t s = b1[o];
    for (int64_t k = 0; k < emb_dim; k++) s += e[k] * w1[o * emb_dim + k];
    h[o] = silu(s);
  }
  for (int64_t o = 0; o < hid; o++) {
    acc_t s = b2[o];
    for (int64_t k = 0; k < hid; k++) s += h[k] * w2[o * hid + k];
    y[o] = (float)s;
  }
  free(e);
  free(h);
}

/* Nearest resize, WGSL_RESIZE_NEAREST wgsl-ops.js:934-942 (floor mapping). */
void or_resize_nearest(const float* x, float* y, int64_t planes, int64_t Hin, int64_t Win,
                       int64_t Hout, int64_t Wout) {
  for (int64_t c = 0; c < planes; c++)
    for (int64_t oy = 0; oy < Hout; oy++)
      for (int64_t ox = 0; ox < Wout; ox++)
        y[(c * Hout + oy) * Wout + ox] =
            x[(c * Hin + (oy * Hin) / Hout) * Win + (ox * Win) / Wout];
}

/* ---------------- seeded inputs ---------------- */

/* SplitMix64 element j of the stream seeded with s, Box-Muller in fp64, the
 * same generator as the library's di_fill_normal. */
static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t or_splitmix_at(uint64_t seed, uint64_t j) {
  return mix64(seed + (j + 1) * 0x9E3779B97F4A7C15ull);
}
void or_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < (n + 1) / 2; k++) {
    uint64_t a = or_splitmix_at(seed, 2 * k), b = or_splitmix_at(seed, 2 * k + 1);
    double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
    double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
    out[2 * k] = (float)(mean + std * (float)(r * cos(th)));
    if (2 * k + 1 < n) out[2 * k + 1] = (float)(mean + std * (float)(r * sin(th)));
  }
}

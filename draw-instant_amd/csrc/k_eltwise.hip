// Element-wise, layout, PRNG and small reduction kernels for gfx950, plus
// their C-ABI entry points.
//
// These serve the executor's generic ops (reference wgsl-ops.js: unary :74-126,
// binary :136-151/:241-252, binaryBcast :156-201, affineBcast :206-237,
// softmax :266-295, reduceMean :958-983, resizeNearest :921-955, transpose
// :993-1044, powScalar :1050-1083, slice :1092-1134, concatCopy :1142-1170)
// and the dtype / layout conversions the fp16 NHWC U-Net path needs.
// All are HBM-bound streaming kernels: one pass, coalesced, grid-stride.
#include "di_device.h"
#include "di_kernels.h"

namespace di {

namespace {

constexpr int kBlock = 256;

inline unsigned grid_for(uint64_t n, int per_thread = 1) {
  uint64_t b = (n + (uint64_t)kBlock * per_thread - 1) / ((uint64_t)kBlock * per_thread);
  if (b < 1) b = 1;
  if (b > 65535ull * 16) b = 65535ull * 16;  // grid-stride covers the rest
  return (unsigned)b;
}

// ---------------- conversions ----------------

template <typename S, typename D>
__global__ void k_convert(const S* __restrict__ src, D* __restrict__ dst, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = (D)(float)src[i];
}

// [N,C,HW] <-> [N,HW,C] tile transpose through LDS (64x64 tiles, 256 threads).
// dir 0: NCHW -> NHWC (dst channel stride C_dst >= C, padded channels zeroed)
// dir 1: NHWC -> NCHW
template <typename S, typename D, int DIR>
__global__ void k_layout(const S* __restrict__ src, D* __restrict__ dst, uint32_t C,
                         uint32_t HW, uint32_t C_dst) {
  __shared__ float tile[64][65];
  const uint32_t n = blockIdx.z;
  const uint32_t c0 = blockIdx.y * 64, p0 = blockIdx.x * 64;
  const uint32_t tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  if (DIR == 0) {
    const S* s = src + (uint64_t)n * C * HW;
    D* d = dst + (uint64_t)n * C_dst * HW;
    for (int r = ty; r < 64; r += 4) {
      uint32_t c = c0 + r, p = p0 + tx;
      tile[r][tx] = (c < C && p < HW) ? (float)s[(uint64_t)c * HW + p] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
      uint32_t p = p0 + r, c = c0 + tx;
      if (p < HW && c < C_dst) d[(uint64_t)p * C_dst + c] = (D)tile[tx][r];
    }
  } else {
    const S* s = src + (uint64_t)n * C * HW;
    D* d = dst + (uint64_t)n * C * HW;
    for (int r = ty; r < 64; r += 4) {
      uint32_t p = p0 + r, c = c0 + tx;
      tile[r][tx] = (c < C && p < HW) ? (float)s[(uint64_t)p * C + c] : 0.0f;
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
      uint32_t c = c0 + r, p = p0 + tx;
      if (p < HW && c < C) d[(uint64_t)c * HW + p] = (D)tile[tx][r];
    }
  }
}

// Seeded normal fill: pair k uses SplitMix64 elements 2k, 2k+1 -> Box-Muller
// in fp64 -> fp32 -> destination dtype (RNE).
template <typename D>
__global__ void k_fill_normal(D* __restrict__ dst, uint64_t n, uint64_t seed, float mean,
                              float std) {
  uint64_t pairs = (n + 1) / 2;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t k = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; k < pairs; k += stride) {
    uint64_t a = splitmix_at(seed, 2 * k), b = splitmix_at(seed, 2 * k + 1);
    double u1 = (double)((a >> 11) + 1) * (1.0 / 9007199254740992.0);  // (0,1]
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);        // [0,1)
    double r = sqrt(-2.0 * log(u1));
    double th = 6.283185307179586 * u2;
    float z0 = (float)(r * cos(th)), z1 = (float)(r * sin(th));
    dst[2 * k] = (D)(mean + std * z0);
    if (2 * k + 1 < n) dst[2 * k + 1] = (D)(mean + std * z1);
  }
}

template <typename D>
__global__ void k_fill_const(D* __restrict__ dst, uint64_t n, float v) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    dst[i] = (D)v;
}

// ---------------- executor element-wise ops ----------------

__device__ __forceinline__ float unary_op(int op, float x) {
  switch (op) {
    case DI_UN_SIGMOID: return 1.0f / (1.0f + __expf(-x));
    case DI_UN_SQRT: return sqrtf(fmaxf(x, 0.0f));
    case DI_UN_NEG: return -x;
    case DI_UN_ABS: return fabsf(x);
    case DI_UN_SIN: return sinf(x);
    case DI_UN_COS: return cosf(x);
    case DI_UN_EXP: return expf(x);
    case DI_UN_LOG: return logf(fmaxf(x, 1e-12f));
    case DI_UN_SILU: return silu_f(x);
    case DI_UN_GELU: return gelu_erf_f(x);
    case DI_UN_ERF: return erf_as(x);
    case DI_UN_GELU_TANH: return gelu_tanh_f(x);
  }
  return x;
}

// Sign-aware pow of BINARY_EXPRS.Pow (wgsl-ops.js:132).
__device__ __forceinline__ float pow_signed(float a, float b) {
  float r = powf(fabsf(a), b);
  bool neg = a < 0.0f && (b - floorf(b)) == 0.0f && (((int)b) & 1) == 1;
  return neg ? -r : r;
}

__device__ __forceinline__ float binary_op(int op, float a, float b) {
  switch (op) {
    case DI_BIN_ADD: return a + b;
    case DI_BIN_SUB: return a - b;
    case DI_BIN_MUL: return a * b;
    case DI_BIN_DIV: return a / b;
    case DI_BIN_POW: return pow_signed(a, b);
    case DI_BIN_MAX: return fmaxf(a, b);
    case DI_BIN_MIN: return fminf(a, b);
  }
  return a;
}

template <typename T>
__global__ void k_unary(int op, const T* __restrict__ x, T* __restrict__ y, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (T)unary_op(op, (float)x[i]);
}

template <typename T>
__global__ void k_binary(int op, const T* __restrict__ a, const T* __restrict__ b,
                         T* __restrict__ y, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = (T)binary_op(op, (float)a[i], (float)b[i]);
}

struct Idx4 {
  uint32_t rank;
  uint32_t dim[4];
  uint32_t s0[4];
  uint32_t s1[4];
};

// Decompose flat output index into rank<=4 coordinates (wgsl-ops.js:176-182).
__device__ __forceinline__ void unravel(const Idx4& c, uint64_t i, uint32_t idx[4]) {
  uint64_t rem = i;
  idx[0] = idx[1] = idx[2] = idx[3] = 0;
  if (c.rank >= 4) { idx[3] = rem % c.dim[3]; rem /= c.dim[3]; }
  if (c.rank >= 3) { idx[2] = rem % c.dim[2]; rem /= c.dim[2]; }
  if (c.rank >= 2) { idx[1] = rem % c.dim[1]; rem /= c.dim[1]; }
  idx[0] = (uint32_t)rem;
}

template <typename T>
__global__ void k_binary_bcast(int op, const T* __restrict__ a, const T* __restrict__ b,
                               T* __restrict__ y, Idx4 c, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t idx[4];
    unravel(c, i, idx);
    uint64_t ao = 0, bo = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      ao += (uint64_t)idx[d] * c.s0[d];
      bo += (uint64_t)idx[d] * c.s1[d];
    }
    y[i] = (T)binary_op(op, (float)a[ao], (float)b[bo]);
  }
}

template <typename T>
__global__ void k_affine_bcast(const T* __restrict__ a, const T* __restrict__ g,
                               const T* __restrict__ bt, T* __restrict__ y, Idx4 c,
                               uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t idx[4];
    unravel(c, i, idx);
    uint64_t ao = 0, bo = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      ao += (uint64_t)idx[d] * c.s0[d];
      bo += (uint64_t)idx[d] * c.s1[d];
    }
    y[i] = (T)((float)a[ao] * (float)g[bo] + (float)bt[bo]);
  }
}

// Transpose: s0 = input strides, s1 = perm (wgsl-ops.js:1019-1031).
template <typename T>
__global__ void k_transpose(const T* __restrict__ x, T* __restrict__ y, Idx4 c, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t o[4], in[4] = {0, 0, 0, 0};
    unravel(c, i, o);
    for (uint32_t d = 0; d < c.rank; d++) in[c.s1[d]] = o[d];
    uint64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) off += (uint64_t)in[d] * c.s0[d];
    y[i] = x[off];
  }
}

// Slice: s0 = input strides, s1 = start (wgsl-ops.js:1109-1122).
template <typename T>
__global__ void k_slice(const T* __restrict__ x, T* __restrict__ y, Idx4 c, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t o[4];
    unravel(c, i, o);
    uint64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; d++) off += (uint64_t)(c.s1[d] + o[d]) * c.s0[d];
    y[i] = x[off];
  }
}

// Striped concat copy (wgsl-ops.js:1142-1157).
template <typename T>
__global__ void k_concat(const T* __restrict__ x, T* __restrict__ y, uint32_t stripe_in,
                         uint32_t stripe_out, uint32_t offset_out, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t row = i / stripe_in, col = i % stripe_in;
    y[row * stripe_out + offset_out + col] = x[i];
  }
}

// Nearest resize with floor index mapping (wgsl-ops.js:934-942).
template <typename T>
__global__ void k_resize(const T* __restrict__ x, T* __restrict__ y, uint32_t Hin,
                         uint32_t Win, uint32_t Hout, uint32_t Wout, uint64_t n) {
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t ox = i % Wout;
    uint64_t t = i / Wout;
    uint32_t oy = t % Hout;
    uint64_t oc = t / Hout;
    uint32_t ix = (uint32_t)(((uint64_t)ox * Win) / Wout);
    uint32_t iy = (uint32_t)(((uint64_t)oy * Hin) / Hout);
    y[i] = x[(oc * Hin + iy) * Win + ix];
  }
}

// powScalar (wgsl-ops.js:1058-1071): x<0 with non-integer e gives 0.
template <typename T>
__global__ void k_pow_scalar(const T* __restrict__ x, T* __restrict__ y, float e, uint64_t n) {
  float ei = floorf(e);
  bool is_int = fabsf(e - ei) < 1e-6f;
  bool odd = is_int && ((((int)ei) & 1) == 1);
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    float v = (float)x[i];
    float r;
    if (v < 0.0f && !is_int) r = 0.0f;
    else r = ((v < 0.0f && odd) ? -1.0f : 1.0f) * powf(fabsf(v), e);
    y[i] = (T)r;
  }
}

// Row softmax, one wavefront per row (replaces one-thread-per-row
// WGSL_SOFTMAX wgsl-ops.js:266-283; same max-subtract formula).
template <typename T>
__global__ void k_softmax(const T* __restrict__ x, T* __restrict__ y, uint32_t inner,
                          uint32_t rows) {
  uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const T* xr = x + (uint64_t)row * inner;
  T* yr = y + (uint64_t)row * inner;
  float m = -3.0e38f;
  for (uint32_t j = lane; j < inner; j += kWave) m = fmaxf(m, (float)xr[j]);
  m = wave_max(m);
  float s = 0.0f;
  for (uint32_t j = lane; j < inner; j += kWave) s += __expf((float)xr[j] - m);
  s = wave_sum(s);
  float inv = 1.0f / s;
  for (uint32_t j = lane; j < inner; j += kWave) yr[j] = (T)(__expf((float)xr[j] - m) * inv);
}

// fp16 rows of inner = 512 * NV elements (NV <= 8): one wavefront per row
// holding the row in registers (NV 16-byte vectors per lane), so the row is
// read once and written once.
template <int NV>
__global__ __launch_bounds__(256) void k_softmax_f16_reg(const f16* __restrict__ x,
                                                         f16* __restrict__ y, uint32_t rows) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  if (row >= rows) return;
  constexpr uint32_t inner = 512 * NV;
  const f16* xr = x + (uint64_t)row * inner;
  f16x8 v[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) v[i] = *(const f16x8*)(xr + (i * kWave + lane) * 8);
  float m = -3.0e38f;
#pragma unroll
  for (int i = 0; i < NV; i++)
#pragma unroll
    for (int e = 0; e < 8; e++) m = fmaxf(m, (float)v[i][e]);
  m = wave_max(m);
  float ex[NV][8], s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; i++)
#pragma unroll
    for (int e = 0; e < 8; e++) {
      ex[i][e] = __expf((float)v[i][e] - m);
      s += ex[i][e];
    }
  s = wave_sum(s);
  const float inv = 1.0f / s;
  f16* yr = y + (uint64_t)row * inner;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = (f16)(ex[i][e] * inv);
    *(f16x8*)(yr + (i * kWave + lane) * 8) = o;
  }
}

template <typename T>
__global__ void k_reduce_mean(const T* __restrict__ x, T* __restrict__ y, uint32_t inner,
                              uint32_t rows) {
  uint32_t row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const T* xr = x + (uint64_t)row * inner;
  float s = 0.0f;
  for (uint32_t j = lane; j < inner; j += kWave) s += (float)xr[j];
  s = wave_sum(s);
  if (lane == 0) y[row] = (T)(s / (float)inner);
}

}  // namespace

// y = a + b over n fp32 values (derived parameters, e.g. summed biases)
__global__ void k_add_f32(const float* __restrict__ a, const float* __restrict__ b,
                          float* __restrict__ y, uint64_t n) {
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x)
    y[i] = a[i] + b[i];
}

void launch_convert(hipStream_t s, const void* src, int sdt, void* dst, int ddt, uint64_t n) {
  unsigned g = grid_for(n, 4);
  if (sdt == DI_F32 && ddt == DI_F16)
    k_convert<float, f16><<<g, kBlock, 0, s>>>((const float*)src, (f16*)dst, n);
  else if (sdt == DI_F16 && ddt == DI_F32)
    k_convert<f16, float><<<g, kBlock, 0, s>>>((const f16*)src, (float*)dst, n);
  else if (sdt == DI_F32)
    k_convert<float, float><<<g, kBlock, 0, s>>>((const float*)src, (float*)dst, n);
  else
    k_convert<f16, f16><<<g, kBlock, 0, s>>>((const f16*)src, (f16*)dst, n);
}

template <typename S, typename D>
static void layout_dispatch(hipStream_t s, const void* src, void* dst, int dir, uint32_t N,
                            uint32_t C, uint32_t HW, uint32_t C_dst) {
  uint32_t cspan = dir == 0 ? C_dst : C;
  dim3 grid((HW + 63) / 64, (cspan + 63) / 64, N);
  if (dir == 0)
    k_layout<S, D, 0><<<grid, 256, 0, s>>>((const S*)src, (D*)dst, C, HW, C_dst);
  else
    k_layout<S, D, 1><<<grid, 256, 0, s>>>((const S*)src, (D*)dst, C, HW, C);
}

void launch_layout(hipStream_t s, const void* src, int sdt, int slay, void* dst, int ddt,
                   int dlay, uint32_t N, uint32_t C, uint32_t H, uint32_t W,
                   uint32_t C_dst) {
  uint32_t HW = H * W;
  if (slay == dlay) {
    launch_convert(s, src, sdt, dst, ddt, (uint64_t)N * C * HW);
    return;
  }
  int dir = (slay == DI_NCHW) ? 0 : 1;
  if (sdt == DI_F32 && ddt == DI_F16) layout_dispatch<float, f16>(s, src, dst, dir, N, C, HW, C_dst);
  else if (sdt == DI_F16 && ddt == DI_F32) layout_dispatch<f16, float>(s, src, dst, dir, N, C, HW, C_dst);
  else if (sdt == DI_F32) layout_dispatch<float, float>(s, src, dst, dir, N, C, HW, C_dst);
  else layout_dispatch<f16, f16>(s, src, dst, dir, N, C, HW, C_dst);
}

void launch_fill_normal(hipStream_t s, void* dst, int dt, uint64_t n, uint64_t seed, float mean,
                        float std) {
  unsigned g = grid_for((n + 1) / 2);
  if (dt == DI_F32) k_fill_normal<float><<<g, kBlock, 0, s>>>((float*)dst, n, seed, mean, std);
  else k_fill_normal<f16><<<g, kBlock, 0, s>>>((f16*)dst, n, seed, mean, std);
}

void launch_fill_const(hipStream_t s, void* dst, int dt, uint64_t n, float v) {
  unsigned g = grid_for(n);
  if (dt == DI_F32) k_fill_const<float><<<g, kBlock, 0, s>>>((float*)dst, n, v);
  else k_fill_const<f16><<<g, kBlock, 0, s>>>((f16*)dst, n, v);
}

void launch_add_f32(hipStream_t s, const float* a, const float* b, float* y, uint64_t n) {
  k_add_f32<<<grid_for(n), kBlock, 0, s>>>(a, b, y, n);
}

}  // namespace di

using namespace di;

// ---------------- C ABI ----------------


namespace {

int fill_idx4(Idx4* c, uint32_t rank, const uint32_t* dim, const uint32_t* s0,
              const uint32_t* s1, const char* what) {
  DI_REQUIRE(rank >= 1 && rank <= 4, DI_EINVAL, "%s: rank %u outside [1,4]", what, rank);
  DI_REQUIRE(dim && s0 && s1, DI_EINVAL, "%s: null shape arrays", what);
  c->rank = rank;
  for (int d = 0; d < 4; d++) {
    c->dim[d] = d < (int)rank ? dim[d] : 1;
    c->s0[d] = d < (int)rank ? s0[d] : 0;
    c->s1[d] = d < (int)rank ? s1[d] : 0;
  }
  return DI_OK;
}

// Largest element offset a strided read can touch (for bounds validation).
uint64_t max_offset(const Idx4& c, const uint32_t* extra_start) {
  uint64_t off = 0;
  for (uint32_t d = 0; d < c.rank; d++)
    off += (uint64_t)((extra_start ? extra_start[d] : 0) + c.dim[d] - 1) * c.s0[d];
  return off;
}

}  // namespace

namespace di {

void launch_softmax(hipStream_t s, const void* x, void* y, uint32_t inner, uint32_t rows,
                    int dt) {
  if (rows == 0) return;
  const unsigned g = (rows + 3) / 4;
  const bool al16 = (((uintptr_t)x | (uintptr_t)y) & 15) == 0;
  if (dt == DI_F16 && al16 && inner % 512 == 0 && inner <= 4096) {
    const f16* xp = (const f16*)x;
    f16* yp = (f16*)y;
    switch (inner / 512) {
      case 1: k_softmax_f16_reg<1><<<g, 256, 0, s>>>(xp, yp, rows); return;
      case 2: k_softmax_f16_reg<2><<<g, 256, 0, s>>>(xp, yp, rows); return;
      case 4: k_softmax_f16_reg<4><<<g, 256, 0, s>>>(xp, yp, rows); return;
      case 8: k_softmax_f16_reg<8><<<g, 256, 0, s>>>(xp, yp, rows); return;
      default: break;
    }
  }
  if (dt == DI_F32) k_softmax<float><<<g, 256, 0, s>>>((const float*)x, (float*)y, inner, rows);
  else k_softmax<f16><<<g, 256, 0, s>>>((const f16*)x, (f16*)y, inner, rows);
}

void launch_transpose_f16(hipStream_t s, const f16* x, uint32_t ldx, uint32_t sx, f16* y,
                          uint32_t batch, uint32_t rows, uint32_t cols) {
  Idx4 c;
  const uint32_t dim[3] = {batch, cols, rows}, s0[3] = {sx, ldx, 1}, perm[3] = {0, 2, 1};
  (void)fill_idx4(&c, 3, dim, s0, perm, "launch_transpose_f16");
  const uint64_t n = (uint64_t)batch * rows * cols;
  if (n) k_transpose<f16><<<grid_for(n), kBlock, 0, s>>>(x, y, c, n);
}

}  // namespace di

extern "C" {

int32_t di_convert(di_ctx* ctx, di_handle src, int32_t sdt, di_handle dst, int32_t ddt,
                   uint64_t n) {
  DI_CTX(ctx);
  DI_DTYPE(sdt);
  DI_DTYPE(ddt);
  DI_BUF(ctx, src, s, n * dtype_size(sdt));
  DI_BUF(ctx, dst, d, n * dtype_size(ddt));
  if (n == 0) return DI_OK;
  launch_convert(ctx->stream, s->ptr, sdt, d->ptr, ddt, n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_layout_convert(di_ctx* ctx, di_handle src, int32_t sdt, int32_t slay, di_handle dst,
                          int32_t ddt, int32_t dlay, uint32_t N, uint32_t C, uint32_t H,
                          uint32_t W) {
  DI_CTX(ctx);
  DI_DTYPE(sdt);
  DI_DTYPE(ddt);
  DI_REQUIRE((slay == DI_NCHW || slay == DI_NHWC) && (dlay == DI_NCHW || dlay == DI_NHWC),
             DI_EINVAL, "di_layout_convert: bad layout %d -> %d", slay, dlay);
  DI_REQUIRE(N && C && H && W, DI_EINVAL, "di_layout_convert: zero dimension");
  uint64_t n = (uint64_t)N * C * H * W;
  DI_BUF(ctx, src, s, n * dtype_size(sdt));
  DI_BUF(ctx, dst, d, n * dtype_size(ddt));
  DI_REQUIRE(s->ptr != d->ptr || slay == dlay, DI_EINVAL,
             "di_layout_convert: in-place transpose not supported");
  launch_layout(ctx->stream, s->ptr, sdt, slay, d->ptr, ddt, dlay, N, C, H, W, C);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_fill_normal(di_ctx* ctx, di_handle h, int32_t dt, uint64_t n, uint64_t seed,
                       float mean, float std) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_BUF(ctx, h, b, n * dtype_size(dt));
  if (n == 0) return DI_OK;
  launch_fill_normal(ctx->stream, b->ptr, dt, n, seed, mean, std);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_unary(di_ctx* ctx, int32_t op, di_handle X, di_handle Y, uint64_t n, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(op >= DI_UN_SIGMOID && op <= DI_UN_GELU_TANH, DI_EINVAL, "unknown unary op %d", op);
  DI_BUF(ctx, X, x, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  if (n == 0) return DI_OK;
  unsigned g = grid_for(n, 4);
  if (dt == DI_F32) k_unary<float><<<g, kBlock, 0, ctx->stream>>>(op, (const float*)x->ptr, (float*)y->ptr, n);
  else k_unary<f16><<<g, kBlock, 0, ctx->stream>>>(op, (const f16*)x->ptr, (f16*)y->ptr, n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_binary(di_ctx* ctx, int32_t op, di_handle A, di_handle B, di_handle Y, uint64_t n,
                  int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(op >= DI_BIN_ADD && op <= DI_BIN_MIN, DI_EINVAL, "unknown binary op %d", op);
  DI_BUF(ctx, A, a, n * dtype_size(dt));
  DI_BUF(ctx, B, b, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  if (n == 0) return DI_OK;
  unsigned g = grid_for(n, 4);
  if (dt == DI_F32)
    k_binary<float><<<g, kBlock, 0, ctx->stream>>>(op, (const float*)a->ptr, (const float*)b->ptr, (float*)y->ptr, n);
  else
    k_binary<f16><<<g, kBlock, 0, ctx->stream>>>(op, (const f16*)a->ptr, (const f16*)b->ptr, (f16*)y->ptr, n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_binary_bcast(di_ctx* ctx, int32_t op, di_handle A, di_handle B, di_handle Y,
                        uint32_t rank, const uint32_t* out_dim, const uint32_t* a_stride,
                        const uint32_t* b_stride, uint64_t numel, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(op >= DI_BIN_ADD && op <= DI_BIN_MIN, DI_EINVAL, "unknown binary op %d", op);
  Idx4 c;
  int rc = fill_idx4(&c, rank, out_dim, a_stride, b_stride, "di_binary_bcast");
  if (rc) return rc;
  uint64_t prod = 1;
  for (uint32_t d = 0; d < rank; d++) prod *= out_dim[d];
  DI_REQUIRE(prod == numel, DI_EINVAL, "di_binary_bcast: numel %llu != prod(outDim) %llu",
             (unsigned long long)numel, (unsigned long long)prod);
  if (numel == 0) return DI_OK;
  Idx4 ca = c, cb = c;
  for (int d = 0; d < 4; d++) cb.s0[d] = c.s1[d];
  DI_BUF(ctx, A, a, (max_offset(ca, nullptr) + 1) * dtype_size(dt));
  DI_BUF(ctx, B, b, (max_offset(cb, nullptr) + 1) * dtype_size(dt));
  DI_BUF(ctx, Y, y, numel * dtype_size(dt));
  unsigned g = grid_for(numel);
  if (dt == DI_F32)
    k_binary_bcast<float><<<g, kBlock, 0, ctx->stream>>>(op, (const float*)a->ptr, (const float*)b->ptr, (float*)y->ptr, c, numel);
  else
    k_binary_bcast<f16><<<g, kBlock, 0, ctx->stream>>>(op, (const f16*)a->ptr, (const f16*)b->ptr, (f16*)y->ptr, c, numel);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_affine_bcast(di_ctx* ctx, di_handle A, di_handle gamma, di_handle beta, di_handle Y,
                        uint32_t rank, const uint32_t* out_dim, const uint32_t* a_stride,
                        const uint32_t* bc_stride, uint64_t numel, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  Idx4 c;
  int rc = fill_idx4(&c, rank, out_dim, a_stride, bc_stride, "di_affine_bcast");
  if (rc) return rc;
  uint64_t prod = 1;
  for (uint32_t d = 0; d < rank; d++) prod *= out_dim[d];
  DI_REQUIRE(prod == numel, DI_EINVAL, "di_affine_bcast: numel mismatch");
  if (numel == 0) return DI_OK;
  Idx4 cb = c;
  for (int d = 0; d < 4; d++) cb.s0[d] = c.s1[d];
  uint64_t bc_need = (max_offset(cb, nullptr) + 1) * dtype_size(dt);
  DI_BUF(ctx, A, a, (max_offset(c, nullptr) + 1) * dtype_size(dt));
  DI_BUF(ctx, gamma, g_, bc_need);
  DI_BUF(ctx, beta, b_, bc_need);
  DI_BUF(ctx, Y, y, numel * dtype_size(dt));
  unsigned g = grid_for(numel);
  if (dt == DI_F32)
    k_affine_bcast<float><<<g, kBlock, 0, ctx->stream>>>((const float*)a->ptr, (const float*)g_->ptr, (const float*)b_->ptr, (float*)y->ptr, c, numel);
  else
    k_affine_bcast<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)a->ptr, (const f16*)g_->ptr, (const f16*)b_->ptr, (f16*)y->ptr, c, numel);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_softmax(di_ctx* ctx, di_handle X, di_handle Y, uint32_t inner, uint32_t rows,
                   int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(inner > 0, DI_EINVAL, "di_softmax: inner length 0");
  uint64_t n = (uint64_t)inner * rows;
  DI_BUF(ctx, X, x, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  if (rows == 0) return DI_OK;
  launch_softmax(ctx->stream, x->ptr, y->ptr, inner, rows, dt);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_reduce_mean(di_ctx* ctx, di_handle X, di_handle Y, uint32_t inner, uint32_t rows,
                       int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(inner > 0, DI_EINVAL, "di_reduce_mean: inner length 0");
  DI_BUF(ctx, X, x, (uint64_t)inner * rows * dtype_size(dt));
  DI_BUF(ctx, Y, y, (uint64_t)rows * dtype_size(dt));
  if (rows == 0) return DI_OK;
  unsigned g = (rows + 3) / 4;
  if (dt == DI_F32) k_reduce_mean<float><<<g, 256, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, inner, rows);
  else k_reduce_mean<f16><<<g, 256, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, inner, rows);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_resize_nearest(di_ctx* ctx, di_handle X, di_handle Y, uint32_t planes, uint32_t Hin,
                          uint32_t Win, uint32_t Hout, uint32_t Wout, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(Hin && Win && Hout && Wout, DI_EINVAL, "di_resize_nearest: zero spatial dim");
  uint64_t n = (uint64_t)planes * Hout * Wout;
  DI_BUF(ctx, X, x, (uint64_t)planes * Hin * Win * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  if (n == 0) return DI_OK;
  unsigned g = grid_for(n);
  if (dt == DI_F32) k_resize<float><<<g, kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, Hin, Win, Hout, Wout, n);
  else k_resize<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, Hin, Win, Hout, Wout, n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_transpose(di_ctx* ctx, di_handle X, di_handle Y, uint32_t rank,
                     const uint32_t* out_dim, const uint32_t* in_stride, const uint32_t* perm,
                     uint64_t numel, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  Idx4 c;
  int rc = fill_idx4(&c, rank, out_dim, in_stride, perm, "di_transpose");
  if (rc) return rc;
  uint64_t prod = 1;
  bool seen[4] = {false, false, false, false};
  for (uint32_t d = 0; d < rank; d++) {
    prod *= out_dim[d];
    DI_REQUIRE(perm[d] < rank && !seen[perm[d]], DI_EINVAL, "di_transpose: perm is not a permutation");
    seen[perm[d]] = true;
  }
  DI_REQUIRE(prod == numel, DI_EINVAL, "di_transpose: numel mismatch");
  if (numel == 0) return DI_OK;
  // Input extent: in dim perm[d] has size out_dim[d].
  uint64_t maxoff = 0;
  for (uint32_t d = 0; d < rank; d++) maxoff += (uint64_t)(out_dim[d] - 1) * in_stride[perm[d]];
  DI_BUF(ctx, X, x, (maxoff + 1) * dtype_size(dt));
  DI_BUF(ctx, Y, y, numel * dtype_size(dt));
  unsigned g = grid_for(numel);
  if (dt == DI_F32) k_transpose<float><<<g, kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, c, numel);
  else k_transpose<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, c, numel);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_slice(di_ctx* ctx, di_handle X, di_handle Y, uint32_t rank, const uint32_t* out_dim,
                 const uint32_t* in_stride, const uint32_t* start, uint64_t numel, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  Idx4 c;
  int rc = fill_idx4(&c, rank, out_dim, in_stride, start, "di_slice");
  if (rc) return rc;
  uint64_t prod = 1;
  for (uint32_t d = 0; d < rank; d++) prod *= out_dim[d];
  DI_REQUIRE(prod == numel, DI_EINVAL, "di_slice: numel mismatch");
  if (numel == 0) return DI_OK;
  DI_BUF(ctx, X, x, (max_offset(c, start) + 1) * dtype_size(dt));
  DI_BUF(ctx, Y, y, numel * dtype_size(dt));
  unsigned g = grid_for(numel);
  if (dt == DI_F32) k_slice<float><<<g, kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, c, numel);
  else k_slice<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, c, numel);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_concat_copy(di_ctx* ctx, di_handle X, di_handle Y, uint32_t stripe_in,
                       uint32_t stripe_out, uint32_t offset_out, uint64_t numel, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(stripe_in > 0 && offset_out + stripe_in <= stripe_out, DI_EINVAL,
             "di_concat_copy: stripe %u at offset %u does not fit output stripe %u", stripe_in,
             offset_out, stripe_out);
  DI_REQUIRE(numel % stripe_in == 0, DI_EINVAL, "di_concat_copy: numel not a multiple of stripe");
  if (numel == 0) return DI_OK;
  uint64_t rows = numel / stripe_in;
  DI_BUF(ctx, X, x, numel * dtype_size(dt));
  DI_BUF(ctx, Y, y, ((rows - 1) * stripe_out + offset_out + stripe_in) * dtype_size(dt));
  unsigned g = grid_for(numel);
  if (dt == DI_F32) k_concat<float><<<g, kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, stripe_in, stripe_out, offset_out, numel);
  else k_concat<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, stripe_in, stripe_out, offset_out, numel);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_pow_scalar(di_ctx* ctx, di_handle X, di_handle Y, uint64_t n, float exponent,
                      int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_BUF(ctx, X, x, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  if (n == 0) return DI_OK;
  unsigned g = grid_for(n);
  if (dt == DI_F32) k_pow_scalar<float><<<g, kBlock, 0, ctx->stream>>>((const float*)x->ptr, (float*)y->ptr, exponent, n);
  else k_pow_scalar<f16><<<g, kBlock, 0, ctx->stream>>>((const f16*)x->ptr, (f16*)y->ptr, exponent, n);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"

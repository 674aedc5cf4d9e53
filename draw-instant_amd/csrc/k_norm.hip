// GroupNorm(+SiLU), InstanceNorm and LayerNorm for gfx950, and their C ABI.
//
// Statistics follow the reference kernels exactly in formula (WGSL_GROUPNORM
// wgsl-ops.js:415-456, WGSL_FUSED_GN_SILU fused-resnet.js:138-165,
// WGSL_LAYERNORM wgsl-ops.js:785-800): mean = E[x], var = E[x^2] - mean^2
// clamped at 0, rstd = 1/sqrt(var + eps), y = (x - mean) * rstd * gamma[c] +
// beta[c], optionally followed by SiLU y/(1+e^-y).  Partial sums are fp32.
//
// Work decomposition is MI355X-first instead of the reference's one
// workgroup per group (32 workgroups for 256 CUs, X read twice):
//  * NCHW: each group is split over S workgroups; every workgroup keeps its
//    slice in registers, publishes (sum, sumsq), meets the group's other
//    workgroups at a bounded cross-block barrier and normalises from
//    registers, so X is read from HBM once.  Launched cooperatively so all
//    workgroups are co-resident; the wait is bounded and raises the context
//    fault word instead of hanging.
//  * NHWC fp16 (U-Net activations): one kernel reduces per-channel partials
//    of a pixel chunk (fully coalesced rows of C), the last workgroup to finish
//    folds them into per-group mean/rstd; a second kernel applies the affine
//    (+SiLU) as per-channel scale/shift.  No waiting, safe under graph replay.
#include <cstdlib>

#include "di_device.h"
#include "di_kernels.h"

namespace di {

namespace {

constexpr uint32_t kGnBarBase = 1;              // sync words [1, 1 + 2*kGnMaxGroups)
constexpr uint32_t kGnMaxGroups = 65536;
constexpr uint32_t kLastBlockBase = 1 + 2 * kGnMaxGroups;  // last-block counters
constexpr uint32_t kSpinLimit = 1u << 22;

__device__ __forceinline__ uint32_t ld_acquire(uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_relaxed_f(float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_relaxed_f(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide sum of two values (256 threads = 4 waves). Result valid in thread 0.
__device__ __forceinline__ void block_sum2(float& a, float& b, float* sh /*[2*8]*/) {
  a = wave_sum(a);
  b = wave_sum(b);
  int w = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    sh[w] = a;
    sh[8 + w] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int nw = blockDim.x / kWave;
    a = 0.0f;
    b = 0.0f;
    for (int i = 0; i < nw; i++) {
      a += sh[i];
      b += sh[8 + i];
    }
  }
}

template <typename T, int VEC>
struct Vec;
template <>
struct Vec<float, 4> {
  typedef f32x4 type;
};
template <>
struct Vec<f16, 4> {
  typedef f16x4 type;
};
template <typename T>
struct Vec<T, 1> {
  typedef T type;
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, float* out) {
  if constexpr (VEC == 1) {
    out[0] = (float)p[0];
  } else {
    typename Vec<T, VEC>::type v = *(const typename Vec<T, VEC>::type*)p;
#pragma unroll
    for (int j = 0; j < VEC; j++) out[j] = (float)v[j];
  }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const float* in) {
  if constexpr (VEC == 1) {
    p[0] = (T)in[0];
  } else {
    typename Vec<T, VEC>::type v;
#pragma unroll
    for (int j = 0; j < VEC; j++) v[j] = (T)in[j];
    *(typename Vec<T, VEC>::type*)p = v;
  }
}

// ---------------- NCHW single pass (register-resident slice) ----------------
// grid (S, N*G), 256 threads. Slice s of group ng covers elements
// [s*chunk, min((s+1)*chunk, L)) of the group's contiguous L = cpg*HW block.
template <typename T, int VEC, int MAXI>
__global__ __launch_bounds__(256) void k_gn_nchw_1pass(
    const T* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    T* __restrict__ y, uint32_t G, uint32_t cpg, uint32_t HW, uint32_t S, uint32_t chunk,
    float eps, int silu, float* __restrict__ part, uint32_t* __restrict__ sync) {
  __shared__ float sh[16];
  __shared__ float s_mean, s_rstd;
  const uint32_t s = blockIdx.x, ng = blockIdx.y;
  const uint32_t L = cpg * HW;
  const uint64_t gbase = (uint64_t)ng * L;  // NCHW: group ng = n*G+g is contiguous
  const uint32_t lo = s * chunk, hi = min(lo + chunk, L);
  const uint32_t g = ng % G;

  float v[MAXI][VEC];
  float ts = 0.0f, tq = 0.0f;
#pragma unroll
  for (int k = 0; k < MAXI; k++) {
    uint32_t e = lo + (k * 256 + threadIdx.x) * VEC;
    if (e < hi) {
      load_vec<T, VEC>(x + gbase + e, v[k]);
#pragma unroll
      for (int j = 0; j < VEC; j++) {
        ts += v[k][j];
        tq += v[k][j] * v[k][j];
      }
    }
  }
  block_sum2(ts, tq, sh);
  if (threadIdx.x == 0) {
    float* pp = part + ((uint64_t)ng * S + s) * 2;
    st_relaxed_f(pp, ts);
    st_relaxed_f(pp + 1, tq);
    uint32_t* cnt = sync + kGnBarBase + 2 * ng;
    uint32_t* gen = cnt + 1;
    uint32_t g0 = ld_acquire(gen);
    __threadfence();
    uint32_t arrived = atomicAdd(cnt, 1u);
    if (arrived == S - 1) {
      atomicExch(cnt, 0u);
      __threadfence();
      atomicAdd(gen, 1u);
    } else {
      uint32_t spins = 0;
      while (ld_acquire(gen) == g0) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kSpinLimit) {
          atomicOr(sync + kFaultWord, 1u);
          break;
        }
      }
    }
    __threadfence();
    float sum = 0.0f, sq = 0.0f;
    const float* pg = part + (uint64_t)ng * S * 2;
    for (uint32_t j = 0; j < S; j++) {
      sum += ld_relaxed_f((float*)pg + 2 * j);
      sq += ld_relaxed_f((float*)pg + 2 * j + 1);
    }
    float mean = sum / (float)L;
    float var = fmaxf(sq / (float)L - mean * mean, 0.0f);
    s_mean = mean;
    s_rstd = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
  const float mean = s_mean, rstd = s_rstd;
#pragma unroll
  for (int k = 0; k < MAXI; k++) {
    uint32_t e = lo + (k * 256 + threadIdx.x) * VEC;
    if (e < hi) {
      // VEC divides HW, so the VEC elements of a vector share one channel.
      const uint32_t c = g * cpg + e / HW;
      const float a = rstd * gamma[c], b = beta[c] - mean * a;
      float o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; j++) {
        float t = v[k][j] * a + b;
        o[j] = silu ? silu_f(t) : t;
      }
      store_vec<T, VEC>(y + gbase + e, o);
    }
  }
}

// ---------------- NCHW two-pass fallback (any size) ----------------
// Pass 1: grid (S, N*G) partial sums; the last workgroup of each group folds
// them into (mean, rstd).  Pass 2: grid-stride normalise.
template <typename T>
__global__ __launch_bounds__(256) void k_gn_nchw_stats(const T* __restrict__ x, uint32_t L,
                                                       uint32_t S, uint32_t chunk, float eps,
                                                       float* __restrict__ part,
                                                       float* __restrict__ stats,
                                                       uint32_t* __restrict__ sync) {
  __shared__ float sh[16];
  __shared__ bool last;
  const uint32_t s = blockIdx.x, ng = blockIdx.y;
  const uint64_t gbase = (uint64_t)ng * L;
  const uint32_t lo = s * chunk, hi = min(lo + chunk, L);
  float ts = 0.0f, tq = 0.0f;
  for (uint32_t e = lo + threadIdx.x; e < hi; e += 256) {
    float v = (float)x[gbase + e];
    ts += v;
    tq += v * v;
  }
  block_sum2(ts, tq, sh);
  if (threadIdx.x == 0) {
    float* pp = part + ((uint64_t)ng * S + s) * 2;
    st_relaxed_f(pp, ts);
    st_relaxed_f(pp + 1, tq);
    __threadfence();
    uint32_t* cnt = sync + kLastBlockBase + ng;
    last = atomicAdd(cnt, 1u) == S - 1;
    if (last) {
      __threadfence();
      float sum = 0.0f, sq = 0.0f;
      for (uint32_t j = 0; j < S; j++) {
        sum += ld_relaxed_f(part + ((uint64_t)ng * S + j) * 2);
        sq += ld_relaxed_f(part + ((uint64_t)ng * S + j) * 2 + 1);
      }
      float mean = sum / (float)L;
      float var = fmaxf(sq / (float)L - mean * mean, 0.0f);
      stats[2 * ng] = mean;
      stats[2 * ng + 1] = 1.0f / sqrtf(var + eps);
      atomicExch(cnt, 0u);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void k_gn_nchw_apply(const T* __restrict__ x,
                                                       const float* __restrict__ gamma,
                                                       const float* __restrict__ beta,
                                                       T* __restrict__ y, uint32_t G,
                                                       uint32_t cpg, uint32_t HW, uint64_t n,
                                                       int silu,
                                                       const float* __restrict__ stats) {
  const uint64_t L = (uint64_t)cpg * HW;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint64_t ng = i / L;
    uint32_t c = (uint32_t)(ng % G) * cpg + (uint32_t)((i % L) / HW);
    float t = ((float)x[i] - stats[2 * ng]) * stats[2 * ng + 1] * gamma[c] + beta[c];
    y[i] = (T)(silu ? silu_f(t) : t);
  }
}

// ---------------- NHWC fp16 (U-Net path) ----------------
// Thread layout for a row of C channels: CV = C/8 vectors of 8 halfs;
// cvb = min(CV, 256) threads across the row, R = 256/cvb pixel lanes.
struct NhwcMap {
  uint32_t CV, cvb, R, kv;
};
__host__ __device__ inline NhwcMap nhwc_map(uint32_t C) {
  NhwcMap m;
  m.CV = C / 8;
  m.cvb = m.CV < 256 ? m.CV : 256;
  m.R = 256 / m.cvb;
  m.kv = (m.CV + m.cvb - 1) / m.cvb;
  return m;
}

constexpr int kMaxKV = 2;  // C <= 4096

// grid (chunks, N). Per-channel partial sums of pixel chunk -> per-group
// partials; the last workgroup of image n folds all chunks into mean/rstd.
__global__ __launch_bounds__(256) void k_gn_nhwc_stats(
    NhwcSrc x, uint32_t C, uint32_t G, uint32_t HW, uint32_t ppc, float eps,
    float* __restrict__ part /*[N][chunks][G][2]*/, float* __restrict__ stats /*[N][G][2]*/,
    uint32_t* __restrict__ sync) {
  extern __shared__ float csh[];  // [R][2][C] per pixel-lane, per-channel sum / sumsq
  __shared__ bool last;
  const uint32_t chunk = blockIdx.x, n = blockIdx.y, chunks = gridDim.x;
  const NhwcMap m = nhwc_map(C);
  const uint32_t p0 = chunk * ppc, p1 = min(p0 + ppc, HW);
  const uint32_t lane_cv = threadIdx.x % m.cvb, pl = threadIdx.x / m.cvb;
  if (pl < m.R) {
    float s[kMaxKV][8], q[kMaxKV][8];
#pragma unroll
    for (int k = 0; k < kMaxKV; k++)
#pragma unroll
      for (int j = 0; j < 8; j++) s[k][j] = q[k][j] = 0.0f;
    for (uint32_t p = p0 + pl; p < p1; p += m.R) {
      const uint64_t pix = (uint64_t)n * HW + p;
#pragma unroll
      for (int k = 0; k < kMaxKV; k++) {
        uint32_t cv = lane_cv + k * m.cvb;
        if (k < (int)m.kv && cv < m.CV) {
          f16x8 v = x.load8(pix, cv * 8);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            float f = (float)v[j];
            s[k][j] += f;
            q[k][j] += f * f;
          }
        }
      }
    }
    // every (pixel-lane, channel) slot is written by exactly one thread
#pragma unroll
    for (int k = 0; k < kMaxKV; k++) {
      uint32_t cv = lane_cv + k * m.cvb;
      if (k < (int)m.kv && cv < m.CV) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          csh[(pl * 2) * C + cv * 8 + j] = s[k][j];
          csh[(pl * 2 + 1) * C + cv * 8 + j] = q[k][j];
        }
      }
    }
  }
  __syncthreads();
  const uint32_t cpg = C / G;
  if (threadIdx.x < G) {
    uint32_t g = threadIdx.x;
    float a = 0.0f, b = 0.0f;
    for (uint32_t r = 0; r < m.R; r++)  // fixed order: deterministic
      for (uint32_t c = g * cpg; c < (g + 1) * cpg; c++) {
        a += csh[(r * 2) * C + c];
        b += csh[(r * 2 + 1) * C + c];
      }
    float* pp = part + (((uint64_t)n * chunks + chunk) * G + g) * 2;
    st_relaxed_f(pp, a);
    st_relaxed_f(pp + 1, b);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    __threadfence();
    uint32_t* cnt = sync + kLastBlockBase + kGnMaxGroups + n;
    last = atomicAdd(cnt, 1u) == chunks - 1;
    if (last) atomicExch(cnt, 0u);
  }
  __syncthreads();
  if (last && threadIdx.x < G) {
    __threadfence();
    uint32_t g = threadIdx.x;
    float a = 0.0f, b = 0.0f;
    for (uint32_t k = 0; k < chunks; k++) {
      float* pp = part + (((uint64_t)n * chunks + k) * G + g) * 2;
      a += ld_relaxed_f(pp);
      b += ld_relaxed_f(pp + 1);
    }
    float L = (float)cpg * (float)HW;
    float mean = a / L;
    float var = fmaxf(b / L - mean * mean, 0.0f);
    stats[((uint64_t)n * G + g) * 2] = mean;
    stats[((uint64_t)n * G + g) * 2 + 1] = 1.0f / sqrtf(var + eps);
  }
}

// grid (chunks, N): y = x * a[c] + b[c] (+SiLU) with a = rstd*gamma,
// b = beta - mean*rstd*gamma folded per channel in LDS.
__global__ __launch_bounds__(256) void k_gn_nhwc_apply(
    NhwcSrc x, const float* __restrict__ gamma, const float* __restrict__ beta,
    f16* __restrict__ y, uint32_t C, uint32_t G, uint32_t HW, uint32_t ppc, int silu,
    const float* __restrict__ stats) {
  extern __shared__ float ab[];  // [2*C]
  const uint32_t chunk = blockIdx.x, n = blockIdx.y;
  const uint32_t cpg = C / G;
  for (uint32_t c = threadIdx.x; c < C; c += 256) {
    uint32_t g = c / cpg;
    float mean = stats[((uint64_t)n * G + g) * 2], rstd = stats[((uint64_t)n * G + g) * 2 + 1];
    float a = rstd * gamma[c];
    ab[c] = a;
    ab[C + c] = beta[c] - mean * a;
  }
  __syncthreads();
  const uint32_t CV = C / 8;
  const uint32_t p0 = chunk * ppc, p1 = min(p0 + ppc, HW);
  const uint64_t base = ((uint64_t)n * HW + p0) * C;
  const uint32_t nv = (p1 - p0) * CV;
  for (uint32_t i = threadIdx.x; i < nv; i += 256) {
    uint32_t cv = i % CV;
    uint64_t off = base + (uint64_t)i * 8;
    f16x8 v = x.load8((uint64_t)n * HW + p0 + i / CV, cv * 8);
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float t = (float)v[j] * ab[cv * 8 + j] + ab[C + cv * 8 + j];
      o[j] = (f16)(silu ? silu_f(t) : t);
    }
    *(f16x8*)(y + off) = o;
  }
}

// ---------------- LayerNorm: one wavefront per row ----------------
template <typename T>
__global__ __launch_bounds__(256) void k_layer_norm(const T* __restrict__ x,
                                                    const float* __restrict__ gamma,
                                                    const float* __restrict__ beta,
                                                    T* __restrict__ y, uint32_t rows,
                                                    uint32_t inner, float eps) {
  uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
  int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const T* xr = x + (uint64_t)row * inner;
  T* yr = y + (uint64_t)row * inner;
  constexpr int V = sizeof(T) == 2 ? 8 : 4;
  float s = 0.0f, q = 0.0f;
  if (inner % V == 0) {
    for (uint32_t j = lane * V; j < inner; j += kWave * V) {
      float v[V];
      if constexpr (V == 8) {
        f16x8 t = *(const f16x8*)(xr + j);
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = (float)t[k];
      } else {
        f32x4 t = *(const f32x4*)(xr + j);
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = t[k];
      }
#pragma unroll
      for (int k = 0; k < V; k++) {
        s += v[k];
        q += v[k] * v[k];
      }
    }
  } else {
    for (uint32_t j = lane; j < inner; j += kWave) {
      float v = (float)xr[j];
      s += v;
      q += v * v;
    }
  }
  s = wave_sum(s);
  q = wave_sum(q);
  float mean = s / (float)inner;
  float var = fmaxf(q / (float)inner - mean * mean, 0.0f);
  float rstd = 1.0f / sqrtf(var + eps);
  for (uint32_t j = lane; j < inner; j += kWave)
    yr[j] = (T)(((float)xr[j] - mean) * rstd * gamma[j] + beta[j]);
}

template <typename T, int VEC, int MAXI>
int try_1pass(Ctx* c, const void* x, const float* gamma, const float* beta, void* y,
              uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu,
              bool* launched) {
  *launched = false;
  const uint32_t L = cpg * HW;
  const uint32_t NG = N * G;
  if (NG > kGnMaxGroups || (VEC > 1 && HW % VEC != 0)) return DI_OK;
  auto kern = k_gn_nchw_1pass<T, VEC, MAXI>;
  int per_cu = 0;
  DI_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 256, 0));
  const uint64_t resident = (uint64_t)per_cu * c->num_cus;
  // Aim for ~2 workgroups per CU over all groups, within register capacity.
  uint32_t S = (uint32_t)((2ull * c->num_cus + NG - 1) / NG);
  const uint32_t per_block_max = 256 * VEC * MAXI;
  uint32_t S_min = (L + per_block_max - 1) / per_block_max;
  if (S < S_min) S = S_min;
  if (S < 1) S = 1;
  uint32_t chunk = (L + S - 1) / S;
  chunk = (chunk + VEC - 1) / VEC * VEC;
  S = (L + chunk - 1) / chunk;
  if ((uint64_t)S * NG > resident || chunk > per_block_max) return DI_OK;
  void* ws = nullptr;
  int rc = workspace(c, (uint64_t)NG * S * 2 * sizeof(float), &ws);
  if (rc) return rc;
  const T* xp = (const T*)x;
  T* yp = (T*)y;
  float* part = (float*)ws;
  uint32_t* sync = c->sync_words;
  int silu_i = silu ? 1 : 0;
  void* args[] = {(void*)&xp, (void*)&gamma, (void*)&beta, (void*)&yp, (void*)&G, (void*)&cpg,
                  (void*)&HW, (void*)&S, (void*)&chunk, (void*)&eps, (void*)&silu_i,
                  (void*)&part, (void*)&sync};
  // All S*NG workgroups fit on the device at once (checked above against the
  // occupancy calculator), so a regular launch keeps them co-resident; the
  // barrier's wait is bounded in any case.
  if (getenv("DI_GN_COOP"))
    DI_HIP(hipLaunchCooperativeKernel((const void*)kern, dim3(S, NG), dim3(256), args, 0,
                                      c->stream));
  else
    kern<<<dim3(S, NG), 256, 0, c->stream>>>(xp, gamma, beta, yp, G, cpg, HW, S, chunk, eps,
                                             silu_i, part, sync);
  *launched = true;
  return DI_OK;
}

template <typename T>
int gn_nchw(Ctx* c, const void* x, const float* gamma, const float* beta, void* y, uint32_t N,
            uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu) {
  bool done = false;
  int rc = try_1pass<T, 4, 8>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, &done);
  if (rc || done) return rc;
  rc = try_1pass<T, 1, 16>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, &done);
  if (rc || done) return rc;
  // Two-pass fallback.
  const uint32_t L = cpg * HW, NG = N * G;
  DI_REQUIRE(NG <= kGnMaxGroups, DI_EUNSUPPORTED, "group norm: %u groups exceed %u", NG,
             kGnMaxGroups);
  uint32_t S = (uint32_t)((2ull * c->num_cus + NG - 1) / NG);
  uint32_t chunk = (L + S - 1) / S;
  if (chunk < 1024) chunk = 1024;
  S = (L + chunk - 1) / chunk;
  void* ws = nullptr;
  rc = workspace(c, ((uint64_t)NG * S * 2 + (uint64_t)NG * 2) * sizeof(float), &ws);
  if (rc) return rc;
  float* part = (float*)ws;
  float* stats = part + (uint64_t)NG * S * 2;
  k_gn_nchw_stats<T><<<dim3(S, NG), 256, 0, c->stream>>>((const T*)x, L, S, chunk, eps, part,
                                                          stats, c->sync_words);
  DI_LAUNCH_CHECK();
  uint64_t n = (uint64_t)NG * L;
  uint64_t blocks = (n + 1023) / 1024;
  if (blocks > 65535ull * 8) blocks = 65535ull * 8;
  k_gn_nchw_apply<T><<<(unsigned)blocks, 256, 0, c->stream>>>(
      (const T*)x, gamma, beta, (T*)y, G, cpg, HW, n, silu ? 1 : 0, stats);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // namespace

int launch_group_norm_nchw(Ctx* c, const void* x, const float* gamma, const float* beta,
                           void* y, uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW,
                           float eps, bool silu, int dt) {
  if (dt == DI_F32) return gn_nchw<float>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu);
  return gn_nchw<f16>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu);
}

uint32_t gn_nhwc_chunks(uint32_t HW, uint32_t C) {
  (void)C;
  uint32_t ppc = (HW + 63) / 64;  // at most 64 chunks per image
  return (HW + ppc - 1) / ppc;
}

uint64_t gn_nhwc_ws_floats(uint32_t N, uint32_t C, uint32_t G, uint32_t HW) {
  return (uint64_t)N * gn_nhwc_chunks(HW, C) * G * 2 + (uint64_t)N * G * 2;
}

void launch_group_norm_nhwc(hipStream_t s, NhwcSrc x, const float* gamma, const float* beta,
                            void* y, uint32_t N, uint32_t C, uint32_t G, uint32_t HW, float eps,
                            bool silu, float* ws, uint32_t* sync) {
  uint32_t chunks = gn_nhwc_chunks(HW, C);
  uint32_t ppc = (HW + chunks - 1) / chunks;
  float* part = ws;
  float* stats = ws + (uint64_t)N * chunks * G * 2;
  const NhwcMap m = nhwc_map(C);
  size_t lds = 2 * C * sizeof(float);
  k_gn_nhwc_stats<<<dim3(chunks, N), 256, lds * m.R, s>>>(x, C, G, HW, ppc, eps, part, stats, sync);
  k_gn_nhwc_apply<<<dim3(chunks, N), 256, lds, s>>>(x, gamma, beta, (f16*)y, C, G, HW, ppc,
                                                    silu ? 1 : 0, stats);
}

void launch_layer_norm(hipStream_t s, const void* x, const float* gamma, const float* beta,
                       void* y, uint32_t rows, uint32_t inner, float eps, int dt) {
  unsigned g = (rows + 3) / 4;
  if (dt == DI_F32)
    k_layer_norm<float><<<g, 256, 0, s>>>((const float*)x, gamma, beta, (float*)y, rows, inner, eps);
  else
    k_layer_norm<f16><<<g, 256, 0, s>>>((const f16*)x, gamma, beta, (f16*)y, rows, inner, eps);
}

}  // namespace di

using namespace di;

extern "C" {

int32_t di_group_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                      uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps,
                      int32_t flags, int32_t dt, int32_t layout) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(layout == DI_NCHW || layout == DI_NHWC, DI_EINVAL, "di_group_norm: bad layout %d",
             layout);
  DI_REQUIRE(N > 0 && G > 0 && cpg > 0 && HW > 0, DI_EINVAL,
             "di_group_norm: zero dimension (N=%u G=%u cpg=%u HW=%u)", N, G, cpg, HW);
  DI_REQUIRE((flags & ~DI_NORM_SILU) == 0, DI_EINVAL, "di_group_norm: unknown flags 0x%x", flags);
  DI_REQUIRE(eps >= 0.0f, DI_EINVAL, "di_group_norm: negative eps");
  const uint32_t C = G * cpg;
  const uint64_t n = (uint64_t)N * C * HW;
  DI_BUF(ctx, X, x, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  DI_BUF(ctx, gamma, g, (uint64_t)C * 4);
  DI_BUF(ctx, beta, b, (uint64_t)C * 4);
  DI_REQUIRE(x->ptr != y->ptr, DI_EINVAL, "di_group_norm: Y may not alias X");
  bool silu = (flags & DI_NORM_SILU) != 0;
  if (layout == DI_NCHW) {
    int rc = launch_group_norm_nchw(ctx, x->ptr, (const float*)g->ptr, (const float*)b->ptr,
                                    y->ptr, N, G, cpg, HW, eps, silu, dt);
    if (rc) return rc;
  } else {
    DI_REQUIRE(dt == DI_F16, DI_EUNSUPPORTED, "di_group_norm: NHWC requires fp16");
    DI_REQUIRE(C % 8 == 0 && C <= 4096 && G <= 256, DI_EUNSUPPORTED,
               "di_group_norm: NHWC needs C %% 8 == 0, C <= 4096, G <= 256 (C=%u G=%u)", C, G);
    DI_REQUIRE(N <= kGnMaxGroups, DI_EUNSUPPORTED, "di_group_norm: batch too large");
    void* ws = nullptr;
    int rc = workspace(ctx, gn_nhwc_ws_floats(N, C, G, HW) * sizeof(float), &ws);
    if (rc) return rc;
    NhwcSrc src{(const f16*)x->ptr, (const f16*)x->ptr, C, C, C};
    launch_group_norm_nhwc(ctx->stream, src, (const float*)g->ptr, (const float*)b->ptr, y->ptr,
                           N, C, G, HW, eps, silu, (float*)ws, ctx->sync_words);
  }
  DI_LAUNCH_CHECK();
  return DI_OK;
}

int32_t di_gn_silu(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                   uint32_t N, uint32_t C, uint32_t G, uint32_t HW, float eps, int32_t dt,
                   int32_t layout) {
  DI_REQUIRE(G > 0 && C % G == 0, DI_EINVAL, "di_gn_silu: C=%u not divisible by G=%u", C, G);
  return di_group_norm(ctx, X, gamma, beta, Y, N, G, C / G, HW, eps, DI_NORM_SILU, dt, layout);
}

int32_t di_instance_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                         uint32_t N, uint32_t C, uint32_t HW, float eps, int32_t dt) {
  return di_group_norm(ctx, X, gamma, beta, Y, N, C, 1, HW, eps, 0, dt, DI_NCHW);
}

int32_t di_layer_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                      uint32_t rows, uint32_t inner, float eps, int32_t dt) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(inner > 0, DI_EINVAL, "di_layer_norm: inner length 0");
  DI_REQUIRE(eps >= 0.0f, DI_EINVAL, "di_layer_norm: negative eps");
  const uint64_t n = (uint64_t)rows * inner;
  DI_BUF(ctx, X, x, n * dtype_size(dt));
  DI_BUF(ctx, Y, y, n * dtype_size(dt));
  DI_BUF(ctx, gamma, g, (uint64_t)inner * 4);
  DI_BUF(ctx, beta, b, (uint64_t)inner * 4);
  if (rows == 0) return DI_OK;
  launch_layer_norm(ctx->stream, x->ptr, (const float*)g->ptr, (const float*)b->ptr, y->ptr,
                    rows, inner, eps, dt);
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // extern "C"

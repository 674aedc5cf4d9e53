// GroupNorm(+SiLU), InstanceNorm and LayerNorm for gfx950, and their C ABI.
//
// Statistics follow the reference kernels exactly in formula (WGSL_GROUPNORM
// wgsl-ops.js:415-456, WGSL_FUSED_GN_SILU fused-resnet.js:138-165,
// WGSL_LAYERNORM wgsl-ops.js:785-800): mean = E[x], var = E[x^2] - mean^2
// clamped at 0, rstd = 1/sqrt(var + eps), y = (x - mean) * rstd * gamma[c] +
// beta[c], optionally followed by SiLU y/(1+e^-y).  Partial sums are fp32.
//
// Work decomposition is MI355X-first instead of the reference's one
// workgroup per group (32 workgroups for 256 CUs, serial reductions): a
// group norm is either two kernels with no inter-workgroup communication,
//  1. partial sums: ~1024 workgroups each reduce a slice of the input to
//     (sum, sumsq) per group and write them to a workspace, no atomics;
//  2. fold + apply: every workgroup folds the partials it needs in one fixed
//     order (so all workgroups agree bit-for-bit), then normalises its slice
// (X read twice; the second read is usually served by the 256 MB Infinity
// Cache), or, for NCHW tensors of up to 64 groups, one kernel whose slices
// exchange their partial sums through epoch-tagged words (k_gn_nchw_xchg),
// or one kernel whose workgroups each re-read their whole group
// (k_gn_nchw_fused).  All are deterministic and safe under graph replay.
//
// Latency, not bandwidth, bounds these kernels at U-Net sizes (2.5-10 MB per
// call), so each issues all of a round's loads (x, partials, gamma/beta)
// before consuming any: `sched_barrier` stops the scheduler from sinking the
// loads next to their uses, which would serialise them.
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "di_device.h"
#include "di_gemv_dev.h"
#include "di_kernels.h"

namespace di {

namespace {

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// Block-wide sum of two values (256 threads = 4 waves), in a fixed order.
// Result valid in thread 0.
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
struct Vec<f16, 8> {
  typedef f16x8 type;
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

// ---------------- NCHW (each group is one contiguous block) ----------------
// grid (S, N*G): slice s of group ng covers elements [s*chunk, min((s+1)*chunk,
// L)) of the group's L = cpg*HW elements; every slice is non-empty and VEC
// divides HW (so a vector never straddles a channel) and chunk.
constexpr int kNchwU = 4;  // vectors per thread per round

template <typename T, int VEC>
__global__ __launch_bounds__(256) void k_gn_nchw_partial(const T* __restrict__ x, uint32_t L,
                                                          uint32_t chunk,
                                                          float* __restrict__ part) {
  __shared__ float sh[16];
  const uint32_t s = blockIdx.x, ng = blockIdx.y, S = gridDim.x;
  const T* xg = x + (uint64_t)ng * L;
  const uint32_t lo = s * chunk, hi = min(lo + chunk, L);
  float ts = 0.0f, tq = 0.0f;
  for (uint32_t b = lo; b < hi; b += 256 * VEC * kNchwU) {
    float v[kNchwU][VEC];
#pragma unroll
    for (int u = 0; u < kNchwU; u++) {
      const uint32_t e = b + (u * 256 + threadIdx.x) * VEC;
      load_vec<T, VEC>(xg + (e < hi ? e : lo), v[u]);
    }
    sched_fence();
#pragma unroll
    for (int u = 0; u < kNchwU; u++) {
      const bool ok = b + (u * 256 + threadIdx.x) * VEC < hi;
#pragma unroll
      for (int j = 0; j < VEC; j++) {
        const float f = ok ? v[u][j] : 0.0f;
        ts += f;
        tq += f * f;
      }
    }
  }
  block_sum2(ts, tq, sh);
  if (threadIdx.x == 0) {
    part[((uint64_t)ng * S + s) * 2] = ts;
    part[((uint64_t)ng * S + s) * 2 + 1] = tq;
  }
}

// Same grid.  Folds the group's S <= 256 partials (one load per thread, fixed
// order), then y = x * a[c] + b[c] (+SiLU) over the slice.  The first round of
// x and its gamma/beta are loaded before the fold.
template <typename T, int VEC>
__global__ __launch_bounds__(256) void k_gn_nchw_apply(const T* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta,
                                                        T* __restrict__ y, uint32_t G,
                                                        uint32_t cpg, uint32_t HW, uint32_t chunk,
                                                        float eps, int silu,
                                                        const float* __restrict__ part) {
  __shared__ float sh[16];
  __shared__ float s_mean, s_rstd;
  const uint32_t s = blockIdx.x, ng = blockIdx.y, S = gridDim.x;
  const uint32_t L = cpg * HW;
  const uint64_t gbase = (uint64_t)ng * L;
  const uint32_t c0 = (ng % G) * cpg;
  const uint32_t lo = s * chunk, hi = min(lo + chunk, L);
  float v[kNchwU][VEC], gm[kNchwU], bt[kNchwU];
  auto load_round = [&](uint32_t b) {
#pragma unroll
    for (int u = 0; u < kNchwU; u++) {
      uint32_t e = b + (u * 256 + threadIdx.x) * VEC;
      e = e < hi ? e : lo;
      load_vec<T, VEC>(x + gbase + e, v[u]);
      gm[u] = gamma[c0 + e / HW];
      bt[u] = beta[c0 + e / HW];
    }
  };
  load_round(lo);
  float ps = 0.0f, pq = 0.0f;
  if (threadIdx.x < S) {
    ps = part[((uint64_t)ng * S + threadIdx.x) * 2];
    pq = part[((uint64_t)ng * S + threadIdx.x) * 2 + 1];
  }
  sched_fence();
  block_sum2(ps, pq, sh);
  if (threadIdx.x == 0) {
    const float mean = ps / (float)L;
    const float var = fmaxf(pq / (float)L - mean * mean, 0.0f);
    s_mean = mean;
    s_rstd = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
  const float mean = s_mean, rstd = s_rstd;
  for (uint32_t b = lo; b < hi; b += 256 * VEC * kNchwU) {
    if (b != lo) {
      load_round(b);
      sched_fence();
    }
#pragma unroll
    for (int u = 0; u < kNchwU; u++) {
      const uint32_t e = b + (u * 256 + threadIdx.x) * VEC;
      if (e < hi) {
        const float a = rstd * gm[u], sb = bt[u] - mean * a;
        float o[VEC];
#pragma unroll
        for (int j = 0; j < VEC; j++) {
          const float t = v[u][j] * a + sb;
          o[j] = silu ? silu_f(t) : t;
        }
        store_vec<T, VEC>(y + gbase + e, o);
      }
    }
  }
}

// Single-launch NCHW GroupNorm for groups of up to 16 x 1024 vectors:
// workgroup w of S per group reads the WHOLE group (one round of U vector
// loads per thread, all in flight at once), reduces (sum, sumsq) in a fixed
// order - so the S workgroups of a group derive bit-identical statistics -
// then normalises its own slice [s*chunk, min((s+1)*chunk, L)), re-read from
// the cache.  No workspace and no inter-workgroup communication: the extra
// reads replace the partials pass.  Workgroups are numbered so that the S
// slices of a group run on one XCD (blocks are dealt round-robin over the 8
// XCDs), where every read after the first hits that XCD's L2.
constexpr int kFusedT = 1024;

template <typename T, int VEC, int U>
__global__ __launch_bounds__(kFusedT) void k_gn_nchw_fused(
    const T* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    T* __restrict__ y, uint32_t G, uint32_t cpg, uint32_t HW, uint32_t S, uint32_t chunk,
    float eps, int silu) {
  __shared__ float sh[2 * (kFusedT / kWave)];
  __shared__ float s_mean, s_rstd;
  const uint32_t tid = threadIdx.x;
  const uint32_t NT = gridDim.x, bid = blockIdx.x, xcd = bid & 7u, idx = bid >> 3;
  const uint32_t per = NT >> 3, extra = NT & 7u;
  const uint32_t w = xcd < extra ? xcd * (per + 1) + idx : extra * (per + 1) + (xcd - extra) * per + idx;
  const uint32_t ng = w / S, s = w % S;
  const uint32_t L = cpg * HW;
  const uint64_t gbase = (uint64_t)ng * L;
  float v[U][VEC];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t e = (u * kFusedT + tid) * VEC;
    load_vec<T, VEC>(x + gbase + (e < L ? e : 0), v[u]);
  }
  sched_fence();
  float ts = 0.0f, tq = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const bool ok = (u * kFusedT + tid) * VEC < L;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const float f = ok ? v[u][j] : 0.0f;
      ts += f;
      tq += f * f;
    }
  }
  ts = wave_sum(ts);
  tq = wave_sum(tq);
  const uint32_t wv = tid / kWave;
  if (tid % kWave == 0) {
    sh[wv] = ts;
    sh[kFusedT / kWave + wv] = tq;
  }
  __syncthreads();
  if (tid == 0) {
    float a = 0.0f, b = 0.0f;
    for (int i = 0; i < kFusedT / kWave; i++) {
      a += sh[i];
      b += sh[kFusedT / kWave + i];
    }
    const float mean = a / (float)L;
    const float var = fmaxf(b / (float)L - mean * mean, 0.0f);
    s_mean = mean;
    s_rstd = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
  const float mean = s_mean, rstd = s_rstd;
  const uint32_t c0 = (ng % G) * cpg;
  const uint32_t lo = s * chunk, hi = min(lo + chunk, L);
  for (uint32_t b = lo; b < hi; b += kFusedT * VEC * 2) {
    float t[2][VEC], gm[2], bt[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
      uint32_t e = b + (u * kFusedT + tid) * VEC;
      e = e < hi ? e : lo;
      load_vec<T, VEC>(x + gbase + e, t[u]);
      gm[u] = gamma[c0 + e / HW];
      bt[u] = beta[c0 + e / HW];
    }
    sched_fence();
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const uint32_t e = b + (u * kFusedT + tid) * VEC;
      if (e < hi) {
        const float a = rstd * gm[u], sb = bt[u] - mean * a;
        float o[VEC];
#pragma unroll
        for (int j = 0; j < VEC; j++) {
          const float z = t[u][j] * a + sb;
          o[j] = silu ? silu_f(z) : z;
        }
        store_vec<T, VEC>(y + gbase + e, o);
      }
    }
  }
}

// Single-launch NCHW GroupNorm whose workgroups read only their own slice and
// exchange the slice statistics (the record protocol of di_device.h):
// kXchgSlices workgroups per group, each holding its slice (<= kXU rounds of
// kXT vectors) in registers, reduce (sum, sumsq) in a fixed order, publish
// them under the launch's epoch and poll the group's record; the kXchgSlices
// partials are summed in slice order by every workgroup alike, so the slices
// normalise with bit-identical statistics.  Should a slice not arrive within
// `spin` polls (a workgroup not resident, or spin = 0), the workgroup
// recomputes every slice's partials itself from the input with the same
// thread mapping and reduction order - the same bits, from one group's worth
// of extra reads - so the kernel always ends.  The arrival fetch-add is
// issued after the slice's loads: its result is waited for at once, which
// would hold back loads issued after it.
constexpr int kXT = 256;  // threads per workgroup
constexpr uint32_t kXS = kXchgSlices;

template <typename T, int VEC, int U>
__device__ __forceinline__ void xslice_load(const T* __restrict__ x, uint32_t lo, uint32_t hi,
                                            float (&v)[U][VEC]) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t e = lo + (u * kXT + threadIdx.x) * VEC;
    load_vec<T, VEC>(x + (e < hi ? e : 0u), v[u]);
  }
}

// (sum, sumsq) of the slice [lo, hi) held in v, in a fixed order; valid in
// thread 0.  Contains a barrier.
template <int VEC, int U>
__device__ __forceinline__ float2 xslice_partial(const float (&v)[U][VEC], uint32_t lo,
                                                 uint32_t hi, float* sh) {
  float ts = 0.0f, tq = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const bool ok = lo + (u * kXT + threadIdx.x) * VEC < hi;
#pragma unroll
    for (int j = 0; j < VEC; j++) {
      const float f = ok ? v[u][j] : 0.0f;
      ts += f;
      tq += f * f;
    }
  }
  block_sum2(ts, tq, sh);
  return float2{ts, tq};
}

template <typename T, int VEC, int U>
__global__ __launch_bounds__(kXT) void k_gn_nchw_xchg(
    const T* __restrict__ x, const float* __restrict__ gamma, const float* __restrict__ beta,
    T* __restrict__ y, uint64_t* __restrict__ xchg, uint32_t G, uint32_t cpg, uint32_t HW,
    uint32_t chunk, float eps, int silu, uint32_t spin) {
  __shared__ float sh[16];
  __shared__ float sv[2 * kXS];
  __shared__ uint32_t s_o;
  __shared__ int s_ok;
  __shared__ float s_mean, s_rstd;
  const uint32_t tid = threadIdx.x;
  // the kXS slices of a group on one XCD (blocks are dealt round-robin over
  // the 8 XCDs): their polls and re-reads stay in one L2
  const uint32_t NT = gridDim.x, bid = blockIdx.x, xcd = bid & 7u, idx = bid >> 3;
  const uint32_t per = NT >> 3, extra = NT & 7u;
  const uint32_t w = xcd < extra ? xcd * (per + 1) + idx : extra * (per + 1) + (xcd - extra) * per + idx;
  const uint32_t ng = w / kXS, s = w % kXS;
  const uint32_t L = cpg * HW;
  uint64_t* const rec = xchg + (uint64_t)ng * kXchgWords;
  const T* const xg = x + (uint64_t)ng * L;
  auto bounds = [&](uint32_t j, uint32_t& lo, uint32_t& hi) {
    lo = min(j * chunk, L);
    hi = min(lo + chunk, L);
  };
  uint32_t lo, hi;
  bounds(s, lo, hi);
  const uint32_t c0 = (ng % G) * cpg;
  float v[U][VEC], gm[U], bt[U];
  xslice_load<T, VEC, U>(xg, lo, hi, v);
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t e = lo + (u * kXT + tid) * VEC;
    const uint32_t c = c0 + (e < hi ? e : 0u) / HW;
    gm[u] = gamma[c];
    bt[u] = beta[c];
  }
  sched_fence();
  if (tid == 0) s_o = xchg_arrive(rec);
  const float2 p = xslice_partial<VEC, U>(v, lo, hi, sh);  // barrier: s_o visible
  const uint64_t ep = (uint64_t)(s_o / kXS + 1u) << 32;
  const bool all = xchg_publish_poll(rec, ep, s, p.x, p.y, spin, sv);
  if (tid == 0) s_ok = all ? 1 : 0;
  __syncthreads();
  if (!s_ok) {
    // recompute every slice's partials exactly as its own workgroup does
    for (uint32_t j = 0; j < kXS; j++) {
      uint32_t l2, h2;
      bounds(j, l2, h2);
      float t[U][VEC];
      xslice_load<T, VEC, U>(xg, l2, h2, t);
      sched_fence();
      const float2 q = xslice_partial<VEC, U>(t, l2, h2, sh);
      if (tid == 0) {
        sv[2 * j] = q.x;
        sv[2 * j + 1] = q.y;
      }
      __syncthreads();  // sh is reused by the next slice
    }
  }
  if (tid == 0) {
    float a = 0.0f, b = 0.0f;
    for (uint32_t j = 0; j < kXS; j++) {
      a += sv[2 * j];
      b += sv[2 * j + 1];
    }
    const float mean = a / (float)L;
    const float var = fmaxf(b / (float)L - mean * mean, 0.0f);
    s_mean = mean;
    s_rstd = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
  const float mean = s_mean, rstd = s_rstd;
  T* const yg = y + (uint64_t)ng * L;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t e = lo + (u * kXT + tid) * VEC;
    if (e < hi) {
      const float a = rstd * gm[u], sb = bt[u] - mean * a;
      float o[VEC];
#pragma unroll
      for (int j = 0; j < VEC; j++) {
        const float z = v[u][j] * a + sb;
        o[j] = silu ? silu_f(z) : z;
      }
      store_vec<T, VEC>(yg + e, o);
    }
  }
}

// ---------------- NHWC fp16 (U-Net path) ----------------
// Thread layout for a row of C channels: CV = C/8 vectors of 8 halfs;
// cvb = min(CV, 256) threads across the row, R = 256/cvb pixel lanes, and
// KV = ceil(CV/cvb) <= 2 vectors per thread.  Every thread keeps the same
// channels for all its pixels.
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

// Per-thread view of its (up to KV) channel vectors in the two-source input.
template <int KV>
struct NhwcLane {
  const f16* base[KV];
  uint64_t ld[KV];
  bool ok[KV];
  uint32_t cv[KV];
  __device__ NhwcLane(const NhwcSrc& x, const NhwcMap& m, uint32_t lane_cv) {
#pragma unroll
    for (int k = 0; k < KV; k++) {
      cv[k] = lane_cv + k * m.cvb;
      ok[k] = cv[k] < m.CV;
      const uint32_t c = ok[k] ? cv[k] * 8 : 0;  // clamped: loads stay in bounds
      const bool first = c < x.c1;
      base[k] = first ? x.p1 + c : x.p2 + (c - x.c1);
      ld[k] = first ? x.ld1 : x.ld2;
    }
  }
  __device__ __forceinline__ f16x8 load(int k, uint64_t pix) const {
    return *(const f16x8*)(base[k] + pix * ld[k]);
  }
};

// pixel loads in flight per thread: 8 vectors of 16 bytes
template <int KV>
constexpr int gn_unroll() {
  return 8 / KV;
}

// Pass 1, grid (chunks, N): per-(chunk, group) partial sum / sum of squares
// part[n][chunk][g][2], written without atomics.  A round's loads use pixel
// indices clamped into the chunk and are masked afterwards.
template <int KV>
__global__ __launch_bounds__(256) void k_gn_nhwc_partial(NhwcSrc x, uint32_t C, uint32_t G,
                                                          uint32_t HW, uint32_t ppc,
                                                          float* __restrict__ part) {
  extern __shared__ float csh[];  // [R][2][C]: per pixel lane, per-channel sum / sumsq
  const uint32_t chunk = blockIdx.x, n = blockIdx.y, chunks = gridDim.x;
  const NhwcMap m = nhwc_map(C);
  const uint32_t p0 = chunk * ppc, p1 = min(p0 + ppc, HW);
  const uint32_t lane_cv = threadIdx.x % m.cvb, pl = threadIdx.x / m.cvb;
  if (pl < m.R) {
    const NhwcLane<KV> ln(x, m, lane_cv);
    float s[KV][8], q[KV][8];
#pragma unroll
    for (int k = 0; k < KV; k++)
#pragma unroll
      for (int j = 0; j < 8; j++) s[k][j] = q[k][j] = 0.0f;
    const uint32_t cnt = p0 + pl < p1 ? (p1 - p0 - pl + m.R - 1) / m.R : 0;
    const uint64_t pix0 = (uint64_t)n * HW + p0 + pl;
    constexpr int U = gn_unroll<KV>();
    for (uint32_t i = 0; i < cnt; i += U) {
      f16x8 v[U][KV];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t ii = min(i + u, cnt - 1);
#pragma unroll
        for (int k = 0; k < KV; k++) v[u][k] = ln.load(k, pix0 + (uint64_t)ii * m.R);
      }
      sched_fence();
#pragma unroll
      for (int u = 0; u < U; u++) {
#pragma unroll
        for (int k = 0; k < KV; k++) {
          const bool valid = (i + u < cnt) && ln.ok[k];
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float f = valid ? (float)v[u][k][j] : 0.0f;
            s[k][j] += f;
            q[k][j] += f * f;
          }
        }
      }
    }
#pragma unroll
    for (int k = 0; k < KV; k++) {
      if (ln.ok[k]) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          csh[pl * 2 * C + ln.cv[k] * 8 + j] = s[k][j];
          csh[pl * 2 * C + C + ln.cv[k] * 8 + j] = q[k][j];
        }
      }
    }
  }
  __syncthreads();
  // per channel and statistic: sum over pixel lanes in fixed order (in place
  // into row 0; entry i is touched by one thread only)
  for (uint32_t i = threadIdx.x; i < 2 * C; i += 256) {
    float a = csh[i];
    for (uint32_t r = 1; r < m.R; r++) a += csh[r * 2 * C + i];
    csh[i] = a;
  }
  __syncthreads();
  const uint32_t cpg = C / G;
  for (uint32_t t = threadIdx.x; t < 2 * G; t += 256) {
    const uint32_t g = t >> 1, st = t & 1;
    float a = 0.0f;
    for (uint32_t c = g * cpg; c < (g + 1) * cpg; c++) a += csh[st * C + c];
    part[(((uint64_t)n * chunks + chunk) * G) * 2 + t] = a;
  }
}

// Sum of partials pn[k*P + pair] for k = sl, sl+step, ... < nk, in that order,
// with 16 loads in flight at a time.
__device__ __forceinline__ float gn_fold(const float* __restrict__ pn, uint32_t P, uint32_t pair,
                                         uint32_t sl, uint32_t step, uint32_t nk) {
  float a = 0.0f;
  for (uint32_t k0 = sl; k0 < nk; k0 += 16 * step) {
    float t[16];
#pragma unroll
    for (int u = 0; u < 16; u++) {
      const uint32_t k = k0 + u * step;
      t[u] = pn[(uint64_t)(k < nk ? k : sl) * P + pair];
    }
    sched_fence();
#pragma unroll
    for (int u = 0; u < 16; u++) a += (k0 + u * step < nk) ? t[u] : 0.0f;
  }
  return a;
}

// Apply pass from producer statistics (no partial pass): the kernel that
// wrote x also wrote, per 64-pixel chunk and per channel, the sum and sum of
// squares of the values it stored (GnStats; two sources for a channel
// concat).  Grid (pixel blocks, C / SW, N): workgroup (pb, slice, n) folds the
// statistics of its slice's channels over image n's chunks in chunk order,
// then per group over the group's channels in channel order (so every
// workgroup of a group computes the same mean / rstd), and applies
// y = x*a[c] + b[c] (+SiLU) to its pixel block.  SW is a multiple of cpg and
// of 8.  Thread t keeps vector t % NV of the slice for pixels t / NV + R*i.
constexpr int kGnSliceMax = 128;
// statistics of images with more than kGnFoldMin chunks (above 128 x 128
// pixels) are pre-folded to about kGnFoldTarget chunks
constexpr uint32_t kGnFoldMin = 256, kGnFoldTarget = 128;
constexpr uint32_t kGnApplyWgs = 256;
constexpr uint32_t kGnSideX = 2560;  // B * K floats of a side-job GEMV's input

// Pre-fold of producer statistics for large images: every apply workgroup
// otherwise re-reads all HW / 64 chunks of its channel slice (2 MB per
// workgroup at 512 x 512).  out[n][k][c][2] = sum over chunks
// [k * F, min((k + 1) * F, cpi)) of st[n][chunk][c][2]; one thread per
// (channel, statistic) pair, consecutive threads on consecutive floats.
__global__ __launch_bounds__(256) void k_gn_stats_fold(GnStats st, float* __restrict__ out,
                                                       uint32_t C, uint32_t cpi, uint32_t F,
                                                       uint32_t cpo) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x, k = blockIdx.y, n = blockIdx.z;
  if (i >= 2 * C) return;
  const uint32_t c = i / 2, sti = i % 2;
  const bool first = c < st.c1;
  const float* base = first ? st.s1 : st.s2;
  const uint64_t ld = first ? st.ld1 : st.ld2;
  const uint64_t cc = first ? c : c - st.c1;
  const uint32_t k0 = k * F, k1 = min(k0 + F, cpi);
  const float* p = base + ((uint64_t)n * cpi * ld + cc) * 2 + sti;
  const uint64_t step = ld * 2;
  // eight independent partial sums keep eight loads in flight
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  uint32_t j = k0;
  for (; j + 8 <= k1; j += 8) {
#pragma unroll
    for (int u = 0; u < 8; u++) a[u] += p[(uint64_t)(j + u) * step];
  }
  for (; j < k1; j++) a[0] += p[(uint64_t)j * step];
  out[(((uint64_t)n * cpo + k) * C + c) * 2 + sti] =
      ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// cpi: statistics chunks per image in st (HW / 64 as the GEMM epilogue wrote
// them, or fewer after k_gn_stats_fold).
// NU: statistics chunks each lane loads in the first, straight-line batch
// (the host picks the smallest of 1 / 2 / 4 / 8 that covers the image's
// chunks, since every load issued costs the CU's load path whether or not
// it is used); chunks beyond NU lanes' worth are taken by a loop.
// SIDE: z-planes past the batch's run the GEMV gv (B <= 2 rows of K <=
// 1280, eight weight rows per wavefront: every ResNet's time_emb_proj of a
// U-Net step) as a side job, which saves that GEMV a launch of its own.
template <int NU, bool SIDE>
__global__ __launch_bounds__(256) void k_gn_nhwc_apply_st(
    NhwcSrc x, GnStats st, const float* __restrict__ gamma, const float* __restrict__ beta,
    f16* __restrict__ y, uint32_t C, uint32_t cpg, uint32_t SW, uint32_t HW, uint32_t ppb,
    float eps, int silu, uint32_t cpi, uint32_t N, GemvArgs gv) {
  if constexpr (SIDE) {
    if (blockIdx.z >= N) {
      __shared__ float gxs[kGnSideX];
      gemv_vec_block<f16, 3, 8, 2, false>(
          gv, gxs, ((blockIdx.z - N) * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x);
      return;
    }
  }
  __shared__ float chs[2][kGnSliceMax];
  __shared__ float gms[2][kGnSliceMax];
  __shared__ __attribute__((aligned(16))) float sgb[2][kGnSliceMax];  // gamma, beta of the slice
  const uint32_t tid = threadIdx.x, n = blockIdx.z, c0 = blockIdx.y * SW;
  // apply mapping; the first round of pixels and gamma / beta are loaded
  // before the fold so the two memory round trips overlap.  Quotients of
  // the thread index by the slice's vector / quad counts come from a float
  // reciprocal (exact for these sizes: the product stays 0.5 / d away from
  // an integer, far beyond its rounding error), not from an integer
  // division sequence: with one wave per SIMD each of those costs ~0.1 us.
  const uint32_t NV = SW / 8, R = 256 / NV;
  const uint32_t lane = (uint32_t)(((float)tid + 0.5f) * __builtin_amdgcn_rcpf((float)NV));
  const uint32_t v = tid - lane * NV;
  const bool act = lane < R;
  const uint32_t c = c0 + v * 8;
  const uint32_t p0 = blockIdx.x * ppb, p1 = min(p0 + ppb, HW);
  const uint64_t pix0 = (uint64_t)n * HW;
  // per channel: sums over the image's chunks.  Thread t takes channel quad
  // t % Q (4 channels x 2 statistics = two 16-byte loads per chunk) and the
  // chunks k = t / Q, + KL, ... (all loads in flight at once); the KL chunk
  // lanes are then added in lane order.  The first batch of eight chunks
  // (all of them at U-Net sizes) is issued before the pixel and gamma / beta
  // loads in straight-line code, so neither memory round trip waits for the
  // other; a loop over further chunks would wait for every load at its top.
  __shared__ float fold[256 * 8];
  const uint32_t Q = SW / 4, KL = 256 / Q;
  const uint32_t kl = (uint32_t)(((float)tid + 0.5f) * __builtin_amdgcn_rcpf((float)Q));
  const uint32_t qd = tid - kl * Q, cq = c0 + qd * 4;
  const bool sfirst = cq < st.c1;  // 4-channel quads never straddle c1 (c1 % 8 == 0)
  const uint64_t sld = sfirst ? st.ld1 : st.ld2;
  const float* sp = (sfirst ? st.s1 : st.s2) + ((uint64_t)n * cpi * sld + (sfirst ? cq : cq - st.c1)) * 2;
  // Every thread issues these loads (threads without a chunk / pixel share
  // in-range addresses and drop the results): a load under a branch makes
  // the compiler wait for all loads where the branch rejoins.
  f32x4 t0[NU][2];
  {
    // chunk lanes past KL or past the image's cpi chunks read chunk 0
    const uint32_t klc = kl < KL ? kl : 0u;
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const uint32_t k = klc + u * KL < cpi ? klc + u * KL : 0u;
      t0[u][0] = *(const f32x4*)(sp + (uint64_t)k * sld * 2);
      t0[u][1] = *(const f32x4*)(sp + (uint64_t)k * sld * 2 + 4);
    }
  }
  // gamma / beta of the slice, one quad per thread (threads past SW / 4
  // repeat quad 0), staged in LDS for the apply instead of every thread
  // loading its own eight channels: after the statistics, ahead of the
  // pixels (loads retire in order: the statistics are needed first)
  const uint32_t gq = tid < SW / 4 ? tid : 0u;
  const f32x4 gmq = *(const f32x4*)(gamma + c0 + gq * 4);
  const f32x4 btq = *(const f32x4*)(beta + c0 + gq * 4);
  sched_fence();
  constexpr int U = 4;
  f16x8 pre[U];
  {
    const uint32_t lc = act ? lane : 0u;
#pragma unroll
    for (int u = 0; u < U; u++) pre[u] = x.load8(pix0 + min(p0 + lc + u * R, p1 - 1), c);
  }
  sched_fence();
  {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // branch-free: a load consumed under a branch is waited for there with
    // every load issued after it
#pragma unroll
    for (int u = 0; u < NU; u++) {
      const bool use = kl < KL && kl + u * KL < cpi;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        acc[e] += use ? t0[u][0][e] : 0.0f;
        acc[e + 4] += use ? t0[u][1][e] : 0.0f;
      }
    }
    if (kl < KL) {
      for (uint32_t k0 = kl + NU * KL; k0 < cpi; k0 += 8 * KL) {
        f32x4 t[8][2];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          const uint32_t k = k0 + u * KL < cpi ? k0 + u * KL : kl;
          t[u][0] = *(const f32x4*)(sp + (uint64_t)k * sld * 2);
          t[u][1] = *(const f32x4*)(sp + (uint64_t)k * sld * 2 + 4);
        }
        sched_fence();
#pragma unroll
        for (int u = 0; u < 8; u++) {
          if (k0 + u * KL < cpi) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
              acc[e] += t[u][0][e];
              acc[e + 4] += t[u][1][e];
            }
          }
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) fold[tid * 8 + e] = acc[e];
  }
  if (tid < SW / 4) {
    *(f32x4*)&sgb[0][tid * 4] = gmq;
    *(f32x4*)&sgb[1][tid * 4] = btq;
  }
  __syncthreads();
  // acc layout per quad: (s, q) of channels 4qd .. 4qd+3 interleaved
  for (uint32_t i = tid; i < 2 * SW; i += 256) {
    const uint32_t cl = i % SW, sti = i / SW, qd = cl / 4, e = (cl % 4) * 2 + sti;
    float a = 0.0f;
    for (uint32_t kl = 0; kl < KL; kl++) a += fold[(kl * Q + qd) * 8 + e];
    chs[sti][cl] = a;
  }
  __syncthreads();
  const uint32_t GS = SW / cpg;
  for (uint32_t g = tid; g < GS; g += 256) {
    float ps = 0.0f, pq = 0.0f;
    for (uint32_t cl = g * cpg; cl < (g + 1) * cpg; cl++) {
      ps += chs[0][cl];
      pq += chs[1][cl];
    }
    const float L = (float)cpg * (float)HW;
    const float mean = ps / L;
    const float var = fmaxf(pq / L - mean * mean, 0.0f);
    gms[0][g] = mean;
    gms[1][g] = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
  if (!act) return;
  float a[8], b[8];
  // groups of the eight channels v * 8 + j: one division, then steps
  uint32_t gl = (v * 8) / cpg, gr = v * 8 - gl * cpg;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    a[j] = gms[1][gl] * sgb[0][v * 8 + j];
    b[j] = sgb[1][v * 8 + j] - gms[0][gl] * a[j];
    if (++gr == cpg) {
      gr = 0;
      gl++;
    }
  }
  for (uint32_t p = p0 + lane; p < p1; p += U * R) {
    f16x8 t[U];
    if (p == p0 + lane) {
#pragma unroll
      for (int u = 0; u < U; u++) t[u] = pre[u];
    } else {
#pragma unroll
      for (int u = 0; u < U; u++) t[u] = x.load8(pix0 + min(p + u * R, p1 - 1), c);
    }
    sched_fence();
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (p + u * R < p1) {
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float r = (float)t[u][j] * a[j] + b[j];
          o[j] = (f16)(silu ? silu_f(r) : r);
        }
        *(f16x8*)(y + (pix0 + p + u * R) * C + c) = o;
      }
    }
  }
}

// Pass 2, grid (achunks, N): every workgroup folds the image's partials in
// the same fixed order into mean/rstd per group (so all workgroups agree
// bit-for-bit) and applies y = x*a[c] + b[c] (+SiLU), a = rstd*gamma[c],
// b = beta[c] - mean*a, to its pixel range.  The first round of pixels and
// the thread's gamma/beta are loaded before the fold.
template <int KV>
__global__ __launch_bounds__(256) void k_gn_nhwc_apply(
    NhwcSrc x, const float* __restrict__ gamma, const float* __restrict__ beta,
    f16* __restrict__ y, uint32_t C, uint32_t G, uint32_t HW, uint32_t ppc, uint32_t schunks,
    float eps, int silu, const float* __restrict__ part) {
  __shared__ float red[256];
  __shared__ float gstat[2 * 256];  // per group: sums, then (mean, rstd)
  const uint32_t chunk = blockIdx.x, n = blockIdx.y;
  const NhwcMap m = nhwc_map(C);
  const uint32_t lane_cv = threadIdx.x % m.cvb, pl = threadIdx.x / m.cvb;
  const bool active = pl < m.R;
  const NhwcLane<KV> ln(x, m, active ? lane_cv : 0);
  const uint32_t p0 = chunk * ppc, p1 = min(p0 + ppc, HW);
  const uint32_t cnt = active && p0 + pl < p1 ? (p1 - p0 - pl + m.R - 1) / m.R : 0;
  constexpr int U = gn_unroll<KV>();
  // Unconditional loads at pixel indices clamped into [p0, p1) (every chunk is
  // non-empty), so no lane branches around them.
  const uint64_t img = (uint64_t)n * HW;
  const uint32_t pfirst = min(p0 + (active ? pl : 0), p1 - 1);
  f16x8 v[U][KV];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint64_t pix = img + min(pfirst + u * m.R, p1 - 1);
#pragma unroll
    for (int k = 0; k < KV; k++) v[u][k] = ln.load(k, pix);
  }
  f32x4 gam[KV][2], bet[KV][2];
#pragma unroll
  for (int k = 0; k < KV; k++) {
    const uint32_t c = (ln.ok[k] ? ln.cv[k] : 0) * 8;
    gam[k][0] = *(const f32x4*)(gamma + c);
    gam[k][1] = *(const f32x4*)(gamma + c + 4);
    bet[k][0] = *(const f32x4*)(beta + c);
    bet[k][1] = *(const f32x4*)(beta + c + 4);
  }
  sched_fence();
  const uint32_t P = 2 * G;  // (group, statistic) pairs
  const float* pn = part + (uint64_t)n * schunks * P;
  const uint32_t slices = P <= 256 ? 256 / P : 1;
  if (P <= 256) {
    if (threadIdx.x < P * slices)
      red[threadIdx.x] = gn_fold(pn, P, threadIdx.x % P, threadIdx.x / P, slices, schunks);
  } else {
    for (uint32_t pair = threadIdx.x; pair < P; pair += 256)
      gstat[pair] = gn_fold(pn, P, pair, 0, 1, schunks);
  }
  __syncthreads();
  if (P <= 256 && threadIdx.x < P) {
    float a = 0.0f;
    for (uint32_t sl = 0; sl < slices; sl++) a += red[sl * P + threadIdx.x];
    gstat[threadIdx.x] = a;
  }
  __syncthreads();
  const uint32_t cpg = C / G;
  const float L = (float)cpg * (float)HW;
  if (G <= 128 && threadIdx.x < G) {
    const float mean = gstat[2 * threadIdx.x] / L;
    const float var = fmaxf(gstat[2 * threadIdx.x + 1] / L - mean * mean, 0.0f);
    red[threadIdx.x] = mean;
    red[128 + threadIdx.x] = 1.0f / sqrtf(var + eps);
  }
  // G <= 128 keeps mean/rstd in `red`; larger G reuses gstat in place.
  __syncthreads();
  if (G > 128) {
    for (uint32_t g = threadIdx.x; g < G; g += 256) {
      const float mean = gstat[2 * g] / L;
      const float var = fmaxf(gstat[2 * g + 1] / L - mean * mean, 0.0f);
      gstat[2 * g] = mean;
      gstat[2 * g + 1] = 1.0f / sqrtf(var + eps);
    }
    __syncthreads();
  }
  if (!active) return;
  float sa[KV][8], sb[KV][8];
#pragma unroll
  for (int k = 0; k < KV; k++) {
    const uint32_t cb = (ln.ok[k] ? ln.cv[k] : 0) * 8;
    uint32_t g = cb / cpg;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      while (cb + j >= (g + 1) * cpg) g++;
      const float mean = G > 128 ? gstat[2 * g] : red[g];
      const float rstd = G > 128 ? gstat[2 * g + 1] : red[128 + g];
      const float gj = j < 4 ? gam[k][0][j] : gam[k][1][j - 4];
      const float bj = j < 4 ? bet[k][0][j] : bet[k][1][j - 4];
      sa[k][j] = rstd * gj;
      sb[k][j] = bj - mean * sa[k][j];
    }
  }
  for (uint32_t i = 0; i < cnt; i += U) {
    if (i > 0) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint64_t pix = img + min(pfirst + (i + u) * m.R, p1 - 1);
#pragma unroll
        for (int k = 0; k < KV; k++) v[u][k] = ln.load(k, pix);
      }
      sched_fence();
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (i + u >= cnt) break;
      const uint64_t pix = img + pfirst + (i + u) * m.R;
#pragma unroll
      for (int k = 0; k < KV; k++) {
        if (!ln.ok[k]) continue;
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const float t = (float)v[u][k][j] * sa[k][j] + sb[k][j];
          o[j] = (f16)(silu ? silu_f(t) : t);
        }
        *(f16x8*)(y + pix * C + ln.cv[k] * 8) = o;
      }
    }
  }
}

// ---------------- LayerNorm: one wavefront per row ----------------
// fp16 rows with inner % 8 == 0 and inner <= 64*8*kLnMaxV stay in registers
// (one read, vector stores); other shapes take the generic two-read loop.
constexpr int kLnMaxV = 4;

template <int NV>
__global__ __launch_bounds__(256) void k_layer_norm_f16_reg(const f16* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            f16* __restrict__ y, uint32_t rows,
                                                            uint32_t inner, float eps) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const f16* xr = x + (uint64_t)row * inner;
  f16* yr = y + (uint64_t)row * inner;
  f16x8 v[NV];
  f32x4 gm[NV][2], bt[NV][2];
  float s = 0.0f, q = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; k++) {
    uint32_t j = (lane + k * kWave) * 8;
    j = j < inner ? j : 0;  // clamped: every lane loads in bounds
    v[k] = *(const f16x8*)(xr + j);
    gm[k][0] = *(const f32x4*)(gamma + j);
    gm[k][1] = *(const f32x4*)(gamma + j + 4);
    bt[k][0] = *(const f32x4*)(beta + j);
    bt[k][1] = *(const f32x4*)(beta + j + 4);
  }
  sched_fence();
#pragma unroll
  for (int k = 0; k < NV; k++) {
    if ((lane + k * kWave) * 8 < inner) {
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float f = (float)v[k][e];
        s += f;
        q += f * f;
      }
    }
  }
  s = wave_sum(s);
  q = wave_sum(q);
  const float mean = s / (float)inner;
  const float var = fmaxf(q / (float)inner - mean * mean, 0.0f);
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int k = 0; k < NV; k++) {
    const uint32_t j = (lane + k * kWave) * 8;
    if (j < inner) {
      const f32x4 g0 = gm[k][0], g1 = gm[k][1], b0 = bt[k][0], b1 = bt[k][1];
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        o[e] = (f16)(((float)v[k][e] - mean) * rstd * g0[e] + b0[e]);
        o[e + 4] = (f16)(((float)v[k][e + 4] - mean) * rstd * g1[e] + b1[e]);
      }
      *(f16x8*)(yr + j) = o;
    }
  }
}

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

// Slice count per group for the NCHW kernels: ~1024 workgroups in total, at
// least one vector per thread, at most 256 (one partial per thread in the fold).
void nchw_slices(uint32_t L, uint32_t NG, uint32_t vec, uint32_t* S_out, uint32_t* chunk_out) {
  uint32_t S = (1024 + NG - 1) / NG;
  const uint32_t smax = (L + 256 * vec - 1) / (256 * vec);
  if (S > smax) S = smax;
  if (S > 256) S = 256;
  if (S < 1) S = 1;
  uint32_t chunk = (L + S - 1) / S;
  chunk = (chunk + vec - 1) / vec * vec;
  *S_out = (L + chunk - 1) / chunk;
  *chunk_out = chunk;
}

// `fixed` (with `fixed_bytes`) replaces the context workspace for the
// partials when non-null.
template <typename T, int VEC>
int gn_nchw_launch(Ctx* c, const void* x, const float* gamma, const float* beta, void* y,
                   uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu,
                   float* fixed, uint64_t fixed_bytes) {
  const uint32_t L = cpg * HW, NG = N * G;
  uint32_t S, chunk;
  nchw_slices(L, NG, VEC, &S, &chunk);
  const uint64_t need = (uint64_t)NG * S * 2 * sizeof(float);
  void* ws = fixed;
  if (fixed) {
    DI_REQUIRE(need <= fixed_bytes, DI_EUNSUPPORTED,
               "group norm: %llu bytes of partials exceed the %llu-byte static scratch",
               (unsigned long long)need, (unsigned long long)fixed_bytes);
  } else {
    int rc = workspace(c, need, &ws);
    if (rc) return rc;
  }
  float* part = (float*)ws;
  k_gn_nchw_partial<T, VEC><<<dim3(S, NG), 256, 0, c->stream>>>((const T*)x, L, chunk, part);
  k_gn_nchw_apply<T, VEC><<<dim3(S, NG), 256, 0, c->stream>>>(
      (const T*)x, gamma, beta, (T*)y, G, cpg, HW, chunk, eps, silu ? 1 : 0, part);
  return DI_OK;
}

// Slices per group for the single-launch kernel (0: use the two-kernel
// path): the grid should cover the CUs, and every slice re-reads its whole
// group, so no more slices than that.  Groups of more than 64 Ki elements
// (64 floats in registers per thread) or of less than one round of 1024
// vectors (most of a 1024-thread workgroup idle), and fewer than 8 groups
// (too few workgroups whichever way), take the two-kernel path.
// largest per-group round count gn_fused instantiates for a vector width
constexpr uint32_t gn_fused_max_rounds(uint32_t vec) { return vec <= 4 ? 16u : 8u; }

uint32_t gn_fused_slices(uint32_t NG, uint32_t L, uint32_t vec) {
  static const int env = [] {
    const char* e = getenv("DI_GN_FUSED");
    return e ? atoi(e) : 1;
  }();
  if (!env || NG < 8 || L > 64u * kFusedT || L < kFusedT * vec || NG > (1u << 20)) return 0;
  // every round of a group needs an instantiated unroll (gn_fused)
  if ((L + kFusedT * vec - 1) / (kFusedT * vec) > gn_fused_max_rounds(vec)) return 0;
  static const uint32_t env_s = [] {  // tuning override: DI_GN_SLICES=n
    const char* e = getenv("DI_GN_SLICES");
    return e ? (uint32_t)atoi(e) : 0u;
  }();
  uint32_t S = env_s ? env_s : 256 / NG;
  if (S < 1) S = 1;
  if (S > 16) S = 16;
  const uint32_t smax = (L + kFusedT * vec - 1) / (kFusedT * vec);  // at least a round each
  return S < smax ? S : smax;
}

template <typename T, int VEC, int U>
void gn_fused_launch(hipStream_t st, const T* x, const float* gamma, const float* beta, T* y,
                     uint32_t NG, uint32_t G, uint32_t cpg, uint32_t HW, uint32_t S, float eps,
                     bool silu) {
  const uint32_t L = cpg * HW;
  // the kernel reads U rounds of kFusedT * VEC elements per group
  if ((L + kFusedT * VEC - 1) / (kFusedT * VEC) > (uint32_t)U) {
    fprintf(stderr, "gn_fused_launch: %u elements per group exceed %d rounds\n", L, U);
    abort();
  }
  uint32_t chunk = (L + S - 1) / S;
  chunk = (chunk + VEC - 1) / VEC * VEC;
  const uint32_t Sr = (L + chunk - 1) / chunk;  // non-empty slices
  k_gn_nchw_fused<T, VEC, U><<<NG * Sr, kFusedT, 0, st>>>(x, gamma, beta, y, G, cpg, HW, Sr,
                                                           chunk, eps, silu ? 1 : 0);
}

// Launches the single-pass kernel with an unroll U >= the group's rounds of
// kFusedT * VEC elements; returns false (nothing launched) for more rounds
// than any instantiation holds, which gn_fused_slices never plans.
template <typename T, int VEC>
bool gn_fused(hipStream_t st, const T* x, const float* gamma, const float* beta, T* y,
              uint32_t NG, uint32_t G, uint32_t cpg, uint32_t HW, uint32_t S, float eps,
              bool silu) {
  const uint32_t rounds = (cpg * HW + kFusedT * VEC - 1) / (kFusedT * VEC);
  static_assert(gn_fused_max_rounds(VEC) == (VEC <= 4 ? 16u : 8u), "unrolls below");
  if (rounds > gn_fused_max_rounds(VEC)) return false;
#define DI_GN_FUSED_U(u) \
  gn_fused_launch<T, VEC, u>(st, x, gamma, beta, y, NG, G, cpg, HW, S, eps, silu)
  if (rounds <= 1) DI_GN_FUSED_U(1);
  else if (rounds <= 2) DI_GN_FUSED_U(2);
  else if (rounds <= 3) DI_GN_FUSED_U(3);
  else if (rounds <= 4) DI_GN_FUSED_U(4);
  else if (rounds <= 6) DI_GN_FUSED_U(6);
  else if (rounds <= 8) DI_GN_FUSED_U(8);
  else if constexpr (VEC <= 4) {
    if (rounds <= 10) DI_GN_FUSED_U(10);
    else if (rounds <= 12) DI_GN_FUSED_U(12);
    else DI_GN_FUSED_U(16);
  }
#undef DI_GN_FUSED_U
  return true;
}

// The exchange kernel for NG <= kXchgNchwRecs groups whose slices fit kXU rounds
// of kXT vectors; false: nothing launched.  Read at every call (tests switch
// them between calls): DI_GN_XCHG=0 turns the kernel off, DI_GN_XCHG_SPIN
// sets the poll limit (0 forces the recomputing path).
constexpr uint32_t kXU = 8;
template <typename T, int VEC>
bool gn_xchg(Ctx* c, const T* x, const float* gamma, const float* beta, T* y, uint32_t NG,
             uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu) {
  const char* e_on = getenv("DI_GN_XCHG");
  const char* e_spin = getenv("DI_GN_XCHG_SPIN");
  const uint32_t spin = e_spin ? (uint32_t)strtoul(e_spin, nullptr, 10) : 20000u;
  const uint32_t L = cpg * HW;
  if ((e_on && !atoi(e_on)) || !c->gn_xchg || NG == 0 || NG > kXchgNchwRecs || L < kXS * kXT)
    return false;
  uint32_t chunk = (L + kXS - 1) / kXS;
  chunk = (chunk + VEC - 1) / VEC * VEC;
  const uint32_t rounds = (chunk + kXT * VEC - 1) / (kXT * VEC);
  if (rounds > kXU) return false;
  uint64_t* const xa = (uint64_t*)c->gn_xchg;
#define DI_GN_XCHG_U(u)                                                                        \
  k_gn_nchw_xchg<T, VEC, u><<<NG * kXS, kXT, 0, c->stream>>>(x, gamma, beta, y, xa, G, cpg, HW, \
                                                              chunk, eps, silu ? 1 : 0, spin)
  if (rounds <= 1) DI_GN_XCHG_U(1);
  else if (rounds <= 2) DI_GN_XCHG_U(2);
  else if (rounds <= 3) DI_GN_XCHG_U(3);
  else if (rounds <= 4) DI_GN_XCHG_U(4);
  else if (rounds <= 5) DI_GN_XCHG_U(5);
  else DI_GN_XCHG_U(8);
#undef DI_GN_XCHG_U
  return true;
}

template <typename T>
int gn_nchw(Ctx* c, const void* x, const float* gamma, const float* beta, void* y, uint32_t N,
            uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu, float* fixed,
            uint64_t fixed_bytes) {
  DI_REQUIRE((uint64_t)N * G <= 65535u, DI_EUNSUPPORTED, "group norm: %llu groups exceed 65535",
             (unsigned long long)N * G);
  DI_REQUIRE((uint64_t)cpg * HW < (1ull << 31), DI_EUNSUPPORTED,
             "group norm: %llu elements per group exceed 2^31", (unsigned long long)cpg * HW);
  constexpr int V = 16 / sizeof(T);
  if (HW % V == 0 &&
      gn_xchg<T, V>(c, (const T*)x, gamma, beta, (T*)y, N * G, G, cpg, HW, eps, silu))
    return DI_OK;
  if (HW % V == 0) {
    const uint32_t S = gn_fused_slices(N * G, cpg * HW, V);
    if (S && gn_fused<T, V>(c->stream, (const T*)x, gamma, beta, (T*)y, N * G, G, cpg, HW, S,
                            eps, silu))
      return DI_OK;
  }
  if (HW % V == 0)
    return gn_nchw_launch<T, V>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, fixed,
                                fixed_bytes);
  return gn_nchw_launch<T, 1>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, fixed,
                              fixed_bytes);
}

int gn_nchw_dt(Ctx* c, const void* x, const float* gamma, const float* beta, void* y,
               uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps, bool silu, int dt,
               float* fixed, uint64_t fixed_bytes) {
  if (dt == DI_F32)
    return gn_nchw<float>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, fixed, fixed_bytes);
  return gn_nchw<f16>(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, fixed, fixed_bytes);
}

}  // namespace

uint64_t gn_xchg_bytes() {
  return (uint64_t)(kXchgNchwRecs + kXchgRedRecs + kXchgRed4Recs) * kXchgWords * sizeof(uint64_t);
}

int launch_group_norm_nchw(Ctx* c, const void* x, const float* gamma, const float* beta,
                           void* y, uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW,
                           float eps, bool silu, int dt) {
  return gn_nchw_dt(c, x, gamma, beta, y, N, G, cpg, HW, eps, silu, dt, nullptr, 0);
}

uint32_t gn_nhwc_chunks(uint32_t N, uint32_t HW) {
  // ~256 partial-statistics workgroups over the batch, at most 64 per image
  // (every apply workgroup folds one image's partials).
  uint32_t c = (256 + N - 1) / N;
  if (c > 64) c = 64;
  if (c > HW) c = HW;
  const uint32_t ppc = (HW + c - 1) / c;
  return (HW + ppc - 1) / ppc;
}

uint64_t gn_nhwc_ws_floats(uint32_t N, uint32_t C, uint32_t G, uint32_t HW) {
  (void)C;
  return (uint64_t)N * gn_nhwc_chunks(N, HW) * G * 2;
}

void launch_group_norm_nhwc(hipStream_t s, NhwcSrc x, const float* gamma, const float* beta,
                            void* y, uint32_t N, uint32_t C, uint32_t G, uint32_t HW, float eps,
                            bool silu, float* ws) {
  const uint32_t sch = gn_nhwc_chunks(N, HW);
  const uint32_t sppc = (HW + sch - 1) / sch;
  const NhwcMap m = nhwc_map(C);
  // apply: ~2 workgroups per CU over the batch, >= 2 pixels per pixel lane
  uint32_t ach = (512 + N - 1) / N;
  const uint32_t maxch = (HW + 2 * m.R - 1) / (2 * m.R);
  if (ach > maxch) ach = maxch;
  if (ach < 1) ach = 1;
  const uint32_t appc = (HW + ach - 1) / ach;
  ach = (HW + appc - 1) / appc;
  const size_t lds_p = (size_t)2 * C * m.R * sizeof(float);
  const int si = silu ? 1 : 0;
  if (m.kv == 1) {
    k_gn_nhwc_partial<1><<<dim3(sch, N), 256, lds_p, s>>>(x, C, G, HW, sppc, ws);
    k_gn_nhwc_apply<1><<<dim3(ach, N), 256, 0, s>>>(x, gamma, beta, (f16*)y, C, G, HW, appc, sch,
                                                     eps, si, ws);
  } else {
    k_gn_nhwc_partial<2><<<dim3(sch, N), 256, lds_p, s>>>(x, C, G, HW, sppc, ws);
    k_gn_nhwc_apply<2><<<dim3(ach, N), 256, 0, s>>>(x, gamma, beta, (f16*)y, C, G, HW, appc, sch,
                                                     eps, si, ws);
  }
}

bool gn_stats_slice(uint32_t C, uint32_t G, uint32_t HW, uint32_t* sw) {
  if (G == 0 || C % G != 0 || HW % 64 != 0) return false;
  const uint32_t cpg = C / G;
  uint32_t l = cpg;
  while (l % 8 != 0) l += cpg;  // lcm(cpg, 8)
  for (uint32_t w = l; w <= (uint32_t)kGnSliceMax; w += l) {
    if (C % w == 0 && (w >= 64 || w == C || w + l > (uint32_t)kGnSliceMax)) {
      *sw = w;
      return true;
    }
  }
  return false;
}

uint64_t gn_fold_ws_floats(uint32_t N, uint32_t C, uint32_t HW) {
  const uint32_t cpi = HW / 64;
  if (cpi <= kGnFoldMin) return 0;
  const uint32_t F = (cpi + kGnFoldTarget - 1) / kGnFoldTarget;
  return (uint64_t)N * ((cpi + F - 1) / F) * C * 2;
}

bool gn_side_gemv_ok(const GemvArgs& g) {
  return g.vec_ok && g.x_mode != GEMV_X_SINUSOID && g.N > 0 && g.K % 8 == 0 &&
         g.K <= 64 * 8 * 3 && g.B >= 1 && g.B <= 2 && (uint64_t)g.B * g.K <= kGnSideX;
}

bool launch_group_norm_nhwc_st(hipStream_t s, NhwcSrc x, const GnStats& st_in, const float* gamma,
                               const float* beta, void* y, uint32_t N, uint32_t C, uint32_t G,
                               uint32_t HW, float eps, bool silu, float* fold_ws,
                               const GemvArgs* side) {
  uint32_t sw = 0;
  if (!gn_stats_slice(C, G, HW, &sw) || x.c1 % 8 != 0 || (st_in.c1 < C && st_in.c1 % 8 != 0))
    return false;
  GnStats st = st_in;
  uint32_t cpi = HW / 64;
  if (fold_ws && cpi > kGnFoldMin) {
    const uint32_t F = (cpi + kGnFoldTarget - 1) / kGnFoldTarget, cpo = (cpi + F - 1) / F;
    k_gn_stats_fold<<<dim3((2 * C + 255) / 256, cpo, N), 256, 0, s>>>(st_in, fold_ws, C, cpi, F,
                                                                     cpo);
    st = GnStats{fold_ws, fold_ws, C, C, C};
    cpi = cpo;
  }
  const uint32_t slices = C / sw, R = 256 / (sw / 8);
  // about 256 workgroups over the batch, 512 for tensors of 16 MiB and more
  // (measured: U-Net step and VAE decode; DI_GN_WGS overrides, for tuning
  // sweeps), at least one pixel per lane
  static const int wgs_env = [] {
    const char* e = getenv("DI_GN_WGS");
    return e ? atoi(e) : 0;
  }();
  const uint32_t wgs = wgs_env > 0 ? (uint32_t)wgs_env
                       : (uint64_t)N * HW * C * 2 >= (16ull << 20) ? 2 * kGnApplyWgs
                                                                    : kGnApplyWgs;
  uint32_t pbs = wgs / (N * slices);
  const uint32_t maxpb = (HW + R - 1) / R;
  if (pbs > maxpb) pbs = maxpb;
  if (pbs < 1) pbs = 1;
  const uint32_t ppb = (HW + pbs - 1) / pbs;
  pbs = (HW + ppb - 1) / ppb;
  // statistics chunks per lane: KL lanes per channel quad
  const uint32_t kl_lanes = 256 / (sw / 4), need = (cpi + kl_lanes - 1) / kl_lanes;
  // a side-job GEMV takes whole extra z-planes of pbs x slices blocks
  const bool sj = side && gn_side_gemv_ok(*side);
  const uint32_t plane = pbs * slices;
  const uint32_t zs = sj ? (gemv_side_blocks(side->N, 8) + plane - 1) / plane : 0;
  const dim3 grid(pbs, slices, N + zs);
  GemvArgs none;
  none.N = 0;
  const GemvArgs& gv = sj ? *side : none;
#define DI_GN_ST(NUV)                                                                            \
  if (sj)                                                                                        \
    k_gn_nhwc_apply_st<NUV, true><<<grid, 256, 0, s>>>(x, st, gamma, beta, (f16*)y, C, C / G, sw, \
                                                       HW, ppb, eps, silu ? 1 : 0, cpi, N, gv);  \
  else                                                                                           \
    k_gn_nhwc_apply_st<NUV, false><<<grid, 256, 0, s>>>(x, st, gamma, beta, (f16*)y, C, C / G,    \
                                                        sw, HW, ppb, eps, silu ? 1 : 0, cpi, N,  \
                                                        gv);
  if (need <= 1) {
    DI_GN_ST(1)
  } else if (need <= 2) {
    DI_GN_ST(2)
  } else if (need <= 4) {
    DI_GN_ST(4)
  } else {
    DI_GN_ST(8)
  }
#undef DI_GN_ST
  return true;
}

void launch_layer_norm(hipStream_t s, const void* x, const float* gamma, const float* beta,
                       void* y, uint32_t rows, uint32_t inner, float eps, int dt) {
  const unsigned g = (rows + 3) / 4;
  if (dt == DI_F16 && inner % 8 == 0 && inner <= 64u * 8u * kLnMaxV) {
    const f16* xp = (const f16*)x;
    f16* yp = (f16*)y;
    const uint32_t nv = (inner / 8 + 63) / 64;
    if (nv == 1)
      k_layer_norm_f16_reg<1><<<g, 256, 0, s>>>(xp, gamma, beta, yp, rows, inner, eps);
    else if (nv == 2)
      k_layer_norm_f16_reg<2><<<g, 256, 0, s>>>(xp, gamma, beta, yp, rows, inner, eps);
    else
      k_layer_norm_f16_reg<4><<<g, 256, 0, s>>>(xp, gamma, beta, yp, rows, inner, eps);
  } else if (dt == DI_F32) {
    k_layer_norm<float><<<g, 256, 0, s>>>((const float*)x, gamma, beta, (float*)y, rows, inner, eps);
  } else {
    k_layer_norm<f16><<<g, 256, 0, s>>>((const f16*)x, gamma, beta, (f16*)y, rows, inner, eps);
  }
}

// ---- LayerNorm folded into the consuming projection ----
// Row statistics: (sum, sum of squares) of each fp16 row, one wavefront per
// row (inner % 8 == 0).
__global__ __launch_bounds__(256) void k_row_stats_f16(const f16* __restrict__ x,
                                                       float* __restrict__ out, uint32_t rows,
                                                       uint32_t inner) {
  const uint32_t row = blockIdx.x * 4 + threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const f16* xr = x + (uint64_t)row * inner;
  float s = 0.0f, q = 0.0f;
  for (uint32_t j = lane * 8; j < inner; j += kWave * 8) {
    const f16x8 v = *(const f16x8*)(xr + j);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float f = (float)v[e];
      s += f;
      q += f * f;
    }
  }
  s = wave_sum(s);
  q = wave_sum(q);
  if (lane == 0) *(float2*)(out + (uint64_t)row * 2) = float2{s, q};
}

void launch_row_stats(hipStream_t s, const f16* x, float* out, uint32_t rows, uint32_t inner) {
  k_row_stats_f16<<<(rows + 3) / 4, 256, 0, s>>>(x, out, rows, inner);
}

// Weight fold, one wavefront per output row n (K % 8 == 0):
// wf[n][k] = fp16(gamma[k] * w[n][k]), sum[n] = sum_k wf[n][k] (the rounded
// values, so the epilogue's mean term matches what the GEMM multiplies) and
// cst[n] = sum_k beta[k] * w[n][k] + bias[n].
__global__ __launch_bounds__(256) void k_ln_fold(const f16* __restrict__ w,
                                                 const float* __restrict__ gamma,
                                                 const float* __restrict__ beta,
                                                 const float* __restrict__ bias,
                                                 f16* __restrict__ wf, float* __restrict__ sum,
                                                 float* __restrict__ cst, uint32_t N, uint32_t K) {
  const uint32_t n = blockIdx.x * 4 + threadIdx.x / kWave;
  const uint32_t lane = threadIdx.x % kWave;
  if (n >= N) return;
  const f16* wr = w + (uint64_t)n * K;
  f16* fr = wf + (uint64_t)n * K;
  float sw = 0.0f, cb = 0.0f;
  for (uint32_t k = lane * 8; k < K; k += kWave * 8) {
    const f16x8 v = *(const f16x8*)(wr + k);
    const f32x4 g[2] = {*(const f32x4*)(gamma + k), *(const f32x4*)(gamma + k + 4)};
    const f32x4 b[2] = {*(const f32x4*)(beta + k), *(const f32x4*)(beta + k + 4)};
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float wv = (float)v[e];
      o[e] = (f16)(wv * g[e >> 2][e & 3]);
      sw += (float)o[e];
      cb += b[e >> 2][e & 3] * wv;
    }
    *(f16x8*)(fr + k) = o;
  }
  sw = wave_sum(sw);
  cb = wave_sum(cb);
  if (lane == 0) {
    sum[n] = sw;
    cst[n] = cb + (bias ? bias[n] : 0.0f);
  }
}

void launch_ln_fold(hipStream_t s, const f16* w, const float* gamma, const float* beta,
                    const float* bias, f16* wf, float* sum, float* cst, uint32_t N, uint32_t K) {
  k_ln_fold<<<(N + 3) / 4, 256, 0, s>>>(w, gamma, beta, bias, wf, sum, cst, N, K);
}

// ---------------- static scratch (di_group_norm_noalloc) ----------------
// Partials of the no-allocation entry point live in this file-scope device
// array instead of the context workspace: each GPU the library runs on holds
// one copy until the process ends.  Host code never uses the array's name as
// an address; it uses the device address hipGetSymbolAddress returns, looked
// up once per device (with that device current) and kept per device.
constexpr uint64_t kScratchBytes = 1ull << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the context's device (current on entry).
int scratch_ptr(Ctx* c, float** out) {
  DI_REQUIRE(c->device >= 0 && c->device < kMaxDevices, DI_EUNSUPPORTED,
             "static scratch: device %d out of range", c->device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[c->device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    DI_REQUIRE(e == hipSuccess && p != nullptr, DI_EHIP,
               "hipGetSymbolAddress(scratch) on device %d failed: %s", c->device,
               hipGetErrorString(e));
    g_scratch_ptr[c->device] = p;
  }
  *out = (float*)g_scratch_ptr[c->device];
  return DI_OK;
}

}  // namespace

// Shared body of di_group_norm and di_group_norm_noalloc: `fixed` (non-null)
// holds the partials instead of the context workspace.
int group_norm_impl(Ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                    uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps, int32_t flags,
                    int32_t dt, int32_t layout, float* fixed, uint64_t fixed_bytes);

}  // namespace di

using namespace di;

int di::group_norm_impl(Ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                        uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps,
                        int32_t flags, int32_t dt, int32_t layout, float* fixed,
                        uint64_t fixed_bytes) {
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
    int rc = gn_nchw_dt(ctx, x->ptr, (const float*)g->ptr, (const float*)b->ptr, y->ptr, N, G,
                        cpg, HW, eps, silu, dt, fixed, fixed_bytes);
    if (rc) return rc;
  } else {
    DI_REQUIRE(dt == DI_F16, DI_EUNSUPPORTED, "di_group_norm: NHWC requires fp16");
    DI_REQUIRE(C % 8 == 0 && C <= 4096 && G <= 256, DI_EUNSUPPORTED,
               "di_group_norm: NHWC needs C %% 8 == 0, C <= 4096, G <= 256 (C=%u G=%u)", C, G);
    DI_REQUIRE(N <= 65535u, DI_EUNSUPPORTED, "di_group_norm: batch too large");
    const uint64_t need = gn_nhwc_ws_floats(N, C, G, HW) * sizeof(float);
    void* ws = fixed;
    if (fixed) {
      DI_REQUIRE(need <= fixed_bytes, DI_EUNSUPPORTED,
                 "group norm: %llu bytes of partials exceed the %llu-byte static scratch",
                 (unsigned long long)need, (unsigned long long)fixed_bytes);
    } else {
      int rc = workspace(ctx, need, &ws);
      if (rc) return rc;
    }
    NhwcSrc src{(const f16*)x->ptr, (const f16*)x->ptr, C, C, C};
    launch_group_norm_nhwc(ctx->stream, src, (const float*)g->ptr, (const float*)b->ptr, y->ptr,
                           N, C, G, HW, eps, silu, (float*)ws);
  }
  DI_LAUNCH_CHECK();
  return DI_OK;
}

extern "C" {

int32_t di_group_norm(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta, di_handle Y,
                      uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW, float eps,
                      int32_t flags, int32_t dt, int32_t layout) {
  DI_CTX(ctx);
  return group_norm_impl(ctx, X, gamma, beta, Y, N, G, cpg, HW, eps, flags, dt, layout, nullptr,
                         0);
}

int32_t di_group_norm_noalloc(di_ctx* ctx, di_handle X, di_handle gamma, di_handle beta,
                              di_handle Y, uint32_t N, uint32_t G, uint32_t cpg, uint32_t HW,
                              float eps, int32_t flags, int32_t dt, int32_t layout) {
  DI_CTX(ctx);
  float* fixed = nullptr;
  int rc = scratch_ptr(ctx, &fixed);
  if (rc) return rc;
  return group_norm_impl(ctx, X, gamma, beta, Y, N, G, cpg, HW, eps, flags, dt, layout, fixed,
                         kScratchBytes);
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

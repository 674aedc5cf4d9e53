// MFMA GEMM and implicit-GEMM convolution for gfx950, with fused epilogues.
//
//   C[b][m][n] = epi( alpha * sum_k A[b][m][k] * B[b][n][k] )
//
// One template covers every contraction of the U-Net path:
//  * linear projections (proj_in/out, Q/K/V, to_out, GEGLU, FF out, temb)
//    with A dense rows (tokens x channels, NHWC activations are tokens);
//  * convolutions as implicit GEMM: m = output pixel, n = output channel,
//    k = (ky, kx, ci) over an NHWC fp16 input and OHWI weights, so both
//    operands are read as 16-byte k-contiguous vectors; the gather supports
//    stride 2 (downsample), a fused 2x nearest upsample of the input
//    (Upsample2D), and a channel concat of two sources (up-block skips);
//  * the reference's fp32 ops (matmul wgsl-ops.js:477-556, gemm :821-897,
//    convMM :584-698 with its (ci, ky, kx) k order on NCHW) through an fp32
//    MFMA variant with exact fp32 products.
// Epilogue: alpha, per-column bias, per-(batch, column) bias (ResNet temb),
// residual add, GELU(erf) / GEGLU / SiLU, fp16 or fp32 store, NHWC or NCHW.
//
// Tiling: 256 threads = 4 wavefronts in a WGM x WGN grid; block tile BM x BN;
// K staged 128 bytes per row per stage through double-buffered LDS with the
// next stage prefetched into registers while the MFMAs of the current one
// run (one barrier per stage).  fp16 uses v_mfma_f32_16x16x32_f16 (lane l
// holds row l%16, k (l/16)*8..+7; C rows (l/16)*4..+3, col l%16), fp32 uses
// v_mfma_f32_16x16x4_f32 (k = l/16).  Split-K writes fp32 partials that a
// second kernel reduces and passes through the same epilogue.
//
// This header holds the device code (the kernel template, its loaders and
// epilogues) and the launchers of each instantiation family; the families
// are compiled in separate translation units (k_gemm_*.hip) so the build
// runs in parallel, and k_gemm.hip holds the host-side planning, the
// split-K reducers and launch_gemm.
#pragma once

#include <cmath>
#include <cstdio>
#include <cstdlib>

#include <type_traits>

#include "di_device.h"
#include "di_gemm.h"
#include "di_kernels.h"

namespace di {

namespace {


template <typename T>
struct Mfma;

template <>
struct Mfma<f16> {
  static constexpr int KV = 8;   // elements per 16-byte vector
  static constexpr int KM = 32;  // k per MFMA
  static constexpr int FK = 8;   // k per lane fragment
  typedef f16x8 vec;
  typedef f16x8 frag;
  __device__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<float> {
  static constexpr int KV = 4;
  static constexpr int KM = 4;
  static constexpr int FK = 1;
  typedef f32x4 vec;
  typedef float frag;
  __device__ static f32x4 mma(frag a, frag b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ typename Mfma<T>::frag ld_frag(const T* p) {
  return *(const typename Mfma<T>::frag*)p;
}

template <typename T>
__device__ __forceinline__ typename Mfma<T>::vec zero_vec() {
  typename Mfma<T>::vec v;
#pragma unroll
  for (int j = 0; j < Mfma<T>::KV; j++) v[j] = (T)0;
  return v;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // raw buffer, stride 0; dword3 0x00020000 is the gfx9-family data format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <typename V>
__device__ __forceinline__ V buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// voff per lane, soff uniform (scalar register): the per-stage advance costs
// no vector instructions
template <typename V>
__device__ __forceinline__ V buf_load16s(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// ---- epilogue (shared by the GEMM kernel and the split-K reducer) ----
template <typename T>
__device__ __forceinline__ float epi_value(const GemmArgs& g, uint32_t bz, uint32_t m, uint32_t n,
                                           float acc) {
  float v = acc * g.alpha;
  if (g.bias) v += g.bias[n];
  if (g.bias2) v += g.bias2[(uint64_t)(m / g.rows_b2) * g.ld_b2 + n];
  return v;
}

__device__ __forceinline__ float apply_act(int act, float v) {
  if (act == ACT_GELU) return gelu_erf_f(v);
  if (act == ACT_SILU) return silu_f(v);
  if (act == ACT_GELU_TANH) return gelu_tanh_f(v);
  return v;
}

// Final store of one output element (after activation / GEGLU combination).
// The residual has the layout and row stride conventions of C.
__device__ __forceinline__ void store_out(const GemmArgs& g, uint32_t bz, uint32_t m, uint32_t n,
                                          uint32_t ncols, float v) {
  uint64_t off, roff;
  if (g.c_nchw) {
    uint32_t img = m / g.c_hw, p = m % g.c_hw;
    uint64_t e = ((uint64_t)img * ncols + n) * g.c_hw + p;
    off = (uint64_t)bz * g.sc + e;
    roff = (uint64_t)bz * g.sr + e;
  } else {
    off = (uint64_t)bz * g.sc + (uint64_t)m * g.ldc + n;
    roff = (uint64_t)bz * g.sr + (uint64_t)m * g.ldr + n;
  }
  if (g.res) v += g.res_f32 ? ((const float*)g.res)[roff] : (float)((const f16*)g.res)[roff];
  if (g.c_f32) ((float*)g.c)[off] = v;
  else ((f16*)g.c)[off] = (f16)v;
}

// ---- vector epilogue (8 consecutive columns per thread) ----
__device__ __forceinline__ void act8(int act, float* v) {
  switch (act) {
    case ACT_GELU:
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = gelu_erf_f(v[j]);
      break;
    case ACT_SILU:
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = silu_f(v[j]);
      break;
    case ACT_GELU_TANH:
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = gelu_tanh_f(v[j]);
      break;
    default:
      break;
  }
}

__device__ __forceinline__ f32x4 ld4(const float* p) { return *(const f32x4*)p; }

// LayerNorm fold (g.ln_rows): mean and rstd of A row m from its row
// statistics, summed in column-tile order.  The first kLnBatch pairs are
// loaded together (indices clamped to the row), so one memory latency
// covers rows of up to kLnBatch column tiles; ln_load issues them and
// ln_reduce consumes them, which lets a caller overlap the latency.
constexpr int kLnBatch = 8;

__device__ __forceinline__ void ln_load(const GemmArgs& g, uint32_t m, float2* v) {
  const float2* p = (const float2*)g.ln_rows + (uint64_t)m * g.ln_nt;
#pragma unroll
  for (int i = 0; i < kLnBatch; i++) v[i] = p[min((uint32_t)i, g.ln_nt - 1)];
}

__device__ __forceinline__ void ln_reduce(const GemmArgs& g, uint32_t m, const float2* v,
                                          float& mean, float& rstd) {
  float s = 0.0f, q = 0.0f;
#pragma unroll
  for (int i = 0; i < kLnBatch; i++) {
    if ((uint32_t)i < g.ln_nt) {
      s += v[i].x;
      q += v[i].y;
    }
  }
  const float2* p = (const float2*)g.ln_rows + (uint64_t)m * g.ln_nt;
  for (uint32_t t = kLnBatch; t < g.ln_nt; t++) {
    const float2 w = p[t];
    s += w.x;
    q += w.y;
  }
  mean = s / (float)g.K;
  const float var = fmaxf(q / (float)g.K - mean * mean, 0.0f);
  rstd = 1.0f / sqrtf(var + g.ln_eps);
}

__device__ __forceinline__ void ln_coef(const GemmArgs& g, uint32_t m, float& mean, float& rstd) {
  float2 v[kLnBatch];
  ln_load(g, m, v);
  ln_reduce(g, m, v, mean, rstd);
}

// x[j] = rstd * (x[j] - mean * s[j]) for one 8-column vector.
__device__ __forceinline__ void ln_fold8(float* x, float mean, float rstd, const f32x4* s) {
#pragma unroll
  for (int j = 0; j < 8; j++) x[j] = rstd * (x[j] - mean * s[j >> 2][j & 3]);
}

// x = act(x*alpha + bias[n..n+8) + bias2[(m/rows_b2)*ld_b2 + n..]) for one
// vector whose operand loads (bb = bias, tb = bias2) were issued earlier.
__device__ __forceinline__ void epi_math8(const GemmArgs& g, float* x, const f32x4* bb,
                                          const f32x4* tb) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    float v = x[j] * g.alpha;
    if (g.bias) v += bb[j >> 2][j & 3];
    if (g.bias2) v += tb[j >> 2][j & 3];
    x[j] = v;
  }
  act8(g.act, x);
}

// Epilogue extras of the dense buffer-load kernels (template parameter EX):
// EX_ROWSTATS writes g.rstats, EX_LNFOLD applies the LayerNorm fold of
// g.ln_*.  Separate instantiations keep their registers out of every other
// GEMM's allocation.
enum { EX_NONE = 0, EX_ROWSTATS = 1, EX_LNFOLD = 2 };

// Barrier for hand-offs through LDS inside a workgroup: waits for the
// wave's LDS operations only and meets the other waves, leaving global
// loads in flight (__syncthreads also waits for those); the signal fences
// keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt not waited on
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// The vector epilogue's operands (bias, temb bias, residual) for one batch
// of up to 4 output vectors of a thread: vector v0 + u is 8 columns of one
// row of the BM x BN tile.  A kernel loads the first batch with epi_prefetch
// before it stages the C tile in LDS, so the loads' latency overlaps the
// staging.
template <int BM, int BN, int NT>
struct EpiOps {
  static constexpr int VPR8 = BN / 8;
  static constexpr int NV = (BM * VPR8 + NT - 1) / NT;
  static constexpr int CH = NV < 4 ? NV : 4;  // vectors per load batch
  f32x4 bb[CH][2], tb[CH][2];
  f16x8 rr[CH];
};

template <int BM, int BN, int NT>
__device__ __forceinline__ void epi_load(const GemmArgs& g, uint32_t m0, uint32_t n0, uint32_t bz,
                                         int v0, EpiOps<BM, BN, NT>& o) {
  using O = EpiOps<BM, BN, NT>;
  const int tid = threadIdx.x;
  const f16* R = (const f16*)g.res + (uint64_t)bz * g.sr;
#pragma unroll
  for (int u = 0; u < O::CH; u++) {
    const int idx = tid + (v0 + u) * NT;
    const int r = idx / O::VPR8, c8 = (idx % O::VPR8) * 8;
    const uint32_t m = m0 + r, n = n0 + c8;
    const bool ok = v0 + u < O::NV && idx < BM * O::VPR8 && m < g.M && n < g.N;
    const uint32_t mc = ok ? m : m0, nc = ok ? n : n0;
    if (g.bias) {
      o.bb[u][0] = ld4(g.bias + nc);
      o.bb[u][1] = ld4(g.bias + nc + 4);
    }
    if (g.bias2) {
      const float* t = g.bias2 + (uint64_t)(mc / g.rows_b2) * g.ld_b2 + nc;
      o.tb[u][0] = ld4(t);
      o.tb[u][1] = ld4(t + 4);
    }
    if (g.res) o.rr[u] = *(const f16x8*)(R + (uint64_t)mc * g.ldr + nc);
  }
}

// Column n's place in one split's [M][N] block of partials: partial (m, n)
// sits at m * stride + offset, row-major (stride N, offset n) or in column
// groups of g.part_cpg (GemmArgs::part_cpg).  Callers take it once per
// column, outside their row loops.  The group index comes from a float
// reciprocal: exact for n < 2^21 (the product stays 0.5 / part_cpg away
// from an integer, far beyond its rounding error).
struct PartCol {
  uint32_t stride;
  uint64_t offset;
};
__device__ __forceinline__ PartCol part_col(const GemmArgs& g, uint32_t n) {
  if (!g.part_cpg) return PartCol{g.N, n};
  const uint32_t gi =
      (uint32_t)(((float)n + 0.5f) * __builtin_amdgcn_rcpf((float)g.part_cpg));
  return PartCol{g.part_cpg, (uint64_t)gi * g.M * g.part_cpg + (n - gi * g.part_cpg)};
}

// GEGLU vector v of a thread: 8 outputs of tile row r from hidden columns
// cl .. cl + 7 and gate columns cl + 16 .. cl + 23 (32-column groups
// [16 hidden | 16 gate]), written at output column f
template <int BN, int NT>
struct GegluVec {
  static constexpr int VPRG = BN / 16;
  int r, cl;
  __device__ __forceinline__ GegluVec(int v) {
    const int idx = (int)threadIdx.x + v * NT;
    r = idx / VPRG;
    const int q = idx % VPRG;
    cl = (q >> 1) * 32 + (q & 1) * 8;
  }
};

// All of a thread's GEGLU operand loads (hidden / gate bias, residual) into
// o.bb / o.tb / o.rr, one entry per vector (BM * BN / 16 / NT of them, at
// most EpiOps' batch), at clamped in-range addresses
template <int BM, int BN, int NT>
__device__ __forceinline__ void epi_load_geglu(const GemmArgs& g, uint32_t m0, uint32_t n0,
                                               uint32_t bz, EpiOps<BM, BN, NT>& o) {
  using O = EpiOps<BM, BN, NT>;
  constexpr int VPRG = BN / 16, NVG = (BM * VPRG + NT - 1) / NT;
  static_assert(NVG <= O::CH, "GEGLU vectors fit the operand batch");
  const f16* R = (const f16*)g.res + (uint64_t)bz * g.sr;
#pragma unroll
  for (int v = 0; v < NVG; v++) {
    const GegluVec<BN, NT> e(v);
    const uint32_t m = m0 + e.r, nh = n0 + e.cl;
    const bool ok = (int)threadIdx.x + v * NT < BM * VPRG && m < g.M && nh < g.N;
    const uint32_t nhc = ok ? nh : n0, f = (nhc / 32) * 16 + (nhc % 32);
    if (g.bias) {
      o.bb[v][0] = ld4(g.bias + nhc);
      o.bb[v][1] = ld4(g.bias + nhc + 4);
      o.tb[v][0] = ld4(g.bias + nhc + 16);
      o.tb[v][1] = ld4(g.bias + nhc + 20);
    }
    if (g.res) o.rr[v] = *(const f16x8*)(R + (uint64_t)(ok ? m : m0) * g.ldr + f);
  }
}

// First-batch operands for gemm_epilogue_vec, or nothing when that
// epilogue will not use them (split-K partials).
template <int BM, int BN, int NT>
__device__ __forceinline__ void epi_prefetch(const GemmArgs& g, uint32_t m0, uint32_t n0, uint32_t bz,
                                             EpiOps<BM, BN, NT>& o) {
  if (g.splits > 1 || g.act == ACT_GEGLU) return;
  epi_load<BM, BN, NT>(g, m0, n0, bz, 0, o);
}

// Writes (GEGLU-combined when act == GEGLU) results for the rows/columns of
// one C tile staged in LDS as fp32 sC[BM][LDC], or as the sum of NSUM
// partial tiles of that layout tstride floats apart (added in tile order),
// where a kernel stages its k parts separately.  Split-K partials are
// stored as fp32 vectors instead.  All operand loads of a batch of vectors
// are issued before any is consumed; `pre` holds the first batch's when the
// kernel prefetched them (epi_prefetch with the same tile).  EX_LNFOLD with
// sln: sln holds (mean, rstd) of each tile row, then ln_s of each tile
// column, and the LayerNorm fold rstd * (sum - mean * ln_s[n]) is applied
// to the summed tile (without sln the caller has applied it while staging).
template <int BM, int BN, int LDC, int NT, int EX, int NSUM = 1>
__device__ __forceinline__ void gemm_epilogue_vec(const GemmArgs& g, const float* sC, uint32_t m0,
                                                  uint32_t n0, uint32_t bz, uint32_t split,
                                                  const EpiOps<BM, BN, NT>* pre = nullptr,
                                                  int tstride = 0, const float* sln = nullptr) {
  const int tid = threadIdx.x;
  auto tile4 = [&](int i) {
    f32x4 v = ld4(&sC[i]);
#pragma unroll
    for (int t = 1; t < NSUM; t++) v += ld4(&sC[i + t * tstride]);
    return v;
  };
  if (g.splits > 1) {
    constexpr int VPR4 = BN / 4;
    constexpr int NV = (BM * VPR4 + NT - 1) / NT;
    float* P = g.part + ((uint64_t)(split + g.part_slot0) * g.batch + bz) * (uint64_t)g.M * g.N;
    if constexpr (NT % VPR4 == 0) {
      // a thread keeps one 4-column slot for all its vectors
      const int c4 = (tid % VPR4) * 4, r0 = tid / VPR4;
      const uint32_t n = n0 + c4;
      const PartCol pc = part_col(g, n);
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int r = r0 + v * (NT / VPR4);
        const uint32_t m = m0 + r;
        if (r < BM && m < g.M && n < g.N)
          *(f32x4*)&P[(uint64_t)m * pc.stride + pc.offset] = tile4(r * LDC + c4);
      }
    } else {
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int idx = tid + v * NT;
        if (idx < BM * VPR4) {
          const int r = idx / VPR4, c4 = (idx % VPR4) * 4;
          const uint32_t m = m0 + r, n = n0 + c4;
          const PartCol pc = part_col(g, n);
          if (m < g.M && n < g.N) *(f32x4*)&P[(uint64_t)m * pc.stride + pc.offset] = tile4(r * LDC + c4);
        }
      }
    }
    return;
  }
  f16* C = (f16*)g.c + (uint64_t)bz * g.sc;
  if (g.act == ACT_GEGLU) {
    // 32-column groups [16 hidden | 16 gate]; a vector is 8 outputs from
    // hidden columns cl..cl+7 and gate columns cl+16..cl+23.  Its operands
    // were prefetched (or are loaded here, all before any is consumed).
    constexpr int VPRG = BN / 16;
    constexpr int NV = (BM * VPRG + NT - 1) / NT;
    EpiOps<BM, BN, NT> ops;
    epi_load_geglu<BM, BN, NT>(g, m0, n0, bz, ops);
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const GegluVec<BN, NT> e(v);
      const int r = e.r, cl = e.cl;
      const uint32_t m = m0 + r, nh = n0 + cl;
      const bool ok = tid + v * NT < BM * VPRG && m < g.M && nh < g.N;
      const uint32_t f = (nh / 32) * 16 + (nh % 32);
      float h[8], gt[8];
      const int rt = tid + v * NT < BM * VPRG ? r : 0;
      {
        const int i = rt * LDC + cl;
        const f32x4 h0 = tile4(i), h1 = tile4(i + 4), g0 = tile4(i + 16), g1 = tile4(i + 20);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          h[j] = h0[j];
          h[j + 4] = h1[j];
          gt[j] = g0[j];
          gt[j + 4] = g1[j];
        }
      }
      if (EX == EX_LNFOLD && sln) {
        const float2 mr = *(const float2*)&sln[2 * rt];
#pragma unroll
        for (int j = 0; j < 8; j++) {
          h[j] = mr.y * (h[j] - mr.x * sln[2 * BM + cl + j]);
          gt[j] = mr.y * (gt[j] - mr.x * sln[2 * BM + cl + 16 + j]);
        }
      }
      // bias only (no bias2 / activation on GEGLU projections)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float hv = h[j] * g.alpha + (g.bias ? ops.bb[v][j >> 2][j & 3] : 0.0f);
        const float gv = gt[j] * g.alpha + (g.bias ? ops.tb[v][j >> 2][j & 3] : 0.0f);
        h[j] = hv * gelu_erf_f(gv);
        if (g.res) h[j] += (float)ops.rr[v][j];
      }
      if (ok) {
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = (f16)h[j];
        *(f16x8*)(C + (uint64_t)m * g.ldc + f) = o;
      }
    }
    return;
  }
  using O = EpiOps<BM, BN, NT>;
  constexpr int VPR8 = O::VPR8, NV = O::NV, CH = O::CH;
#pragma unroll
  for (int v0 = 0; v0 < NV; v0 += CH) {
    O ops;
    if (v0 == 0 && pre) ops = *pre;
    else epi_load<BM, BN, NT>(g, m0, n0, bz, v0, ops);
    auto& bb = ops.bb;
    auto& tb = ops.tb;
    auto& rr = ops.rr;
    uint32_t mm[CH], nn[CH];
    bool okv[CH];
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const int idx = tid + (v0 + u) * NT;
      const int r = idx / VPR8, c8 = (idx % VPR8) * 8;
      mm[u] = m0 + r;
      nn[u] = n0 + c8;
      okv[u] = v0 + u < NV && idx < BM * VPR8 && mm[u] < g.M && nn[u] < g.N;
    }
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const int idx = tid + (v0 + u) * NT;
      const int r = idx / VPR8, c8 = (idx % VPR8) * 8;
      float rs = 0.0f, rq = 0.0f;
      if (okv[u]) {
        float x[8];
        const f32x4 a0 = tile4(r * LDC + c8), a1 = tile4(r * LDC + c8 + 4);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          x[j] = a0[j];
          x[j + 4] = a1[j];
        }
        if (EX == EX_LNFOLD && sln) {
          const float2 mr = *(const float2*)&sln[2 * r];
          const f32x4 l0 = ld4(&sln[2 * BM + c8]), l1 = ld4(&sln[2 * BM + c8 + 4]);
#pragma unroll
          for (int j = 0; j < 4; j++) {
            x[j] = mr.y * (x[j] - mr.x * l0[j]);
            x[j + 4] = mr.y * (x[j + 4] - mr.x * l1[j]);
          }
        }
        epi_math8(g, x, bb[u], tb[u]);
        f16x8 o;
#pragma unroll
        for (int j = 0; j < 8; j++) o[j] = (f16)(g.res ? x[j] + (float)rr[u][j] : x[j]);
        *(f16x8*)(C + (uint64_t)mm[u] * g.ldc + nn[u]) = o;
        if (g.stats) {
          // the stored values, for the column statistics of the tile
          float* w = const_cast<float*>(&sC[r * LDC + c8]);
          *(f32x4*)w = f32x4{(float)o[0], (float)o[1], (float)o[2], (float)o[3]};
          *(f32x4*)(w + 4) = f32x4{(float)o[4], (float)o[5], (float)o[6], (float)o[7]};
        }
        if constexpr (EX == EX_ROWSTATS) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const float f = (float)o[j];
            rs += f;
            rq += f * f;
          }
        }
      }
      if constexpr (EX == EX_ROWSTATS) {
        // row statistics over the tile's columns: the VPR8 lanes holding
        // one row are consecutive (VPR8 divides the wavefront)
        static_assert(64 % VPR8 == 0 || BN == 160, "row groups inside a wavefront");
        if constexpr (64 % VPR8 == 0) {
#pragma unroll
          for (int o = 1; o < VPR8; o <<= 1) {
            rs += __shfl_xor(rs, o);
            rq += __shfl_xor(rq, o);
          }
          if (c8 == 0 && v0 + u < NV && idx < BM * VPR8 && mm[u] < g.M)
            *(float2*)(g.rstats + ((uint64_t)mm[u] * ((g.N + BN - 1) / BN) + n0 / BN) * 2) =
                float2{rs, rq};
        }
      }
    }
  }
}

// GroupNorm statistics of an output tile (g.stats): for each 64-row chunk of
// the tile and each column, the sum and sum of squares of the stored fp16
// values over the chunk's rows < M, written to stats[(chunk * N + n) * 2 +
// {0, 1}] with chunk = global row / 64.  sC holds the stored values
// (written back by the epilogue).  TPI adjacent lanes share a column, each
// summing every TPI-th row, and add their sums by lane swaps in a fixed
// order: a lone thread per column spent a dependent add per row, with one
// or two waves of the workgroup busy.
template <int BM, int BN, int LDC, int NT>
__device__ __forceinline__ void gemm_tile_stats(const GemmArgs& g, const float* sC, uint32_t m0,
                                                uint32_t n0) {
  static_assert(BM % 64 == 0, "whole 64-row chunks");
  constexpr int NCH = BM / 64, ITEMS = NCH * BN;
  constexpr int TPI = NT / ITEMS >= 8 ? 8 : NT / ITEMS >= 4 ? 4 : NT / ITEMS >= 2 ? 2 : 1;
  for (int i = threadIdx.x; i < ITEMS * TPI; i += NT) {  // whole TPI groups
    const int item = i / TPI, part = i % TPI;
    const int ch = item / BN, n = item % BN;
    const uint32_t r0 = m0 + ch * 64;
    const bool ok = r0 < g.M && n0 + n < g.N;
    const int rows = ok ? (int)min(64u, g.M - r0) : 0;
    float s = 0.0f, q = 0.0f;
    // a constant trip count (rows past the tile's count add zeros), so the
    // LDS reads are issued together rather than one round trip per row
#pragma unroll
    for (int k = 0; k < 64 / TPI; k++) {
      const int r = part + k * TPI;
      const float v = r < rows ? sC[(ch * 64 + r) * LDC + n] : 0.0f;
      s += v;
      q += v * v;
    }
#pragma unroll
    for (int o = 1; o < TPI; o <<= 1) {
      s += __shfl_xor(s, o);
      q += __shfl_xor(q, o);
    }
    if (ok && part == 0) {
      float* st = g.stats + ((uint64_t)(r0 / 64) * g.N + n0 + n) * 2;
      st[0] = s;
      st[1] = q;
    }
  }
}

// The argument block (GemmArgs, 328 bytes: six scalar-cache lines) in one
// round trip at entry, instead of three serialised misses before the first
// operand load.
__device__ __forceinline__ void args_warm(const GemmArgs& g) { kernarg_warm(g); }

// ---- the GEMM kernel ----
// TB: storage type of B.  The fp32 kernels also take fp16 B (weights kept
// in fp16), widened exactly to fp32 as each vector is loaded.
template <typename T, int BM, int BN, int WGM, int WGN, int AM, int BMD, bool FAST, int D, int KS,
          int EX, typename TB = T>
__global__ __launch_bounds__(64 * WGM * WGN * KS) void k_gemm(GemmArgs g) {
  static_assert(EX == EX_NONE || (FAST && AM == A_DENSE), "epilogue extras: dense fast path");
  static_assert(std::is_same<TB, T>::value || (!FAST && std::is_same<T, float>::value &&
                                               std::is_same<TB, f16>::value),
                "fp16 B with fp32 A: bounds-checked fp32 kernels only");
  using MT = Mfma<T>;
  constexpr int KV = MT::KV;
  constexpr int BK = 128 / sizeof(T);  // k elements per stage (128 bytes per row)
  constexpr int VPR = BK / KV;         // 16-byte vectors per row per stage (8)
  // LDS rows are BK elements (128 bytes, 8 chunks of 16 bytes) with the
  // chunk position XOR-swizzled by (row >> 1) & 7: the 8 lanes writing one row
  // and the 16 lanes reading one fragment column (16 rows) hit distinct banks.
  constexpr int LDK = BK;
  // WGM x WGN output wave tiles (4 or 8).  KS = 2: two wavefronts per output
  // wave tile, each computing half of every stage's k steps (the halves are
  // summed through LDS at the end).  A lone workgroup per CU then still has
  // two (4 tiles) or four (8 tiles) waves per SIMD, so LDS reads and barrier
  // waits of one wave overlap the MFMAs of another.
  constexpr int NWQ = WGM * WGN;
  constexpr int NT = 64 * NWQ * KS;    // threads
  // A / B vectors per thread per stage; when a tile has fewer vectors than
  // threads, the first BM * VPR (BN * VPR) threads - whole wavefronts - load
  constexpr int NVA = (BM * VPR + NT - 1) / NT;
  constexpr int NVB = (BN * VPR + NT - 1) / NT;
  constexpr bool A_PART = NVA * NT != BM * VPR, B_PART = NVB * NT != BN * VPR;
  constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int KSTEPS = BK / MT::KM;  // MFMA k steps per stage
  static_assert(NWQ == 4 || NWQ == 8, "4 or 8 wavefronts per k half");
  static_assert(KS == 1 || (FAST && KSTEPS % KS == 0), "k halves: fast path, whole k steps");
  static_assert(NVA >= 1 && NVB >= 1 && TM >= 1 && TN >= 1, "tile too small");
  static_assert((!A_PART || (FAST && NVA == 1 && BM * VPR % 64 == 0)) &&
                    (!B_PART || (FAST && NVB == 1 && BN * VPR % 64 == 0)),
                "partial vector loads: fast path, whole wavefronts");

  // Pipeline buffers sA[2][BM*LDK], sB[2][BN*LDK]; reused by the fp32 C tile
  // of the vector epilogue.
  constexpr int kSmemPipe = 2 * (BM + BN) * LDK;
  constexpr int kSmemC = BM * (BN + 4) * 4 / (int)sizeof(T);  // fp32 C tile of the vector epilogue
  // Side by side: the two k halves stage their fp32 C tiles at once and the
  // vector epilogue adds them as it reads (one barrier, no read-modify-write
  // pass), where the second tile costs no workgroup residency (a CU holds
  // workgroups in two 80 KiB halves of its LDS).  The LayerNorm fold is then
  // applied by the vector epilogue to the summed tile.
  constexpr int kPer80K = (int)(80 * 1024 / sizeof(T));
  constexpr int kSmem1 = kSmemPipe > kSmemC ? kSmemPipe : kSmemC;
  constexpr int kSmem2 = kSmemPipe > 2 * kSmemC ? kSmemPipe : 2 * kSmemC;
  constexpr bool SBS = sizeof(T) == 2 && KS == 2 && kSmem2 <= kPer80K &&
                       kPer80K / kSmem2 == kPer80K / kSmem1;
  __shared__ __attribute__((aligned(16))) T smem[SBS ? kSmem2 : kSmem1];
  // LayerNorm fold: (mean, rstd) of each tile row, then ln_s of each column
  __shared__ __attribute__((aligned(16))) float sLn[EX == EX_LNFOLD ? 2 * BM + BN : 2];
  T (*sA)[BM * LDK] = reinterpret_cast<T (*)[BM * LDK]>(smem);
  T (*sB)[BN * LDK] = reinterpret_cast<T (*)[BN * LDK]>(smem + 2 * BM * LDK);
  // element offset of (row r, k element e) inside one buffer
  auto lds_at = [](int r, int e) {
    return r * LDK + (((e / KV) ^ ((r >> 1) & 7)) * KV) + e % KV;
  };

  args_warm(g);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wq = wave % NWQ, kh = wave / NWQ;  // output wave tile, k half
  const bool a_ld = !A_PART || tid < BM * VPR, b_ld = !B_PART || tid < BN * VPR;
  const int wm0 = (wq / WGN) * WM, wn0 = (wq % WGN) * WN;

  // Tile order: N fastest, so consecutive tiles share A rows.  Workgroups are
  // dealt round-robin to the 8 XCDs (each with its own L2); remap so that
  // each XCD gets a contiguous run of tiles and shares their A / B reads.
  const uint32_t n_tiles = (g.N + BN - 1) / BN;
  const uint32_t n_wg = gridDim.x;
  uint32_t tile = blockIdx.x;
  {
    const uint32_t per = n_wg / 8, rem = n_wg % 8, xcd = tile % 8, slot = tile / 8;
    tile = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  }
  const uint32_t m0 = (tile / n_tiles) * BM, n0 = (tile % n_tiles) * BN;
  const uint32_t splits = g.splits;
  const uint32_t bz = blockIdx.z / splits, split = blockIdx.z % splits;
  const uint32_t k_begin = split * g.k_split;
  const uint32_t k_end = min(g.K, k_begin + g.k_split);
  // a trailing split may start past K: it contributes zeros to the reduction
  const int n_stages = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;

  const T* A = (const T*)g.a + (uint64_t)bz * g.sa;
  const T* A2 = (const T*)g.a2 + (uint64_t)bz * g.sa2;
  const TB* B = (const TB*)g.b + (uint64_t)bz * g.sb;
  // one vector of B: KV elements of TB (widened to T)
  auto ld_bvec = [](const TB* p) -> typename MT::vec {
    if constexpr (std::is_same<TB, T>::value) {
      return *(const typename MT::vec*)p;
    } else {
      return __builtin_convertvector(*(const f16x4*)p, f32x4);
    }
  };

  // ---- per-thread A addressing (rows fixed for the whole K loop) ----
  const int kc = tid % VPR;  // same k-vector slot for all of this thread's vectors
  int64_t a_row_off[NVA];     // dense: row offset; conv: image pixel base
  int a_iy0[NVA], a_ix0[NVA];
  bool a_row_ok[NVA];
#pragma unroll
  for (int i = 0; i < NVA; i++) {
    uint32_t r = (tid + i * NT) / VPR;
    uint32_t m = m0 + r;
    a_row_ok[i] = a_ld && m < g.M;
    if constexpr (AM == A_DENSE) {
      a_row_off[i] = (int64_t)m;
      a_iy0[i] = a_ix0[i] = 0;
    } else {
      uint32_t hw = g.Ho * g.Wo;
      uint32_t img = m / hw, p = m % hw;
      uint32_t oy = p / g.Wo, ox = p % g.Wo;
      a_row_off[i] = (int64_t)img;
      a_iy0[i] = (int)(oy * g.stride) - (int)g.pad;
      a_ix0[i] = (int)(ox * g.stride) - (int)g.pad;
    }
  }
  // conv k tracking: k = tap * Cin + ci for NHWC
  uint32_t ci = 0, ky = 0, kx = 0;
  if constexpr (AM == A_CONV_NHWC) {
    uint32_t k0 = k_begin + kc * KV;
    uint32_t tap = k0 / g.Cin;
    ci = k0 % g.Cin;
    ky = tap / g.ks;
    kx = tap % g.ks;
  }
  const uint32_t Hi = g.H * g.up, Wi = g.W * g.up;
  const bool a_fast = g.a_vec_ok;
  const bool b_fast = g.b_vec_ok;

  // ---- FAST path (fp16, B_NK, dense or NHWC conv with Cin % 64 == 0):
  // every load is an unconditional raw buffer load; invalid elements get an
  // offset past the buffer's range and read as zero, so the loads carry no
  // branches and the compiler can keep exact vmcnt waits for the pipeline.
  constexpr uint32_t kInv = 0x80000000u;
  const __amdgpu_buffer_rsrc_t rA = make_rsrc(A, g.a_bytes), rA2 = make_rsrc(A2, g.a2_bytes),
                               rB = make_rsrc(B, g.b_bytes);
  uint32_t fa1[NVA], fa2[NVA], fb[NVB];
  uint32_t fimg[NVA];
  uint32_t f_ci0 = 0, f_ky = 0, f_kx = 0;  // conv: per-stage tap and channel base (uniform)
  const uint32_t upsh = g.up == 2 ? 1 : 0;
  if constexpr (FAST) {
#pragma unroll
    for (int i = 0; i < NVA; i++) {
      const uint32_t m = m0 + (tid + i * NT) / VPR;
      // row base + this thread's k chunk at k_begin; stages add a scalar offset
      fa1[i] = a_row_ok[i] ? m * (uint32_t)g.lda * 2u + (k_begin + kc * KV) * 2u : kInv;
      fa2[i] = a_row_ok[i] ? m * (uint32_t)g.lda2 * 2u : kInv;
      fimg[i] = (uint32_t)a_row_off[i] * g.H;
    }
#pragma unroll
    for (int i = 0; i < NVB; i++) {
      const uint32_t n = n0 + (tid + i * NT) / VPR;
      fb[i] = b_ld && n < g.N ? n * (uint32_t)g.ldb * 2u + (k_begin + kc * KV) * 2u : kInv;
    }
    if constexpr (AM == A_CONV_NHWC) {
      const uint32_t tap0 = k_begin / g.Cin;
      f_ci0 = k_begin % g.Cin;
      f_ky = tap0 / g.ks;
      f_kx = tap0 % g.ks;
    }
  }

  struct Stage {
    typename MT::vec a[NVA];
    typename MT::vec b[NVB];
  };

  auto load_a = [&](int stage, Stage& st) {
    const uint32_t kbase = k_begin + stage * BK;
#pragma unroll
    for (int i = 0; i < NVA; i++) {
      typename MT::vec v = zero_vec<T>();
      const uint32_t k = kbase + kc * KV;
      if constexpr (AM == A_DENSE) {
        if (a_row_ok[i]) {
          if (a_fast && k + KV <= k_end) {
            if (k < g.c1) v = *(const typename MT::vec*)(A + a_row_off[i] * g.lda + k);
            else v = *(const typename MT::vec*)(A2 + a_row_off[i] * g.lda2 + (k - g.c1));
          } else {
#pragma unroll
            for (int j = 0; j < KV; j++) {
              uint32_t kk = k + j;
              if (kk < k_end)
                v[j] = kk < g.c1 ? A[a_row_off[i] * g.lda + kk] : A2[a_row_off[i] * g.lda2 + kk - g.c1];
            }
          }
        }
      } else if constexpr (AM == A_CONV_NHWC) {
        // fast path only (Cin % 8 == 0 checked by the host)
        int iy = a_iy0[i] + (int)ky, ix = a_ix0[i] + (int)kx;
        if (a_row_ok[i] && k < k_end && iy >= 0 && iy < (int)Hi && ix >= 0 && ix < (int)Wi) {
          uint32_t sy = (uint32_t)iy / g.up, sx = (uint32_t)ix / g.up;
          uint64_t pix = ((uint64_t)a_row_off[i] * g.H + sy) * g.W + sx;
          if (ci < g.c1) v = *(const typename MT::vec*)(A + pix * g.lda + ci);
          else v = *(const typename MT::vec*)(A2 + pix * g.lda2 + (ci - g.c1));
        }
      } else {  // A_CONV_NCHW, reference k order (ci, ky, kx), element gathers
        if (a_row_ok[i]) {
          const uint32_t kk2 = g.ks * g.ks;
#pragma unroll
          for (int j = 0; j < KV; j++) {
            uint32_t kk = k + j;
            if (kk < k_end) {
              uint32_t c = kk / kk2, r = kk % kk2;
              int iy = a_iy0[i] + (int)(r / g.ks), ix = a_ix0[i] + (int)(r % g.ks);
              if (iy >= 0 && iy < (int)Hi && ix >= 0 && ix < (int)Wi) {
                uint32_t sy = (uint32_t)iy / g.up, sx = (uint32_t)ix / g.up;
                v[j] = A[(((uint64_t)a_row_off[i] * g.Cin + c) * g.H + sy) * g.W + sx];
              }
            }
          }
        }
      }
      st.a[i] = v;
    }
    if constexpr (AM == A_CONV_NHWC) {
      ci += BK;
      while (ci >= g.Cin) {
        ci -= g.Cin;
        if (++kx == g.ks) {
          kx = 0;
          ++ky;
        }
      }
    }
  };

  auto load_b = [&](int stage, Stage& st) {
    const uint32_t kbase = k_begin + stage * BK;
#pragma unroll
    for (int i = 0; i < NVB; i++) {
      typename MT::vec v = zero_vec<T>();
      if constexpr (BMD == B_NK) {
        uint32_t r = (tid + i * NT) / VPR;
        uint32_t n = n0 + r, k = kbase + kc * KV;
        if (n < g.N) {
          if (b_fast && k + KV <= k_end) {
            v = ld_bvec(B + (uint64_t)n * g.ldb + k);
          } else {
#pragma unroll
            for (int j = 0; j < KV; j++)
              if (k + j < k_end) v[j] = B[(uint64_t)n * g.ldb + k + j];
          }
        }
      } else {  // B_KN: vector along n at fixed k; transposed into LDS at store
        constexpr int VPK = BN / KV;  // vectors per k row
        uint32_t kr = (tid + i * NT) / VPK, nc = (tid + i * NT) % VPK;
        uint32_t k = kbase + kr, n = n0 + nc * KV;
        if (k < k_end) {
          if (b_fast && n + KV <= g.N) {
            v = ld_bvec(B + (uint64_t)k * g.ldb + n);
          } else {
#pragma unroll
            for (int j = 0; j < KV; j++)
              if (n + j < g.N) v[j] = B[(uint64_t)k * g.ldb + n + j];
          }
        }
      }
      st.b[i] = v;
    }
  };

  auto store_stage = [&](int buf, const Stage& st) {
#pragma unroll
    for (int i = 0; i < NVA; i++) {
      uint32_t r = (tid + i * NT) / VPR;
      if (a_ld) *(typename MT::vec*)&sA[buf][lds_at(r, kc * KV)] = st.a[i];
    }
#pragma unroll
    for (int i = 0; i < NVB; i++) {
      if (!b_ld) break;
      if constexpr (BMD == B_NK) {
        uint32_t r = (tid + i * NT) / VPR;
        *(typename MT::vec*)&sB[buf][lds_at(r, kc * KV)] = st.b[i];
      } else {
        constexpr int VPK = BN / KV;
        uint32_t kr = (tid + i * NT) / VPK, nc = (tid + i * NT) % VPK;
#pragma unroll
        for (int j = 0; j < KV; j++) sB[buf][lds_at(nc * KV + j, kr)] = st.b[i][j];
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; a++)
#pragma unroll
    for (int b = 0; b < TN; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fk = (lane >> 4) * MT::FK;
  auto compute = [&](int buf) {
#pragma unroll
    for (int ks = 0; ks < KSTEPS / KS; ks++) {
      const int kk = (kh * (KSTEPS / KS) + ks) * MT::KM;
      typename MT::frag af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; a++) af[a] = ld_frag<T>(&sA[buf][lds_at(wm0 + a * 16 + fr, kk + fk)]);
#pragma unroll
      for (int b = 0; b < TN; b++) bf[b] = ld_frag<T>(&sB[buf][lds_at(wn0 + b * 16 + fr, kk + fk)]);
#pragma unroll
      for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++) acc[a][b] = MT::mma(af[a], bf[b], acc[a][b]);
    }
  };
  // FAST loads need K % BK == 0 (gemm_fast_ok), so every stage of a split is
  // whole: no per-lane k bound.  Stages past the split's end (the ring's
  // padding) read whatever lies beyond (zeros past the buffer) and are never
  // computed; rows past M / N carry an out-of-range offset and read zeros.
  auto load_fast = [&](int stage, Stage& st) {
    const uint32_t sk = (uint32_t)stage * (BK * 2u);
    if constexpr (AM == A_DENSE) {
      // single source (gemm_fast_ok): one descriptor, so it stays uniform; a
      // per-stage choice between two descriptors merged with a per-lane
      // condition makes the compiler emit a waterfall loop around every load
#pragma unroll
      for (int i = 0; i < NVA; i++) st.a[i] = buf_load16s<typename MT::vec>(rA, fa1[i], sk);
    } else {
      const bool s2 = f_ci0 >= g.c1;
      const uint32_t cb = ((s2 ? f_ci0 - g.c1 : f_ci0) + kc * KV) * 2u;
      const uint32_t ld2 = (uint32_t)(s2 ? g.lda2 : g.lda) * 2u;
      const int Hi_ = (int)(g.H << upsh), Wi_ = (int)(g.W << upsh);
#pragma unroll
      for (int i = 0; i < NVA; i++) {
        const int iy = a_iy0[i] + (int)f_ky, ix = a_ix0[i] + (int)f_kx;
        const bool ok = a_row_ok[i] && iy >= 0 && iy < Hi_ && ix >= 0 && ix < Wi_;
        const uint32_t pix = (fimg[i] + ((uint32_t)iy >> upsh)) * g.W + ((uint32_t)ix >> upsh);
        st.a[i] = buf_load16<typename MT::vec>(s2 ? rA2 : rA, ok ? pix * ld2 + cb : kInv);
      }
      f_ci0 += BK;
      if (f_ci0 >= g.Cin) {
        f_ci0 = 0;
        if (++f_kx == g.ks) {
          f_kx = 0;
          ++f_ky;
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NVB; i++) st.b[i] = buf_load16s<typename MT::vec>(rB, fb[i], sk);
  };
  auto load = [&](int stage, Stage& st) {
    if constexpr (FAST) {
      load_fast(stage, st);
    } else {
      load_a(stage, st);
      load_b(stage, st);
    }
  };

  // FAST path: a ring of D register stages and two LDS buffers.  Sub-step s
  // first writes stage s+1 (loaded D sub-steps earlier) into LDS buffer
  // (s+1)%2, refills that register slot with stage s+1+D, then computes stage
  // s from buffer s%2; one barrier per stage.  Writing before computing keeps
  // the LDS-write latency and the global-load wait off the end of the stage,
  // where they would sit in front of the barrier.  Buffer (s+1)%2 was last
  // read by compute(s-1), which every wave finished before the previous
  // barrier.  Loads past the last stage read zeros (offsets out of range) and
  // stages past the end skip their MFMA work, so the loop body has no branches
  // around loads and the waitcnt pass keeps exact vmcnt counts.
  // LayerNorm fold (no split): the LN_T = NT / BM consecutive threads of
  // tile row r = tid / LN_T each fetch every LN_T-th (sum, sum of squares)
  // pair of the row (LN_U at once, after the first stages' loads are
  // issued), combine them with lane shuffles once stage 0 is in LDS and
  // leave (mean, rstd) in sLn; threads < BN add the column sums ln_s[n0 + tid].
  // The prologue barrier publishes both before the main loop.
  constexpr int LN_T = NT / BM, LN_U = 3;
  static_assert(LN_T >= 1 && LN_T <= 64 && (LN_T & (LN_T - 1)) == 0, "row groups in a wavefront");
  float2 ln_v[EX == EX_LNFOLD ? LN_U : 1];
  float ln_col = 0.0f;
  const uint32_t ln_r = (uint32_t)tid / LN_T, ln_p = (uint32_t)tid % LN_T;
  const float2* ln_row = (const float2*)g.ln_rows + (uint64_t)min(m0 + ln_r, g.M - 1) * g.ln_nt;
  auto ln_issue = [&]() {
    if constexpr (EX == EX_LNFOLD) {
#pragma unroll
      for (int i = 0; i < LN_U; i++) ln_v[i] = ln_row[min(ln_p + i * LN_T, g.ln_nt - 1)];
      if (tid < BN) ln_col = g.ln_s[min(n0 + (uint32_t)tid, g.N - 1)];
    }
  };
  auto ln_publish = [&]() {
    if constexpr (EX == EX_LNFOLD) {
      float sm = 0.0f, sq = 0.0f;
#pragma unroll
      for (int i = 0; i < LN_U; i++) {
        if (ln_p + i * LN_T < g.ln_nt) {
          sm += ln_v[i].x;
          sq += ln_v[i].y;
        }
      }
      for (uint32_t t = ln_p + LN_U * LN_T; t < g.ln_nt; t += LN_T) {
        const float2 w = ln_row[t];
        sm += w.x;
        sq += w.y;
      }
#pragma unroll
      for (int o = 1; o < LN_T; o <<= 1) {
        sm += __shfl_xor(sm, o);
        sq += __shfl_xor(sq, o);
      }
      if (ln_p == 0) {
        const float mean = sm / (float)g.K;
        const float var = fmaxf(sq / (float)g.K - mean * mean, 0.0f);
        *(float2*)&sLn[2 * ln_r] = float2{mean, 1.0f / sqrtf(var + g.ln_eps)};
      }
      if (tid < BN) sLn[2 * BM + tid] = ln_col;
    }
  };
  Stage r0, r1;
  if constexpr (FAST) {
    static_assert(D % 2 == 0, "even ring depth: LDS buffer = stage parity");
    Stage r[D];
    if (n_stages > 0) {
#pragma unroll
      for (int j = 0; j < D; j++) load(j, r[j]);
      ln_issue();
      store_stage(0, r[0]);
      load(D, r[0]);
      ln_publish();  // after stage D's loads are issued: its wait covers stage 1 only
      __syncthreads();
      // steady state: whole rounds of D stages, no conditions (a conditional
      // compute makes the compiler copy the accumulators around it)
      int s0 = 0;
      for (; s0 + D <= n_stages; s0 += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
          store_stage((j + 1) & 1, r[(j + 1) % D]);
          load(s0 + j + 1 + D, r[(j + 1) % D]);
          // issue the loads here, not after the MFMAs (the scheduler would
          // otherwise sink them and shorten the prefetch distance)
          __builtin_amdgcn_sched_barrier(0);
          compute(j & 1);
          __syncthreads();
        }
      }
      // tail: the last n_stages % D stages (stage s0 + j in LDS buffer j & 1)
      const int rem = n_stages - s0;
#pragma unroll
      for (int j = 0; j + 1 < D; j++) {
        if (j < rem) {
          if (j + 1 < rem) store_stage((j + 1) & 1, r[(j + 1) % D]);
          compute(j & 1);
          __syncthreads();
        }
      }
    }
  } else {
  if (n_stages > 0) {
    load(0, r0);
    store_stage(0, r0);
  }
  if (n_stages > 1) load(1, r1);
  if (n_stages > 2) load(2, r0);
  __syncthreads();
  for (int s = 0; s < n_stages; s += 2) {
    compute(0);
    if (s + 1 < n_stages) store_stage(1, r1);
    __syncthreads();
    if (s + 3 < n_stages) load(s + 3, r1);
    if (s + 1 >= n_stages) break;
    compute(1);
    if (s + 2 < n_stages) store_stage(0, r0);
    __syncthreads();
    if (s + 4 < n_stages) load(s + 4, r0);
  }
  }

  // ---- epilogue ----
  const uint32_t rq = (lane >> 4) * 4;
  if constexpr (sizeof(T) == 2) {
    if (g.vec_epi) {
      constexpr int LDC = BN + 4;
      static_assert((SBS ? 2 : 1) * BM * LDC * 4 <= (int)sizeof(smem), "C tiles fit the LDS allocation");
      float* sC = reinterpret_cast<float*>(smem);
      // bias / temb bias / residual loads in flight while the tile is staged
      EpiOps<BM, BN, NT> pre;
      epi_prefetch<BM, BN, NT>(g, m0, n0, bz, pre);
      lds_barrier();  // every wave is done reading the last stage
      if constexpr (SBS) {
        float* const sCh = sC + kh * (BM * LDC);
#pragma unroll
        for (int a = 0; a < TM; a++)
#pragma unroll
          for (int b = 0; b < TN; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) sCh[(wm0 + a * 16 + rq + i) * LDC + wn0 + b * 16 + fr] = acc[a][b][i];
        lds_barrier();
        gemm_epilogue_vec<BM, BN, LDC, NT, EX, 2>(g, sC, m0, n0, bz, split, &pre, BM * LDC, sLn);
        if (g.stats && splits == 1) {
          lds_barrier();
          gemm_tile_stats<BM, BN, LDC, NT>(g, sC, m0, n0);
        }
        return;
      }
      // LayerNorm fold (EX_LNFOLD, launched without split-K): the (mean,
      // rstd) of this thread's accumulator rows and ln_s of its columns
      float2 lmr[EX == EX_LNFOLD ? TM : 1][4];
      float lsc[EX == EX_LNFOLD ? TN : 1];
      if constexpr (EX == EX_LNFOLD) {
#pragma unroll
        for (int a = 0; a < TM; a++)
#pragma unroll
          for (int i = 0; i < 4; i++) lmr[a][i] = *(const float2*)&sLn[2 * (wm0 + a * 16 + rq + i)];
#pragma unroll
        for (int b = 0; b < TN; b++) lsc[b] = sLn[2 * BM + wn0 + b * 16 + fr];
      }
      // k half 0 writes the C tile, k half 1 (same positions) adds to it
#pragma unroll
      for (int h = 0; h < KS; h++) {
        if (kh == h) {
#pragma unroll
          for (int a = 0; a < TM; a++)
#pragma unroll
            for (int b = 0; b < TN; b++)
#pragma unroll
              for (int i = 0; i < 4; i++) {
                float& c = sC[(wm0 + a * 16 + rq + i) * LDC + wn0 + b * 16 + fr];
                float v = h == 0 ? acc[a][b][i] : c + acc[a][b][i];
                // LayerNorm fold once the k halves are summed:
                // rstd * (acc - mean * ln_s[n])
                if constexpr (EX == EX_LNFOLD)
                  if (h == KS - 1) v = lmr[a][i].y * (v - lmr[a][i].x * lsc[b]);
                c = v;
              }
        }
        lds_barrier();
      }
      gemm_epilogue_vec<BM, BN, LDC, NT, EX>(g, sC, m0, n0, bz, split, &pre);
      if (g.stats && splits == 1) {
        lds_barrier();
        gemm_tile_stats<BM, BN, LDC, NT>(g, sC, m0, n0);
      }
      return;
    }
  }
  if constexpr (KS > 1) {
    // k half 1 hands its sums to half 0 through LDS; half 0 runs the epilogue
    constexpr int LDC = BN + 4;
    float* sC = reinterpret_cast<float*>(smem);
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            sC[(wm0 + a * 16 + rq + i) * LDC + wn0 + b * 16 + fr] = acc[a][b][i];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
      for (int b = 0; b < TN; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[a][b][i] += sC[(wm0 + a * 16 + rq + i) * LDC + wn0 + b * 16 + fr];
  }
  if (splits > 1) {
    float* P = g.part + ((uint64_t)(split + g.part_slot0) * g.batch + bz) * (uint64_t)g.M * g.N;
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
      for (int b = 0; b < TN; b++) {
        uint32_t n = n0 + wn0 + b * 16 + fr;
        const PartCol pc = part_col(g, n);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t m = m0 + wm0 + a * 16 + rq + i;
          if (m < g.M && n < g.N) P[(uint64_t)m * pc.stride + pc.offset] = acc[a][b][i];
        }
      }
    return;
  }
  if (g.act == ACT_GEGLU) {
    // columns come in 32-wide groups: [16 hidden | 16 gate] of the same outputs
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
      for (int b = 0; b + 1 < TN; b += 2) {
        uint32_t nh = n0 + wn0 + b * 16 + fr;
        uint32_t f = (nh / 32) * 16 + (nh % 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t m = m0 + wm0 + a * 16 + rq + i;
          if (m < g.M && nh + 16 < g.N) {
            float h = epi_value<T>(g, bz, m, nh, acc[a][b][i]);
            float gt = epi_value<T>(g, bz, m, nh + 16, acc[a][b + 1][i]);
            store_out(g, bz, m, f, g.N / 2, h * gelu_erf_f(gt));
          }
        }
      }
    return;
  }
#pragma unroll
  for (int a = 0; a < TM; a++)
#pragma unroll
    for (int b = 0; b < TN; b++) {
      uint32_t n = n0 + wn0 + b * 16 + fr;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        uint32_t m = m0 + wm0 + a * 16 + rq + i;
        if (m < g.M && n < g.N)
          store_out(g, bz, m, n, g.N, apply_act(g.act, epi_value<T>(g, bz, m, n, acc[a][b][i])));
      }
    }
}

template <typename T, int BM, int BN, int WGM, int WGN, int AM, int BMD, bool FAST, int D = 2,
          int KS = 1, int EX = EX_NONE, typename TB = T>
void launch_cfg(const GemmArgs& g, hipStream_t s) {
  uint32_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  k_gemm<T, BM, BN, WGM, WGN, AM, BMD, FAST, D, KS, EX, TB>
      <<<dim3(tiles, 1, g.batch * g.splits), 64 * WGM * WGN * KS, 0, s>>>(g);
}

// Generic (bounds-checked) variants: two tile shapes.
template <typename T, int AM, int BMD, typename TB = T>
void launch_slow(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  if (tile_cfg == TILE_64x64 || tile_cfg == TILE_128x64 || tile_cfg == TILE_64x128 ||
      tile_cfg == TILE_64x160 || tile_cfg == TILE_64x64_K2 || tile_cfg == TILE_128x64_K2 ||
      tile_cfg == TILE_64x128_K2 || tile_cfg == TILE_64x128_W16 || tile_cfg == TILE_128x64_W16 ||
      tile_cfg == TILE_64x64_W16)
    launch_cfg<T, 64, 64, 2, 2, AM, BMD, false, 2, 1, EX_NONE, TB>(g, s);
  else
    launch_cfg<T, 128, 128, 2, 2, AM, BMD, false, 2, 1, EX_NONE, TB>(g, s);
}

// Buffer-load variants: every tile shape, ring depth D, epilogue extras EX.
template <int AM, int D, int EX = EX_NONE>
void launch_fast_d(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  switch (tile_cfg) {
    case TILE_128x128: launch_cfg<f16, 128, 128, 2, 2, AM, B_NK, true, D, 1, EX>(g, s); break;
    case TILE_128x64: launch_cfg<f16, 128, 64, 2, 2, AM, B_NK, true, D, 1, EX>(g, s); break;
    case TILE_64x160: launch_cfg<f16, 64, 160, 2, 2, AM, B_NK, true, D, 1, EX>(g, s); break;
    case TILE_64x128: launch_cfg<f16, 64, 128, 2, 2, AM, B_NK, true, D, 1, EX>(g, s); break;
    case TILE_64x64_K2: launch_cfg<f16, 64, 64, 2, 2, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_128x64_K2: launch_cfg<f16, 128, 64, 2, 2, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_64x128_K2: launch_cfg<f16, 64, 128, 2, 2, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_64x128_W16: launch_cfg<f16, 64, 128, 2, 4, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_128x64_W16: launch_cfg<f16, 128, 64, 4, 2, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_128x128_W16: launch_cfg<f16, 128, 128, 2, 4, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_64x64_W16: launch_cfg<f16, 64, 64, 2, 4, AM, B_NK, true, D, 2, EX>(g, s); break;
    case TILE_64x32_K2: launch_cfg<f16, 64, 32, 2, 2, AM, B_NK, true, D, 2, EX>(g, s); break;
    default: launch_cfg<f16, 64, 64, 2, 2, AM, B_NK, true, D, 1, EX>(g, s); break;
  }
}
}  // namespace

}  // namespace di

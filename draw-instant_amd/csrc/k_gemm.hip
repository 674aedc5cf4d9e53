// Host side of the MFMA GEMM / implicit-GEMM conv (k_gemm_kernel.h): plan
// selection, the split-K reducers and launch_gemm, which dispatches to the
// instantiation families of k_gemm_*.hip.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "k_gemm_kernel.h"
#include "k_gemm_families.h"

namespace di {

namespace {

// Split-K reduction + epilogue: one thread per output element.
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g) {
  args_warm(g);
  const uint32_t ncols = g.act == ACT_GEGLU ? g.N / 2 : g.N;
  const uint64_t total = (uint64_t)g.batch * g.M * ncols;
  const uint64_t mn = (uint64_t)g.M * g.N;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint32_t col = i % ncols;
    uint64_t t = i / ncols;
    uint32_t m = t % g.M;
    uint32_t bz = (uint32_t)(t / g.M);
    auto sum_at = [&](uint32_t n) {
      float s = 0.0f;
      for (uint32_t sp = 0; sp < g.splits; sp++)
        s += g.part[((uint64_t)sp * g.batch + bz) * mn + (uint64_t)m * g.N + n];
      return s;
    };
    if (g.act == ACT_GEGLU) {
      uint32_t nh = (col / 16) * 32 + col % 16;
      float h = epi_value<f16>(g, bz, m, nh, sum_at(nh));
      float gt = epi_value<f16>(g, bz, m, nh + 16, sum_at(nh + 16));
      store_out(g, bz, m, col, ncols, h * gelu_erf_f(gt));
    } else {
      store_out(g, bz, m, col, ncols, apply_act(g.act, epi_value<f16>(g, bz, m, col, sum_at(col))));
    }
  }
}

// The split-K partials of 8 columns of row m: the first 8 splits' loads are
// issued by splits8_load (with the epilogue operands, before anything is
// consumed, so one memory round trip covers them all) and summed by
// splits8_sum in split order, further splits by a loop there.
struct Parts8 {
  f32x4 t[8][2];
};

__device__ __forceinline__ const float* part_row(const GemmArgs& g, uint32_t bz, uint32_t m,
                                                 uint32_t n) {
  return g.part + (uint64_t)bz * g.M * g.N + (uint64_t)m * g.N + n;
}

__device__ __forceinline__ void splits8_load(const GemmArgs& g, const float* p, Parts8& P) {
  const uint64_t step = (uint64_t)g.batch * g.M * g.N;
#pragma unroll
  for (int u = 0; u < 8; u++) {
    const uint32_t sp = (uint32_t)u < g.splits ? (uint32_t)u : 0u;
    P.t[u][0] = ld4(p + sp * step);
    P.t[u][1] = ld4(p + sp * step + 4);
  }
}

__device__ __forceinline__ void splits8_sum(const GemmArgs& g, const float* p, const Parts8& P,
                                            float* out) {
  const uint64_t step = (uint64_t)g.batch * g.M * g.N;
#pragma unroll
  for (int j = 0; j < 8; j++) out[j] = 0.0f;
#pragma unroll
  for (int u = 0; u < 8; u++) {
    if ((uint32_t)u < g.splits) {  // uniform
#pragma unroll
      for (int j = 0; j < 4; j++) {
        out[j] += P.t[u][0][j];
        out[j + 4] += P.t[u][1][j];
      }
    }
  }
  for (uint32_t s0 = 8; s0 < g.splits; s0 += 8) {
    f32x4 t[8][2];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const uint32_t sp = s0 + u < g.splits ? s0 + u : s0;
      t[u][0] = ld4(p + sp * step);
      t[u][1] = ld4(p + sp * step + 4);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      if (s0 + u < g.splits) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          out[j] += t[u][0][j];
          out[j + 4] += t[u][1][j];
        }
      }
    }
  }
}

// One output vector of the split-K reduction + epilogue (vec_epi): row m,
// output columns c8 .. c8 + 7 (with GEGLU, of the N / 2 combined columns).
// Every load (partials, LayerNorm row statistics and column sums, bias,
// temb bias, residual) is issued before any is consumed.  The stored fp16
// values are returned in v as floats.
__device__ __forceinline__ void splitk_vec8(const GemmArgs& g, uint32_t bz, uint32_t m, uint32_t c8,
                                            float* v) {
  f16* C = (f16*)g.c + (uint64_t)bz * g.sc + (uint64_t)m * g.ldc + c8;
  const f16* R = (const f16*)g.res + (uint64_t)bz * g.sr + (uint64_t)m * g.ldr + c8;
  float x[8];
  float mean = 0.0f, rstd = 0.0f;
  float2 lv[kLnBatch];
  if (g.act == ACT_GEGLU) {
    const uint32_t nh = (c8 / 16) * 32 + c8 % 16;
    const float* ph = part_row(g, bz, m, nh);
    const float* pg = part_row(g, bz, m, nh + 16);
    Parts8 Ph, Pg;
    splits8_load(g, ph, Ph);
    splits8_load(g, pg, Pg);
    f32x4 sh[2] = {}, sg[2] = {}, bh[2] = {}, bg[2] = {};
    if (g.bias) {
      bh[0] = ld4(g.bias + nh);
      bh[1] = ld4(g.bias + nh + 4);
      bg[0] = ld4(g.bias + nh + 16);
      bg[1] = ld4(g.bias + nh + 20);
    }
    // the LayerNorm loads last: the compiler may start their reduction inside
    // this branch, and a wait there must find every other load in flight
    if (g.ln_rows) {
      sh[0] = ld4(g.ln_s + nh);
      sh[1] = ld4(g.ln_s + nh + 4);
      sg[0] = ld4(g.ln_s + nh + 16);
      sg[1] = ld4(g.ln_s + nh + 20);
      ln_load(g, m, lv);
    }
    float gt[8];
    splits8_sum(g, ph, Ph, x);
    splits8_sum(g, pg, Pg, gt);
    if (g.ln_rows) {
      ln_reduce(g, m, lv, mean, rstd);
      ln_fold8(x, mean, rstd, sh);
      ln_fold8(gt, mean, rstd, sg);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float hv = x[j] * g.alpha + bh[j >> 2][j & 3];
      const float gv = gt[j] * g.alpha + bg[j >> 2][j & 3];
      x[j] = hv * gelu_erf_f(gv);
    }
  } else {
    const float* pp = part_row(g, bz, m, c8);
    Parts8 P;
    splits8_load(g, pp, P);
    f32x4 bb[2] = {}, tb[2] = {}, ls[2] = {};
    if (g.bias) {
      bb[0] = ld4(g.bias + c8);
      bb[1] = ld4(g.bias + c8 + 4);
    }
    if (g.bias2) {
      const float* tp = g.bias2 + (uint64_t)(m / g.rows_b2) * g.ld_b2 + c8;
      tb[0] = ld4(tp);
      tb[1] = ld4(tp + 4);
    }
    f16x8 rv = {};
    if (g.res) rv = *(const f16x8*)R;
    // the LayerNorm loads last (see the GEGLU branch)
    if (g.ln_rows) {
      ls[0] = ld4(g.ln_s + c8);
      ls[1] = ld4(g.ln_s + c8 + 4);
      ln_load(g, m, lv);
    }
    splits8_sum(g, pp, P, x);
    if (g.ln_rows) {
      ln_reduce(g, m, lv, mean, rstd);
      ln_fold8(x, mean, rstd, ls);
    }
    epi_math8(g, x, bb, tb);
    if (g.res)
#pragma unroll
      for (int j = 0; j < 8; j++) x[j] += (float)rv[j];
  }
  f16x8 o;
#pragma unroll
  for (int j = 0; j < 8; j++) o[j] = (f16)x[j];
  *(f16x8*)C = o;
#pragma unroll
  for (int j = 0; j < 8; j++) v[j] = (float)o[j];
}


// Vector split-K reduction + epilogue (vec_epi): one thread per 8 output
// columns (splitk_vec8).
__global__ __launch_bounds__(256) void k_splitk_reduce_vec(GemmArgs g) {
  args_warm(g);
  const uint32_t ncols = g.act == ACT_GEGLU ? g.N / 2 : g.N;
  const uint32_t vpr = ncols / 8;
  const uint64_t total = (uint64_t)g.batch * g.M * vpr;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const uint32_t c8 = (uint32_t)(i % vpr) * 8;
    const uint64_t t = i / vpr;
    float v[8];
    splitk_vec8(g, (uint32_t)(t / g.M), (uint32_t)(t % g.M), c8, v);
  }
}

// Split-K reduction + epilogue + GroupNorm statistics (g.stats, vec_epi, no
// GEGLU, N % 32 == 0): grid (N / 32, ceil(M / 64), batch); workgroup (x, y)
// owns rows [64y, 64y + 64) x columns [32x, 32x + 32); thread t reduces
// columns 32x + 8*(t % 4) .. +8 of row 64y + t/4.
__global__ __launch_bounds__(256) void k_splitk_reduce_stats(GemmArgs g) {
  args_warm(g);
  constexpr int LDR = 33;
  __shared__ float red[64 * LDR];
  const uint32_t t = threadIdx.x, cv = t % 4, rr = t / 4;
  const uint32_t n = blockIdx.x * 32 + cv * 8, bz = blockIdx.z;
  const uint32_t m = blockIdx.y * 64 + rr;
  float v[8] = {};
  if (m < g.M) splitk_vec8(g, bz, m, n, v);
#pragma unroll
  for (int j = 0; j < 8; j++) red[rr * LDR + cv * 8 + j] = v[j];
  __syncthreads();
  // column sums (t / 4 < 32) and sums of squares (t / 4 >= 32) of the 64
  // staged rows: four adjacent lanes take every fourth row and add their
  // sums by lane swaps in a fixed order (one thread per column spent a
  // dependent add per row)
  {
    const uint32_t item = t / 4, part = t % 4, col = item % 32, st = item / 32;
    float a = 0.0f;
    // a constant trip count, so the 16 LDS reads are issued together (from a
    // lane-dependent start the loop stays rolled, one LDS round trip per row)
#pragma unroll
    for (uint32_t k = 0; k < 16; k++) {
      const float x = red[(part + 4 * k) * LDR + col];
      a += st ? __fmul_rn(x, x) : x;
    }
    a += __shfl_xor(a, 1);
    a += __shfl_xor(a, 2);
    if (part == 0) {
      const uint64_t chunk = (uint64_t)bz * ((g.M + 63) / 64) + blockIdx.y;
      g.stats[(chunk * g.N + blockIdx.x * 32 + col) * 2 + st] = a;
    }
  }
}

// Split-K reduction fused with the GroupNorm (+SiLU) of its output (GnFuse):
// workgroup (group, image) sums the partials of the group's cpg channels
// over the image's HW = RS IM rows in split order and applies x * alpha +
// bias (+ temb bias) (+ residual, RES) as the vector reducer does (the same
// fp16 values, stored as the output when f.raw), then takes the group's
// mean and variance of those fp16 values (E[x^2] - E[x]^2, clamped at 0:
// GroupNorm's statistics) inside the workgroup and writes GN(x) (+SiLU)
// to f.y.  Thread t of RS Q (<= 640):
// channel quad q = t % Q (Q = cpg / 4), rows t / Q + RS i, i < IM (HW = RS
// IM), from partials the GEMM stored in column groups of cpg, so a wave
// reads 1 KB contiguous per load.  The split count S
// is a template parameter: the IM x S partial loads are straight-line code
// in batches of at most 24, each batch issued before any of it is added (a
// loop over splits would make the compiler wait for every load at its top).
// NS > 1: NS workgroups per (group, image) (x = group * NS + slice), each
// taking HW / NS = RS IM consecutive rows, exchange their (sum, sumsq)
// through the group's record in f.xchg's region for NS (the protocol of
// di_device.h) and sum the slices' partials in slice order, so all agree
// bit for bit.  Should a slice not arrive within f.spin polls, the
// workgroup recomputes every other slice's sums from the split-K partials
// (written by the launch before) with the same code and order: the same
// bits, so the kernel always ends.
template <int IM, int S, bool RES, int NS>
__global__ __launch_bounds__(640) void k_splitk_reduce_gn(GemmArgs g, GnFuse f, uint32_t Q,
                                                          uint32_t RS) {
  args_warm(g);
  kernarg_warm(f);
  __shared__ float red[2][10];
  __shared__ __attribute__((aligned(16))) float sst[64 * 40];  // one chunk, f.stats only
  constexpr bool XCH = NS > 1;
  static_assert(NS == 1 || NS == 4 || NS == kXchgSlices, "record regions");
  __shared__ float sv[2 * NS];                                 // XCH: the slices' sums
  __shared__ uint32_t s_o;
  __shared__ int s_ok;
  const uint32_t tid = threadIdx.x, n = blockIdx.y;
  const uint32_t grp = blockIdx.x / NS, sl = blockIdx.x % NS;
  const uint32_t hws = RS * IM, hw = hws * NS;  // rows: slice, image
  // tid / Q from a float reciprocal: exact for tid < 1024 (the product stays
  // 0.5 / Q away from an integer, far beyond its rounding error)
  const uint32_t r0 = (uint32_t)(((float)tid + 0.5f) * __builtin_amdgcn_rcpf((float)Q));
  const uint32_t q = tid - r0 * Q, c = grp * Q * 4 + q * 4;
  const uint64_t img0 = (uint64_t)n * hw;  // the image's first row
  uint64_t* const rec =
      XCH ? f.xchg + ((NS == 4 ? kXchgRedRecs : 0u) + (uint64_t)n * f.groups + grp) * kXchgWords
          : nullptr;
  // per-channel and residual operands first: loads retire in order, and
  // these are needed only after the partials.  Without a temb bias the bias
  // is loaded twice rather than a load under a branch; the empty asm hides
  // where the pointer came from, else the compiler turns the second load
  // into a copy of the first, which waits for it before any later load
  const f32x4 bb = ld4(g.bias + c);
  uint64_t tbase = (uint64_t)(g.bias2 ? g.bias2 + (uint64_t)n * g.ld_b2 : g.bias);
  asm volatile("" : "+s"(tbase));
  typedef __attribute__((address_space(1))) const f32x4 gf32x4;  // global, not flat
  const f32x4 tb = *(gf32x4*)(tbase + (uint64_t)c * 4);
  const f32x4 gm = ld4(f.gamma + c);
  const f32x4 bt = ld4(f.beta + c);
  // the stored values h of slice j's rows (this thread's) and their sum and
  // sum of squares; `arrive`: the exchange's arrival fetch-add goes out
  // after the slice's loads (its result is waited for at once, which would
  // hold back loads issued after it)
  auto slice = [&](uint32_t j, f16x4(&h)[IM], float& sum, float& sq, bool arrive) {
    const uint64_t row0 = img0 + (uint64_t)j * hws + r0;
    f16x4 rr[RES ? IM : 1];
    if constexpr (RES) {
      const f16* R = (const f16*)g.res + row0 * g.ldr + c;
#pragma unroll
      for (int i = 0; i < IM; i++) rr[i] = *(const f16x4*)(R + (uint64_t)i * RS * g.ldr);
    }
    // partials in column groups (part_cpg = cpg): the group's rows are
    // contiguous, thread t reads quads t, t + RS Q, ... of the slice
    const float* p = g.part + ((uint64_t)grp * g.M + row0) * (Q * 4) + q * 4;
    const uint64_t sstep = (uint64_t)g.M * g.N, rstep = (uint64_t)RS * Q * 4;
    constexpr int NL = IM * S, NB = NL <= 24 ? NL : IM >= 8 ? 16 : 24;
    f32x4 acc[IM];
#pragma unroll
    for (int i = 0; i < IM; i++) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b0 = 0; b0 < NL; b0 += NB) {
      f32x4 t[NB];
#pragma unroll
      for (int u = 0; u < NB; u++) {
        const int jj = b0 + u;  // split jj / IM of row step jj % IM: splits in order per row
        if (jj < NL) t[u] = ld4(p + (uint64_t)(jj / IM) * sstep + (uint64_t)(jj % IM) * rstep);
      }
      if constexpr (XCH) {
        if (arrive && b0 + NB >= NL && tid == 0) s_o = xchg_arrive(rec);
      }
      // the whole batch is issued before the scheduler may start its adds
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < NB; u++) {
        const int jj = b0 + u;
        if (jj < NL) acc[jj % IM] += t[u];
      }
    }
    sum = 0.0f;
    sq = 0.0f;
#pragma unroll
    for (int i = 0; i < IM; i++) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float v = acc[i][k] * g.alpha;
        v += bb[k];
        if (g.bias2) v += tb[k];
        if constexpr (RES) v += (float)rr[i][k];
        h[i][k] = (f16)v;
        const float x = (float)h[i][k];
        sum += x;
        sq += __fmul_rn(x, x);
      }
    }
  };
  f16x4 h[IM];
  float sum, sq;
  slice(sl, h, sum, sq, true);
  sum = wave_sum(sum);
  sq = wave_sum(sq);
  if (tid % 64 == 0) {
    red[0][tid / 64] = sum;
    red[1][tid / 64] = sq;
  }
  const uint64_t row0 = img0 + (uint64_t)sl * hws + r0;
  if (f.stats) {
    // per 64-row chunk and channel (sum, sum of squares) of the stored
    // values, the GemmArgs::stats layout: row step i holds the slice's
    // chunks i * RS / 64 .. + RS / 64 - 1.  Step by step through LDS
    // ([RS][cpg] floats, RS * cpg = 16 * blockDim <= 64 * 40): 8 adjacent
    // lanes per (chunk, statistic, channel) each take every eighth row of
    // the chunk, added by lane swaps in a fixed order (RS cpg / 32 tasks
    // x 8 lanes = every thread).
    const uint32_t cpg = Q * 4, task = tid >> 3, part = tid & 7;
    const uint32_t cs = (uint32_t)(((float)task + 0.5f) * __builtin_amdgcn_rcpf((float)cpg));
    const uint32_t ch = task - cs * cpg, lc = cs >> 1, st = cs & 1;
    const uint64_t chunk0 = (img0 + (uint64_t)sl * hws) / 64 + lc;
#pragma unroll
    for (int i = 0; i < IM; i++) {
      *(f32x4*)&sst[r0 * cpg + q * 4] =
          f32x4{(float)h[i][0], (float)h[i][1], (float)h[i][2], (float)h[i][3]};
      __syncthreads();
      float a = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float x = sst[(lc * 64 + part + 8 * k) * cpg + ch];
        a += st ? __fmul_rn(x, x) : x;
      }
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
      a += __shfl_xor(a, 4);
      if (part == 0)
        f.stats[((chunk0 + (uint64_t)i * (RS / 64)) * g.N + grp * cpg + ch) * 2 + st] = a;
      __syncthreads();
    }
  }
  __syncthreads();
  float ps = 0.0f, pq = 0.0f;
  for (uint32_t w = 0; w < blockDim.x / 64; w++) {
    ps += red[0][w];
    pq += red[1][w];
  }
  if constexpr (XCH) {
    const uint64_t ep = (uint64_t)(s_o / NS + 1u) << 32;  // s_o: before the barrier
    const bool all = xchg_publish_poll<NS>(rec, ep, sl, ps, pq, f.spin, sv);
    if (tid == 0) s_ok = all ? 1 : 0;
    __syncthreads();
    if (!s_ok) {
      for (uint32_t j = 0; j < NS; j++) {
        if (j == sl) {
          if (tid == 0) {
            sv[2 * j] = ps;
            sv[2 * j + 1] = pq;
          }
          continue;
        }
        f16x4 ht[IM];
        float s2, q2;
        slice(j, ht, s2, q2, false);
        s2 = wave_sum(s2);
        q2 = wave_sum(q2);
        __syncthreads();  // every read of red before is done
        if (tid % 64 == 0) {
          red[0][tid / 64] = s2;
          red[1][tid / 64] = q2;
        }
        __syncthreads();
        if (tid == 0) {
          float a = 0.0f, b = 0.0f;
          for (uint32_t w = 0; w < blockDim.x / 64; w++) {
            a += red[0][w];
            b += red[1][w];
          }
          sv[2 * j] = a;
          sv[2 * j + 1] = b;
        }
      }
      __syncthreads();
    }
    ps = 0.0f;
    pq = 0.0f;
    for (uint32_t j = 0; j < NS; j++) {
      ps += sv[2 * j];
      pq += sv[2 * j + 1];
    }
  }
  const float L = (float)(Q * 4) * (float)hw;
  const float mean = ps / L;
  const float var = fmaxf(pq / L - mean * mean, 0.0f);
  const float rstd = 1.0f / sqrtf(var + f.eps);
  float a[4], b[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    a[j] = rstd * gm[j];
    b[j] = bt[j] - mean * a[j];
  }
  if (f.raw) {
    f16* C = (f16*)g.c + row0 * g.ldc + c;
#pragma unroll
    for (int i = 0; i < IM; i++) *(f16x4*)(C + (uint64_t)i * RS * g.ldc) = h[i];
  }
  f16* y = (f16*)f.y + row0 * f.ldy + c;
#pragma unroll
  for (int i = 0; i < IM; i++) {
    f16x4 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float r = (float)h[i][j] * a[j] + b[j];
      o[j] = (f16)(f.silu ? silu_f(r) : r);
    }
    *(f16x4*)(y + (uint64_t)i * RS * f.ldy) = o;
  }
}

// (row steps, split count) pairs the fused reducer is built for (16 row
// steps would spill its accumulators to scratch); with the exchange, eight
// slices (images of 512 or 1024 rows: slices of 64 or 128) and four (256
// rows: slices of 64)
#define DI_RGN_CASES(X)                                                                   \
  X(1, 2) X(1, 3) X(1, 4) X(1, 5) X(1, 6) X(1, 8) X(1, 12) X(2, 2) X(2, 3) X(2, 4) X(2, 5) \
  X(2, 6) X(2, 8) X(2, 12) X(4, 2) X(4, 3) X(4, 4) X(4, 5) X(4, 6) X(4, 8) X(4, 12)       \
  X(8, 2) X(8, 3) X(8, 4) X(8, 5) X(8, 6)
#define DI_RGNX_CASES(X) \
  X(1, 2) X(1, 3) X(1, 4) X(1, 5) X(1, 6) X(2, 2) X(2, 3) X(2, 4) X(2, 5) X(2, 6)
#define DI_RGNX4_CASES(X) X(1, 2) X(1, 3) X(1, 4) X(1, 5) X(1, 6) X(1, 8) X(1, 12)

bool splitk_gn_built(uint32_t im, uint32_t splits, uint32_t ns) {
#define DI_RGN_HAS(IMV, SV) if (im == IMV && splits == SV) return true;
  if (ns == kXchgSlices) {
    DI_RGNX_CASES(DI_RGN_HAS)
  } else if (ns == 4) {
    DI_RGNX4_CASES(DI_RGN_HAS)
  } else {
    DI_RGN_CASES(DI_RGN_HAS)
  }
#undef DI_RGN_HAS
  return false;
}

// Rows per step of the fused reducer: the most (a multiple of 64 dividing
// hw) with at most 640 threads.
uint32_t splitk_gn_rs(uint32_t q, uint32_t hw) {
  uint32_t rs = 64;
  while (2 * rs * q <= 640 && hw % (2 * rs) == 0) rs *= 2;
  return rs;
}

// Workgroups per (group, image) of the fused reducer: eight exchanging their
// statistics for images of more than 256 rows, four for 256 rows, else one
// (DI_GN_REDUCE_XCHG=0: one always)
uint32_t splitk_gn_slices(const GnFuse& f) {
  const char* e = getenv("DI_GN_REDUCE_XCHG");
  if (!f.xchg || (e && e[0] == '0')) return 1;
  return f.hw > 256 ? kXchgSlices : f.hw == 256 ? 4u : 1u;
}

void launch_splitk_reduce_gn(const GemmArgs& g, const GnFuse& f, hipStream_t s) {
  const uint32_t ns = splitk_gn_slices(f), hws = f.hw / ns;
  const uint32_t q = g.N / f.groups / 4, rs = splitk_gn_rs(q, hws), im = hws / rs;
  const dim3 grid(f.groups * ns, g.M / f.hw), block(rs * q);
#define DI_RGN_LAUNCH_NS(IMV, SV, NSV)                                              \
  if (im == IMV && g.splits == SV) {                                                \
    if (g.res)                                                                      \
      k_splitk_reduce_gn<IMV, SV, true, NSV><<<grid, block, 0, s>>>(g, f, q, rs);  \
    else                                                                            \
      k_splitk_reduce_gn<IMV, SV, false, NSV><<<grid, block, 0, s>>>(g, f, q, rs); \
    return;                                                                         \
  }
#define DI_RGN_LAUNCH(IMV, SV) DI_RGN_LAUNCH_NS(IMV, SV, 1)
#define DI_RGNX_LAUNCH(IMV, SV) DI_RGN_LAUNCH_NS(IMV, SV, 8)
#define DI_RGNX4_LAUNCH(IMV, SV) DI_RGN_LAUNCH_NS(IMV, SV, 4)
  static_assert(kXchgSlices == 8, "DI_RGNX_LAUNCH");
  if (ns == kXchgSlices) {
    DI_RGNX_CASES(DI_RGNX_LAUNCH)
  } else if (ns == 4) {
    DI_RGNX4_CASES(DI_RGNX4_LAUNCH)
  } else {
    DI_RGN_CASES(DI_RGN_LAUNCH)
  }
#undef DI_RGN_LAUNCH_NS
#undef DI_RGN_LAUNCH
#undef DI_RGNX_LAUNCH
#undef DI_RGNX4_LAUNCH
  // splitk_gn_ok admits only built pairs: reaching here would leave the
  // output unwritten
  fprintf(stderr, "launch_splitk_reduce_gn: no instantiation for %u row steps x %u splits\n", im,
          g.splits);
  abort();
}

const uint32_t kTileM[TILE_COUNT] = {64, 128, 64, 128, 128, 64, 64, 128, 64, 64, 128, 128, 64, 128, 64};
const uint32_t kTileN[TILE_COUNT] = {64, 64, 128, 128, 160, 160, 64, 64, 128, 128, 64, 128, 64, 64, 32};
// Relative per-CU MFMA efficiency of each tile shape (the 2x2 wavefront tile
// sets LDS bytes per MFMA cycle); tuned by measurement.
const double kTileEff[TILE_COUNT] = {0.35, 0.5, 0.5, 0.8, 0.85, 0.55, 0.35, 0.5, 0.5,
                                      0.5, 0.5, 0.8, 0.35, 0.8, 0.25};
bool vec_epi_ok(const GemmArgs& g, int elem, int tile_cfg);

}  // namespace

namespace {

// Measured plans for the U-Net step's GEMM shapes (a timed sweep); other
// shapes use the cost model below.
struct TunedPlan {
  uint32_t M, N, K, conv, ks, stride, up, geglu;
  int tile;
  uint32_t splits;
};
const TunedPlan kTuned[] = {
#include "gemm_tuned.inc"
    {0, 0, 0, 0, 0, 0, 0, 0, TILE_64x64, 1},  // end
};

bool tuned_plan(const GemmArgs& g, GemmPlan* out) {
  const uint32_t conv = g.Cin > 0 ? 1 : 0;
  const uint32_t ks = conv ? g.ks : 0, stride = conv ? g.stride : 0, up = conv ? g.up : 0;
  const uint32_t geglu = g.act == ACT_GEGLU ? 1 : 0;
  for (const TunedPlan& t : kTuned) {
    if (t.M == g.M && t.N == g.N && t.K == g.K && t.conv == conv && t.ks == ks &&
        t.stride == stride && t.up == up && t.geglu == geglu && t.M != 0) {
      *out = GemmPlan{t.tile, t.splits};
      return true;
    }
  }
  return false;
}

}  // namespace

// DI_GEMM_TILE / DI_GEMM_SPLITS (tuning runs): a value that is not a whole
// number, names no built tile (or the halo conv for a conv it cannot take),
// or asks for splits outside [1, 64] is ignored, so no override can index
// the tile tables out of range.
static void env_plan_override(const GemmArgs& g, int elem, const char* env_tile,
                              const char* env_split, GemmPlan* plan) {
  if (env_tile) {
    char* end = nullptr;
    const long t = strtol(env_tile, &end, 10);
    const bool ok = end != env_tile && *end == '\0' && t >= 0 && t < TILE_COUNT &&
                    t != TILE_128x160 &&
                    (t != TILE_CONV3_HALO ||
                     (conv3_halo_ok(g) && vec_epi_ok(g, elem, TILE_CONV3_HALO)));
    if (ok) plan->tile = (int)t;
  }
  if (env_split) {
    char* end = nullptr;
    const long sp = strtol(env_split, &end, 10);
    if (end != env_split && *end == '\0' && sp >= 1 && sp <= 64) plan->splits = (uint32_t)sp;
  }
  if (plan->splits < 1) plan->splits = 1;
}

GemmPlan gemm_plan(const GemmArgs& g, int elem, int num_cus) {
  // DI_GEMM_PLAN="M,N,K,tile,splits;..." fixes the plan of the listed fp16
  // shapes only (tuning runs of the whole step; tile 13 = the halo conv)
  if (const char* env_plan = getenv("DI_GEMM_PLAN"); env_plan && elem == DI_F16) {
    for (const char* p = env_plan; p && *p;) {
      unsigned m, n, k, t, sp;
      if (sscanf(p, "%u,%u,%u,%u,%u", &m, &n, &k, &t, &sp) == 5 && m == g.M && n == g.N &&
          k == g.K && t < TILE_COUNT && t != TILE_128x160 && sp >= 1)
        return GemmPlan{(int)t, sp};
      p = strchr(p, ';');
      if (p) p++;
    }
  }
  const char* env_tile = getenv("DI_GEMM_TILE");
  const char* env_split = getenv("DI_GEMM_SPLITS");
  GemmPlan best{TILE_64x64, 1};
  // 3x3 convs the halo kernel takes, from 5 channel chunks up (with fewer,
  // measured on the VAE's 128- / 256-channel convs, the pipeline prologue
  // dominates and the implicit GEMM's larger tiles win); DI_CONV_HALO=0
  // turns it off for A/B runs
  const char* env_halo = getenv("DI_CONV_HALO");
  if (elem == DI_F16 && !env_tile && (!env_halo || atoi(env_halo) != 0) && g.Cin >= 320 &&
      conv3_halo_ok(g) && vec_epi_ok(g, elem, TILE_CONV3_HALO)) {
    // channel-chunk splits bring the workgroup count near 224 (measured best
    // at 16x16 / 32x32 / 64x64: 200-240 workgroups, one per CU)
    const uint32_t tiles = (g.M / 128) * (g.N / 64), nch = g.Cin / 64;
    uint32_t hs = 1;
    for (uint32_t sp = 2; sp <= nch && sp <= 16; sp++) {
      if (nch % sp) continue;
      const int64_t d = llabs((int64_t)tiles * sp - 224), db = llabs((int64_t)tiles * hs - 224);
      if (d < db) hs = sp;
    }
    const char* env_hs = getenv("DI_CONV_HALO_SPLITS");
    if (env_hs) hs = (uint32_t)atoi(env_hs);
    if (hs >= 1 && nch % hs == 0) return GemmPlan{TILE_CONV3_HALO, hs};
  }
  if (elem == DI_F16 && tuned_plan(g, &best)) {
    env_plan_override(g, elem, env_tile, env_split, &best);
    return best;
  }
  if (elem == DI_F32) {
    uint64_t t = (uint64_t)((g.M + 127) / 128) * ((g.N + 127) / 128) * g.batch;
    best.tile = t >= (uint64_t)num_cus / 2 ? TILE_128x128 : TILE_64x64;
    return best;
  }
  const double cus = num_cus;
  double best_t = 1e300;
  for (int tc = 0; tc < TILE_COUNT; tc++) {
    if (tc == TILE_128x160) continue;  // spills registers: not built
    if (tc >= TILE_64x128_W16) continue;  // sixteen-wave tiles: measured table only
    if (g.act == ACT_GEGLU && kTileN[tc] == 160) continue;  // GEGLU pairs need even TN
    const uint64_t mt = (g.M + kTileM[tc] - 1) / kTileM[tc], nt = (g.N + kTileN[tc] - 1) / kTileN[tc];
    const uint64_t T = mt * nt * g.batch;
    for (uint32_t s = 1; s <= 32; s++) {
      const uint32_t kper = ((g.K + s - 1) / s + 63) / 64 * 64;
      if (s > 1 && kper < 256) break;
      const double rounds = ceil((double)T * s / cus);
      // cycles per work unit at the tile's efficiency (4096 fp16 FLOP/clk/CU)
      // plus a fixed prologue / epilogue cost
      const double cyc = 2.0 * kTileM[tc] * kTileN[tc] * kper / (4096.0 * kTileEff[tc]) + 3000.0;
      double t = rounds * cyc;
      if (s > 1)  // fp32 partials written and read back (~4 TB/s) plus a launch
        t += (double)g.batch * g.M * g.N * 4.0 * (s + 1) / (4.0e12 / 2.4e9) + 5000.0;
      if (t < best_t * 0.97) {
        best_t = t;
        best = GemmPlan{tc, s};
      }
    }
  }
  env_plan_override(g, elem, env_tile, env_split, &best);
  return best;
}

namespace {

template <typename S>
__global__ void k_repack(const S* __restrict__ w, f16* __restrict__ out, uint32_t Cout,
                         uint32_t Cin, uint32_t ks, uint32_t Cin_pad) {
  const uint32_t taps = ks * ks;
  const uint64_t total = (uint64_t)Cout * taps * Cin_pad;
  uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    uint32_t ci = i % Cin_pad;
    uint64_t t = i / Cin_pad;
    uint32_t tap = t % taps;
    uint32_t oc = (uint32_t)(t / taps);
    out[i] = ci < Cin ? (f16)(float)w[((uint64_t)oc * Cin + ci) * taps + tap] : (f16)0.0f;
  }
}

}  // namespace

void launch_repack_oihw_ohwi(hipStream_t s, const void* w, int wdt, void* out, uint32_t Cout,
                             uint32_t Cin, uint32_t ks, uint32_t Cin_pad) {
  uint64_t total = (uint64_t)Cout * ks * ks * Cin_pad;
  uint64_t blocks = (total + 255) / 256;
  if (blocks > 65535ull * 8) blocks = 65535ull * 8;
  if (wdt == DI_F32)
    k_repack<float><<<(unsigned)blocks, 256, 0, s>>>((const float*)w, (f16*)out, Cout, Cin, ks, Cin_pad);
  else
    k_repack<f16><<<(unsigned)blocks, 256, 0, s>>>((const f16*)w, (f16*)out, Cout, Cin, ks, Cin_pad);
}

uint64_t gemm_ws_bytes(const GemmArgs& g) {
  const uint64_t slots = g.part_slots ? g.part_slots : g.splits;
  return g.splits > 1 ? slots * g.batch * g.M * g.N * sizeof(float) : 0;
}

bool gemm_fast_ok(const GemmArgs& g, int elem, int a_mode, int b_mode) {
  // a2 == nullptr: single source (launch_gemm then sets a2 = a)
  const uint32_t a2_bytes = g.a2 ? g.a2_bytes : g.a_bytes;
  const bool single = !g.a2 || g.c1 == 0xffffffffu || g.a2 == g.a;
  if (elem != DI_F16 || b_mode != B_NK || !g.b_vec_ok) return false;
  if (g.a_bytes == 0 || a2_bytes == 0 || g.b_bytes == 0) return false;  // extents unknown
  if (g.K % 64 != 0) return false;  // whole 64-element stages (no per-lane k bound)
  if (a_mode == A_DENSE) return g.a_vec_ok && single;
  if (a_mode == A_CONV_NHWC) return g.Cin % 64 == 0 && (single || g.c1 % 64 == 0) && (g.up == 1 || g.up == 2);
  return false;
}

namespace {
bool vec_epi_ok(const GemmArgs& g, int elem, int tile_cfg) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  return elem == DI_F16 && !g.c_nchw && !g.c_f32 && g.N % 8 == 0 && g.ldc % 8 == 0 &&
         g.sc % 8 == 0 && al16(g.c) && (!g.bias || al16(g.bias)) &&
         (!g.bias2 || (al16(g.bias2) && g.ld_b2 % 4 == 0)) &&
         (!g.res || (!g.res_f32 && g.ldr % 8 == 0 && g.sr % 8 == 0 && al16(g.res))) &&
         (g.act != ACT_GEGLU || g.N % 32 == 0) && tile_cfg != TILE_128x160;
}
}  // namespace

bool gemm_stats_ok(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg) {
  return gemm_fast_ok(g, elem, a_mode, b_mode) && vec_epi_ok(g, elem, tile_cfg) &&
         g.act != ACT_GEGLU && g.batch == 1 && (g.splits <= 1 || g.N % 32 == 0);
}

bool gemm_rstats_ok(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg) {
  GemmArgs h = g;
  h.splits = 1;
  // row groups of the vector epilogue must divide a wavefront (not 160
  // wide); at least 32 columns per tile, so that [rows][ceil(N / 32)] pairs
  // hold the layout (the callers' buffers are sized so)
  return gemm_stats_ok(h, elem, a_mode, b_mode, tile_cfg) && g.splits <= 1 &&
         kTileN[tile_cfg] >= 32 && 64 % (kTileN[tile_cfg] / 8) == 0;
}

bool gemm_lnfold_ok(const GemmArgs& g, int elem, int tile_cfg) {
  // without split-K the fold runs in the buffer-load kernel's epilogue, with
  // it in the vector split-K reducer
  return vec_epi_ok(g, elem, tile_cfg) && g.batch == 1 && !g.stats && !g.rstats && g.ln_s &&
         ((uintptr_t)g.ln_s & 15) == 0 && ((uintptr_t)g.ln_rows & 7) == 0 && g.ln_nt > 0 && g.K > 0 &&
         (g.splits > 1 || gemm_fast_ok(g, elem, A_DENSE, B_NK));
}

uint32_t gemm_rstats_tiles(const GemmArgs& g, int tile_cfg) {
  return (g.N + kTileN[tile_cfg] - 1) / kTileN[tile_cfg];
}

bool splitk_gn_ok(const GemmArgs& g, const GnFuse& f) {
  if (g.splits <= 1 || g.batch != 1 || !f.groups || !f.hw || !f.gamma || !f.beta || !f.y)
    return false;
  // images of more than 256 rows: kXchgSlices workgroups per (group,
  // image) exchanging their statistics (with the raw output one workgroup
  // per group did not pay: at 32 x 32 the fused conv2 reducer took 11.2 us
  // against 5.0 + 5.0 us for the reducer and apply it replaces)
  const uint32_t ns = splitk_gn_slices(f);
  if (f.raw && f.hw > 256 && ns == 1) return false;
  const uint32_t hws = f.hw / ns;  // rows per workgroup
  if (ns > 1 && (f.hw % ns != 0 || (uint64_t)(g.M / f.hw) * f.groups >
                                       (ns == 4 ? kXchgRed4Recs : kXchgRedRecs)))
    return false;
  // statistics of the stored values only with the raw output
  if (f.stats && (!f.raw || ((uintptr_t)f.stats & 7) != 0)) return false;
  const uint32_t cpg = g.N / f.groups, slots = g.part_slots ? g.part_slots : g.splits;
  return g.N % f.groups == 0 && cpg % 4 == 0 && cpg <= 40 && hws % 64 == 0 &&
         splitk_gn_built(hws / splitk_gn_rs(cpg / 4, hws), slots, ns) && g.M % f.hw == 0 &&
         g.bias && (!g.bias2 || (g.rows_b2 == f.hw && g.ld_b2 % 4 == 0)) &&
         (!g.res || (!g.res_f32 && g.ldr % 4 == 0 && ((uintptr_t)g.res & 7) == 0)) &&
         (!f.raw || (g.c && g.ldc % 4 == 0 && ((uintptr_t)g.c & 7) == 0)) &&
         g.act == ACT_NONE && !g.c_f32 && !g.c_nchw && f.ldy % 4 == 0 &&
         ((uintptr_t)f.y & 7) == 0 && ((uintptr_t)g.bias & 15) == 0 &&
         ((uintptr_t)g.bias2 & 15) == 0 && ((uintptr_t)f.gamma & 15) == 0 &&
         ((uintptr_t)f.beta & 15) == 0;
}

void launch_gemm(GemmArgs g, int elem, int a_mode, int b_mode, int tile_cfg, hipStream_t s,
                 const GnFuse* gn) {
  // k_split in elements, multiple of the stage depth
  const uint32_t bk = elem == DI_F32 ? 32 : 64;
  if (g.splits < 1) g.splits = 1;
  uint32_t per = (g.K + g.splits - 1) / g.splits;
  g.k_split = (per + bk - 1) / bk * bk;
  if (g.rows_b2 == 0) g.rows_b2 = 0xffffffffu;
  if (!g.a2) {
    g.a2 = g.a;
    g.lda2 = g.lda;
    g.sa2 = g.sa;
    g.a2_bytes = g.a_bytes;
    if (g.c1 == 0) g.c1 = 0xffffffffu;
  }
  const bool trace = getenv("DI_TRACE_GEMM") != nullptr;
  if (trace)
    fprintf(stderr,
            "[di_gemm] M=%u N=%u K=%u batch=%u amode=%d bmode=%d elem=%d cin=%u hw=%ux%u ks=%u "
            "stride=%u up=%u tile=%d splits=%u act=%d fast=%d\n",
            g.M, g.N, g.K, g.batch, a_mode, b_mode, elem, g.Cin, g.H, g.W, g.ks, g.stride, g.up,
            tile_cfg, g.splits, g.act, (int)gemm_fast_ok(g, elem, a_mode, b_mode));
  g.vec_epi = vec_epi_ok(g, elem, tile_cfg);
  const bool fast = gemm_fast_ok(g, elem, a_mode, b_mode);
  bool halo = false;
  if (tile_cfg == TILE_CONV3_HALO) {
    halo = fast && a_mode == A_CONV_NHWC && g.vec_epi && conv3_halo_ok(g) &&
           (g.Cin / 64) % g.splits == 0;
    if (!halo) {
      tile_cfg = TILE_64x128_K2;  // a caller-chosen plan the halo kernel does not take
      g.vec_epi = vec_epi_ok(g, elem, tile_cfg);
    }
  }
  if (halo) {
    launch_conv3_halo(g, s);
  } else if (fast) {
    if (a_mode == A_DENSE && g.ln_rows && g.splits <= 1) gemm_fast_dense_ex(g, tile_cfg, s);
    else if (a_mode == A_DENSE && g.rstats) gemm_fast_dense_ex(g, tile_cfg, s);
    else if (a_mode == A_DENSE) gemm_fast_dense(g, tile_cfg, s);
    else gemm_fast_conv(g, tile_cfg, s);
  } else {
    gemm_slow(g, elem, a_mode, b_mode, tile_cfg, s);
  }
  if (g.splits > 1 && g.part_only) return;  // a later launch's reducer sums the slots
  if (g.splits > 1 && g.part_slots) g.splits = g.part_slots;  // the reducers sum every slot
  if (g.splits > 1 && gn) {
    launch_splitk_reduce_gn(g, *gn, s);  // g.part_cpg set by the caller
  } else if (g.splits > 1 && g.stats) {
    k_splitk_reduce_stats<<<dim3(g.N / 32, (g.M + 63) / 64, g.batch), 256, 0, s>>>(g);
  } else if (g.splits > 1) {
    uint32_t ncols = g.act == ACT_GEGLU ? g.N / 2 : g.N;
    uint64_t total = (uint64_t)g.batch * g.M * ncols;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65535ull * 8) blocks = 65535ull * 8;
    if (g.vec_epi) {
      uint64_t vblocks = (total / 8 + 255) / 256;
      if (vblocks > 65535ull * 8) vblocks = 65535ull * 8;
      k_splitk_reduce_vec<<<(unsigned)vblocks, 256, 0, s>>>(g);
    } else {
      k_splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(g);
    }
  }
}

}  // namespace di

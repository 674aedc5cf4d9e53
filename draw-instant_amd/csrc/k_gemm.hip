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

// ---- the GEMM kernel ----
template <typename T, int BM, int BN, int WGM, int WGN, int AM, int BMD>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs g) {
  using MT = Mfma<T>;
  constexpr int KV = MT::KV;
  constexpr int BK = 128 / sizeof(T);  // k elements per stage (128 bytes per row)
  constexpr int VPR = BK / KV;         // 16-byte vectors per row per stage (8)
  constexpr int LDK = BK + KV;         // padded LDS row (elements)
  constexpr int NVA = BM * VPR / 256;  // A vectors per thread per stage
  constexpr int NVB = BN * VPR / 256;
  constexpr int WM = BM / WGM, WN = BN / WGN;  // wave tile
  constexpr int TM = WM / 16, TN = WN / 16;
  static_assert(WGM * WGN == 4, "4 wavefronts");
  static_assert(NVA >= 1 && NVB >= 1 && TM >= 1 && TN >= 1, "tile too small");

  __shared__ __attribute__((aligned(16))) T sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) T sB[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WGN) * WM, wn0 = (wave % WGN) * WN;

  // tile coordinates: N fastest so neighbouring workgroups share A rows
  const uint32_t n_tiles = (g.N + BN - 1) / BN;
  const uint32_t tile = blockIdx.x;
  const uint32_t m0 = (tile / n_tiles) * BM, n0 = (tile % n_tiles) * BN;
  const uint32_t splits = g.splits;
  const uint32_t bz = blockIdx.z / splits, split = blockIdx.z % splits;
  const uint32_t k_begin = split * g.k_split;
  const uint32_t k_end = min(g.K, k_begin + g.k_split);
  // a trailing split may start past K: it contributes zeros to the reduction
  const int n_stages = k_end > k_begin ? (int)((k_end - k_begin + BK - 1) / BK) : 0;

  const T* A = (const T*)g.a + (uint64_t)bz * g.sa;
  const T* A2 = (const T*)g.a2 + (uint64_t)bz * g.sa2;
  const T* B = (const T*)g.b + (uint64_t)bz * g.sb;

  // ---- per-thread A addressing (rows fixed for the whole K loop) ----
  const int kc = tid % VPR;  // same k-vector slot for all of this thread's vectors
  int64_t a_row_off[NVA];     // dense: row offset; conv: image pixel base
  int a_iy0[NVA], a_ix0[NVA];
  bool a_row_ok[NVA];
#pragma unroll
  for (int i = 0; i < NVA; i++) {
    uint32_t r = (tid + i * 256) / VPR;
    uint32_t m = m0 + r;
    a_row_ok[i] = m < g.M;
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

  typename MT::vec ra[NVA], rb[NVB];

  auto load_a = [&](int stage) {
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
      ra[i] = v;
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

  auto load_b = [&](int stage) {
    const uint32_t kbase = k_begin + stage * BK;
#pragma unroll
    for (int i = 0; i < NVB; i++) {
      typename MT::vec v = zero_vec<T>();
      if constexpr (BMD == B_NK) {
        uint32_t r = (tid + i * 256) / VPR;
        uint32_t n = n0 + r, k = kbase + kc * KV;
        if (n < g.N) {
          if (b_fast && k + KV <= k_end) {
            v = *(const typename MT::vec*)(B + (uint64_t)n * g.ldb + k);
          } else {
#pragma unroll
            for (int j = 0; j < KV; j++)
              if (k + j < k_end) v[j] = B[(uint64_t)n * g.ldb + k + j];
          }
        }
      } else {  // B_KN: vector along n at fixed k; transposed into LDS at store
        constexpr int VPK = BN / KV;  // vectors per k row
        uint32_t kr = (tid + i * 256) / VPK, nc = (tid + i * 256) % VPK;
        uint32_t k = kbase + kr, n = n0 + nc * KV;
        if (k < k_end) {
          if (b_fast && n + KV <= g.N) {
            v = *(const typename MT::vec*)(B + (uint64_t)k * g.ldb + n);
          } else {
#pragma unroll
            for (int j = 0; j < KV; j++)
              if (n + j < g.N) v[j] = B[(uint64_t)k * g.ldb + n + j];
          }
        }
      }
      rb[i] = v;
    }
  };

  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NVA; i++) {
      uint32_t r = (tid + i * 256) / VPR;
      *(typename MT::vec*)&sA[buf][r * LDK + kc * KV] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NVB; i++) {
      if constexpr (BMD == B_NK) {
        uint32_t r = (tid + i * 256) / VPR;
        *(typename MT::vec*)&sB[buf][r * LDK + kc * KV] = rb[i];
      } else {
        constexpr int VPK = BN / KV;
        uint32_t kr = (tid + i * 256) / VPK, nc = (tid + i * 256) % VPK;
#pragma unroll
        for (int j = 0; j < KV; j++) sB[buf][(nc * KV + j) * LDK + kr] = rb[i][j];
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; a++)
#pragma unroll
    for (int b = 0; b < TN; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n_stages > 0) {
    load_a(0);
    load_b(0);
    store_stage(0);
  }
  __syncthreads();

  const int fr = lane & 15, fk = (lane >> 4) * MT::FK;
  for (int s = 0; s < n_stages; s++) {
    const int cur = s & 1;
    if (s + 1 < n_stages) {
      load_a(s + 1);
      load_b(s + 1);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += MT::KM) {
      typename MT::frag af[TM], bf[TN];
#pragma unroll
      for (int a = 0; a < TM; a++) af[a] = ld_frag<T>(&sA[cur][(wm0 + a * 16 + fr) * LDK + kk + fk]);
#pragma unroll
      for (int b = 0; b < TN; b++) bf[b] = ld_frag<T>(&sB[cur][(wn0 + b * 16 + fr) * LDK + kk + fk]);
#pragma unroll
      for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++) acc[a][b] = MT::mma(af[a], bf[b], acc[a][b]);
    }
    if (s + 1 < n_stages) store_stage(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const uint32_t rq = (lane >> 4) * 4;
  if (splits > 1) {
    float* P = g.part + ((uint64_t)split * g.batch + bz) * (uint64_t)g.M * g.N;
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
      for (int b = 0; b < TN; b++) {
        uint32_t n = n0 + wn0 + b * 16 + fr;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          uint32_t m = m0 + wm0 + a * 16 + rq + i;
          if (m < g.M && n < g.N) P[(uint64_t)m * g.N + n] = acc[a][b][i];
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

// Split-K reduction + epilogue: one thread per output element.
__global__ __launch_bounds__(256) void k_splitk_reduce(GemmArgs g) {
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

template <typename T, int BM, int BN, int WGM, int WGN, int AM, int BMD>
void launch_cfg(const GemmArgs& g, hipStream_t s) {
  uint32_t tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  k_gemm<T, BM, BN, WGM, WGN, AM, BMD><<<dim3(tiles, 1, g.batch * g.splits), 256, 0, s>>>(g);
}

template <typename T, int AM, int BMD>
void launch_tile(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  switch (tile_cfg) {
    case TILE_128x128: launch_cfg<T, 128, 128, 2, 2, AM, BMD>(g, s); break;
    case TILE_128x64: launch_cfg<T, 128, 64, 2, 2, AM, BMD>(g, s); break;
    case TILE_64x128: launch_cfg<T, 64, 128, 2, 2, AM, BMD>(g, s); break;
    default: launch_cfg<T, 64, 64, 2, 2, AM, BMD>(g, s); break;
  }
}

uint64_t tiles_of(const GemmArgs& g, int cfg) {
  uint32_t bm = (cfg == TILE_128x128 || cfg == TILE_128x64) ? 128 : 64;
  uint32_t bn = (cfg == TILE_128x128 || cfg == TILE_64x128) ? 128 : 64;
  return (uint64_t)((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn) * g.batch;
}

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

int gemm_pick_tile(const GemmArgs& g, int num_cus) {
  // Largest tile that still gives every CU a workgroup; else 64x64.
  if (tiles_of(g, TILE_128x128) >= (uint64_t)num_cus) return TILE_128x128;
  if (tiles_of(g, TILE_128x64) >= (uint64_t)num_cus) return TILE_128x64;
  if (tiles_of(g, TILE_64x128) >= (uint64_t)num_cus) return TILE_64x128;
  return TILE_64x64;
}

uint32_t gemm_pick_splits(const GemmArgs& g, int tile_cfg, int num_cus) {
  uint64_t t = tiles_of(g, tile_cfg);
  uint32_t k_stages = (g.K + 63) / 64;
  uint32_t s = 1;
  while (t * s * 2 <= (uint64_t)num_cus && k_stages / (s * 2) >= 8 && s < 16) s *= 2;
  return s;
}

uint64_t gemm_ws_bytes(const GemmArgs& g) {
  return g.splits > 1 ? (uint64_t)g.splits * g.batch * g.M * g.N * sizeof(float) : 0;
}

void launch_gemm(GemmArgs g, int elem, int a_mode, int b_mode, int tile_cfg, hipStream_t s) {
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
    if (g.c1 == 0) g.c1 = 0xffffffffu;
  }
#define DI_GEMM_CASE(T, AMv, BMv)                        \
  if (a_mode == AMv && b_mode == BMv) {                  \
    launch_tile<T, AMv, BMv>(g, tile_cfg, s);            \
  }
  if (elem == DI_F16) {
    DI_GEMM_CASE(f16, A_DENSE, B_NK)
    else DI_GEMM_CASE(f16, A_DENSE, B_KN)
    else DI_GEMM_CASE(f16, A_CONV_NHWC, B_NK)
  } else {
    DI_GEMM_CASE(float, A_DENSE, B_NK)
    else DI_GEMM_CASE(float, A_DENSE, B_KN)
    else DI_GEMM_CASE(float, A_CONV_NCHW, B_NK)
  }
#undef DI_GEMM_CASE
  if (g.splits > 1) {
    uint32_t ncols = g.act == ACT_GEGLU ? g.N / 2 : g.N;
    uint64_t total = (uint64_t)g.batch * g.M * ncols;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65535ull * 8) blocks = 65535ull * 8;
    k_splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(g);
  }
}

}  // namespace di

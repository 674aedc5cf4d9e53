// 3x3 stride-1 NHWC fp16 convolution for gfx950 with the input halo staged
// once per channel chunk (the U-Net's and VAE's wide-resolution convs).
//
// The implicit GEMM of k_gemm_kernel.h re-reads every input pixel for each
// of the nine taps, and at B = 1 a CU's global-load throughput (measured
// ~40 B/clk through the vector memory path, whether the data lands in VGPRs
// or goes straight to LDS) bounds the kernel, not the MFMAs or HBM.  Here a
// workgroup owns 128 output pixels = R whole image rows of width W (R =
// 128 / W), or a 128-pixel run of one row of a wider image, and 64 output
// channels; with a fused 2x nearest upsample the patch pixels map to the
// source at half resolution.  For each 64-channel input chunk it loads
// the (R + 2) x (W + 2) pixel patch around its rows once (out-of-image
// pixels arrive as zeros: the padding) and runs the chunk's nine taps from
// it, each tap a 128 x 64 x 64 MFMA step whose A fragments are the patch
// rows shifted by (ky, kx).  Bytes loaded per stage drop from 24 KB to
// 8 KB of weights + ~3.7 KB of patch.
//
// Loads go global -> LDS directly (buffer_load ... lds: lane l of a wave
// writes 16 bytes at base + 16 l), so the XOR chunk swizzle of the LDS rows
// is applied on the global side: the lane that fills physical chunk p of row
// r loads logical chunk p ^ (r & 7).  A fragment read covers 16 consecutive
// rows from any start row (the tap shifts the patch rows by 0..2 + k * PW)
// and 4 chunks; per-row XOR keeps that free of bank conflicts on gfx950
// for every start row, where XOR by row pairs costs 1.33 extra LDS cycles
// per read unless the start row is a multiple of 16 (measured with the
// SQ_LDS_BANK_CONFLICT counter).  Six weight buffers, two patch buffers;
// iteration s (stage s = chunk * 9 + tap) reads the MFMA fragments of stage
// s + 1, runs the MFMAs of stage s, issues the weights of stage s + 5 and,
// at the first taps, pieces of the next chunk's patch.  Every second
// iteration waits until the loads the next two iterations read have landed
// (loads retire in order) and for its own LDS reads, and meets the barrier:
// one barrier per 16 MFMAs of a wave instead of per 8.  The schedule
// (k_conv3_sched.h) is replayed on the host by a test.
// Eight waves: four 32-row wave tiles x two k halves; the halves
// are summed through LDS and the shared vector epilogue of the GEMM kernel
// (bias, temb bias, residual, SiLU, GroupNorm statistics) writes the tile,
// whose rows are contiguous output pixels.  With split-K (small spatial
// sizes, few tiles) each split takes a range of channel chunks and the
// epilogue writes fp32 partials for the GEMM's split-K reducer.
#include <type_traits>

#include "di_gemv_dev.h"
#include "di_kernels.h"
#include "k_conv3_sched.h"
#include "k_gemm_kernel.h"

namespace di {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;

using namespace conv3;

// s_waitcnt with vmcnt = VM and lgkmcnt = LG (expcnt not waited on)
template <int VM, int LG>
__device__ __forceinline__ void cv_wait() {
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (LG << 8));
}

// f(integral_constant<int, I>) for I = B .. E-1: loop bodies whose wait
// counts and buffer indices must be compile-time constants
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int W>
__global__ __launch_bounds__(CV_NT) void k_conv3_halo(GemmArgs g) {
  using G = ConvGeo<W>;
  __shared__ __attribute__((aligned(1024))) char smem[G::SMEM];
  args_warm(g);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wq = wave & 3, kh = wave >> 2;  // 32-row wave tile, k half
  const int wm0 = wq * 32;

  const uint32_t n_tiles = g.N / CV_BN;
  uint32_t tile = blockIdx.x;
  {
    // deal contiguous runs of tiles to each XCD (its own L2): neighbours
    // share the patch (same pixels) or the weights
    const uint32_t n_wg = gridDim.x, per = n_wg / 8, rem = n_wg % 8, xcd = tile % 8,
                   slot = tile / 8;
    tile = xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
  }
  const uint32_t m0 = (tile / n_tiles) * CV_BM, n0 = (tile % n_tiles) * CV_BN;
  // output image Ho x Wo (the 2x nearest upsample of the H x W source when
  // g.up == 2); the tile is R rows x W pixels from (y0, x0), W = min(Wo, 128)
  const uint32_t HWo = g.Ho * g.Wo;
  const uint32_t img = m0 / HWo, y0 = (m0 % HWo) / g.Wo, x0 = (m0 % HWo) % g.Wo;
  const uint32_t ush = g.up == 2 ? 1u : 0u;
  // split-K over input-channel chunks: split blockIdx.y takes chunks
  // [cb0, cb0 + nch) (the host picks splits dividing Cin / 64)
  const uint32_t split = blockIdx.y;
  const int nch = (int)(g.Cin / 64 / g.splits);
  const int cb0 = (int)split * nch;
  const int n_stages = nch * 9;

  constexpr uint32_t kInv = 0x80000000u;
  const __amdgpu_buffer_rsrc_t rA = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(g.a), (short)0, (int)g.a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rA2 = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(g.a2), (short)0, (int)g.a2_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rB = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(g.b), (short)0, (int)g.b_bytes, 0x00020000);

  char* const patch = smem;                                 // [2][PROWS][128 B]
  char* const wbuf = smem + 2 * G::PROWS * CV_ROW;          // [G::NBB][64][128 B]

  // ---- this lane's DMA slots ----
  const int lrow = lane >> 3, lpos = lane & 7;
  // weights: row n0 + wave * 8 + lrow, logical chunk lpos ^ swizzle
  const int brow = wave * 8 + lrow;
  const uint32_t fb = (n0 + brow) * (uint32_t)g.ldb * 2u + (uint32_t)(lpos ^ (brow & 7)) * 16u;
  // patch pieces: patch row i * 64 + wave * 8 + lrow
  uint32_t ppix[G::NP], pchk[G::NP];
#pragma unroll
  for (int i = 0; i < G::NP; i++) {
    const int r = i * 64 + wave * 8 + lrow;
    const int iy = (int)y0 - 1 + r / G::PW, ix = (int)x0 - 1 + r % G::PW;
    const bool ok = r < G::PR && iy >= 0 && iy < (int)g.Ho && ix >= 0 && ix < (int)g.Wo;
    ppix[i] = ok ? (img * g.H + ((uint32_t)iy >> ush)) * g.W + ((uint32_t)ix >> ush) : kInv;
    pchk[i] = (uint32_t)(lpos ^ (r & 7)) * 16u;
  }
  // stage s = local chunk * 9 + tap; chunks below are global.  Stages past
  // the split (issued by the last iterations, never read) and the chunk
  // after its last get an out-of-range per-lane offset (kInv, checked
  // against the buffer's range; fb < 2 GiB): their DMAs write zeros without
  // touching memory and still count as loads for the waits
  auto dma_weights = [&](int stage, int buf) {
    const bool live = stage < n_stages;
    const uint32_t c = (uint32_t)(cb0 + stage / 9), t = (uint32_t)stage % 9u;
    const uint32_t koff = live ? (t * g.Cin + c * 64u) * 2u : 0u;  // uniform
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rB, (lds_ptr)(wbuf + buf * CV_BBUF + wave * 8 * CV_ROW),
                                             16, live ? fb : kInv, koff, 0, 0);
  };
  auto dma_patch = [&](int chunk, int piece) {
    const uint32_t cb = (uint32_t)chunk * 64u;
    const bool s2 = cb >= g.c1;
    const uint32_t ld2 = (uint32_t)(s2 ? g.lda2 : g.lda) * 2u;
    const uint32_t ch2 = (s2 ? cb - g.c1 : cb) * 2u;
    const uint32_t p = ppix[piece];
    const uint32_t off = p != kInv && chunk < cb0 + nch ? p * ld2 + ch2 + pchk[piece] : kInv;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        s2 ? rA2 : rA,
        (lds_ptr)(patch + (chunk & 1) * G::PROWS * CV_ROW + (piece * 64 + wave * 8) * CV_ROW), 16,
        off, 0, 0, 0);
  };

  // ---- MFMA fragments (16x16x32 f16: lane row lane % 16, k (lane / 16) * 8) ----
  const int fr = lane & 15;
  const int cidx = kh * 4 + (lane >> 4);  // logical 16-byte k chunk of this lane
  int pr0[2];
#pragma unroll
  for (int a = 0; a < 2; a++) {
    const int p = wm0 + a * 16 + fr;
    pr0[a] = (p / W) * G::PW + p % W;
  }
  struct Frags {
    f16x8 a[2];
    f16x8 b[4];
  };
  auto read_frags = [&](int chunk, int tap, int buf, Frags& f) {
    const f16* pa = (const f16*)(patch + (chunk & 1) * G::PROWS * CV_ROW);
    const int shift = (tap / 3) * G::PW + tap % 3;
#pragma unroll
    for (int a = 0; a < 2; a++) {
      const int pr = pr0[a] + shift;
      f.a[a] = *(const f16x8*)&pa[pr * 64 + ((cidx ^ (pr & 7)) * 8)];
    }
    const f16* pb = (const f16*)(wbuf + buf * CV_BBUF);
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int rr = b * 16 + fr;
      f.b[b] = *(const f16x8*)&pb[rr * 64 + ((cidx ^ (rr & 7)) * 8)];
    }
  };
  f32x4 acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int b = 0; b < 4; b++)
        acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.a[a], f.b[b], acc[a][b], 0, 0, 0);
  };

  // ---- prologue: patch of the first chunk, weights of stages 0..NBB-2 ----
  Frags F[2];
#pragma unroll
  for (int i = 0; i < G::NP; i++) dma_patch(cb0, i);
#pragma unroll
  for (int b = 0; b + 1 < G::NBB; b++) dma_weights(b, b);
  cv_wait<G::prologue_allow, 15>();
  __builtin_amdgcn_s_barrier();
  read_frags(cb0, 0, 0, F[0]);
  cv_wait<63, 0>();
  __builtin_amdgcn_s_barrier();

  // ---- steady state: two chunks (18 stages) per round, static tap,
  // weight-buffer and fragment-set indices.  Iteration s issues the weights
  // of stage s + NBB - 1 into the buffer stage s - 1 used.  A barrier follows
  // every BAR-th iteration.  At the barrier after iteration s, leaving the
  // last SLACK iterations' loads outstanding (loads retire in order)
  // completes everything issued up to s - SLACK: the weights of stages up to
  // s + BAR + 1, which the next BAR iterations read, and the patch pieces
  // of the next chunk (issued at its first five taps, read from its last
  // tap on).  A weight buffer is refilled two iterations after its
  // fragments were read, and one of those two iterations ends in a barrier
  // (BAR <= 2) that waits for the wave's LDS reads (lgkmcnt 0); a patch
  // buffer is refilled a whole chunk after.  So no DMA overwrites a buffer
  // with reads in flight.  Near the end of the split the weights of stages
  // past it are still issued (they read in-bounds weights or, past the
  // buffer's range, zeros) and land in buffers no stage reads ----

  int s0 = 0;
  for (; s0 + 18 <= n_stages; s0 += 18) {
    const int c0 = cb0 + s0 / 9;
    static_for<0, 18>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      constexpr int tap = j % 9;
      const int c = c0 + j / 9, cn = c0 + (j + 1) / 9;
      read_frags(cn, (j + 1) % 9, (j + 1) % G::NBB, F[(j + 1) & 1]);
      mma(F[j & 1]);
      dma_weights(s0 + j + G::NBB - 1, (j + G::NBB - 1) % G::NBB);
#pragma unroll
      for (int q = 0; q < G::pieces(tap); q++) dma_patch(c + 1, tap * G::PPT + q);
      if constexpr (j % G::BAR == G::BAR - 1) {
        cv_wait<G::allow(j), 0>();
        __builtin_amdgcn_s_barrier();
      }
    });
  }
  // ---- tail: an odd chunk count leaves the last chunk (9 stages), entered
  // right after a barrier; barriers after its odd iterations as above (the
  // drain below follows the last) ----
  if (s0 < n_stages) {
    const int c = cb0 + s0 / 9;
    static_for<0, 9>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      if constexpr (j + 1 < 9) read_frags(c, j + 1, (j + 1) % G::NBB, F[(j + 1) & 1]);
      mma(F[j & 1]);
      if constexpr (j + G::NBB - 1 < 9)
        dma_weights(s0 + j + G::NBB - 1, (j + G::NBB - 1) % G::NBB);
      if constexpr (j % G::BAR == G::BAR - 1) {
        cv_wait<G::tail_allow(j), 0>();
        __builtin_amdgcn_s_barrier();
      }
    });
  }
  // loads past the last stage may still be landing: drain before the C tile
  // reuses the pipeline's LDS
  cv_wait<0, 0>();
  __syncthreads();

  // ---- epilogue: the two k halves write their fp32 tiles side by side at
  // once; the shared vector epilogue adds them as it reads ----
  float* sC = reinterpret_cast<float*>(smem);
  float* const sCh = sC + kh * (CV_BM * CV_LDC);
  const int rq = (lane >> 4) * 4;
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) sCh[(wm0 + a * 16 + rq + i) * CV_LDC + b * 16 + fr] = acc[a][b][i];
  __syncthreads();
  gemm_epilogue_vec<CV_BM, CV_BN, CV_LDC, CV_NT, EX_NONE, 2>(g, sC, m0, n0, 0, split, nullptr,
                                                             CV_BM * CV_LDC);
  if (g.stats && g.splits == 1) {
    __syncthreads();
    gemm_tile_stats<CV_BM, CV_BN, CV_LDC, CV_NT>(g, sC, m0, n0);
  }
}

// The U-Net's conv_in: 3x3, stride 1, pad 1, from the NCHW fp32 latent
// (CIN channels, here 4) to NHWC fp16 with the bias added, and the
// GroupNorm statistics of the stored values per 64-pixel chunk and channel
// (the layout gemm_tile_stats writes: stats[(chunk * Cout + c) * 2 + {0, 1}]).
// The implicit GEMM took 10 us behind a separate NCHW -> NHWC pass and wrote
// no statistics, so both GroupNorms that read conv_in's output ran a
// statistics pass of their own.  Here the MFMA k index is (tap, channel)
// with the channels padded to 8 - exactly the OHWI weight layout - so a
// lane's B fragment is one 16-byte weight vector and its A fragment one
// tap of one pixel, read from the NCHW tensor (zero outside the image) and
// rounded to fp16 as the GEMM path's layout pass did; 3 k steps of 4 taps
// (the last holding tap 8 only).  Workgroup (64-pixel chunk, 32 channels):
// wave w takes pixels 16w .. 16w + 15, two 16-channel blocks.
constexpr int CI_CS = 32, CI_LDY = CI_CS + 8;

// With cn > 0 the grid has one more row of workgroups (blockIdx.y = Cout /
// CI_CS) that converts cn fp32 values cx -> fp16 cy (the U-Net's context;
// cn % 8 == 0, 16-byte aligned), and with gv.N > 0 rows from gv_row0 on run
// the timestep sinusoid's first GEMV gv (fp16 weights, B K <= kCiGemvX), so
// neither costs a launch of its own.
constexpr uint32_t kCiGemvX = 2560;
template <int CIN>
__global__ __launch_bounds__(256) void k_conv_in(const float* __restrict__ x,
                                                 const f16* __restrict__ w,
                                                 const float* __restrict__ bias,
                                                 f16* __restrict__ y, float* __restrict__ stats,
                                                 uint32_t Cout, uint32_t H, uint32_t W,
                                                 const float* __restrict__ cx,
                                                 f16* __restrict__ cy, uint32_t cn, GemvArgs gv,
                                                 uint32_t gv_row0) {
  static_assert(CIN <= 8, "weights padded to 8 channels per tap");
  if (gv.N && blockIdx.y >= gv_row0) {
    __shared__ float gxs[kCiGemvX];
    gemv_vec_block<f16, 3, 1, 8, true>(gv, gxs, (blockIdx.y - gv_row0) * gridDim.x + blockIdx.x);
    return;
  }
  if (cn && blockIdx.y == Cout / CI_CS) {
    for (uint32_t i = (blockIdx.x * 256 + threadIdx.x) * 8; i < cn; i += gridDim.x * 256 * 8) {
      const f32x4 a = *(const f32x4*)(cx + i), b = *(const f32x4*)(cx + i + 4);
      f16x8 o;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        o[j] = (f16)a[j];
        o[j + 4] = (f16)b[j];
      }
      *(f16x8*)(cy + i) = o;
    }
    return;
  }
  __shared__ __attribute__((aligned(16))) f16 sy[64 * CI_LDY];  // [pixel][co]
  __shared__ float sst[4][CI_CS][2];                             // per-wave channel sums
  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t chunk = blockIdx.x, c0 = blockIdx.y * CI_CS;
  const uint32_t HW = H * W;
  // a chunk lies in one image (HW % 64 == 0)
  const uint32_t img = __builtin_amdgcn_readfirstlane(chunk * 64 / HW);
  const uint32_t p0 = chunk * 64 - img * HW;
  const uint32_t r = lane & 15, g = lane >> 4;
  // A: pixel p0 + 16 wave + r, tap 4 ks + g
  const uint32_t p = p0 + wave * 16 + r;
  const int py = (int)(p / W), px = (int)(p % W);
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(x + (uint64_t)img * CIN * HW), (short)0, (int)(CIN * HW * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<f16*>(w), (short)0, (int)(Cout * 72 * 2), 0x00020000);
  float xa[3][CIN];
  f16x8 bf[3][2];
#pragma unroll
  for (int ks = 0; ks < 3; ks++) {
    const int tap = ks * 4 + (int)g;
    const int yy = py + tap / 3 - 1, xx = px + tap % 3 - 1;
    const bool ok = tap < 9 && yy >= 0 && yy < (int)H && xx >= 0 && xx < (int)W;
    const uint32_t off = ok ? (uint32_t)(yy * (int)W + xx) * 4u : 0x80000000u;
#pragma unroll
    for (int ci = 0; ci < CIN; ci++)
      xa[ks][ci] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rx, off, (int)(ci * HW * 4), 0));
#pragma unroll
    for (int nb = 0; nb < 2; nb++) {
      const uint32_t co = c0 + nb * 16 + r;
      const uint32_t woff = tap < 9 ? (co * 72 + (uint32_t)tap * 8) * 2 : 0x80000000u;
      bf[ks][nb] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(rw, woff, 0, 0));
    }
  }
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int ks = 0; ks < 3; ks++) {
    f16x8 af = {};
#pragma unroll
    for (int ci = 0; ci < CIN; ci++) af[ci] = (f16)xa[ks][ci];
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
      acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[ks][nb], acc[nb], 0, 0, 0);
  }
  // C: lane holds pixels 16 wave + 4 g + i, channel 16 nb + r
#pragma unroll
  for (int nb = 0; nb < 2; nb++) {
    const uint32_t cl = nb * 16 + r;
    const float b = bias[c0 + cl];
    float s = 0.0f, q = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const f16 h = (f16)(acc[nb][i] + b);
      sy[(wave * 16 + g * 4 + i) * CI_LDY + cl] = h;
      s += (float)h;
      q += (float)h * (float)h;
    }
    s += __shfl_xor(s, 16);
    q += __shfl_xor(q, 16);
    s += __shfl_xor(s, 32);
    q += __shfl_xor(q, 32);
    if (g == 0) {
      sst[wave][cl][0] = s;
      sst[wave][cl][1] = q;
    }
  }
  __syncthreads();
  {
    const uint32_t pix = tid >> 2, v = tid & 3;  // 64 pixels x 4 vectors of 8
    *(f16x8*)(y + ((uint64_t)chunk * 64 + pix) * Cout + c0 + v * 8) =
        *(const f16x8*)&sy[pix * CI_LDY + v * 8];
  }
  if (stats && tid < CI_CS) {
    const float s = (sst[0][tid][0] + sst[1][tid][0]) + (sst[2][tid][0] + sst[3][tid][0]);
    const float q = (sst[0][tid][1] + sst[1][tid][1]) + (sst[2][tid][1] + sst[3][tid][1]);
    *(float2*)(stats + ((uint64_t)chunk * Cout + c0 + tid) * 2) = float2{s, q};
  }
}

template <int W>
void launch_w(const GemmArgs& g, hipStream_t s) {
  const uint32_t tiles = (g.M / CV_BM) * (g.N / CV_BN);
  k_conv3_halo<W><<<dim3(tiles, g.splits), CV_NT, 0, s>>>(g);
}

}  // namespace

bool conv3_halo_ok(const GemmArgs& g) {
  const uint32_t Wo = g.Wo, TW = Wo < 128 ? Wo : 128;
  const bool single = g.a2 == nullptr || g.a2 == g.a || g.c1 == 0 || g.c1 == 0xffffffffu;
  return g.Cin > 0 && g.ks == 3 && g.stride == 1 && g.pad == 1 && (g.up == 1 || g.up == 2) &&
         g.Cin % 64 == 0 && (single || g.c1 % 64 == 0) && g.N % CV_BN == 0 &&
         g.Ho == g.H * g.up && Wo == g.W * g.up &&
         (TW == 16 || TW == 32 || TW == 64 || TW == 128) && Wo % TW == 0 &&
         g.Ho % (CV_BM / TW) == 0 && g.M % CV_BM == 0 && g.batch == 1 && g.b_vec_ok &&
         g.a_bytes > 0 && g.b_bytes > 0 && (single || g.a2_bytes > 0) && g.K == 9 * g.Cin;
}

bool conv_in_direct_ok(uint32_t Cin, uint32_t Cout, uint32_t H, uint32_t W) {
  return Cin == 4 && Cout % CI_CS == 0 && (H * W) % 64 == 0;
}

bool conv_in_convert_ok(const float* cx, const void* cy, uint64_t cn) {
  return cn > 0 && cn % 8 == 0 && cn < (1ull << 31) && ((uintptr_t)cx & 15) == 0 &&
         ((uintptr_t)cy & 15) == 0;
}

bool conv_in_gemv_ok(const GemvArgs& g) {
  return g.vec_ok && g.x_mode == GEMV_X_SINUSOID && g.N > 0 && g.K % 8 == 0 && g.K <= 64 * 8 * 3 &&
         g.B >= 1 && g.B <= 8 && (uint64_t)g.B * g.K <= kCiGemvX;
}

void launch_conv_in(hipStream_t s, const float* x, const f16* w, const float* bias, f16* y,
                    float* stats, uint32_t B, uint32_t Cout, uint32_t H, uint32_t W,
                    const float* cx, f16* cy, uint64_t cn, const GemvArgs* gv) {
  const bool conv = conv_in_convert_ok(cx, cy, cn);
  const uint32_t gx = B * H * W / 64, rows = Cout / CI_CS + (conv ? 1 : 0);
  GemvArgs none;
  none.N = 0;
  const bool side = gv && conv_in_gemv_ok(*gv);
  const uint32_t grows = side ? (gemv_side_blocks(gv->N, 1) + gx - 1) / gx : 0;
  k_conv_in<4><<<dim3(gx, rows + grows), 256, 0, s>>>(x, w, bias, y, stats, Cout, H, W, cx, cy,
                                                      conv ? (uint32_t)cn : 0u, side ? *gv : none,
                                                      rows);
}

void launch_conv3_halo(const GemmArgs& g, hipStream_t s) {
  switch (g.Wo < 128 ? g.Wo : 128) {
    case 16: launch_w<16>(g, s); break;
    case 32: launch_w<32>(g, s); break;
    case 64: launch_w<64>(g, s); break;
    default: launch_w<128>(g, s); break;
  }
}

}  // namespace di

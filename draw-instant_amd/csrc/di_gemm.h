// Argument block and launch API of the MFMA GEMM / implicit-GEMM conv kernel
// (k_gemm.hip).  Raw device pointers; callers validate shapes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "di_tembed.h"

namespace di {

enum AMode { A_DENSE = 0, A_CONV_NHWC = 1, A_CONV_NCHW = 2 };
enum BMode { B_NK = 0, B_KN = 1 };
enum Act { ACT_NONE = 0, ACT_GELU = 1, ACT_GEGLU = 2, ACT_SILU = 3, ACT_GELU_TANH = 4 };
enum TileCfg {
  TILE_64x64 = 0,
  TILE_128x64 = 1,
  TILE_64x128 = 2,
  TILE_128x128 = 3,
  TILE_128x160 = 4,
  TILE_64x160 = 5,
  // eight wavefronts: two per output wave tile, splitting each stage's k steps
  TILE_64x64_K2 = 6,
  TILE_128x64_K2 = 7,
  TILE_64x128_K2 = 8,
  // sixteen wavefronts: 2x4 (4x2) output wave tiles, two waves per tile
  TILE_64x128_W16 = 9,
  TILE_128x64_W16 = 10,
  TILE_128x128_W16 = 11,
  TILE_64x64_W16 = 12,
  // 3x3 stride-1 conv with the input halo staged per channel chunk
  // (k_conv3.hip): 128 output pixels (whole rows) x 64 channels
  TILE_CONV3_HALO = 13,
  // eight wavefronts, 2x2 wave tiles of 32 x 16 (two k halves): half the
  // B rows per workgroup of 64x64 K2, so a small-M GEMM spreads its loads
  // over twice the CUs
  TILE_64x32_K2 = 14,
  TILE_COUNT = 15
};

struct GemmPlan {
  int tile;
  uint32_t splits;
};

struct GemmArgs {
  // ---- A operand ----
  const void* a = nullptr;
  const void* a2 = nullptr;  // second source: k (dense) or channel (conv) >= c1
  uint64_t lda = 0, lda2 = 0;  // row / pixel stride in elements
  uint64_t sa = 0, sa2 = 0;    // batch stride in elements
  uint32_t c1 = 0;             // split point (0 with a2 == nullptr: single source)
  // conv geometry (A_CONV_*): source H x W, input upsampled by `up` (1 or 2)
  uint32_t Cin = 0, H = 0, W = 0, Ho = 0, Wo = 0, ks = 1, stride = 1, pad = 0, up = 1;
  // ---- B operand: B_NK = [N][K] (torch Linear / OHWI conv), B_KN = [K][N] ----
  const void* b = nullptr;
  uint64_t ldb = 0, sb = 0;
  // ---- problem ----
  uint32_t M = 0, N = 0, K = 0, batch = 1;
  uint32_t splits = 1, k_split = 0;
  uint32_t a_vec_ok = 1, b_vec_ok = 1;  // whole-vector (KV element) loads legal
  // fp32 problem (elem DI_F32) whose B is stored in fp16 and widened exactly
  // as it loads (fp16-resident weights); bounds-checked kernels only
  int b_f16 = 0;
  // Byte extents of A, A2 (per batch entry) and B for buffer-load range
  // checks; 0 = unknown (generic path).  Must stay below 2 GiB.
  uint32_t a_bytes = 0, a2_bytes = 0, b_bytes = 0;
  // ---- epilogue ----
  float alpha = 1.0f;
  const float* bias = nullptr;   // [N]
  const float* bias2 = nullptr;  // [(m / rows_b2)][ld_b2]
  uint32_t rows_b2 = 0, ld_b2 = 0;
  const void* res = nullptr;  // residual, same layout as C (NHWC rows)
  uint64_t ldr = 0, sr = 0;
  int res_f32 = 0;
  int act = ACT_NONE;
  void* c = nullptr;
  uint64_t ldc = 0, sc = 0;
  int c_f32 = 0;
  int c_nchw = 0;     // store C[(img*N + n)*c_hw + p] with m = img*c_hw + p
  uint32_t c_hw = 1;
  float* part = nullptr;  // split-K partials [splits][batch][M][N]
  // part_cpg > 0: partials in column groups of part_cpg (4 | part_cpg,
  // part_cpg | N), [splits][batch][N / part_cpg][M][part_cpg], so that one
  // group's values are contiguous (the GroupNorm-fused reducer's layout)
  uint32_t part_cpg = 0;
  // Partials shared with another launch (a ResNet's 1x1 shortcut and its
  // conv2): this launch writes slots part_slot0 + split of a buffer of
  // part_slots slots ([part_slots][batch][M][N]; 0: its own splits);
  // part_only = 1 launches no reducer (a later launch's reducer sums every
  // slot), else the reducer sums all part_slots slots.
  uint32_t part_slot0 = 0, part_slots = 0;
  int part_only = 0;
  // Optional GroupNorm statistics of the stored output (see gemm_stats_ok):
  // per 64-row chunk of the M rows and per column, (sum, sum of squares) at
  // stats[((bz * ceil(M/64) + m/64) * N + n) * 2].
  float* stats = nullptr;
  // Optional row statistics of the stored output (vector epilogue, no split):
  // per row m and column tile t = n0 / BN, (sum, sum of squares) at
  // rstats[(m * ceil(N / BN) + t) * 2].
  float* rstats = nullptr;
  // Optional LayerNorm of A folded into the epilogue (see gemm_lnfold_ok):
  // with B = W * gamma (per k), ln_s[n] = sum_k B[n][k] and the bias holding
  // sum_k beta[k] W[n][k] + bias[n], LayerNorm(A) W^T + bias equals
  // rstd[m] * (acc[m][n] - mean[m] * ln_s[n]) + bias[n].  mean / rstd of row
  // m come from ln_rows: ln_nt (sum, sum of squares) pairs per row over its K
  // values (the rstats layout), eps ln_eps.
  const float* ln_rows = nullptr;
  uint32_t ln_nt = 0;
  const float* ln_s = nullptr;
  float ln_eps = 0.0f;
  // Set by launch_gemm: fp16 NHWC output whose rows, bias, temb bias and
  // residual allow 16-byte vectors (the C tile is then staged through LDS
  // and written 8 columns per thread).
  int vec_epi = 0;
};

// Tile shape and split-K factor from a cost model (env DI_GEMM_TILE /
// DI_GEMM_SPLITS override, for tuning sweeps).
GemmPlan gemm_plan(const GemmArgs& g, int elem, int num_cus);
uint64_t gemm_ws_bytes(const GemmArgs& g);
// Whether the buffer-load (FAST) kernel variant applies.
bool gemm_fast_ok(const GemmArgs& g, int elem, int a_mode, int b_mode);
// Byte extent clamped to the buffer-load limit (0 = too large for it).
inline uint32_t gemm_extent(uint64_t bytes) { return bytes < 0x7fff0000ull ? (uint32_t)bytes : 0; }
// The halo conv kernel (TILE_CONV3_HALO, k_conv3.hip): whether it takes
// this NHWC fp16 conv (3x3, stride 1, pad 1, optional 2x nearest upsample,
// Cin % 64 == 0, Cout % 64 == 0, output width 16 / 32 / 64 or a multiple of
// 128, one GEMM batch), and its launch (vector epilogue; split-K over
// channel chunks writes partials for the split-K reducer).
bool conv3_halo_ok(const GemmArgs& g);
void launch_conv3_halo(const GemmArgs& g, hipStream_t s);
// The U-Net's conv_in as a direct kernel from the NCHW fp32 latent (4
// channels) to NHWC fp16 [B*H*W][Cout] (+bias), with GroupNorm statistics
// per 64-pixel chunk and channel into stats (may be null).  Weights OHWI
// fp16 with the input channels padded to 8 per tap.
bool conv_in_direct_ok(uint32_t Cin, uint32_t Cout, uint32_t H, uint32_t W);
// cx / cy / cn: optionally also convert cn fp32 values cx -> fp16 cy in the
// same launch (taken when conv_in_convert_ok; the caller converts otherwise).
// gv: optionally also run that GEMV (the timestep sinusoid's first linear,
// taken when conv_in_gemv_ok; blocks past conv_in's own rows compute it,
// and the caller launches it otherwise).
bool conv_in_convert_ok(const float* cx, const void* cy, uint64_t cn);
bool conv_in_gemv_ok(const GemvArgs& g);
void launch_conv_in(hipStream_t s, const float* x, const _Float16* w, const float* bias,
                    _Float16* y, float* stats, uint32_t B, uint32_t Cout, uint32_t H, uint32_t W,
                    const float* cx = nullptr, _Float16* cy = nullptr, uint64_t cn = 0,
                    const GemvArgs* gv = nullptr);
// GroupNorm (+SiLU) of a split-K conv's output applied by its reducer: the
// output rows are hw-pixel images of N channels in `groups` groups;
// y[rows][ldy] = GN(out) (+SiLU) in fp16, and the output itself only when
// raw is set (no statistics either way).  For a conv whose output feeds
// that GroupNorm (a ResNet's conv1: raw = 0) or that GroupNorm and
// consumers of the raw output that need no statistics (a ResNet's conv2
// whose output enters a transformer: raw = 1).
struct GnFuse {
  const float* gamma = nullptr;
  const float* beta = nullptr;
  void* y = nullptr;
  uint64_t ldy = 0;
  uint32_t groups = 0, hw = 0;
  float eps = 0.0f;
  int silu = 0;
  int raw = 0;
  // with raw: also the GroupNorm statistics of the stored output in the
  // GemmArgs::stats layout (per 64-row chunk and channel), for other
  // GroupNorms that read it; null: none
  float* stats = nullptr;
  // the reducer records of the context's statistics-exchange area
  // (di_device.h) and the poll limit: images of more than 256 rows are then
  // reduced by kXchgSlices workgroups per (group, image); null: one each
  uint64_t* xchg = nullptr;
  uint32_t spin = 0;
};
// Whether the fused reducer takes this call (g with its plan's splits):
// batch 1, split-K with a built (rows per thread, split count) pair, a
// bias, optionally a per-image temb bias and an fp16 residual, no
// activation, 4 | channels per group <= 40, hw a multiple of 64 (64 to 1024
// pixels; at most 256 with raw; statistics only with raw).
bool splitk_gn_ok(const GemmArgs& g, const GnFuse& f);
// elem: DI_F16 or DI_F32 operand element type.  gn: see GnFuse (only with
// g.splits > 1 and splitk_gn_ok).
void launch_gemm(GemmArgs g, int elem, int a_mode, int b_mode, int tile_cfg, hipStream_t s,
                 const GnFuse* gn = nullptr);
// Whether launch_gemm can produce g.stats for this call: buffer-load fp16
// path with the vector epilogue, no GEGLU, batch 1, and N % 32 == 0 when
// split-K is used.
bool gemm_stats_ok(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg);
// Whether launch_gemm can produce g.rstats (same path, no split-K); the
// column-tile count of the layout is then gemm_rstats_tiles(g, tile_cfg).
bool gemm_rstats_ok(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg);
uint32_t gemm_rstats_tiles(const GemmArgs& g, int tile_cfg);
// Whether launch_gemm applies the LayerNorm fold of g.ln_* (fp16 vector
// epilogue, batch 1, no GroupNorm statistics; split-K included).
bool gemm_lnfold_ok(const GemmArgs& g, int elem, int tile_cfg);
// OIHW (any dtype) -> OHWI fp16 with optional zero channel padding Cin -> Cin_pad.
void launch_repack_oihw_ohwi(hipStream_t s, const void* w, int wdt, void* out, uint32_t Cout,
                             uint32_t Cin, uint32_t ks, uint32_t Cin_pad);

}  // namespace di

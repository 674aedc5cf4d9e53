// Flash attention (head dim 64, fp16 in / fp32 accumulate) for gfx950, and
// the attention C ABI.
//
// Computes softmax(Q K^T * scale) V per (batch, head) - the maths of
// WGSL_FUSED_ATTN (fused-attn.js:199-307) and the cross-attention kernel
// WGSL_FUSED (fused-cross-attn.js:112-173) - without materialising scores:
// online softmax over 64-key tiles in the exp2 domain.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16), one wavefront = 16 queries:
//  * S^T = K Q'^T: A = K tile rows (keys) from LDS, B = Q'^T in registers,
//    where Q' = Q * scale * log2(e) (rounded to fp16 once), so scores come
//    out in log2 units.  The accumulator starts at -m (the running row max),
//    so the MFMA itself subtracts the max and p = exp2(S') is one
//    instruction per score.  The C layout leaves lane l with query l%16 and
//    keys 4g..4g+3 (g = l/16) of each 16-key tile;
//  * O^T += V^T P^T: those 8 probabilities of two adjacent key tiles are one
//    B fragment of P^T when the PV product's k index runs over keys in the
//    order {4g..4g+3, 16+4g..16+4g+3} per 32-key block.  V stays row-major in
//    LDS; ds_read_b64_tr_b16 gathers the V^T A fragment in that key order.
//
// VALU and MFMA work of one SIMD overlap only partly on gfx950 (measured), so
// the softmax is kept to the minimum per score: one exp2, one add, half a
// convert.  The running max is taken from the first key tile only.  Later
// tiles run against it unchanged while every probability stays <= 2^15
// (fp16-safe): each lane checks the sum of its 16 probabilities against
// kLaneSumMax, and only when some lane exceeds it (wave-uniform branch) is
// the max raised to the tile's and the tile's probabilities recomputed.  Row
// sums are reduced across the 4 lanes of a query once, at the end.
//
// Each workgroup (4 wavefronts = 64 queries) shares double-buffered K / V
// tiles in LDS (XOR-swizzled 16-byte chunks, conflict-free for the K
// fragment reads and the transposed V reads; 32 KiB per workgroup, four
// resident per CU).  The next tile goes straight from memory into LDS
// (buffer_load ... lds, one 1 KiB row group per instruction, the swizzle
// applied on the global side) during the MFMAs, by buffer loads whose
// descriptor ends at the head's last key: keys past Skv (cross-attention's
// 77) land as zeros and are masked to -inf.
//
// Key groups: where the grid is small (the 32x32 level's 160 workgroups) a
// workgroup runs two groups of four wavefronts on the same 64 queries, each
// group walking half of the key tiles with its own K / V buffers, and merges
// the two (max, row sum, output) triples through LDS at the end.
//
// KV split: a wave of 16 queries that walks all keys is the smallest unit of
// work, and 64x64-latent self-attention has 1280 of them for 1024 SIMDs, so
// some SIMDs would run two while most run one.  The keys are therefore split
// into `splits` ranges (attn_splits picks it so the whole grid is resident
// at once, four workgroups per CU); each workgroup writes its range's output normalised by
// its own row sum (fp16) plus that row sum and max, and k_attn_combine merges
// the ranges: O = sum_s l_s 2^(m_s - M) O_s / sum_s l_s 2^(m_s - M).  Workgroups are numbered so
// that each XCD (blocks are dealt round-robin over the 8 XCDs) gets a
// contiguous range of work, i.e. at most two heads' K / V in its L2.
#include "di_attn.h"
#include "di_device.h"
#include "di_kernels.h"

#include <cstdlib>
#include <type_traits>

namespace di {

namespace {

constexpr int D = 64;              // head dim
constexpr int BKV = 64;            // keys per tile
constexpr int K_BYTES = BKV * D * 2;      // 128-byte rows, XOR-swizzled 16-byte chunks
constexpr int BUF_BYTES = 2 * K_BYTES;    // K tile, then V tile
// a lane's 16 probabilities of one tile sum to at most this without a
// rescale, so none exceeds it either (fp16 max is 65504)
constexpr float kLaneSumMax = 32768.0f;
constexpr uint32_t kLaneSumMaxBits = 0x47000000u;  // bits of 32768.0f
static_assert(__builtin_bit_cast(uint32_t, kLaneSumMax) == kLaneSumMaxBits, "kLaneSumMaxBits");

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void* lds_ptr;

template <int N>
using Int = std::integral_constant<int, N>;

// byte offset of 16-byte chunk c of K row r: chunk index XOR (r/2)%8, so the
// 16 rows read by one 16-lane pass of a fragment load hit distinct banks
__device__ __forceinline__ uint32_t k_off(uint32_t r, uint32_t c) {
  return r * 128u + ((c ^ ((r >> 1) & 7u)) << 4);
}
// V rows: chunk index XOR r%8.  One 32-lane pass of a transposed read covers
// 8 consecutive rows x 2 adjacent chunks (2dt, 2dt+1); the XOR spreads those
// 16 chunk reads over all 64 banks.
__device__ __forceinline__ uint32_t v_off(uint32_t r, uint32_t c) {
  return r * 128u + ((c ^ (r & 7u)) << 4);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // raw buffer, stride 0; dword3 0x00020000 is the gfx9-family data format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ f16x8 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// s_waitcnt vmcnt(0) (expcnt and lgkmcnt at their maxima: not waited on)
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);

// lanes l, l^16, l^32, l^48 hold the same query
__device__ __forceinline__ float max_q4(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_q4(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// KS (1 or 2) key groups of four wavefronts each (KS * 256 threads): the workgroup's
// 64 queries are shared by every group, group kg walks its own contiguous
// run of the key tiles with its own pair of K / V buffers, and the groups'
// (max, row sum, output) are merged through LDS at the end.  KS = 1 is the
// single-group kernel (which may be split over workgroups and merged by
// k_attn_combine).
template <int KS>
__global__ __launch_bounds__(256 * KS, 4) void k_flash_attn(AttnArgs a, uint32_t nqb) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[KS * 2 * BUF_BYTES];  // [kg][buf][K | V]
  kernarg_warm(a);

  const uint32_t tid = threadIdx.x, lane = tid & 63;
  const uint32_t wave = KS == 1 ? tid >> 6 : __builtin_amdgcn_readfirstlane(tid >> 6) & 3u;
  const uint32_t kg = KS == 1 ? 0u : __builtin_amdgcn_readfirstlane(tid >> 8);
  const uint32_t r = lane & 15, g = lane >> 4;

  // XCD-aware numbering: block i runs on XCD i % 8; give XCD x the x-th
  // contiguous slice of the work list (slices differ by at most one block)
  const uint32_t T = gridDim.x, bid = blockIdx.x, xcd = bid & 7u, idx = bid >> 3;
  const uint32_t per = T >> 3, extra = T & 7u;
  const uint32_t w = xcd < extra ? xcd * (per + 1) + idx : extra * (per + 1) + (xcd - extra) * per + idx;
  const uint32_t qb = w % nqb, rest = w / nqb, split = rest % a.splits, hb = rest / a.splits;
  const uint32_t h = hb % a.H, b = hb / a.H;

  const f16* Q = a.q + b * a.bq + h * a.hq;
  const f16* K = a.k + b * a.bk + h * a.hk;
  const f16* V = a.v + b * a.bv + h * a.hv;
  f16* O = a.o + b * a.bo + h * a.ho;

  // Q'^T fragments for the two 32-wide d steps
  const uint32_t qrow = qb * 64 + wave * 16 + r;
  f16x8 qf[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    f16x8 t = {};
    if (qrow < a.Sq) t = *(const f16x8*)(Q + (uint64_t)qrow * a.ldq + ks * 32 + g * 8);
#pragma unroll
    for (int j = 0; j < 8; j++) qf[ks][j] = (f16)((float)t[j] * a.scale_log2);
  }

  // K / V tiles straight into LDS: wave w moves rows 16w .. 16w+15 of each,
  // 8 rows (1 KiB) per instruction; lane l lands at row + l/8, chunk slot l%8,
  // so it fetches the global chunk (l%8) XOR swizzle(row).  The buffer
  // descriptor of tile t starts at key 64t and ends after the head's last
  // key, so rows past Skv land as zeros.
  uint32_t dk[2], dv[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t row = wave * 16 + i * 8 + (lane >> 3), lc = lane & 7;
    dk[i] = row * (uint32_t)a.ldk * 2u + ((lc ^ ((row >> 1) & 7u)) << 4);
    dv[i] = row * (uint32_t)a.ldv * 2u + ((lc ^ (row & 7u)) << 4);
  }
  auto dma_kv = [&](int t, auto buf_c) {
    const uint32_t key0 = (uint32_t)t * BKV, left = a.Skv - key0;
    const __amdgpu_buffer_rsrc_t rK =
        make_rsrc(K + (uint64_t)key0 * a.ldk, (left - 1) * (uint32_t)a.ldk * 2u + D * 2);
    const __amdgpu_buffer_rsrc_t rV =
        make_rsrc(V + (uint64_t)key0 * a.ldv, (left - 1) * (uint32_t)a.ldv * 2u + D * 2);
    unsigned char* base = smem + (kg * 2 + decltype(buf_c)::value) * BUF_BYTES + wave * 16 * 128;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rK, (lds_ptr)(base + i * 8 * 128), 16, dk[i], 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rV, (lds_ptr)(base + K_BYTES + i * 8 * 128), 16,
                                               dv[i], 0, 0, 0);
    }
  };

  float m = 0.0f, l = 0.0f;  // running max (log2 units) and this lane's partial row sum
  f32x4 negm = {0.f, 0.f, 0.f, 0.f};  // -m: the score MFMAs' accumulator start
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K fragment (kt, ks): row kt*16 + r, chunk 4ks + g
  const uint32_t k_rd0 = k_off(r, g), k_rd1 = k_off(r, 4 + g);
  // V^T fragment (dt, ks) by transposed reads (see the header): lane r of
  // 16-lane group g reads 4 elements of key row 4g + r/4 (+16 for the second
  // half, +32 per k step: multiples of 8 rows, same XOR) at columns
  // 16dt + 4(r%4), i.e. chunk 2dt + (r%4)/2, bytes (r%2)*8 of it.
  uint32_t v_rd[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
    v_rd[dt] = K_BYTES + v_off(4 * g + (r >> 2), 2 * dt + ((r & 3) >> 1)) + (r & 1) * 8;

  // this workgroup's key tiles [w0, w1); key group kg takes [t0, t1), the
  // kg-th run of tpg tiles (the host picks KS so that no run is empty).  All
  // groups make tpg iterations, so every wave meets the same barriers
  const int n_tiles = (int)((a.Skv + BKV - 1) / BKV);
  const int tps = (n_tiles + (int)a.splits - 1) / (int)a.splits;
  const int w0 = (int)split * tps, w1 = min(w0 + tps, n_tiles);
  const int tpg = KS == 1 ? w1 - w0 : (w1 - w0 + KS - 1) / KS;
  const int t0 = w0 + (int)kg * tpg, t1 = KS == 1 ? w1 : min(t0 + tpg, w1);

  auto tile = [&](auto cur_c, int t) {
    constexpr int cur = decltype(cur_c)::value;
    const unsigned char* sb = smem + (kg * 2 + cur) * BUF_BYTES;
    if (KS > 1 && t >= t1) {  // this group's run is shorter: only the barrier
      __syncthreads();
      return;
    }
    if (t + 1 < t1) dma_kv(t + 1, Int<cur ^ 1>{});

    // S' = K Q'^T - m
    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      const f16x8 k0 = *(const f16x8*)(sb + k_rd0 + kt * 2048);
      const f16x8 k1 = *(const f16x8*)(sb + k_rd1 + kt * 2048);
      s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qf[0], negm, 0, 0, 0);
      s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qf[1], s[kt], 0, 0, 0);
    }
    if ((uint32_t)(t + 1) * BKV > a.Skv) {
#pragma unroll
      for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          if ((uint32_t)(t * BKV + kt * 16 + 4 * g + i) >= a.Skv) s[kt][i] = -INFINITY;
    }
    // raise the running max by this tile's excess over it (>= 0 after the
    // first tile; on the first, o and l are still zero)
    auto raise_max = [&](bool first) {
      float mx = fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3]));
#pragma unroll
      for (int kt = 1; kt < 4; kt++)
        mx = fmaxf(fmaxf(mx, fmaxf(s[kt][0], s[kt][1])), fmaxf(s[kt][2], s[kt][3]));
      mx = max_q4(mx);
      const float dl = first ? mx : fmaxf(mx, 0.0f);
      m += dl;
      negm -= dl;
#pragma unroll
      for (int kt = 0; kt < 4; kt++) s[kt] -= dl;
      const float alpha = first ? 0.0f : __builtin_amdgcn_exp2f(-dl);
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
    };
    if (t == t0) raise_max(true);
    f16x8 pf[2];
    float ts;
    auto probs = [&]() {
      ts = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float p = __builtin_amdgcn_exp2f(s[kt][i]);
          ts += p;
          pf[kt >> 1][(kt & 1) * 4 + i] = (f16)p;
        }
    };
    probs();
    // a probability above kLaneSumMax (or inf / NaN from an overflowing
    // score) shows in its lane's sum: rescale and redo the tile.  The test
    // compares the sum's bits as an integer (sign cleared), which orders
    // finite < inf < NaN and which -fno-honor-nans cannot fold away.
    if (__builtin_amdgcn_ballot_w64((__float_as_uint(ts) & 0x7fffffffu) > kLaneSumMaxBits) != 0) {
      raise_max(false);
      probs();
    }
    l += ts;
    // O^T += V^T P^T over two 32-key k steps
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
#pragma unroll
      for (int dt = 0; dt < 4; dt++) {
        const unsigned char* vp = sb + v_rd[dt] + ks * 32 * 128;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)vp);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vp + 16 * 128));
        const f16x8 vf = __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf[ks], o[dt], 0, 0, 0);
      }
    }
    // the next tile has landed in LDS (vmcnt 0), every wave is done with this one
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
  };

  if (KS == 1 || t0 < t1) dma_kv(t0, Int<0>{});
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();
  // two tiles per iteration so each LDS buffer has fixed offsets
  for (int i = 0; i < tpg; i += 2) {
    tile(Int<0>{}, t0 + i);
    if (i + 1 < tpg) tile(Int<1>{}, t0 + i + 1);
  }
  l = sum_q4(l);
  if constexpr (KS > 1) {
    // merge the key groups: groups 1..KS-1 leave (m, row sum, unnormalised
    // O) in LDS, lane by lane (float j of lane l at [slot][j][l]); group 0
    // rescales every part to the largest max and adds them.  The K / V
    // buffers are free: every group's last tile ended in a barrier after its
    // loads completed
    constexpr int NF = 18;  // o[4] (16 floats), m, l
    float* xs = reinterpret_cast<float*>(smem);
    if (kg > 0) {
      float* dst = xs + ((kg - 1) * 4 + wave) * NF * 64 + lane;
#pragma unroll
      for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) dst[(dt * 4 + i) * 64] = o[dt][i];
      dst[16 * 64] = m;
      dst[17 * 64] = l;
    }
    __syncthreads();
    if (kg > 0) return;
    float ms[KS], ls[KS];
    ms[0] = m;
    ls[0] = l;
    float mx = m;
#pragma unroll
    for (int k = 1; k < KS; k++) {
      const float* src = xs + ((k - 1) * 4 + wave) * NF * 64 + lane;
      ms[k] = src[16 * 64];
      ls[k] = src[17 * 64];
      mx = fmaxf(mx, ms[k]);
    }
    float wk = __builtin_amdgcn_exp2f(m - mx);
    l = ls[0] * wk;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] *= wk;
#pragma unroll
    for (int k = 1; k < KS; k++) {
      const float* src = xs + ((k - 1) * 4 + wave) * NF * 64 + lane;
      wk = __builtin_amdgcn_exp2f(ms[k] - mx);
      l += ls[k] * wk;
#pragma unroll
      for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[dt][i] += src[(dt * 4 + i) * 64] * wk;
    }
  }
  if (qrow < a.Sq) {
    const float inv = 1.0f / l;
    f16* dst = O + (uint64_t)qrow * a.ldo;
    if (a.splits > 1) {
      // this key range's normalised output and (max, row sum), per row
      // (b, h, q) of the [splits][B*H*Sq] workspace
      const uint64_t prow = ((uint64_t)split * a.rows + (uint64_t)hb * a.Sq + qrow);
      dst = a.part_o + prow * D;
      if (g == 0) *(float2*)(a.part_ml + prow * 2) = float2{m, l};
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
      f16x4 ov;
#pragma unroll
      for (int i = 0; i < 4; i++) ov[i] = (f16)(o[dt][i] * inv);
      *(f16x4*)(dst + dt * 16 + g * 4) = ov;
    }
  }
}

// Merge the key ranges of a split launch: one thread per 8 outputs (a
// 16-byte chunk) of a (b, h, q) row; all SP ranges are loaded up front.
template <int SP>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
  kernarg_warm(a);
  const uint32_t i = blockIdx.x * 256 + threadIdx.x, row = i >> 3, c = i & 7;
  if (row >= a.rows) return;
  float2 ml[SP];
  f16x8 v[SP];
#pragma unroll
  for (int sp = 0; sp < SP; sp++) {
    const uint64_t prow = (uint64_t)sp * a.rows + row;
    ml[sp] = *(const float2*)(a.part_ml + prow * 2);
    v[sp] = *(const f16x8*)(a.part_o + prow * D + c * 8);
  }
  float mx = ml[0].x;
#pragma unroll
  for (int sp = 1; sp < SP; sp++) mx = fmaxf(mx, ml[sp].x);
  float wsum = 0.0f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < SP; sp++) {
    const float w = ml[sp].y * __builtin_amdgcn_exp2f(ml[sp].x - mx);
    wsum += w;
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] += w * (float)v[sp][j];
  }
  const float inv = 1.0f / wsum;
  const uint32_t q = row % a.Sq, hb = row / a.Sq, h = hb % a.H, b = hb / a.H;
  f16x8 out;
#pragma unroll
  for (int j = 0; j < 8; j++) out[j] = (f16)(acc[j] * inv);
  *(f16x8*)(a.o + b * a.bo + h * a.ho + (uint64_t)q * a.ldo + c * 8) = out;
}

}  // namespace

constexpr uint32_t kMaxSplits = 8;

uint32_t attn_splits(const Ctx* c, uint32_t B, uint32_t H, uint32_t Sq, uint32_t Skv) {
  // Largest split that keeps the grid resident at once and every range >= 16
  // key tiles (shorter ranges lose more to the merge than they gain).  A CU's 160 KiB of LDS holds workgroups in two 80 KiB halves
  // (measured: 32 KiB workgroups reside 4 per CU, not 5), so the budget is
  // 4 workgroups per CU.
  const uint32_t blocks = ((Sq + 63) / 64) * H * B, cap = 4u * (uint32_t)c->num_cus;
  const uint32_t n_tiles = (Skv + BKV - 1) / BKV;
  uint32_t sp = blocks ? cap / blocks : 1;
  sp = sp < n_tiles / 16 ? sp : n_tiles / 16;
  sp = sp < kMaxSplits ? sp : kMaxSplits;
  if (sp < 2) return 1;
  // ranges of tps = ceil(n_tiles / sp) tiles: drop the ones that would be empty
  const uint32_t tps = (n_tiles + sp - 1) / sp;
  return (n_tiles + tps - 1) / tps;
}

uint32_t attn_key_groups(const Ctx* c, uint32_t B, uint32_t H, uint32_t Sq, uint32_t Skv,
                         uint32_t splits) {
  // Two key groups inside a workgroup (64 KiB of LDS: two workgroups per CU)
  // when the grid stays resident with them and each wave would otherwise
  // walk 8 or more key tiles: the serial chain halves without a merge
  // launch.  Measured per launch (one process, interleaved): 32x32-level
  // self-attention (10 heads, 16 tiles) 10.9 -> 9.1 us, 8 tiles 7.2 ->
  // 6.6 us; with 2 - 4 tiles (the cross-attentions, the 16x16 level) the
  // extra waves and the merge cost 0.2 - 0.7 us, and four groups were no
  // faster than two at 16 tiles and slower at 8.  Larger grids with more
  // tiles take the key-range split over workgroups instead (attn_splits).
  if (splits > 1) return 1;
  const uint32_t blocks = ((Sq + 63) / 64) * H * B, n = (Skv + BKV - 1) / BKV;
  uint32_t ks = n >= 8 && blocks <= 2u * (uint32_t)c->num_cus ? 2u : 1u;
  // tuning override: DI_ATTN_KGROUPS=1|2, read per call so that one process
  // can time both
  if (const char* env = getenv("DI_ATTN_KGROUPS")) {
    const uint32_t want = (uint32_t)atoi(env);
    if ((want == 1 || want == 2) && want <= n) ks = want;
  }
  return ks;
}

void launch_attention(const AttnArgs& a, uint32_t B, hipStream_t s) {
  const uint32_t nqb = (a.Sq + 63) / 64;
  const dim3 grid(nqb * a.H * B * a.splits);
  if (a.splits == 1 && a.key_groups == 2) k_flash_attn<2><<<grid, 512, 0, s>>>(a, nqb);
  else k_flash_attn<1><<<grid, 256, 0, s>>>(a, nqb);
  const dim3 cg((uint32_t)((a.rows * 8 + 255) / 256));
  switch (a.splits) {
    case 1: break;
    case 2: k_attn_combine<2><<<cg, 256, 0, s>>>(a); break;
    case 3: k_attn_combine<3><<<cg, 256, 0, s>>>(a); break;
    case 4: k_attn_combine<4><<<cg, 256, 0, s>>>(a); break;
    case 5: k_attn_combine<5><<<cg, 256, 0, s>>>(a); break;
    case 6: k_attn_combine<6><<<cg, 256, 0, s>>>(a); break;
    case 7: k_attn_combine<7><<<cg, 256, 0, s>>>(a); break;
    default: k_attn_combine<8><<<cg, 256, 0, s>>>(a); break;
  }
}

int run_attention(Ctx* c, AttnArgs a, uint32_t B) {
  // K / V rows of one head are addressed with 32-bit byte offsets
  const uint64_t ld = a.ldk > a.ldv ? a.ldk : a.ldv;
  if ((uint64_t)(a.Skv + BKV) * ld * 2 >= (1ull << 31)) {
    set_error("attention: Skv %u x row stride %llu too large", a.Skv, (unsigned long long)ld);
    return DI_EUNSUPPORTED;
  }
  a.splits = attn_splits(c, B, a.H, a.Sq, a.Skv);
  // tuning override: DI_ATTN_SPLITS=n (clamped so no key range is empty)
  static const char* env_splits = getenv("DI_ATTN_SPLITS");
  if (env_splits) {
    const uint32_t n_tiles = (a.Skv + BKV - 1) / BKV, want = (uint32_t)atoi(env_splits);
    uint32_t sp = want < 1 ? 1 : (want > n_tiles ? n_tiles : want);
    sp = sp < kMaxSplits ? sp : kMaxSplits;
    const uint32_t tps = (n_tiles + sp - 1) / sp;
    a.splits = (n_tiles + tps - 1) / tps;
  }
  a.key_groups = attn_key_groups(c, B, a.H, a.Sq, a.Skv, a.splits);
  a.rows = (uint64_t)B * a.H * a.Sq;
  void* ws = nullptr;
  uint64_t cap = 0;
  if (a.splits > 1) {
    const uint64_t ob = a.splits * a.rows * D * 2;
    const int rc = pool_alloc(c, ob + a.splits * a.rows * 8, &ws, &cap);
    if (rc) return rc;
    a.part_o = (f16*)ws;
    a.part_ml = (float*)((char*)ws + ob);
  }
  launch_attention(a, B, c->stream);
  if (ws) pool_release(c, ws, cap);
  return DI_OK;
}

}  // namespace di

using namespace di;

namespace {

// Strides for the two reference layouts.
void layout_strides(int layout, uint32_t H, uint32_t S, uint64_t* ld, uint64_t* hs, uint64_t* bs) {
  if (layout == DI_ATTN_BSHD) {  // fused-attn.js [B, S, H, d]
    *ld = (uint64_t)H * D;
    *hs = D;
    *bs = (uint64_t)S * H * D;
  } else {  // fused-cross-attn.js [B, H, S, d]
    *ld = D;
    *hs = (uint64_t)S * D;
    *bs = (uint64_t)H * S * D;
  }
}

int attention_entry(di_ctx* ctx, di_handle Q, di_handle K, di_handle V, di_handle Out, uint32_t B,
                    uint32_t H, uint32_t Sq, uint32_t Skv, uint32_t d, int32_t layout, float scale,
                    int32_t dt, const char* fn) {
  DI_CTX(ctx);
  DI_DTYPE(dt);
  DI_REQUIRE(d == 64, DI_EUNSUPPORTED, "%s: head dim %u (flash kernel is built for 64)", fn, d);
  DI_REQUIRE(B && H && Sq && Skv, DI_EINVAL, "%s: zero dimension", fn);
  DI_REQUIRE(layout == DI_ATTN_BSHD || layout == DI_ATTN_BHSD, DI_EINVAL, "%s: bad layout %d", fn,
             layout);
  // K / V rows of one head are addressed with 32-bit byte offsets
  DI_REQUIRE((uint64_t)(Skv + 64) * H * d * 2 < (1ull << 31), DI_EUNSUPPORTED,
             "%s: Skv*H = %llu too large", fn, (unsigned long long)Skv * H);
  const uint64_t nq = (uint64_t)B * H * Sq * d, nkv = (uint64_t)B * H * Skv * d;
  const size_t es = dtype_size(dt);
  DI_BUF(ctx, Q, q, nq * es);
  DI_BUF(ctx, K, k, nkv * es);
  DI_BUF(ctx, V, v, nkv * es);
  DI_BUF(ctx, Out, o, nq * es);
  AttnArgs a;
  a.H = H;
  a.Sq = Sq;
  a.Skv = Skv;
  a.scale_log2 = (scale > 0.0f ? scale : 1.0f / sqrtf((float)d)) * 1.4426950408889634f;
  layout_strides(layout, H, Sq, &a.ldq, &a.hq, &a.bq);
  layout_strides(layout, H, Skv, &a.ldk, &a.hk, &a.bk);
  a.ldv = a.ldk;
  a.hv = a.hk;
  a.bv = a.bk;
  a.ldo = a.ldq;
  a.ho = a.hq;
  a.bo = a.bq;
  if (dt == DI_F16) {
    a.q = (const f16*)q->ptr;
    a.k = (const f16*)k->ptr;
    a.v = (const f16*)v->ptr;
    a.o = (f16*)o->ptr;
    const int rc = run_attention(ctx, a, B);
    if (rc) return rc;
    DI_LAUNCH_CHECK();
    return DI_OK;
  }
  // fp32 tensors: stage through fp16 (MFMA operands), write fp32.
  void *tq = nullptr, *tk = nullptr, *tv = nullptr, *to = nullptr;
  uint64_t cq, ck, cv, co;
  int rc = pool_alloc(ctx, nq * 2, &tq, &cq);
  if (!rc) rc = pool_alloc(ctx, nkv * 2, &tk, &ck);
  if (!rc) rc = pool_alloc(ctx, nkv * 2, &tv, &cv);
  if (!rc) rc = pool_alloc(ctx, nq * 2, &to, &co);
  if (!rc) {
    launch_convert(ctx->stream, q->ptr, DI_F32, tq, DI_F16, nq);
    launch_convert(ctx->stream, k->ptr, DI_F32, tk, DI_F16, nkv);
    launch_convert(ctx->stream, v->ptr, DI_F32, tv, DI_F16, nkv);
    a.q = (const f16*)tq;
    a.k = (const f16*)tk;
    a.v = (const f16*)tv;
    a.o = (f16*)to;
    rc = run_attention(ctx, a, B);
    if (!rc) launch_convert(ctx->stream, to, DI_F16, o->ptr, DI_F32, nq);
  }
  if (tq) pool_release(ctx, tq, cq);
  if (tk) pool_release(ctx, tk, ck);
  if (tv) pool_release(ctx, tv, cv);
  if (to) pool_release(ctx, to, co);
  if (rc) return rc;
  DI_LAUNCH_CHECK();
  return DI_OK;
}

}  // namespace

extern "C" {

int32_t di_attn_self(di_ctx* ctx, di_handle Q, di_handle K, di_handle V, di_handle O, uint32_t B,
                     uint32_t H, uint32_t S, uint32_t d, int32_t layout, float scale, int32_t dt) {
  return attention_entry(ctx, Q, K, V, O, B, H, S, S, d, layout, scale, dt, "di_attn_self");
}

int32_t di_attn_cross(di_ctx* ctx, di_handle Q, di_handle K, di_handle V, di_handle O, uint32_t B,
                      uint32_t H, uint32_t Sq, uint32_t Skv, uint32_t d, int32_t layout,
                      float scale, int32_t dt) {
  return attention_entry(ctx, Q, K, V, O, B, H, Sq, Skv, d, layout, scale, dt, "di_attn_cross");
}

}  // extern "C"

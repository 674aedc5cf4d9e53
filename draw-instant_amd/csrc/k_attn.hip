// Flash attention (head dim 64, fp16 in / fp32 accumulate) for gfx950, and
// the attention C ABI.
//
// Computes softmax(Q K^T * scale) V per (batch, head) - the maths of
// WGSL_FUSED_ATTN (fused-attn.js:199-307) and the cross-attention kernel
// WGSL_FUSED (fused-cross-attn.js:112-173) - without materialising scores:
// online softmax over 64-key tiles (running max m, sum l, rescaled O), in
// the exp2 domain with scale*log2(e) folded into one multiply.
//
// MFMA mapping (v_mfma_f32_16x16x32_f16), one wavefront = 16 queries:
//  * S^T = K Q^T: A = K tile rows (keys) from LDS, B = Q^T kept in registers.
//    The C layout leaves lane l with query r = l%16 and keys 4g..4g+3
//    (g = l/16) of each 16-key tile;
//  * O^T += V^T P^T: those 8 probabilities of two adjacent key tiles are
//    exactly one B fragment of P^T if the k index of the PV product runs over
//    keys in the order {4g..4g+3, 16+4g..16+4g+3} per 32-key block.  V is
//    staged in LDS transposed ([d][slot]) in that same slot order, so the PV
//    product needs no shuffles of P and reads V^T as 16-byte fragments.
// Each workgroup (4 wavefronts = 64 queries) shares double-buffered K / V^T
// tiles in LDS, the next tile prefetched into registers during the MFMAs.
// Keys past Skv (cross-attention's 77) are masked to -inf.
#include "di_attn.h"
#include "di_device.h"
#include "di_kernels.h"

namespace di {

namespace {

constexpr int D = 64;       // head dim
constexpr int BKV = 64;     // keys per tile
constexpr int LDS_ROW = 72; // padded row (elements)

__device__ __forceinline__ uint32_t v_slot(uint32_t kk) {
  const uint32_t block = kk >> 5, w = kk & 31, t = w >> 4, rr = w & 15;
  return block * 32 + (rr >> 2) * 8 + (rr & 3) + 4 * t;
}

__global__ __launch_bounds__(256) void k_flash_attn(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) f16 sK[2][BKV * LDS_ROW];
  __shared__ __attribute__((aligned(16))) f16 sV[2][D * LDS_ROW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, g = lane >> 4;
  const uint32_t b = blockIdx.z, h = blockIdx.y;
  const uint32_t q0 = blockIdx.x * 64 + wave * 16;
  const f16* Q = a.q + b * a.bq + h * a.hq;
  const f16* K = a.k + b * a.bk + h * a.hk;
  const f16* V = a.v + b * a.bv + h * a.hv;
  f16* O = a.o + b * a.bo + h * a.ho;

  // Q^T fragments for the two 32-wide d steps
  f16x8 qf[2];
  const uint32_t qrow = q0 + r;
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    if (qrow < a.Sq) qf[ks] = *(const f16x8*)(Q + (uint64_t)qrow * a.ldq + ks * 32 + g * 8);
    else
#pragma unroll
      for (int j = 0; j < 8; j++) qf[ks][j] = (f16)0.0f;
  }

  f16x8 rk[2], rv[2];
  auto load_kv = [&](int t) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t vi = tid + i * 256, kk = vi >> 3, dc = vi & 7;
      const uint32_t key = t * BKV + kk;
      if (key < a.Skv) {
        rk[i] = *(const f16x8*)(K + (uint64_t)key * a.ldk + dc * 8);
        rv[i] = *(const f16x8*)(V + (uint64_t)key * a.ldv + dc * 8);
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) rk[i][j] = rv[i][j] = (f16)0.0f;
      }
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const uint32_t vi = tid + i * 256, kk = vi >> 3, dc = vi & 7;
      *(f16x8*)&sK[buf][kk * LDS_ROW + dc * 8] = rk[i];
      const uint32_t slot = v_slot(kk);
#pragma unroll
      for (int j = 0; j < 8; j++) sV[buf][(dc * 8 + j) * LDS_ROW + slot] = rv[i][j];
    }
  };

  float m = -INFINITY, l = 0.0f;
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n_tiles = (int)((a.Skv + BKV - 1) / BKV);
  load_kv(0);
  store_kv(0);
  __syncthreads();
  for (int t = 0; t < n_tiles; t++) {
    const int cur = t & 1;
    if (t + 1 < n_tiles) load_kv(t + 1);
    // scores S^T for 4 key tiles of 16
    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        f16x8 kf = *(const f16x8*)&sK[cur][(kt * 16 + r) * LDS_ROW + ks * 32 + g * 8];
        s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], s[kt], 0, 0, 0);
      }
    }
    // online softmax (exp2 domain); lanes r, r+16, r+32, r+48 share a query
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const uint32_t key = t * BKV + kt * 16 + g * 4 + i;
        float v = key < a.Skv ? s[kt][i] * a.scale_log2 : -INFINITY;
        s[kt][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    float rs = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float p = __builtin_amdgcn_exp2f(s[kt][i] - m_new);
        s[kt][i] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    l = l * alpha + rs;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
    // O^T += V^T P^T over two 32-key k steps
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      f16x8 pf;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        pf[j] = (f16)s[2 * ks][j];
        pf[j + 4] = (f16)s[2 * ks + 1][j];
      }
#pragma unroll
      for (int dt = 0; dt < 4; dt++) {
        f16x8 vf = *(const f16x8*)&sV[cur][(dt * 16 + r) * LDS_ROW + ks * 32 + g * 8];
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pf, o[dt], 0, 0, 0);
      }
    }
    if (t + 1 < n_tiles) store_kv(cur ^ 1);
    __syncthreads();
  }
  if (qrow < a.Sq) {
    const float inv = 1.0f / l;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
      f16x4 ov;
#pragma unroll
      for (int i = 0; i < 4; i++) ov[i] = (f16)(o[dt][i] * inv);
      *(f16x4*)(O + (uint64_t)qrow * a.ldo + dt * 16 + g * 4) = ov;
    }
  }
}

}  // namespace

void launch_attention(const AttnArgs& a, uint32_t B, hipStream_t s) {
  dim3 grid((a.Sq + 63) / 64, a.H, B);
  k_flash_attn<<<grid, 256, 0, s>>>(a);
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
    launch_attention(a, B, ctx->stream);
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
    launch_attention(a, B, ctx->stream);
    launch_convert(ctx->stream, to, DI_F16, o->ptr, DI_F32, nq);
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

// Flash-attention launch API (k_attn.hip).  Head dim 64, fp16 tensors addressed
// as q + b*bq + h*hq + s*ldq + d (same for k, v, o), which covers [B,S,H,d],
// [B,H,S,d] and strided token-major views such as a fused QKV buffer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "di_device.h"

namespace di {

struct AttnArgs {
  const f16* q = nullptr;
  const f16* k = nullptr;
  const f16* v = nullptr;
  f16* o = nullptr;
  uint64_t ldq = 0, ldk = 0, ldv = 0, ldo = 0;  // token row stride
  uint64_t hq = 0, hk = 0, hv = 0, ho = 0;      // head stride
  uint64_t bq = 0, bk = 0, bv = 0, bo = 0;      // batch stride
  uint32_t H = 1, Sq = 0, Skv = 0;
  float scale_log2 = 0.0f;  // softmax scale * log2(e)
  // key-range split (set by run_attention): workspace of `splits` x rows
  // normalised fp16 outputs [rows][64] and (max, row sum) float pairs, where
  // rows = B * H * Sq enumerates (b, h, q) with q fastest
  uint32_t splits = 1;
  // key groups inside a workgroup (1 or 2; set by run_attention, only
  // without a split): see k_flash_attn
  uint32_t key_groups = 1;
  uint64_t rows = 0;
  f16* part_o = nullptr;
  float* part_ml = nullptr;
};

struct Ctx;

// Picks the split, takes the workspace from the context's pool and enqueues
// the attention (and, when split, the merge) on the context's stream.
int run_attention(Ctx* c, AttnArgs a, uint32_t B);
uint32_t attn_splits(const Ctx* c, uint32_t B, uint32_t H, uint32_t Sq, uint32_t Skv);
uint32_t attn_key_groups(const Ctx* c, uint32_t B, uint32_t H, uint32_t Sq, uint32_t Skv,
                         uint32_t splits);
// Enqueue with a.splits / a.rows / workspace already set.
void launch_attention(const AttnArgs& a, uint32_t B, hipStream_t s);

}  // namespace di

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
};

void launch_attention(const AttnArgs& a, uint32_t B, hipStream_t s);

}  // namespace di

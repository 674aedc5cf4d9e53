// Instantiation families of the k_gemm template (k_gemm_kernel.h), each
// compiled in its own translation unit so the library builds in parallel.
#pragma once

#include <hip/hip_runtime.h>

#include "di_gemm.h"

namespace di {

// fp16 buffer-load path, dense A (k_gemm_dense.hip).
void gemm_fast_dense(const GemmArgs& g, int tile_cfg, hipStream_t s);
// The same path with an epilogue extra: the LayerNorm fold (g.ln_rows, no
// split) or the output row statistics (g.rstats) (k_gemm_dense_ex.hip).
void gemm_fast_dense_ex(const GemmArgs& g, int tile_cfg, hipStream_t s);
// fp16 buffer-load path, implicit-GEMM NHWC conv (k_gemm_conv.hip).
void gemm_fast_conv(const GemmArgs& g, int tile_cfg, hipStream_t s);
// Bounds-checked kernels: fp16 (dense / B_KN / NHWC conv), fp32 and fp32
// with fp16-resident B (dense / B_KN / NCHW conv) (k_gemm_slow.hip).
void gemm_slow(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg, hipStream_t s);

}  // namespace di

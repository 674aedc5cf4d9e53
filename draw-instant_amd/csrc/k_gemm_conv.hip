// k_gemm instantiations: fp16 buffer-load path, implicit-GEMM NHWC conv.
#include "k_gemm_families.h"
#include "k_gemm_kernel.h"

namespace di {

void gemm_fast_conv(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  launch_fast_d<A_CONV_NHWC, 2>(g, tile_cfg, s);
}

}  // namespace di

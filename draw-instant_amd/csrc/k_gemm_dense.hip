// k_gemm instantiations: fp16 buffer-load path, dense A, no epilogue extras.
#include "k_gemm_families.h"
#include "k_gemm_kernel.h"

namespace di {

void gemm_fast_dense(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  launch_fast_d<A_DENSE, 2>(g, tile_cfg, s);
}

}  // namespace di

// k_gemm instantiations: fp16 buffer-load path, dense A, with the LayerNorm
// fold or the output row statistics in the epilogue.
#include "k_gemm_families.h"
#include "k_gemm_kernel.h"

namespace di {

void gemm_fast_dense_ex(const GemmArgs& g, int tile_cfg, hipStream_t s) {
  if (g.ln_rows && g.splits <= 1) launch_fast_d<A_DENSE, 2, EX_LNFOLD>(g, tile_cfg, s);
  else launch_fast_d<A_DENSE, 2, EX_ROWSTATS>(g, tile_cfg, s);
}

}  // namespace di

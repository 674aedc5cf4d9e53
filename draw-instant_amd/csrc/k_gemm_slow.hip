// k_gemm instantiations: the bounds-checked kernels (fp16 operands the
// buffer-load path does not take, the reference's fp32 ops, fp32 with
// fp16-resident B).
#include "k_gemm_families.h"
#include "k_gemm_kernel.h"

namespace di {

void gemm_slow(const GemmArgs& g, int elem, int a_mode, int b_mode, int tile_cfg, hipStream_t s) {
  if (elem == DI_F16) {
    if (a_mode == A_DENSE && b_mode == B_NK) launch_slow<f16, A_DENSE, B_NK>(g, tile_cfg, s);
    else if (a_mode == A_DENSE && b_mode == B_KN) launch_slow<f16, A_DENSE, B_KN>(g, tile_cfg, s);
    else if (a_mode == A_CONV_NHWC && b_mode == B_NK)
      launch_slow<f16, A_CONV_NHWC, B_NK>(g, tile_cfg, s);
  } else if (g.b_f16) {
    if (a_mode == A_DENSE && b_mode == B_NK) launch_slow<float, A_DENSE, B_NK, f16>(g, tile_cfg, s);
    else if (a_mode == A_DENSE && b_mode == B_KN)
      launch_slow<float, A_DENSE, B_KN, f16>(g, tile_cfg, s);
    else if (a_mode == A_CONV_NCHW && b_mode == B_NK)
      launch_slow<float, A_CONV_NCHW, B_NK, f16>(g, tile_cfg, s);
  } else {
    if (a_mode == A_DENSE && b_mode == B_NK) launch_slow<float, A_DENSE, B_NK>(g, tile_cfg, s);
    else if (a_mode == A_DENSE && b_mode == B_KN) launch_slow<float, A_DENSE, B_KN>(g, tile_cfg, s);
    else if (a_mode == A_CONV_NCHW && b_mode == B_NK)
      launch_slow<float, A_CONV_NCHW, B_NK>(g, tile_cfg, s);
  }
}

}  // namespace di

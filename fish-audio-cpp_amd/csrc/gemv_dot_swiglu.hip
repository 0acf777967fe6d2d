// gemv_dot_swiglu.hip -- instantiates the N == 1 GEMV with the SwiGLU pair
// epilogue (two rows per wave: an interleaved w1 / w3 row pair), with plain
// (pro 0) or residual + RMSNorm (pro 2) in-kernel quantization.
#include "gemv_kernels.h"

namespace fa {
namespace gv {

DotFn dot_swiglu(int pro, int K, int kd, int lgl, bool sep) {
    if (sep)   // separate w1 / w3, each with its own quantization companions
        return pro == 2 ? dot_for_xv<2, true, kDotWavesQx, 2, 2>(K, kd, lgl)
                        : dot_for_xv<2, true, kDotWavesQx, 0, 2>(K, kd, lgl);
    return pro == 2 ? dot_for_xv<2, true, kDotWavesQx, 2, 1>(K, kd, lgl)
                    : dot_for_xv<2, true, kDotWavesQx, 0, 1>(K, kd, lgl);
}

}  // namespace gv
}  // namespace fa

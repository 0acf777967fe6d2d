// gemv_dot_pro.hip -- instantiates the N == 1 GEMV with a fused prologue in
// front of its quantizer: SiLU * mul (pro 1) or residual + RMSNorm (pro 2).
#include "gemv_kernels.h"

namespace fa {
namespace gv {

DotFn dot_pro(int R, int pro, int K, int kd, int lgl) {
    if (R == 1)
        return pro == 1 ? dot_for_xv<1, true, kDotWavesQx, 1, 0>(K, kd, lgl)
                        : dot_for_xv<1, true, kDotWavesQx, 2, 0>(K, kd, lgl);
    return pro == 1 ? dot_for_xv<2, true, kDotWavesQx, 1, 0>(K, kd, lgl)
                    : dot_for_xv<2, true, kDotWavesQx, 2, 0>(K, kd, lgl);
}

}  // namespace gv
}  // namespace fa

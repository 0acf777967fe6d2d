// gemv_dot.hip -- instantiates the N == 1 GEMV on staged int8 activations
// and with plain in-kernel quantization (kernels in gemv_kernels.h).
#include "gemv_kernels.h"

namespace fa {
namespace gv {

DotFn dot_plain(int R, bool qx, int K, int kd, int lgl) {
    if (R == 1)
        return qx ? dot_for_xv<1, true, kDotWavesQx, 0, 0>(K, kd, lgl)
                  : dot_for_xv<1, false, kDotWaves, 0, 0>(K, kd, lgl);
    return qx ? dot_for_xv<2, true, kDotWavesQx, 0, 0>(K, kd, lgl)
              : dot_for_xv<2, false, kDotWaves, 0, 0>(K, kd, lgl);
}

}  // namespace gv
}  // namespace fa

// gemv_mfma_fused.hip -- instantiations of the 2 <= N <= 16 MFMA kernel with
// in-kernel quantization of the fp16 tokens and / or the SwiGLU pair
// epilogue (the kernel is in gemv_kernels.h).
#include "gemv_kernels.h"

namespace fa {
namespace gv {
namespace {

template <int SPG, int MAXG, bool LC, int QX, int EPI>
MfmaFn<false> inst() {
    constexpr int lim = QX == 2 ? kMfmaQxStepsSmooth : kMfmaQxSteps;
    if constexpr (QX != 0 && SPG * MAXG > lim) return nullptr;
    else return gemv_mfma_kernel<SPG, MAXG, LC, false, 12, QX, EPI>;
}

template <int SPG, bool LC, int QX, int EPI>
MfmaFn<false> for_maxg(int maxg) {
    switch (maxg) {
        case 1: return inst<SPG, 1, LC, QX, EPI>();
        case 2: return inst<SPG, 2, LC, QX, EPI>();
        case 3: return inst<SPG, 3, LC, QX, EPI>();
        case 4: return inst<SPG, 4, LC, QX, EPI>();
        case 6: return inst<SPG, 6, LC, QX, EPI>();
        case 8: return inst<SPG, 8, LC, QX, EPI>();
        case 12: return inst<SPG, 12, LC, QX, EPI>();
        case 16: return inst<SPG, 16, LC, QX, EPI>();
        case 20: return inst<SPG, 20, LC, QX, EPI>();
        default: return nullptr;
    }
}

template <bool LC, int QX, int EPI>
MfmaFn<false> for_spg(int spg, int maxg) {
    switch (spg) {
        case 1: return for_maxg<1, LC, QX, EPI>(maxg);
        case 2: return for_maxg<2, LC, QX, EPI>(maxg);
        case 4: return for_maxg<4, LC, QX, EPI>(maxg);
        case 8: return for_maxg<8, LC, QX, EPI>(maxg);
        default: return nullptr;
    }
}

template <int QX, int EPI>
MfmaFn<false> for_lc(bool lc, int spg, int maxg) {
    return lc ? for_spg<true, QX, EPI>(spg, maxg) : for_spg<false, QX, EPI>(spg, maxg);
}

}  // namespace

MfmaFn<false> mfma_fused(int qx, int epi, bool lc, int spg, int maxg) {
    if (epi == 0) {
        if (qx == 1) return for_lc<1, 0>(lc, spg, maxg);
        if (qx == 2) return for_lc<2, 0>(lc, spg, maxg);
    } else if (epi == 1) {
        if (qx == 0) return for_lc<0, 1>(lc, spg, maxg);
        if (qx == 1) return for_lc<1, 1>(lc, spg, maxg);
        if (qx == 2) return for_lc<2, 1>(lc, spg, maxg);
    }
    return nullptr;
}

}  // namespace gv
}  // namespace fa

// gemv.hip -- decode-shaped W8A8 linear (N <= 16 tokens): plan, launch and
// the instantiations of the small-batch MFMA kernel.  The kernels and the
// design notes are in gemv_kernels.h; the N == 1 kernel families are
// instantiated in gemv_dot*.hip.
#include "gemv_kernels.h"

#include <atomic>

namespace fa {
using namespace gv;
namespace {

template <int SPG, bool LC, bool D>
MfmaFn<D> mfma_for_maxg(int maxg) {
    switch (maxg) {
        case 1: return gemv_mfma_kernel<SPG, 1, LC, D>;
        case 2: return gemv_mfma_kernel<SPG, 2, LC, D>;
        case 3: return gemv_mfma_kernel<SPG, 3, LC, D>;
        case 4: return gemv_mfma_kernel<SPG, 4, LC, D>;
        case 6: return gemv_mfma_kernel<SPG, 6, LC, D>;
        case 8: return gemv_mfma_kernel<SPG, 8, LC, D>;
        case 12: return gemv_mfma_kernel<SPG, 12, LC, D>;
        case 16: return gemv_mfma_kernel<SPG, 16, LC, D>;
        default: return gemv_mfma_kernel<SPG, 20, LC, D>;
    }
}

template <bool LC, bool D>
MfmaFn<D> mfma_for_spg(int spg, int maxg) {
    switch (spg) {
        case 1: return mfma_for_maxg<1, LC, D>(maxg);
        case 2: return mfma_for_maxg<2, LC, D>(maxg);
        case 4: return mfma_for_maxg<4, LC, D>(maxg);
        default: return mfma_for_maxg<8, LC, D>(maxg);
    }
}

template <bool D>
MfmaFn<D> mfma_for(bool lc, int spg, int maxg) {
    return lc ? mfma_for_spg<true, D>(spg, maxg) : mfma_for_spg<false, D>(spg, maxg);
}

int round_maxg(int m) {
    static const int opts[] = {1, 2, 3, 4, 6, 8, 12, 16, 20};
    for (int o : opts)
        if (m <= o) return o;
    return 20;
}

}  // namespace

int device_cus() {
    static std::atomic<int> cached[64];   // zero-initialised (static storage)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return 0;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

namespace {
std::atomic<int> g_plan_rejects{0};
}

GemvPlan plan_gemv(int M, int N, int K, int g, int G, bool qx, int pro, int epi, bool smooth) {
    // A plan outside the kernels' assumptions is a planning bug: it is
    // counted and dropped (kind 0), so the caller takes its other path
    // (separate quantizer, the prefill kernels) instead of failing.
    GemvPlan p = plan_gemv_raw(M, N, K, g, G, qx, pro, epi, smooth);
    if (p.kind != 0 && !gemv_plan_valid(p, M, N, K, g, G)) {
        g_plan_rejects.fetch_add(1, std::memory_order_relaxed);
        return GemvPlan{};
    }
    return p;
}

int gemv_plan_rejects() { return g_plan_rejects.load(std::memory_order_relaxed); }

GemvPlan plan_gemv_raw(int M, int N, int K, int g, int G, bool qx, int pro, int epi, bool smooth) {
    GemvPlan p{};
    if (pro != 0 && (!qx || N != 1 || K > 3 * 8 * 64 * kDotWavesQx || K % 8 != 0)) return p;
    if (epi != 0 && (M & 1)) return p;
    if (epi != 0 && N == 1 && (!qx || pro == 1)) return p;
    if (epi == 2 && N != 1) return p;
    if (N == 1 && (g == 64 || g == 128 || g == 256 || g == 512) && K % 16 == 0 && K <= 32768) {
        const int lgroups = g / 16;
        // rows per wave (measured on MI355X over the layer shapes at g256):
        // one row streams best on staged int8 codes; with in-kernel
        // quantization (8-wave workgroups, each quantizing the token) two
        // rows halve the workgroups and win on the large shapes; the SwiGLU
        // pair needs two
        const bool two = epi || (qx && (M >= 8192 || K >= 8192));
        p.kind = (two && lgroups <= 32) ? 2 : 1;
        if (epi && p.kind != 2) return GemvPlan{};
        p.epi = epi;
        const int R = p.kind;
        if (lgroups > 64 / R) return GemvPlan{};
        const int PB = (64 / R) * 16;
        const int passes = (K + PB - 1) / PB;
        // ring depth: all passes of a row when they are few, else 5 (deeper
        // rings cost more occupancy than they gain, measured on MI355X)
        p.kd = passes <= 3 ? 3 : passes <= 4 ? 4 : 5;
        const int nwv = qx ? kDotWavesQx : kDotWaves;
        p.grid = ceil_div(M, nwv * R);   // row blocks
        p.block = nwv * 64;
        const int Kp = (K + 15) & ~15;
        p.lds = (size_t)Kp + (size_t)((G + 3) & ~3) * sizeof(float);   // xs padded for float4 reads
        if (pro == 2) p.lds += (size_t)Kp * 2 + 33 * sizeof(float);      // fp16 row, warp sums
        if (epi == 2)   // the fp16 row area, then the up weight's codes and scales
            p.lds = (((size_t)Kp + (size_t)((G + 3) & ~3) * 4 + (size_t)Kp * 2 + 33 * 4 + 15) &
                     ~(size_t)15) + (size_t)Kp + (size_t)((G + 3) & ~3) * 4;
        p.pro = pro;
        if (g < 16) return GemvPlan{};
        if (p.lds > 64 * 1024) return GemvPlan{};
        int lg = 0;
        while ((1 << lg) < g) ++lg;
        p.lg = lg;            // log2(g)
        p.passes = passes;
        return p;
    }
    if (N >= 1 && N <= 16 && (g == 64 || g == 128 || g == 256 || g == 512) && K % 64 == 0) {
        const int tiles = ceil_div(M, kTile);
        // Waves per 16-row tile (measured on MI355X): with many tiles two
        // waves split the groups; with few tiles (o and down projections) up
        // to eight, and the terms go through LDS to one chain lane per output.
        // A wave holds at most 20 groups.
        int nw = tiles >= 384 ? 2 : (G >= 64 ? 8 : 2);
        if (nw < ceil_div(G, 20)) nw = ceil_div(G, 20);
        if (nw > G) nw = G;
        if (nw > 8) nw = 8;
        const int qx_lim = smooth ? kMfmaQxStepsSmooth : kMfmaQxSteps;
        if (qx) {
            // in-kernel quantization holds the wave's fp16 values (8 VGPRs a
            // step, 16 with smooth_inv) until they become codes: more waves
            // per tile when the range is too long
            while (nw < 8 && nw < G && (g / 64) * round_maxg(ceil_div(G, nw)) > qx_lim) ++nw;
            if ((g / 64) * round_maxg(ceil_div(G, nw)) > qx_lim) return GemvPlan{};
        }
        if (ceil_div(G, nw) > 20) return GemvPlan{};
        p.kind = 3;
        p.spg = g / 64;
        p.maxg = round_maxg(ceil_div(G, nw));
        p.grid = tiles;
        p.block = nw * 64;
        const int ns = N <= 8 ? 8 : 16;
        const size_t lds_lc = (size_t)(2 * kTile * G + G * ns * kTile) * sizeof(float);
        p.lc = tiles < 384 && lds_lc <= 64 * 1024;
        p.lds = p.lc ? lds_lc : (size_t)(2 * kTile * G + kTile * kTile) * sizeof(float);
        if (p.lds > 64 * 1024) return GemvPlan{};
        p.epi = epi;
        if (qx) p.qx = smooth ? 2 : 1;
        return p;
    }
    return GemvPlan{};
}

bool gemv_plan_valid(const GemvPlan& p, int M, int N, int K, int g, int G) {
    // What the kernels take for granted about their grid and shapes; a plan
    // outside it is a planning bug and is refused before any launch.
    if (M <= 0 || N <= 0 || K <= 0 || g <= 0 || G != ceil_div(K, g)) return false;
    if (p.block <= 0 || p.block % 64 != 0 || p.grid <= 0) return false;
    if (p.kind == 1 || p.kind == 2) {
        const int R = p.kind;
        const int nwv = p.block / 64;
        if (N != 1 || (nwv != kDotWaves && nwv != kDotWavesQx)) return false;
        if (g != 64 && g != 128 && g != 256 && g != 512) return false;
        if ((1 << p.lg) != g || g / 16 > 64 / R) return false;      // a group fits a row's lanes
        if (K % 16 != 0 || K > 32768) return false;
        if (p.passes != ceil_div(K, (64 / R) * 16)) return false;
        if (p.kd < 3 || p.kd > 5) return false;
        if ((long long)p.grid * nwv * R < M) return false;         // every row has a wave
        if (p.pro != 0 && K > 3 * 8 * 64 * kDotWavesQx) return false;
        if (p.epi != 0 && (R != 2 || (M & 1))) return false;
        return p.lds <= 64 * 1024;
    }
    if (p.kind == 3) {
        const int nw = p.block / 64;
        if (N > 16 || nw > 8 || K % 64 != 0 || p.spg * 64 != g) return false;
        if (p.spg != 1 && p.spg != 2 && p.spg != 4 && p.spg != 8) return false;
        if (p.grid != ceil_div(M, kTile)) return false;
        if (ceil_div(G, nw) > p.maxg || p.maxg > 20 || nw > G) return false;  // each wave's groups
        if (kTile * G > 5 * p.block) return false;                // scale staging: 5 per thread
        if (p.qx && p.spg * p.maxg > (p.qx == 2 ? kMfmaQxStepsSmooth : kMfmaQxSteps)) return false;
        if (p.epi != 0 && (p.epi != 1 || (M & 1))) return false;
        const int ns = N <= 8 ? 8 : 16;
        const size_t lds = p.lc ? (size_t)(2 * kTile * G + G * ns * kTile) * sizeof(float)
                                : (size_t)(2 * kTile * G + kTile * kTile) * sizeof(float);
        return p.lds == lds && p.lds <= 64 * 1024;
    }
    return false;
}

hipError_t launch_gemv(const GemvPlan& p, const int8_t* W, const uint16_t* w_scale,
                       const int8_t* x_q, const float* x_scale, const uint16_t* X,
                       const uint16_t* act_scale, const uint16_t* smooth_inv, uint16_t* Y,
                       int32_t* dbg_partials, int dbg_row0, int dbg_rows, int dbg_tok0,
                       int dbg_toks, int M, int N, int K, int g, int G, hipStream_t stream,
                       const uint16_t* x2, const uint16_t* gamma, float eps, uint16_t* h_out,
                       const int8_t* w3, const uint16_t* w3_scale, const uint16_t* act_scale3,
                       const uint16_t* smooth_inv3) {
    DbgWindow dbg{dbg_partials, dbg_row0, dbg_rows, dbg_tok0, dbg_toks};
    const ProArgs pro{x2, gamma, h_out, eps, w3, w3_scale, act_scale3, smooth_inv3};
    if (!gemv_plan_valid(p, M, N, K, g, G)) return hipErrorInvalidValue;
    if (p.kind == 1 || p.kind == 2) {
        const bool qx = X != nullptr;
        const int lgl = p.lg - 4;   // log2(lanes per group)
        if (qx != (p.block == kDotWavesQx * 64)) return hipErrorInvalidValue;   // planned for the other input
        if (p.pro == 2 && !gamma) return hipErrorInvalidValue;
        if (p.epi && (p.kind != 2 || !qx || (M & 1))) return hipErrorInvalidValue;
        if (p.epi == 2 && (!w3 || !w3_scale)) return hipErrorInvalidValue;
        DotFn fn = p.epi ? dot_swiglu(p.pro, K, p.kd, lgl, p.epi == 2)
                 : p.pro ? dot_pro(p.kind, p.pro, K, p.kd, lgl)
                         : dot_plain(p.kind, qx, K, p.kd, lgl);
        // One workgroup per row block on staged codes.  With in-kernel
        // quantization at most two workgroups per CU, each walking several
        // row blocks, so each quantizes the token once for several blocks
        // (measured on MI355X: qkv 6.25 -> 5.84 us, gate_up 11.4 -> 10.7 us,
        // the 36-layer stack 1.42 -> 1.30 ms).
        const int cap = qx ? 2 * device_cus() : 0;
        const int grid = cap > 0 && p.grid > cap ? cap : p.grid;
        hipLaunchKernelGGL(fn, dim3(grid), dim3(p.block), p.lds, stream, W, w_scale, x_q, x_scale,
                           X, act_scale, smooth_inv, Y, dbg, M, K, p.lg, G, p.passes, p.grid, pro);
    } else if (p.kind == 3) {
        if (p.pro || (p.qx != 0) != (X != nullptr)) return hipErrorInvalidValue;
        if ((p.qx == 2) != (smooth_inv != nullptr)) return hipErrorInvalidValue;
        if (p.epi && (M & 1)) return hipErrorInvalidValue;
        const bool d = dbg_partials != nullptr;
        if (d && (p.qx || p.epi)) return hipErrorInvalidValue;   // debug window: staged codes
        if (d) {
            hipLaunchKernelGGL(mfma_for<true>(p.lc, p.spg, p.maxg), dim3(p.grid), dim3(p.block), p.lds,
                               stream, W, w_scale, x_q, x_scale, X, act_scale, smooth_inv, Y, dbg,
                               M, N, K, G);
        } else {
            MfmaFn<false> fn = (p.qx || p.epi) ? mfma_fused(p.qx, p.epi, p.lc, p.spg, p.maxg)
                                               : mfma_for<false>(p.lc, p.spg, p.maxg);
            if (!fn) return hipErrorInvalidValue;
            hipLaunchKernelGGL(fn, dim3(p.grid), dim3(p.block), p.lds, stream, W, w_scale, x_q,
                               x_scale, X, act_scale, smooth_inv, Y, dbg, M, N, K, G);
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fa

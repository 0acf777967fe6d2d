// gemv.hip -- decode-shaped W8A8 linear (N <= 16 tokens) on CDNA4 int8 MFMA.
//
// Replaces the reference's int8_matvec_dequant_kernel / int8_smallbatch
// kernel and, for 5 <= N <= 16, its per-group cuBLAS loop
// (src/kernels/int8_gemm.cu:245-380, 439-498).
//
// Shape of the work: one wave owns a tile of 16 weight rows and a contiguous
// range of K-groups (a "split").  Each lane streams 16 bytes of one weight row
// per 64-wide K step (lane -> row lane&15, byte offset 16*(lane>>4)), so a
// wave reads 16 rows x 64 B per step with 128-bit loads.  The activations of
// up to 16 tokens ride in the MFMA's second operand with the same byte
// mapping, so v_mfma_i32_16x16x64_i8 yields the exact int32 dot product of
// every (row, token) pair over those 64 bytes.  A K-group of g bytes is g/64
// chained MFMAs; after its last one the int32 partial P_g is scaled in
// registers: acc = fma(float(P_g) * w_scale, x_scale, acc) -- the order the
// reference's accumulate kernel uses (int8_gemm.cu:231, contracted by nvcc).
//
// Loads run two blocks of 8 K-steps ahead of the MFMAs (ping-pong register
// buffers), and the split's weight/activation scales are staged in LDS once.
// When a tile is split over several waves, each wave writes its fp32 partial
// to scratch; the last wave to finish (per-tile arrival counter) adds the
// partials in split order -- a fixed order, so results are deterministic --
// writes fp16 and re-arms the counter for the next launch.
#include "common.h"

namespace fa {
namespace {

constexpr int kRows = 16;         // weight rows per wave tile
constexpr int kBlk = 8;           // K-steps (64 B each) per load block
constexpr int kMaxGroupsPerWave = 64;

struct DbgWindow {
    int32_t* p;
    int row0, rows, tok0, toks;
};

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

template <bool kDbg>
__global__ __launch_bounds__(64) void gemv_mfma_kernel(
    const int8_t* __restrict__ W, const uint16_t* __restrict__ w_scale,
    const int8_t* __restrict__ x_q, const float* __restrict__ x_scale,
    uint16_t* __restrict__ Y, float* __restrict__ part, int* __restrict__ counters,
    DbgWindow dbg, int M, int N, int K, int g, int G, int tiles, int splits, int gps) {
    __shared__ float ws_s[kRows * kMaxGroupsPerWave];
    __shared__ float xs_s[kRows * kMaxGroupsPerWave];
    __shared__ int s_last;

    const int lane = threadIdx.x;
    const int tile = blockIdx.x % tiles;
    const int split = blockIdx.x / tiles;
    const int g_begin = split * gps;
    const int g_end = min(G, g_begin + gps);
    const int ng = g_end - g_begin;
    const int row0 = tile * kRows;
    const int spg = g >> 6;               // MFMA K-steps per group
    const int nsteps = ng * spg;

    const int lr = lane & 15;             // A: weight row in tile; B: token
    const int kq = (lane >> 4) * 16;      // byte offset inside a 64-B step
    const int row_ld = min(row0 + lr, M - 1);
    const bool tok_ok = lr < N;
    const size_t kbase = (size_t)g_begin * g + kq;
    const int8_t* wp = W + (size_t)row_ld * K + kbase;
    const int8_t* xp = x_q + (size_t)(tok_ok ? lr : 0) * K + kbase;

    v4i a0[kBlk], b0[kBlk], a1[kBlk], b1[kBlk];
    const v4i zero = {0, 0, 0, 0};

    auto load_block = [&](v4i (&a)[kBlk], v4i (&b)[kBlk], int blk) {
#pragma unroll
        for (int s = 0; s < kBlk; ++s) {
            const int step = blk * kBlk + s;
            if (step < nsteps) {
                a[s] = ld16(wp + (size_t)step * 64);
                b[s] = tok_ok ? ld16(xp + (size_t)step * 64) : zero;
            } else {
                a[s] = zero;
                b[s] = zero;
            }
        }
    };

    load_block(a0, b0, 0);

    // Stage this split's scales: w_scale rows of the tile, x_scale of the
    // tokens (fp16 [M] when G == 1, reference int8_gemm.cu:228-230).
    for (int i = lane; i < kRows * ng; i += 64) {
        const int r = i / ng, j = i - r * ng;
        const int row = min(row0 + r, M - 1);
        ws_s[r * kMaxGroupsPerWave + j] =
            h2f(G == 1 ? w_scale[row] : w_scale[(size_t)row * G + g_begin + j]);
        xs_s[r * kMaxGroupsPerWave + j] = r < N ? x_scale[(size_t)r * G + g_begin + j] : 0.0f;
    }
    __syncthreads();

    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    v4i P = zero;
    int sig = 0;   // steps done in the current group
    int gj = 0;    // current group, relative to g_begin
    const int orow = 4 * (lane >> 4);   // first of this lane's 4 output rows in the tile

    auto compute_block = [&](const v4i (&a)[kBlk], const v4i (&b)[kBlk], int blk) {
#pragma unroll
        for (int s = 0; s < kBlk; ++s) {
            const int step = blk * kBlk + s;
            if (step < nsteps) {
                P = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s], b[s], P, 0, 0, 0);
                if (++sig == spg) {
                    const float xs = xs_s[lr * kMaxGroupsPerWave + gj];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float ws = ws_s[(orow + r) * kMaxGroupsPerWave + gj];
                        acc[r] = __builtin_fmaf((float)P[r] * ws, xs, acc[r]);
                    }
                    if constexpr (kDbg) {
                        const int t = lr;
                        if (t >= dbg.tok0 && t < dbg.tok0 + dbg.toks && t < N) {
#pragma unroll
                            for (int r = 0; r < 4; ++r) {
                                const int row = row0 + orow + r;
                                if (row >= dbg.row0 && row < dbg.row0 + dbg.rows && row < M)
                                    dbg.p[((size_t)(t - dbg.tok0) * dbg.rows + (row - dbg.row0)) *
                                              G + g_begin + gj] = P[r];
                            }
                        }
                    }
                    P = zero;
                    sig = 0;
                    ++gj;
                }
            }
        }
    };

    const int nblk = (nsteps + kBlk - 1) / kBlk;
    for (int blk = 0; blk < nblk; blk += 2) {
        if (blk + 1 < nblk) load_block(a1, b1, blk + 1);
        compute_block(a0, b0, blk);
        if (blk + 2 < nblk) load_block(a0, b0, blk + 2);
        if (blk + 1 < nblk) compute_block(a1, b1, blk + 1);
    }

    const int t = lr;
    if (splits == 1) {
        if (t < N) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + orow + r;
                if (row < M) Y[(size_t)t * M + row] = f2h(acc[r]);
            }
        }
        return;
    }

    if (t < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + orow + r;
            if (row < M) part[((size_t)split * N + t) * M + row] = acc[r];
        }
    }
    __threadfence();
    if (lane == 0) s_last = atomicAdd(&counters[tile], 1) == splits - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (t < N) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + orow + r;
            if (row < M) {
                float s = 0.0f;
                for (int sp = 0; sp < splits; ++sp) s += part[((size_t)sp * N + t) * M + row];
                Y[(size_t)t * M + row] = f2h(s);
            }
        }
    }
    if (lane == 0) counters[tile] = 0;
}

}  // namespace

GemvPlan plan_gemv(int M, int N, int K, int g, int G) {
    (void)N;
    (void)K;
    (void)g;
    GemvPlan p;
    p.tiles = ceil_div(M, kRows);
    // Aim for ~10 waves per CU over 256 CUs so every CU keeps several 16-row
    // weight streams in flight; never split finer than one group per wave.
    const int target_waves = 2560;
    int s = target_waves / (p.tiles > 0 ? p.tiles : 1);
    if (s < 1) s = 1;
    if (s > G) s = G;
    int gps = ceil_div(G, s);
    if (gps > kMaxGroupsPerWave) gps = kMaxGroupsPerWave;
    p.gps = gps;
    p.splits = ceil_div(G, gps);
    return p;
}

hipError_t launch_gemv(const GemvPlan& p, const int8_t* W, const uint16_t* w_scale,
                       const int8_t* x_q, const float* x_scale, uint16_t* Y, float* part,
                       int* counters, int32_t* dbg_partials, int dbg_row0, int dbg_rows,
                       int dbg_tok0, int dbg_toks, int M, int N, int K, int g, int G,
                       hipStream_t stream) {
    DbgWindow dbg{dbg_partials, dbg_row0, dbg_rows, dbg_tok0, dbg_toks};
    const dim3 grid((unsigned)(p.tiles * p.splits));
    if (dbg_partials)
        hipLaunchKernelGGL((gemv_mfma_kernel<true>), grid, dim3(64), 0, stream, W, w_scale, x_q,
                           x_scale, Y, part, counters, dbg, M, N, K, g, G, p.tiles, p.splits,
                           p.gps);
    else
        hipLaunchKernelGGL((gemv_mfma_kernel<false>), grid, dim3(64), 0, stream, W, w_scale, x_q,
                           x_scale, Y, part, counters, dbg, M, N, K, g, G, p.tiles, p.splits,
                           p.gps);
    return hipGetLastError();
}

}  // namespace fa

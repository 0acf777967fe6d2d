// gemm.hip -- prefill-shaped W8A8 linear (N > 16 tokens) on CDNA4 int8 MFMA,
// plus the any-shape fallback.
//
// Replaces the reference's N > 4 path: G separate cuBLAS int8 GEMMs of depth g
// plus G accumulate passes over an fp32 [M, N] buffer and a final cast
// (src/kernels/int8_gemm.cu:423-505).  Here the whole sum over K-groups stays
// in registers of one kernel:
//
//   workgroup tile 128 weight rows x 128 tokens, 4 waves in 2x2, each wave
//   64 x 64 = 2 x 2 blocks of v_mfma_i32_32x32x32_i8;
//   K advances 64 bytes per stage through double-buffered LDS tiles (row
//   stride 80 B: 16 consecutive rows hit 16 distinct 16-byte bank slots, so
//   the 128-bit fragment reads are conflict-free);
//   a K-group (g bytes) is g/64 stages of exact int32 MFMA accumulation; at
//   its end every int32 partial is scaled in registers,
//       acc = fma(float(P_g) * w_scale[row, g], x_scale[tok, g], acc),
//   the same operation order as the reference's accumulate kernel
//   (int8_gemm.cu:231; nvcc contracts it into one FMA), applied for
//   g = 0, 1, ... in order -- so the fp16 result equals the host oracle's
//   bit for bit;
//   the group's scales ride along with its first stage into LDS.
#include "common.h"

namespace fa {
namespace {

constexpr int BM = 128;        // weight rows per workgroup
constexpr int BN = 128;        // tokens per workgroup
constexpr int kStride = 80;    // LDS bytes per 64-byte K row (16 B pad)

struct DbgWindow {
    int32_t* p;
    int row0, rows, tok0, toks;
};

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

template <bool kDbg>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(
    const int8_t* __restrict__ W, const uint16_t* __restrict__ w_scale,
    const int8_t* __restrict__ x_q, const float* __restrict__ x_scale,
    uint16_t* __restrict__ Y, DbgWindow dbg, int M, int N, int K, int g, int G, int tiles_m) {
    __shared__ __align__(16) int8_t As[2][BM * kStride];
    __shared__ __align__(16) int8_t Bs[2][BN * kStride];
    __shared__ __align__(16) float ws_s[2][BM];
    __shared__ __align__(16) float xs_s[2][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave & 1;
    const int wn = wave >> 1;
    const int tm = blockIdx.x % tiles_m;
    const int tn = blockIdx.x / tiles_m;
    const int m0 = tm * BM;
    const int n0 = tn * BN;

    // Global -> LDS: 2 x 16 B per thread per operand per stage.
    const int8_t* ga[2];
    const int8_t* gb[2];
    int so[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = tid + 256 * j;
        const int r = c >> 2;
        const int kc = (c & 3) * 16;
        ga[j] = W + (size_t)min(m0 + r, M - 1) * K + kc;
        gb[j] = x_q + (size_t)min(n0 + r, N - 1) * K + kc;
        so[j] = r * kStride + kc;
    }

    const int nsteps = K >> 6;
    const int spg = g >> 6;
    v4i ra[2], rb[2];
    float rs = 0.0f;

    auto gload = [&](int step) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            ra[j] = ld16(ga[j] + (size_t)step * 64);
            rb[j] = ld16(gb[j] + (size_t)step * 64);
        }
    };
    auto sload = [&](int gi) {
        if (tid < BM) {
            const int row = min(m0 + tid, M - 1);
            rs = h2f(G == 1 ? w_scale[row] : w_scale[(size_t)row * G + gi]);
        } else {
            const int tok = min(n0 + tid - BM, N - 1);
            rs = x_scale[(size_t)tok * G + gi];
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            *reinterpret_cast<v4i*>(&As[buf][so[j]]) = ra[j];
            *reinterpret_cast<v4i*>(&Bs[buf][so[j]]) = rb[j];
        }
    };
    auto sstore = [&](int sb) {
        if (tid < BM) ws_s[sb][tid] = rs;
        else xs_s[sb][tid - BM] = rs;
    };

    gload(0);
    sload(0);
    lstore(0);
    sstore(0);
    __syncthreads();

    v16i P[2][2];
    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                P[i][j][e] = 0;
                acc[i][j][e] = 0.0f;
            }
        }

    const int frag_row = lane & 31;
    const int frag_k = (lane >> 5) * 16;
    int sig = 0;
    int gi = 0;
    for (int step = 0; step < nsteps; ++step) {
        const int buf = step & 1;
        const bool nxt = step + 1 < nsteps;
        const bool nxt_group = nxt && (sig + 1 == spg);
        if (nxt) gload(step + 1);
        if (nxt_group) sload(gi + 1);

#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            v4i a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const v4i*>(
                    &As[buf][(wm * 64 + i * 32 + frag_row) * kStride + kk * 32 + frag_k]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const v4i*>(
                    &Bs[buf][(wn * 64 + j * 32 + frag_row) * kStride + kk * 32 + frag_k]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    P[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], P[i][j], 0, 0, 0);
        }

        if (++sig == spg) {
            const int sb = gi & 1;
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int tl = wn * 64 + j * 32 + frag_row;
                    const float xs = xs_s[sb][tl];
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int rl = wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        acc[i][j][e] =
                            __builtin_fmaf((float)P[i][j][e] * ws_s[sb][rl], xs, acc[i][j][e]);
                        if constexpr (kDbg) {
                            const int row = m0 + rl, tok = n0 + tl;
                            if (row < M && tok < N && row >= dbg.row0 &&
                                row < dbg.row0 + dbg.rows && tok >= dbg.tok0 &&
                                tok < dbg.tok0 + dbg.toks)
                                dbg.p[((size_t)(tok - dbg.tok0) * dbg.rows + (row - dbg.row0)) *
                                          G + gi] = P[i][j][e];
                        }
                        P[i][j][e] = 0;
                    }
                }
            sig = 0;
            ++gi;
        }

        if (nxt) {
            lstore(buf ^ 1);
            if (nxt_group) sstore(gi & 1);
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int tok = n0 + wn * 64 + j * 32 + frag_row;
            if (tok >= N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) Y[(size_t)tok * M + row] = f2h(acc[i][j][e]);
            }
        }
}

// Any K, any group size, any alignment: one wave per (row, token); lanes
// stride the group, the int32 partial is reduced exactly across the wave and
// scaled in the reference order.  Used only for shapes the MFMA kernels do
// not take (K or g not a multiple of 64, unaligned operands).
template <bool kDbg>
__global__ __launch_bounds__(64) void gemm_generic_kernel(
    const int8_t* __restrict__ W, const uint16_t* __restrict__ w_scale,
    const int8_t* __restrict__ x_q, const float* __restrict__ x_scale,
    uint16_t* __restrict__ Y, DbgWindow dbg, int M, int N, int K, int g, int G) {
    const int row = blockIdx.x;
    const int tok = blockIdx.y;
    const int lane = threadIdx.x;
    const int8_t* wr = W + (size_t)row * K;
    const int8_t* xr = x_q + (size_t)tok * K;
    float acc = 0.0f;
    for (int gi = 0; gi < G; ++gi) {
        const int k0 = gi * g;
        const int k1 = min(k0 + g, K);
        int s = 0;
        for (int k = k0 + lane; k < k1; k += 64) s += (int)wr[k] * (int)xr[k];
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
        const float ws = h2f(G == 1 ? w_scale[row] : w_scale[(size_t)row * G + gi]);
        acc = __builtin_fmaf((float)s * ws, x_scale[(size_t)tok * G + gi], acc);
        if constexpr (kDbg) {
            if (lane == 0 && row >= dbg.row0 && row < dbg.row0 + dbg.rows && tok >= dbg.tok0 &&
                tok < dbg.tok0 + dbg.toks)
                dbg.p[((size_t)(tok - dbg.tok0) * dbg.rows + (row - dbg.row0)) * G + gi] = s;
        }
    }
    if (lane == 0) Y[(size_t)tok * M + row] = f2h(acc);
}

}  // namespace

hipError_t launch_gemm(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                       const float* x_scale, uint16_t* Y, int32_t* dbg_partials, int dbg_row0,
                       int dbg_rows, int dbg_tok0, int dbg_toks, int M, int N, int K, int g, int G,
                       hipStream_t stream) {
    const int tiles_m = ceil_div(M, BM);
    const int tiles_n = ceil_div(N, BN);
    DbgWindow dbg{dbg_partials, dbg_row0, dbg_rows, dbg_tok0, dbg_toks};
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    if (dbg_partials)
        hipLaunchKernelGGL((gemm_mfma_kernel<true>), grid, dim3(256), 0, stream, W, w_scale, x_q,
                           x_scale, Y, dbg, M, N, K, g, G, tiles_m);
    else
        hipLaunchKernelGGL((gemm_mfma_kernel<false>), grid, dim3(256), 0, stream, W, w_scale, x_q,
                           x_scale, Y, dbg, M, N, K, g, G, tiles_m);
    return hipGetLastError();
}

hipError_t launch_gemm_generic(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                               const float* x_scale, uint16_t* Y, int32_t* dbg_partials,
                               int dbg_row0, int dbg_rows, int dbg_tok0, int dbg_toks, int M,
                               int N, int K, int g, int G, hipStream_t stream) {
    DbgWindow dbg{dbg_partials, dbg_row0, dbg_rows, dbg_tok0, dbg_toks};
    const dim3 grid((unsigned)M, (unsigned)N);
    if (dbg_partials)
        hipLaunchKernelGGL((gemm_generic_kernel<true>), grid, dim3(64), 0, stream, W, w_scale, x_q,
                           x_scale, Y, dbg, M, N, K, g, G);
    else
        hipLaunchKernelGGL((gemm_generic_kernel<false>), grid, dim3(64), 0, stream, W, w_scale,
                           x_q, x_scale, Y, dbg, M, N, K, g, G);
    return hipGetLastError();
}

}  // namespace fa

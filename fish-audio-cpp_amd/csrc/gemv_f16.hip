// gemv_f16.hip -- fp16 x fp16 linear with fp32 accumulation for few tokens:
// the FP16 path of DualAREngine::quantized_gemm (dual_ar_engine.cc:338-341),
// i.e. gemm_fp16 (dac_engine.cc:19-32: cublasGemmEx fp16 inputs, fp16 output,
// CUBLAS_COMPUTE_32F), used for the tied-embedding logits head
// (dual_ar_engine.cc:663-665, 155776 x 2560).  HBM-bound: every weight byte is
// read once per call.
//
// One wave streams one weight row: lane l loads 16 bytes (8 fp16) of each
// 1024-byte pass, all of a row's passes (up to 8) issued before the first is
// used; the tokens' fp16 rows sit in LDS, zero-padded to whole passes, and
// each pass adds 4 v_dot2_f32_f16 per token into fp32 lane partials, which a
// DPP / shuffle tree sums at the end of the row.  The summation order differs
// from cuBLAS's (which is unspecified); results agree to fp32 rounding.
#include "common.h"

namespace fa {
namespace {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);   // row_half_mirror
    v += dpp_f<0x140>(v);   // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// NT tokens, PMAX passes of 512 fp16 per row held in flight.
template <int NT, int PMAX>
__global__ __launch_bounds__(256) void gemv_f16_kernel(const uint16_t* __restrict__ W,
                                                       const uint16_t* __restrict__ X,
                                                       uint16_t* __restrict__ Y, int M, int K,
                                                       int ldy, int passes) {
    extern __shared__ __align__(16) uint16_t xs[];   // [NT][passes * 512]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int Kp = passes * 512;
    for (int i = threadIdx.x * 8; i < NT * Kp; i += 256 * 8) {
        const int t = i / Kp, k = i - t * Kp;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (k < K) v = *reinterpret_cast<const uint4*>(X + (size_t)t * K + k);
        *reinterpret_cast<uint4*>(xs + i) = v;
    }
    const int row = blockIdx.x * 4 + wave;
    const int rowc = row < M ? row : M - 1;
    const uint16_t* wr = W + (size_t)rowc * K;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    for (int p0 = 0; p0 < passes; p0 += PMAX) {
        uint4 w[PMAX];
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            const int k = (p0 + j) * 512 + lane * 8;
            // past K the tokens are zero, so any in-row bytes will do
            w[j] = *reinterpret_cast<const uint4*>(wr + (k < K ? k : 0));
        }
        if (p0 == 0) __syncthreads();   // token rows staged (loads above already in flight)
#pragma unroll
        for (int j = 0; j < PMAX; ++j) {
            if (p0 + j >= passes) break;
            const int k = (p0 + j) * 512 + lane * 8;
            const h2v* wa = reinterpret_cast<const h2v*>(&w[j]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint4 xv = *reinterpret_cast<const uint4*>(xs + t * Kp + k);
                const h2v* xa = reinterpret_cast<const h2v*>(&xv);
                float a = acc[t];
#pragma unroll
                for (int e = 0; e < 4; ++e) a = __builtin_amdgcn_fdot2(wa[e], xa[e], a, false);
                acc[t] = a;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float s = wave_sum(acc[t]);
        if (lane == 0 && row < M) Y[(size_t)t * ldy + row] = f2h(s);
    }
}

// Any shape, any alignment: one wave per (row, token), fp32 partials.
__global__ __launch_bounds__(64) void gemm_f16_generic_kernel(const uint16_t* __restrict__ W,
                                                              const uint16_t* __restrict__ X,
                                                              uint16_t* __restrict__ Y, int M,
                                                              int K) {
    const int row = blockIdx.x, tok = blockIdx.y, lane = threadIdx.x;
    float a = 0.0f;
    for (int k = lane; k < K; k += 64)
        a = __builtin_fmaf(h2f(W[(size_t)row * K + k]), h2f(X[(size_t)tok * K + k]), a);
    a = wave_sum(a);
    if (lane == 0) Y[(size_t)tok * M + row] = f2h(a);
}

template <int NT>
void launch_nt(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int K, int ldy,
               hipStream_t stream) {
    const int passes = (K + 511) / 512;
    const dim3 grid((unsigned)((M + 3) / 4));
    const size_t lds = (size_t)NT * passes * 512 * 2;
#define FA_F16(PM)                                                                             \
    hipLaunchKernelGGL((gemv_f16_kernel<NT, PM>), grid, dim3(256), lds, stream, W, X, Y, M, K, \
                       ldy, passes)
    switch (passes) {   // a row's passes all in flight at once (K <= 4096)
        case 1: FA_F16(1); break;
        case 2: FA_F16(2); break;
        case 3: FA_F16(3); break;
        case 4: FA_F16(4); break;
        case 5: FA_F16(5); break;
        case 6: FA_F16(6); break;
        case 7: FA_F16(7); break;
        default: FA_F16(8); break;
    }
#undef FA_F16
}

}  // namespace

bool gemv_f16_ok(int M, int N, int K) {
    (void)M;
    (void)N;
    return K % 8 == 0 && K <= 4096;   // 8 tokens' rows in 64 KB of LDS, a row's passes in flight
}

hipError_t launch_gemm_f16_generic(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N,
                                   int K, hipStream_t stream) {
    hipLaunchKernelGGL(gemm_f16_generic_kernel, dim3((unsigned)M, (unsigned)N), dim3(64), 0,
                       stream, W, X, Y, M, K);
    return hipGetLastError();
}

hipError_t launch_gemv_f16(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                           hipStream_t stream) {
    // tokens in chunks of 8, 4, 2, 1 (each chunk streams W once)
    for (int t0 = 0; t0 < N;) {
        const int left = N - t0;
        const uint16_t* x = X + (size_t)t0 * K;
        uint16_t* y = Y + (size_t)t0 * M;
        if (left >= 8) { launch_nt<8>(W, x, y, M, K, M, stream); t0 += 8; }
        else if (left >= 4) { launch_nt<4>(W, x, y, M, K, M, stream); t0 += 4; }
        else if (left >= 2) { launch_nt<2>(W, x, y, M, K, M, stream); t0 += 2; }
        else { launch_nt<1>(W, x, y, M, K, M, stream); t0 += 1; }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace fa

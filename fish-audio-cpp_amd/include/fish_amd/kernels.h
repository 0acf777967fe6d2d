// kernels.h -- C++ mirror of the reference's kernel API for the W8A8 path
// (src/kernels/kernels.h:11-19, 111-140, 242-259, 324-344), on HIP.
//
// Same names, argument order and meaning; hipStream_t replaces cudaStream_t,
// and the cublasHandle_t slot of int8_dequant_gemm_fp16 becomes an unused
// opaque pointer.  Failures throw std::runtime_error, as CUDA_CHECK does
// (src/utils/cuda_utils.h:10-17).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace fish::kernels {

void rms_norm(const __half* x, const __half* weight, __half* out, int n_tokens, int dim,
              float eps, hipStream_t stream = 0);

void silu_forward(__half* x, int n, hipStream_t stream = 0);
void mul_forward(__half* a, const __half* b, int n, hipStream_t stream = 0);
void residual_add(__half* a, const __half* b, int n, hipStream_t stream = 0);

// W [M, K] int8 row-major; scale fp16 [M] or [M, G]; act_scale fp16 [G] or
// null (dynamic); smooth_inv fp16 [K] or null; X fp16 [N, K] row-major;
// Y fp16 col-major [M, N] (ld = M).
void int8_dequant_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                            const __half* act_scale, const __half* smooth_inv, const __half* X,
                            __half* Y, int M, int N, int K, void* blas_handle_unused,
                            hipStream_t stream = 0);

// Prefill attention side (src/kernels/kernels.h:324-344): the same names and
// argument order; the cublasHandle_t of prefill_attention_gpu becomes an
// unused opaque pointer and `workspace` may be null (the fused kernel needs
// none).
void prefill_attention_gpu(const __half* q, const __half* k, const __half* v, __half* out,
                           __half* workspace, int n_q, int n_kv, int T, int D, float sm_scale,
                           void* blas_handle_unused, hipStream_t stream, int window_size = 0);
void qkv_split_heads(const __half* qkv, __half* q, __half* k, __half* v, int T, int n_heads,
                     int head_dim, hipStream_t stream = 0);
void qkv_split_heads_gqa(const __half* qkv, __half* q, __half* k, __half* v, int T, int n_q,
                         int n_kv, int head_dim, hipStream_t stream = 0);
void merge_heads(const __half* heads, __half* out, int T, int n_heads, int head_dim,
                 hipStream_t stream = 0);
// prefill_attention_gpu + merge_heads in one launch (fa_prefill_attention_merged):
// out token-major [T, n_q * D].
void prefill_attention_merged(const __half* q, const __half* k, const __half* v, __half* out,
                              int n_q, int n_kv, int T, int D, float sm_scale,
                              hipStream_t stream = 0, int window_size = 0);

// Additive fused entry points (no single reference counterpart).
void rms_norm_quant(const __half* x, const __half* weight, float eps, const __half* smooth_inv,
                    const __half* act_scale, int group_size, int8_t* X_q, float* X_scale,
                    __half* out, int n_tokens, int dim, hipStream_t stream = 0);
void silu_mul_quant(const __half* gate, const __half* up, const __half* smooth_inv,
                    const __half* act_scale, int group_size, int8_t* X_q, float* X_scale,
                    __half* out, int n_tokens, int dim, hipStream_t stream = 0);
void int8_gemm_quantized_fp16(const int8_t* W, const __half* scale, int group_size,
                              const int8_t* X_q, const float* X_scale, __half* Y, int M, int N,
                              int K, hipStream_t stream = 0);

// The FP16 weight path of DualAREngine::quantized_gemm: gemm_fp16
// (dac_engine.cc:19-32, same argument order; Y col-major [M_out, N_out]).
void gemm_fp16(int M_out, int N_out, int K, const __half* W, const __half* X, __half* Y,
               void* blas_handle_unused, hipStream_t stream = 0);

// Linear layers with their decode prologue / epilogue fused (fa_w8a8_gemm_rms,
// fa_w8a8_gemm_swiglu, fa_w8a8_gemm_silu_mul in include/fish_w8a8.h): one
// launch each at one token.
void int8_rms_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                        const __half* act_scale, const __half* smooth_inv, const __half* x,
                        const __half* resid, __half* h_out, const __half* gamma, float eps,
                        __half* Y, int M, int N, int K, hipStream_t stream = 0);
void int8_swiglu_gemm_fp16(const int8_t* W13, const __half* scale13, int group_size,
                           const __half* act_scale, const __half* smooth_inv, const __half* x,
                           const __half* resid, __half* h_out, const __half* gamma, float eps,
                           __half* act, int F, int N, int K, hipStream_t stream = 0);
void int8_silu_mul_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                             const __half* act_scale, const __half* smooth_inv,
                             const __half* gate, const __half* up, __half* Y, int M, int N, int K,
                             hipStream_t stream = 0);
// SwiGLU over separate w1 / w3 with their own companions (fa_w8a8_gemm_swiglu_sep).
void int8_swiglu_sep_gemm_fp16(const int8_t* W1, const __half* scale1, const int8_t* W3,
                               const __half* scale3, int group_size, const __half* act_scale1,
                               const __half* smooth_inv1, const __half* act_scale3,
                               const __half* smooth_inv3, const __half* x, const __half* resid,
                               __half* h_out, const __half* gamma, float eps, __half* act, int F,
                               int N, int K, hipStream_t stream = 0);

}  // namespace fish::kernels

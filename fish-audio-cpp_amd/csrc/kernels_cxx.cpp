// kernels_cxx.cpp -- fish::kernels C++ entry points over the C ABI; a failure
// throws std::runtime_error with fa_last_error(), as the reference's
// CUDA_CHECK does (src/utils/cuda_utils.h:10-17).
#include "fish_amd/kernels.h"
#include "../../include/fish_w8a8.h"

#include <stdexcept>
#include <string>

namespace fish::kernels {
namespace {
inline const uint16_t* u16(const __half* p) { return reinterpret_cast<const uint16_t*>(p); }
inline uint16_t* u16(__half* p) { return reinterpret_cast<uint16_t*>(p); }
inline void check(int rc) {
    if (rc != FA_OK) throw std::runtime_error(std::string("fish::kernels: ") + fa_last_error());
}
}  // namespace

void rms_norm(const __half* x, const __half* weight, __half* out, int n_tokens, int dim, float eps,
              hipStream_t stream) {
    check(fa_rms_norm(u16(x), u16(weight), u16(out), n_tokens, dim, eps, stream));
}

void silu_forward(__half* x, int n, hipStream_t stream) { check(fa_silu(u16(x), n, stream)); }

void mul_forward(__half* a, const __half* b, int n, hipStream_t stream) {
    check(fa_mul(u16(a), u16(b), n, stream));
}

void residual_add(__half* a, const __half* b, int n, hipStream_t stream) {
    check(fa_residual_add(u16(a), u16(b), n, stream));
}

void int8_dequant_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                            const __half* act_scale, const __half* smooth_inv, const __half* X,
                            __half* Y, int M, int N, int K, void* /*blas_handle_unused*/,
                            hipStream_t stream) {
    check(fa_w8a8_gemm(W, u16(scale), group_size, u16(act_scale), u16(smooth_inv), u16(X), u16(Y),
                       M, N, K, stream));
}

void rms_norm_quant(const __half* x, const __half* weight, float eps, const __half* smooth_inv,
                    const __half* act_scale, int group_size, int8_t* X_q, float* X_scale,
                    __half* out, int n_tokens, int dim, hipStream_t stream) {
    check(fa_rms_norm_quant(u16(x), u16(weight), eps, u16(smooth_inv), u16(act_scale), group_size,
                            X_q, X_scale, u16(out), n_tokens, dim, stream));
}

void silu_mul_quant(const __half* gate, const __half* up, const __half* smooth_inv,
                    const __half* act_scale, int group_size, int8_t* X_q, float* X_scale,
                    __half* out, int n_tokens, int dim, hipStream_t stream) {
    check(fa_silu_mul_quant(u16(gate), u16(up), u16(smooth_inv), u16(act_scale), group_size, X_q,
                            X_scale, u16(out), n_tokens, dim, stream));
}

void int8_gemm_quantized_fp16(const int8_t* W, const __half* scale, int group_size,
                              const int8_t* X_q, const float* X_scale, __half* Y, int M, int N,
                              int K, hipStream_t stream) {
    check(fa_w8a8_gemm_quantized(W, u16(scale), group_size, X_q, X_scale, u16(Y), M, N, K, stream));
}

void gemm_fp16(int M_out, int N_out, int K, const __half* W, const __half* X, __half* Y,
               void* /*blas_handle_unused*/, hipStream_t stream) {
    check(fa_gemm_fp16(u16(W), u16(X), u16(Y), M_out, N_out, K, stream));
}

void int8_rms_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                        const __half* act_scale, const __half* smooth_inv, const __half* x,
                        const __half* resid, __half* h_out, const __half* gamma, float eps,
                        __half* Y, int M, int N, int K, hipStream_t stream) {
    check(fa_w8a8_gemm_rms(W, u16(scale), group_size, u16(act_scale), u16(smooth_inv), u16(x),
                           u16(resid), u16(h_out), u16(gamma), eps, u16(Y), M, N, K, stream));
}

void int8_swiglu_gemm_fp16(const int8_t* W13, const __half* scale13, int group_size,
                           const __half* act_scale, const __half* smooth_inv, const __half* x,
                           const __half* resid, __half* h_out, const __half* gamma, float eps,
                           __half* act, int F, int N, int K, hipStream_t stream) {
    check(fa_w8a8_gemm_swiglu(W13, u16(scale13), group_size, u16(act_scale), u16(smooth_inv),
                              u16(x), u16(resid), u16(h_out), u16(gamma), eps, u16(act), F, N, K,
                              stream));
}

void int8_silu_mul_gemm_fp16(const int8_t* W, const __half* scale, int group_size,
                             const __half* act_scale, const __half* smooth_inv,
                             const __half* gate, const __half* up, __half* Y, int M, int N, int K,
                             hipStream_t stream) {
    check(fa_w8a8_gemm_silu_mul(W, u16(scale), group_size, u16(act_scale), u16(smooth_inv),
                                u16(gate), u16(up), u16(Y), M, N, K, stream));
}

void int8_swiglu_sep_gemm_fp16(const int8_t* W1, const __half* scale1, const int8_t* W3,
                               const __half* scale3, int group_size, const __half* act_scale1,
                               const __half* smooth_inv1, const __half* act_scale3,
                               const __half* smooth_inv3, const __half* x, const __half* resid,
                               __half* h_out, const __half* gamma, float eps, __half* act, int F,
                               int N, int K, hipStream_t stream) {
    check(fa_w8a8_gemm_swiglu_sep(W1, u16(scale1), W3, u16(scale3), group_size, u16(act_scale1),
                                  u16(smooth_inv1), u16(act_scale3), u16(smooth_inv3), u16(x),
                                  u16(resid), u16(h_out), u16(gamma), eps, u16(act), F, N, K,
                                  stream));
}

void prefill_attention_gpu(const __half* q, const __half* k, const __half* v, __half* out,
                           __half* workspace, int n_q, int n_kv, int T, int D, float sm_scale,
                           void* /*blas_handle_unused*/, hipStream_t stream, int window_size) {
    check(fa_prefill_attention(u16(q), u16(k), u16(v), u16(out), workspace, n_q, n_kv, T, D,
                               sm_scale, stream, window_size));
}

void qkv_split_heads(const __half* qkv, __half* q, __half* k, __half* v, int T, int n_heads,
                     int head_dim, hipStream_t stream) {
    check(fa_qkv_split_heads(u16(qkv), u16(q), u16(k), u16(v), T, n_heads, head_dim, stream));
}

void qkv_split_heads_gqa(const __half* qkv, __half* q, __half* k, __half* v, int T, int n_q,
                         int n_kv, int head_dim, hipStream_t stream) {
    check(fa_qkv_split_heads_gqa(u16(qkv), u16(q), u16(k), u16(v), T, n_q, n_kv, head_dim,
                                 stream));
}

void merge_heads(const __half* heads, __half* out, int T, int n_heads, int head_dim,
                 hipStream_t stream) {
    check(fa_merge_heads(u16(heads), u16(out), T, n_heads, head_dim, stream));
}

void prefill_attention_merged(const __half* q, const __half* k, const __half* v, __half* out,
                              int n_q, int n_kv, int T, int D, float sm_scale, hipStream_t stream,
                              int window_size) {
    check(fa_prefill_attention_merged(u16(q), u16(k), u16(v), u16(out), n_q, n_kv, T, D, sm_scale,
                                      stream, window_size));
}

}  // namespace fish::kernels

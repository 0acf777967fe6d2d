/*
 * w8a8_ref.h -- CPU oracle for the W8A8 linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a scalar C restatement of the reference
 * engine's arithmetic, used as the checker in tests/, in __graft_entry__.smoke()
 * and as the timed CPU baseline in bench.py.  Nothing in the product library
 * (fish-audio-cpp_amd/) links, loads or calls it.
 *
 * Naming follows the reference kernel API (src/kernels/kernels.h:242-259):
 *   M = output features (rows of W), N = tokens, K = input features.
 * fp16 values travel as raw IEEE binary16 bit patterns (uint16_t).
 *
 * Every function cites the reference file:line it restates; the header of
 * w8a8_ref.c lists where each one is pinned.
 */
#ifndef FISH_W8A8_REF_H
#define FISH_W8A8_REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* binary16 <-> binary32, round-to-nearest-even (the CUDA __float2half /
 * numpy astype(float16) rounding the reference relies on). */
float    orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
void     orc_h2f_array(const uint16_t* h, float* f, int64_t n);
void     orc_f2h_array(const float* f, uint16_t* h, int64_t n);

/* group_size <= 0 || > K  ->  K   (src/kernels/int8_gemm.cu:396-397) */
int orc_effective_group(int K, int group_size);
int orc_num_groups(int K, int group_size);

/* Group-size inference from a scale tensor's shape
 * (src/engine/dual_ar_engine.cc:17-24). */
int orc_infer_group_size(int64_t K, int scale_ndim, int64_t scale_groups);

/* tools/quant_utils.py:171-194 quantize_groupwise: fp16 W [rows, K] ->
 * int8 q [rows, K] and fp16 scale [rows, G]. */
void orc_quantize_weights_groupwise(const uint16_t* w, int64_t rows, int64_t K,
                                    int group_size, int8_t* q, uint16_t* scale);

/* src/kernels/int8_gemm.cu:147-211 quantize_activation_groups_kernel:
 * X fp16 [N, K] -> X_q int8 [N, K], X_scale fp32 [N, G]. act_scale (fp16 [G])
 * and smooth_inv (fp16 [K]) may be NULL. */
void orc_quantize_activations(const uint16_t* X, const uint16_t* act_scale,
                              const uint16_t* smooth_inv, int N, int K,
                              int group_size, int8_t* x_q, float* x_scale);

/* Exact int32 per-(token, row, K-group) partial sums, the quantity cuBLAS
 * computes per group at src/kernels/int8_gemm.cu:476-488.
 * P layout: [N tokens][M rows][G groups]. */
void orc_group_partials(const int8_t* W, const int8_t* x_q, int M, int N, int K,
                        int group_size, int32_t* P);

/* Dequant-sum epilogue on already-quantized activations
 * (int8_gemm.cu:213-243): acc = fma(float(P_g) * ws, xs, acc) over ascending g,
 * then fp16 RN.  Y is col-major [M, N] (= row-major [N tokens, M]). */
void orc_gemm_quantized(const int8_t* W, const uint16_t* w_scale, int group_size,
                        const int8_t* x_q, const float* x_scale, uint16_t* Y,
                        int M, int N, int K);

/* Whole reference entry point int8_dequant_gemm_fp16
 * (src/kernels/kernels.h:249-259, int8_gemm.cu:384-511). */
void orc_w8a8_gemm(const int8_t* W, const uint16_t* w_scale, int group_size,
                   const uint16_t* act_scale, const uint16_t* smooth_inv,
                   const uint16_t* X, uint16_t* Y, int M, int N, int K);

/* 1 / sqrt(sum_sq / dim + eps) as rms_norm.cu:44 computes it (rsqrtf replaced
 * by a correctly rounded double 1/sqrt, rounded to float). */
float orc_rms_inv(float sum_sq, int dim, float eps);

/* src/kernels/rms_norm.cu:10-76, with the reference's reduction order. */
void orc_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* out,
                  int n_tokens, int dim, float eps);

/* rms_norm followed by the activation quantizer (the two reference launches
 * at dual_ar_engine.cc:580-583 / 636-640).  out_f16 may be NULL. */
void orc_rms_norm_quant(const uint16_t* x, const uint16_t* weight, float eps,
                        const uint16_t* smooth_inv, const uint16_t* act_scale,
                        int group_size, int8_t* x_q, float* x_scale,
                        uint16_t* out_f16, int n_tokens, int dim);

/* src/kernels/ffn_activations.cu:12-17 / 35-45 (in place on a). */
void orc_silu(uint16_t* x, int64_t n);
void orc_mul(uint16_t* a, const uint16_t* b, int64_t n);
void orc_residual_add(uint16_t* a, const uint16_t* b, int64_t n);

/* silu(gate) -> fp16, * up -> fp16, then the activation quantizer
 * (dual_ar_engine.cc:640-646).  out_f16 may be NULL. */
void orc_silu_mul_quant(const uint16_t* gate, const uint16_t* up,
                        const uint16_t* smooth_inv, const uint16_t* act_scale,
                        int group_size, int8_t* x_q, float* x_scale,
                        uint16_t* out_f16, int n_tokens, int dim);

/* Threads OpenMP will use (for the CPU-baseline report). */
int orc_num_threads(void);
void orc_set_num_threads(int n);

/* fp16 linear as an exact value: Y, sum|w x| [N, M] in double. */
/* Prefill attention side (src/kernels/prefill_attention.cu). */
void orc_qkv_split_gqa(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                       int n_q, int n_kv, int D);
void orc_merge_heads(const uint16_t* heads, uint16_t* out, int T, int H, int D);
void orc_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* out, double* absw, int n_q, int n_kv, int T, int D,
                           float sm_scale, int window);
void orc_gemm_fp16_exact(const uint16_t* W, const uint16_t* X, double* Y, double* absY,
                         int M, int N, int K);

#ifdef __cplusplus
}
#endif
#endif

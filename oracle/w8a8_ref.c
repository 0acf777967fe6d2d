/*
 * w8a8_ref.c -- CPU oracle (scalar C, OpenMP over rows) for the W8A8 path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and the CPU
 * baseline leg of bench.py.  The product library never links or calls it.
 *
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf() and every other float operation rounds on its own.  The
 * reference is compiled by nvcc with its default --fmad=true, which contracts
 * `a * b + c` into one FMA; the places where that happens in the reference are
 * written here as fmaf() and marked "nvcc contracts".
 *
 * Where each function is pinned (tests/test_oracle.py):
 *   orc_h2f / orc_f2h            exhaustive / dense comparison with numpy's
 *                                independent float16 conversion, incl. ties.
 *   orc_quantize_weights_groupwise  hand-computed known answers, invariants
 *                                (max|q| == 127 per nonzero group, |w-q*s|<=s/2),
 *                                the all-zero-group special case.
 *   orc_quantize_activations     known answers (zero group -> s=1e-8, one-hot
 *                                -> +-127, exact .5 ties -> even), static-scale
 *                                and smooth_inv paths, the same invariants.
 *   orc_group_partials           brute-force exact integer dot products
 *                                (numpy int64) and closed forms (all-ones -> g).
 *   orc_gemm_quantized / orc_w8a8_gemm  float64 evaluation of the same sum,
 *                                within 1 fp16 ulp; a scale-index swap, a
 *                                dropped group or a transposed output fails it.
 *   orc_rms_norm                 the reference's own closed-form tests
 *                                (tests/test_kernels.cu:121-247) plus float64.
 *   orc_silu / orc_mul / orc_residual_add  the reference's closed-form tests
 *                                (tests/test_kernels.cu:354-481) plus float64.
 *   orc_gemm_fp16_exact          exact rational sums (Python fractions) on
 *                                small inputs and one-hot closed forms.
 *   orc_qkv_split_gqa / orc_merge_heads  numpy slicing / transposition of the
 *                                same layouts (independent index algebra).
 *   orc_prefill_attention        closed forms (T = 1 -> V row 0; Q = 0 -> the
 *                                mean of V over the causal/window range;
 *                                window 1 -> V row i), a float64 softmax
 *                                evaluation within the stated tolerance, and
 *                                a swapped K/V or a broken mask shown to fail.
 * The reference's CUDA intrinsics rsqrtf/expf are approximations whose
 * constants are not reproduced: this oracle uses (float)(1/sqrt(double)) and
 * (float)exp(double) instead, and the device code uses the same formulas.
 */
#include "w8a8_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 ---- */

float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0x1f) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        float v = (float)m * (1.0f / 16777216.0f);
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                                           /* normal half */
        uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);                  /* RN-even at bit 13 */
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    /* subnormal half (or zero): round |f| * 2^24 to an integer, ties to even;
     * the scaling by a power of two is exact in this range. */
    float a;
    memcpy(&a, &ax, 4);
    float s = a * 16777216.0f;
    uint32_t m = (uint32_t)rintf(s);
    return (uint16_t)(sign | m);
}

void orc_h2f_array(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; ++i) f[i] = orc_h2f(h[i]);
}

void orc_f2h_array(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; ++i) h[i] = orc_f2h(f[i]);
}

/* ------------------------------------------------------------- groups ---- */

int orc_effective_group(int K, int group_size) {
    /* int8_gemm.cu:396 */
    if (group_size <= 0 || group_size > K) return K;
    return group_size;
}

int orc_num_groups(int K, int group_size) {
    /* int8_gemm.cu:397 */
    int g = orc_effective_group(K, group_size);
    return g > 0 ? (K + g - 1) / g : 0;
}

int orc_infer_group_size(int64_t K, int scale_ndim, int64_t scale_groups) {
    /* dual_ar_engine.cc:17-24: 1-D scale or G <= 1 -> K, else ceil(K / G) */
    if (scale_ndim <= 1) return (int)K;
    if (scale_groups <= 1) return (int)K;
    return (int)((K + scale_groups - 1) / scale_groups);
}

/* ------------------------------------------------------- weight quant ---- */

void orc_quantize_weights_groupwise(const uint16_t* w, int64_t rows, int64_t K,
                                    int group_size, int8_t* q, uint16_t* scale) {
    /* tools/quant_utils.py:171-194.  All arithmetic is float32 (numpy >= 2
     * keeps float32 for float32-array op python-float):
     *   amax = max(max|w|, 1e-8);  s = float16(amax / 127)
     *   q = clip(round_half_even(w / float32(s)), -127, 127)
     * An all-zero group gives s = float16(7.9e-11) = 0 and 0/0 = NaN, which
     * numpy's float->int8 cast turns into 0 on x86; this oracle writes 0. */
    int64_t g = group_size;
    int64_t groups = (K + g - 1) / g;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* wr = w + r * K;
        for (int64_t gi = 0; gi < groups; ++gi) {
            int64_t k0 = gi * g, k1 = k0 + g < K ? k0 + g : K;
            float amax = 0.0f;
            for (int64_t k = k0; k < k1; ++k) {
                float a = fabsf(orc_h2f(wr[k]));
                if (a > amax) amax = a;
            }
            if (!(amax > 1e-8f)) amax = 1e-8f;
            uint16_t sh = orc_f2h(amax / 127.0f);
            scale[r * groups + gi] = sh;
            float s = orc_h2f(sh);
            for (int64_t k = k0; k < k1; ++k) {
                float v = orc_h2f(wr[k]) / s;
                int8_t out;
                if (isnan(v)) {
                    out = 0;
                } else {
                    float rv = rintf(v);
                    if (rv > 127.0f) rv = 127.0f;
                    if (rv < -127.0f) rv = -127.0f;
                    out = (int8_t)rv;
                }
                q[r * K + k] = out;
            }
        }
    }
}

/* -------------------------------------------------- activation quant ---- */

static void quantize_row_groups(const float* v, const uint16_t* act_scale, int K,
                                int g, int groups, int8_t* q_row, float* s_row) {
    /* int8_gemm.cu:158-210 for one token row, v already smoothed. */
    for (int gi = 0; gi < groups; ++gi) {
        int k0 = gi * g, k1 = k0 + g < K ? k0 + g : K;
        float s;
        if (act_scale) {
            s = orc_h2f(act_scale[gi]);
            if (s < 1e-8f) s = 1e-8f;
        } else {
            float amax = 0.0f;
            for (int k = k0; k < k1; ++k) amax = fmaxf(amax, fabsf(v[k]));
            s = amax / 127.0f;
            if (s < 1e-8f) s = 1e-8f;
        }
        s_row[gi] = s;
        float inv = 1.0f / s;
        for (int k = k0; k < k1; ++k) {
            float t = rintf(v[k] * inv);   /* __float2int_rn: RN-even */
            if (t > 127.0f) t = 127.0f;
            if (t < -127.0f) t = -127.0f;
            q_row[k] = (int8_t)t;
        }
    }
}

void orc_quantize_activations(const uint16_t* X, const uint16_t* act_scale,
                              const uint16_t* smooth_inv, int N, int K,
                              int group_size, int8_t* x_q, float* x_scale) {
    int g = orc_effective_group(K, group_size);
    int groups = orc_num_groups(K, group_size);
    #pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)(K > 0 ? K : 1));
        #pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            const uint16_t* xr = X + (int64_t)n * K;
            for (int k = 0; k < K; ++k) {
                float t = orc_h2f(xr[k]);
                if (smooth_inv) t *= orc_h2f(smooth_inv[k]);   /* int8_gemm.cu:178,206 */
                v[k] = t;
            }
            quantize_row_groups(v, act_scale, K, g, groups, x_q + (int64_t)n * K,
                                x_scale + (int64_t)n * groups);
        }
        free(v);
    }
}

/* ----------------------------------------------------- int32 partials ---- */

static inline int32_t dot_i8(const int8_t* a, const int8_t* b, int n) {
    int32_t s = 0;
    for (int i = 0; i < n; ++i) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

void orc_group_partials(const int8_t* W, const int8_t* x_q, int M, int N, int K,
                        int group_size, int32_t* P) {
    int g = orc_effective_group(K, group_size);
    int groups = orc_num_groups(K, group_size);
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const int8_t* wr = W + (int64_t)m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* xr = x_q + (int64_t)n * K;
            int32_t* out = P + ((int64_t)n * M + m) * groups;
            for (int gi = 0; gi < groups; ++gi) {
                int k0 = gi * g, k1 = k0 + g < K ? k0 + g : K;
                out[gi] = dot_i8(wr + k0, xr + k0, k1 - k0);
            }
        }
    }
}

/* ----------------------------------------------------------- epilogue ---- */

void orc_gemm_quantized(const int8_t* W, const uint16_t* w_scale, int group_size,
                        const int8_t* x_q, const float* x_scale, uint16_t* Y,
                        int M, int N, int K) {
    /* accumulate_group_kernel (int8_gemm.cu:213-234) applied for g = 0..G-1 in
     * order, then float_to_half_kernel (:236-243).  `accum += float(P)*ws*xs`
     * is contracted by nvcc to fma(float(P)*ws, xs, accum). */
    int g = orc_effective_group(K, group_size);
    int groups = orc_num_groups(K, group_size);
    #pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m) {
        const int8_t* wr = W + (int64_t)m * K;
        for (int n = 0; n < N; ++n) {
            const int8_t* xr = x_q + (int64_t)n * K;
            const float* xs = x_scale + (int64_t)n * groups;
            float acc = 0.0f;
            for (int gi = 0; gi < groups; ++gi) {
                int k0 = gi * g, k1 = k0 + g < K ? k0 + g : K;
                int32_t p = dot_i8(wr + k0, xr + k0, k1 - k0);
                float ws = groups == 1 ? orc_h2f(w_scale[m])
                                       : orc_h2f(w_scale[(int64_t)m * groups + gi]);
                acc = fmaf((float)p * ws, xs[gi], acc);          /* nvcc contracts */
            }
            Y[(int64_t)n * M + m] = orc_f2h(acc);
        }
    }
}

void orc_w8a8_gemm(const int8_t* W, const uint16_t* w_scale, int group_size,
                   const uint16_t* act_scale, const uint16_t* smooth_inv,
                   const uint16_t* X, uint16_t* Y, int M, int N, int K) {
    int g = orc_effective_group(K, group_size);
    int groups = orc_num_groups(K, group_size);
    int8_t* xq = (int8_t*)malloc((size_t)N * (size_t)K + 1);
    float* xs = (float*)malloc(sizeof(float) * ((size_t)N * (size_t)groups + 1));
    orc_quantize_activations(X, act_scale, smooth_inv, N, K, g, xq, xs);
    orc_gemm_quantized(W, w_scale, g, xq, xs, Y, M, N, K);
    free(xq);
    free(xs);
}

/* ------------------------------------------------------------ RMSNorm ---- */

static size_t next_pow2(size_t x) {
    /* src/utils/cuda_utils.h:41-52 */
    if (x == 0) return 1;
    size_t p = 1;
    while (p < x) p <<= 1;
    return p;
}

/* One CUDA warp's __shfl_down_sync tree (offsets 16, 8, 4, 2, 1) as seen by
 * lane 0: v[i] += v[i + off] for the lanes that feed lane 0. */
static float warp32_tree(float* v) {
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) v[i] = v[i] + v[i + off];
    return v[0];
}

static float rms_sum_of_squares(const float* x, int dim) {
    /* rms_norm.cu:22-41 with blockDim = min(next_pow2(dim), 1024) (:69-70).
     * Thread t sums x[t], x[t+T], ... with nvcc-contracted FMAs; each 32-lane
     * warp reduces by the shuffle tree; warp sums go through shared memory and
     * the first warp reduces them by the same tree.  Lanes that a block smaller
     * than 32 threads does not have contribute 0. */
    int T = (int)next_pow2((size_t)dim);
    if (T > 1024) T = 1024;
    int lanes = T < 32 ? 32 : T;
    float local[1024];
    for (int t = 0; t < lanes; ++t) {
        float s = 0.0f;
        if (t < T)
            for (int i = t; i < dim; i += T) s = fmaf(x[i], x[i], s);   /* nvcc contracts */
        local[t] = s;
    }
    int num_warps = (T + 31) / 32;
    float warp_sums[32];
    for (int w = 0; w < 32; ++w) warp_sums[w] = 0.0f;
    for (int w = 0; w < num_warps; ++w) warp_sums[w] = warp32_tree(local + 32 * w);
    return warp32_tree(warp_sums);
}

float orc_rms_inv(float sum_sq, int dim, float eps) {
    /* rms_norm.cu:44 `rsqrtf(total_sum / dim + eps)`; rsqrtf replaced by a
     * double-precision 1/sqrt rounded to float. */
    float t = sum_sq / (float)dim + eps;
    return (float)(1.0 / sqrt((double)t));
}

void orc_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* out,
                  int n_tokens, int dim, float eps) {
    #pragma omp parallel
    {
        float* v = (float*)malloc(sizeof(float) * (size_t)(dim > 0 ? dim : 1));
        #pragma omp for schedule(static)
        for (int n = 0; n < n_tokens; ++n) {
            const uint16_t* xr = x + (int64_t)n * dim;
            for (int i = 0; i < dim; ++i) v[i] = orc_h2f(xr[i]);
            float r = orc_rms_inv(rms_sum_of_squares(v, dim), dim, eps);
            for (int i = 0; i < dim; ++i)
                out[(int64_t)n * dim + i] = orc_f2h((v[i] * r) * orc_h2f(weight[i]));  /* :52-56 */
        }
        free(v);
    }
}

void orc_rms_norm_quant(const uint16_t* x, const uint16_t* weight, float eps,
                        const uint16_t* smooth_inv, const uint16_t* act_scale,
                        int group_size, int8_t* x_q, float* x_scale,
                        uint16_t* out_f16, int n_tokens, int dim) {
    uint16_t* h = out_f16 ? out_f16
                          : (uint16_t*)malloc(sizeof(uint16_t) * ((size_t)n_tokens * dim + 1));
    orc_rms_norm(x, weight, h, n_tokens, dim, eps);
    orc_quantize_activations(h, act_scale, smooth_inv, n_tokens, dim, group_size, x_q, x_scale);
    if (!out_f16) free(h);
}

/* ------------------------------------------------------- elementwise ---- */

static inline float silu_f(float v) {
    /* ffn_activations.cu:15 `val / (1.0f + expf(-val))`; expf replaced by a
     * double exp rounded to float. */
    float e = (float)exp(-(double)v);
    return v / (1.0f + e);
}

void orc_silu(uint16_t* x, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = orc_f2h(silu_f(orc_h2f(x[i])));
}

void orc_mul(uint16_t* a, const uint16_t* b, int64_t n) {
    /* ffn_activations.cu:35-39 */
    for (int64_t i = 0; i < n; ++i) a[i] = orc_f2h(orc_h2f(a[i]) * orc_h2f(b[i]));
}

void orc_residual_add(uint16_t* a, const uint16_t* b, int64_t n) {
    /* ffn_activations.cu:41-45 */
    for (int64_t i = 0; i < n; ++i) a[i] = orc_f2h(orc_h2f(a[i]) + orc_h2f(b[i]));
}

void orc_silu_mul_quant(const uint16_t* gate, const uint16_t* up,
                        const uint16_t* smooth_inv, const uint16_t* act_scale,
                        int group_size, int8_t* x_q, float* x_scale,
                        uint16_t* out_f16, int n_tokens, int dim) {
    int64_t n = (int64_t)n_tokens * dim;
    uint16_t* h = out_f16 ? out_f16 : (uint16_t*)malloc(sizeof(uint16_t) * ((size_t)n + 1));
    memcpy(h, gate, sizeof(uint16_t) * (size_t)n);
    orc_silu(h, n);
    orc_mul(h, up, n);
    orc_quantize_activations(h, act_scale, smooth_inv, n_tokens, dim, group_size, x_q, x_scale);
    if (!out_f16) free(h);
}


/* ------------------------------------------------- prefill attention ---- */

/* qkv_split_gqa_kernel (src/kernels/prefill_attention.cu:38-57): token-major
 * fused QKV [T, (n_q + 2 n_kv) D] -> head-major q [n_q, T, D], k / v
 * [n_kv, T, D]. */
void orc_qkv_split_gqa(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                       int n_q, int n_kv, int D) {
    const int64_t stride = (int64_t)(n_q + 2 * n_kv) * D;
    for (int t = 0; t < T; ++t) {
        const uint16_t* row = qkv + (int64_t)t * stride;
        for (int h = 0; h < n_q; ++h)
            memcpy(q + ((int64_t)h * T + t) * D, row + (int64_t)h * D, (size_t)D * 2);
        for (int h = 0; h < n_kv; ++h) {
            memcpy(k + ((int64_t)h * T + t) * D, row + (int64_t)(n_q + h) * D, (size_t)D * 2);
            memcpy(v + ((int64_t)h * T + t) * D, row + (int64_t)(n_q + n_kv + h) * D,
                   (size_t)D * 2);
        }
    }
}

/* merge_heads_kernel (prefill_attention.cu:68-86): head-major [H, T, D] ->
 * token-major [T, H * D]. */
void orc_merge_heads(const uint16_t* heads, uint16_t* out, int T, int H, int D) {
    for (int t = 0; t < T; ++t)
        for (int h = 0; h < H; ++h)
            memcpy(out + ((int64_t)t * H + h) * D, heads + ((int64_t)h * T + t) * D,
                   (size_t)D * 2);
}

/* prefill_attention_gpu (src/kernels/prefill_attention.cu:226-322) with its stages:
 *   1. S = Q K^T per head (cublasGemmStridedBatchedEx, fp32 compute, fp16
 *      scores); query head h reads kv head h / (n_q / n_kv)
 *      (gqa_expand_kernel, :118-139).  cuBLAS's summation order is
 *      unspecified; here the fp32 sum runs over d = 0 .. D-1 with FMAs.
 *   2. causal_softmax_kernel (:141-224): v = float(S) * sm_scale for
 *      left <= j <= i (left = i - window + 1 when window > 0, else 0), else
 *      -1e30; mx = max; e = exp(v - mx); sum; P = half(e * (1 / sum)).  exp is
 *      (float)exp(double) and the sum runs in j order (the reference's tree
 *      order is a rounding detail inside the stated tolerance).
 *   3. sgemv_kernel (:325-349): O[i, d] = half(sum_j float(P_ij) * float(V_jd)),
 *      j in order, nvcc contracts into an FMA chain.
 * absw, when non-null, receives sum_j float(P_ij) * |float(V_jd)| (float64)
 * per output, the scale of the tolerance the tests apply. */
void orc_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           uint16_t* out, double* absw, int n_q, int n_kv, int T, int D,
                           float sm_scale, int window) {
    const int gs = n_q / n_kv;
    #pragma omp parallel
    {
        float* qr = (float*)malloc(sizeof(float) * (size_t)D);
        float* srow = (float*)malloc(sizeof(float) * (size_t)T);
        uint16_t* prow = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T);
        #pragma omp for schedule(dynamic) collapse(2)
        for (int h = 0; h < n_q; ++h)
            for (int i = 0; i < T; ++i) {
                const uint16_t* Kh = k + (int64_t)(h / gs) * T * D;
                const uint16_t* Vh = v + (int64_t)(h / gs) * T * D;
                const uint16_t* Qi = q + ((int64_t)h * T + i) * D;
                for (int d = 0; d < D; ++d) qr[d] = orc_h2f(Qi[d]);
                const int left = window > 0 ? i - window + 1 : 0;
                float mx = -1e30f;
                for (int j = 0; j < T; ++j) {
                    float acc = 0.0f;
                    const uint16_t* Kj = Kh + (int64_t)j * D;
                    for (int d = 0; d < D; ++d) acc = fmaf(qr[d], orc_h2f(Kj[d]), acc);
                    float val = orc_h2f(orc_f2h(acc));
                    val = (j <= i && j >= left) ? val * sm_scale : -1e30f;
                    srow[j] = val;
                    if (val > mx) mx = val;
                }
                float sum = 0.0f;
                for (int j = 0; j < T; ++j) {
                    const float e = (float)exp((double)(srow[j] - mx));
                    srow[j] = e;
                    sum += e;
                }
                const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
                for (int j = 0; j < T; ++j) prow[j] = orc_f2h(srow[j] * inv);
                for (int d = 0; d < D; ++d) {
                    float acc = 0.0f;
                    double aw = 0.0;
                    for (int j = 0; j < T; ++j) {
                        const float pj = orc_h2f(prow[j]);
                        const float vj = orc_h2f(Vh[(int64_t)j * D + d]);
                        acc = fmaf(pj, vj, acc);   /* nvcc contracts */
                        aw += (double)pj * fabs((double)vj);
                    }
                    out[((int64_t)h * T + i) * D + d] = orc_f2h(acc);
                    if (absw) absw[((int64_t)h * T + i) * D + d] = aw;
                }
            }
        free(qr);
        free(srow);
        free(prow);
    }
}

/* ------------------------------------------------------------ threads ---- */

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* ------------------------------------------------------- fp16 linear ---- */

void orc_gemm_fp16_exact(const uint16_t* W, const uint16_t* X, double* Y, double* absY,
                         int M, int N, int K) {
    /* gemm_fp16 (dac_engine.cc:19-32): cublasGemmEx, fp16 W [M, K] and X
     * [N, K], CUBLAS_COMPUTE_32F, fp16 Y.  cuBLAS's summation order is not
     * specified, so this oracle gives the value it approximates: the sum in
     * double (every fp16 product is exact in double; K <= 2^20 terms keep the
     * double sum within 2^-32 relative of the exact one), plus sum |w x| for
     * the caller's fp32-accumulation tolerance.  Y and absY are [N, M]. */
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)N * M; ++i) {
        const int n = (int)(i / M), m = (int)(i % M);
        double s = 0.0, a = 0.0;
        for (int k = 0; k < K; ++k) {
            const double p = (double)orc_h2f(W[(int64_t)m * K + k]) *
                             (double)orc_h2f(X[(int64_t)n * K + k]);
            s += p;
            a += fabs(p);
        }
        Y[i] = s;
        absY[i] = a;
    }
}

/*
 * fish_w8a8.h -- C ABI of the MI355X-native W8A8 linear-layer path.
 *
 * Drop-in boundary for fish-audio-cpp's int8 linear layers.  Every entry point
 * takes plain device pointers and sizes, enqueues work on `stream` (a
 * hipStream_t; NULL is the default stream) and returns 0 (FA_OK) or a nonzero
 * fa_status; fa_last_error() then describes the failure for the calling
 * thread.  No entry point synchronises the stream, except that growing the
 * per-thread scratch (see fa_workspace_reserve) waits for `stream` once.
 *
 * Index names follow the reference kernel API (src/kernels/kernels.h:242-259):
 *   M = output features (rows of the int8 weight W [M, K], row-major),
 *   N = tokens,  K = input features.
 *   X  fp16 [N, K] row-major;  Y fp16 col-major [M, N] (= row-major [N, M]).
 *   w_scale fp16 [M] (one group) or [M, G] row-major, G = ceil(K / group_size);
 *   group_size <= 0 or > K means one group of K (int8_gemm.cu:396).
 * fp16 buffers are passed as uint16_t bit patterns.
 */
#ifndef FISH_W8A8_H
#define FISH_W8A8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    FA_OK = 0,
    FA_ERR_INVALID_ARG = 1, /* null pointer, bad size or unsupported shape      */
    FA_ERR_HIP = 2,         /* a HIP runtime call or kernel launch failed        */
    FA_ERR_IO = 3,          /* .bin file could not be opened / mapped            */
    FA_ERR_FORMAT = 4,      /* .bin file is malformed (magic, version, bounds)   */
    FA_ERR_NOT_FOUND = 5    /* tensor name not present in the .bin file          */
} fa_status;

/* Message for the last failing call on this thread ("" if none). */
const char* fa_last_error(void);
/* Library version string. */
const char* fa_version(void);

/* ------------------------------------------------------------------------ */
/* W8A8 linear layer.                                                        */
/* ------------------------------------------------------------------------ */

/* Replaces fish::kernels::int8_dequant_gemm_fp16 (src/kernels/kernels.h:249-259,
 * src/kernels/int8_gemm.cu:384-511): quantize X per (token, K-group) to int8
 * (dynamic amax/127 scales, or the static fp16 act_scale [G] when non-NULL;
 * X * smooth_inv [K] first when non-NULL), exact int32 per-group dot products
 * with W, fp32 dequant-sum over groups, fp16 Y.  The cublasHandle_t argument
 * of the reference has no counterpart. */
int fa_w8a8_gemm(const int8_t* W, const uint16_t* w_scale, int group_size,
                 const uint16_t* act_scale, const uint16_t* smooth_inv,
                 const uint16_t* X, uint16_t* Y, int M, int N, int K, void* stream);

/* Scratch maximum of fa_w8a8_gemm_noalloc, per device (32 MiB). */
#define FA_NOALLOC_SCRATCH_BYTES (32u << 20)

/* No counterpart in the reference: fa_w8a8_gemm for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments as fa_w8a8_gemm, and the
 * reference's results bit for bit, as fa_w8a8_gemm gives them by default;
 * the kernel choice can differ (at 2..16 tokens it always quantizes in a
 * separate launch, and it never splits K even when fa_w8a8_set_k_split has
 * opted fa_w8a8_gemm in).  It never calls hipMalloc / hipFree.  Its scratch
 * (x_q, x_scale and the prefill scale tables, fa_noalloc_scratch_bytes()
 * bytes) lives in one statically sized device array of
 * FA_NOALLOC_SCRATCH_BYTES per device, held until the process ends; shapes
 * needing more fail with FA_ERR_INVALID_ARG (one token on aligned buffers
 * needs none).  Every call on a device shares that device's array: calls
 * that overlap in time on one device (two streams, two threads) race. */
int fa_w8a8_gemm_noalloc(const int8_t* W, const uint16_t* w_scale, int group_size,
                         const uint16_t* act_scale, const uint16_t* smooth_inv,
                         const uint16_t* X, uint16_t* Y, int M, int N, int K, void* stream);
/* Scratch bytes fa_w8a8_gemm_noalloc uses for this shape when it quantizes
 * in a separate launch (an upper bound; (size_t)-1 for bad sizes). */
size_t fa_noalloc_scratch_bytes(int M, int N, int K, int group_size);

/* The FP16 weight path of DualAREngine::quantized_gemm
 * (dual_ar_engine.cc:338-341): gemm_fp16 (dac_engine.cc:19-32), i.e.
 * cublasGemmEx with fp16 W [M, K], fp16 X [N, K], fp16 Y (col-major [M, N],
 * ld = M) and CUBLAS_COMPUTE_32F; used for the tied-embedding logits head
 * (get_logits, dual_ar_engine.cc:663-665).  fp32 accumulation in an order of
 * its own (cuBLAS's is unspecified), fp16 round-to-nearest output.  The
 * cublasHandle_t argument has no counterpart. */
int fa_gemm_fp16(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                 void* stream);

/* Fused prologue + linear for the decode step's attention_norm / ffn_norm
 * projections (src/engine/dual_ar_engine.cc:576-648: residual_add, rms_norm,
 * then int8_dequant_gemm_fp16 on the normalised row).  h = x when resid is
 * NULL, else h = fp16(x + resid) (residual_add, ffn_activations.cu:41-45),
 * written to h_out [N, K] (required with resid, optional without; must not
 * overlap x or resid); then rms_norm(h, gamma, eps) (rms_norm.cu:10-58) feeds
 * fa_w8a8_gemm's quantizer and linear.  Results equal those separate calls
 * bit for bit.  At N == 1 it is one launch: every workgroup of the GEMV forms
 * the normalised, quantized token itself.  No reference counterpart as one
 * call; additive. */
int fa_w8a8_gemm_rms(const int8_t* W, const uint16_t* w_scale, int group_size,
                     const uint16_t* act_scale, const uint16_t* smooth_inv,
                     const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                     const uint16_t* gamma, float eps, uint16_t* Y, int M, int N, int K,
                     void* stream);

/* The FFN's gate and up projections with the SwiGLU product in their
 * epilogue: W13 int8 [2F, K] holds w1 and w3 with rows interleaved (row 2i =
 * w1 row i, row 2i+1 = w3 row i; scales [2F, G] likewise), and act fp16 [N, F]
 * gets fp16(fp16(silu(gate_i)) * up_i) with gate_i, up_i the fp16 outputs of
 * the two linears (dual_ar_engine.cc:640-646: two int8_dequant_gemm_fp16,
 * silu_forward, mul_forward).  gamma non-NULL puts fa_w8a8_gemm_rms's prologue
 * (residual add into h_out, RMSNorm) in front; gamma NULL quantizes x as
 * fa_w8a8_gemm does (resid and h_out must then be NULL).  At N == 1 it is one
 * launch.  Uses that exact input quantization for both halves, so it matches
 * the reference whenever w1 and w3 share it (no per-weight smooth_inv).  No
 * reference counterpart as one call; additive. */
int fa_w8a8_gemm_swiglu(const int8_t* W13, const uint16_t* w13_scale, int group_size,
                        const uint16_t* act_scale, const uint16_t* smooth_inv,
                        const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                        const uint16_t* gamma, float eps, uint16_t* act, int F, int N, int K,
                        void* stream);

/* SwiGLU over separate w1 / w3 weights, each with its own quantization
 * companions -- the layout of a calibrated dual_ar.bin, where w1 and w3 carry
 * different `_smooth_inv` (or `_act_scale`) vectors, so their inputs quantize
 * differently and the two cannot share one interleaved weight
 * (tools/step2_export_w8a8.py:477; the engine's two int8_dequant_gemm_fp16
 * calls, src/engine/dual_ar_engine.cc:640-644, with silu_forward and
 * mul_forward).  act [N, F] = fp16(fp16(silu(gate)) * up) with
 * gate = x' @ w1.T quantized with (act_scale1, smooth_inv1) and
 * up = x' @ w3.T quantized with (act_scale3, smooth_inv3); x' is
 * rms_norm(x (+ resid), gamma) when gamma is non-NULL (h_out then receives
 * x + resid, or x), else x.  W1 / W3 are int8 [F, K] with fp16 scales
 * [F, G] each.  One launch at N == 1 (both quantizations in the GEMV
 * prologue); separate launches otherwise.  No counterpart entry point in the
 * reference. */
int fa_w8a8_gemm_swiglu_sep(const int8_t* W1, const uint16_t* w1_scale, const int8_t* W3,
                            const uint16_t* w3_scale, int group_size,
                            const uint16_t* act_scale1, const uint16_t* smooth_inv1,
                            const uint16_t* act_scale3, const uint16_t* smooth_inv3,
                            const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                            const uint16_t* gamma, float eps, uint16_t* act, int F, int N, int K,
                            void* stream);

/* Fused prologue + linear for the FFN down projection: the quantizer sees
 * fp16(fp16(silu(gate)) * up) (silu_forward then mul_forward,
 * ffn_activations.cu:12-17, 35-39), then fa_w8a8_gemm's quantizer and linear.
 * gate, up: fp16 [N, K].  One launch at N == 1.  No reference counterpart as
 * one call; additive. */
int fa_w8a8_gemm_silu_mul(const int8_t* W, const uint16_t* w_scale, int group_size,
                          const uint16_t* act_scale, const uint16_t* smooth_inv,
                          const uint16_t* gate, const uint16_t* up, uint16_t* Y, int M, int N,
                          int K, void* stream);

/* The same linear layer on activations that are already quantized (X_q int8
 * [N, K] row-major, X_scale fp32 [N, G]): the part of int8_gemm.cu:423-505
 * after its quantizer launch (:415-421).  Used after the fused prologues
 * below. */
int fa_w8a8_gemm_quantized(const int8_t* W, const uint16_t* w_scale, int group_size,
                           const int8_t* X_q, const float* X_scale, uint16_t* Y,
                           int M, int N, int K, void* stream);

/* Opt-in K split for prefill grids with few tiles (no reference
 * counterpart).  By default (max_splits <= 1) every output is the
 * reference's single group-ordered fp32 chain, bit for bit, on every device.
 * With max_splits >= 3 the linear layer may split K over up to max_splits
 * (at most 8) workgroups per 128 x 128 tile on grids with fewer tiles than
 * 256 (2560 outputs at 512 tokens: 80 tiles), each split a partial chain
 * over consecutive whole groups, the partial sums added in split order.  The
 * int32 partials stay exact, the result is deterministic and independent of
 * the device's CU count, but the fp16 output is a reassociation of the
 * reference's chain: within 1 fp16 ulp + 2^-20 sum_g |term_g * x_scale_g| of
 * it, which near-zero outputs (|y| << sum_g |term_g|) can take beyond
 * "1 ulp or rtol 1e-3".  Process-wide; returns the previous setting. */
int fa_w8a8_set_k_split(int max_splits);

/* Number of workgroups the linear layer splits K over for this shape under
 * the current fa_w8a8_set_k_split setting: 1 (always, by default) means the
 * reference's single group-ordered chain, bit for bit; n > 1 as described
 * there.  (16-byte aligned operands assumed; fa_w8a8_gemm_noalloc never
 * splits.) */
int fa_w8a8_gemm_k_splits(int M, int N, int K, int group_size);

/* Decode planning query with no reference counterpart (for tests and
 * tools; no device call): the decode GEMV plan for N <= 16 tokens.  qx: the
 * kernel quantizes fp16 tokens itself; pro: 0 plain, 1 SiLU*mul, 2 residual
 * + RMSNorm prologue (one token); epi: 1 SwiGLU pairs, 2 separate w1 / w3;
 * smooth: a smooth_inv vector comes along.  Returns the kernel kind (0: the
 * shape takes another path; 1, 2: the one-token GEMV with 1 or 2 rows per
 * wave; 3: the 2..16-token MFMA GEMV) and, when out is non-NULL, fills
 * out[0..9] = kind, grid, block, LDS bytes, 64-byte steps per group, groups
 * per wave, terms-in-LDS flag, in-kernel quantization (0/1/2), epilogue, and
 * 1 if the plan meets the kernels' grid and shape assumptions.  This reports
 * the planner's own plan; the entry points drop a plan that fails the check
 * and take their other path (separate quantizer, prefill kernels), counting
 * each such drop in fa_debug_gemv_plan_rejects. */
int fa_debug_gemv_plan(int M, int N, int K, int group_size, int qx, int pro, int epi,
                       int smooth, int* out);

/* Number of decode plans dropped since the library loaded because they
 * failed the kernels' grid and shape assumptions (0 unless the planner has a
 * bug; no reference counterpart, for tests). */
int fa_debug_gemv_plan_rejects(void);

/* Verification hook with no reference counterpart (the reference keeps its
 * int32 partials inside cuBLAS, int8_gemm.cu:476-488): runs exactly the kernel
 * fa_w8a8_gemm_quantized would run for this shape, writes Y, and also writes
 * the exact int32 partial of every (token, row, group) in the window
 * [tok0, tok0+toks) x [row0, row0+rows) to
 * partials[((tok - tok0) * rows + (row - row0)) * G + group]. */
int fa_w8a8_gemm_partials(const int8_t* W, const uint16_t* w_scale, int group_size,
                          const int8_t* X_q, const float* X_scale, uint16_t* Y,
                          int32_t* partials, int row0, int rows, int tok0, int toks,
                          int M, int N, int K, void* stream);

/* ------------------------------------------------------------------------ */
/* Activation quantizer and fused prologues.                                 */
/* ------------------------------------------------------------------------ */

/* quantize_activation_groups_kernel (src/kernels/int8_gemm.cu:147-211):
 * X fp16 [N, K] -> X_q int8 [N, K], X_scale fp32 [N, G]. */
int fa_quantize_activations(const uint16_t* X, const uint16_t* act_scale,
                            const uint16_t* smooth_inv, int8_t* X_q, float* X_scale,
                            int N, int K, int group_size, void* stream);

/* fish::kernels::rms_norm (src/kernels/kernels.h:11-19, rms_norm.cu:60-76). */
int fa_rms_norm(const uint16_t* x, const uint16_t* weight, uint16_t* out,
                int n_tokens, int dim, float eps, void* stream);

/* rms_norm fused with the activation quantizer: the two launches the
 * reference makes before wqkv and w1/w3 (dual_ar_engine.cc:580-583, 636-643)
 * in one kernel.  out (the fp16 normalised rows) may be NULL. */
int fa_rms_norm_quant(const uint16_t* x, const uint16_t* weight, float eps,
                      const uint16_t* smooth_inv, const uint16_t* act_scale, int group_size,
                      int8_t* X_q, float* X_scale, uint16_t* out,
                      int n_tokens, int dim, void* stream);

/* residual_add fused in front of fa_rms_norm_quant: h <- fp16(h + resid) in
 * place (residual_add, ffn_activations.cu:41-45), then the normalised, group-
 * quantized rows of the new h.  Replaces the residual_add, rms_norm and
 * quantizer launches the reference makes between sublayers
 * (dual_ar_engine.cc:632-636, and :647 then :580 of the next layer) with one. */
int fa_residual_rms_norm_quant(uint16_t* h, const uint16_t* resid, const uint16_t* weight,
                               float eps, const uint16_t* smooth_inv, const uint16_t* act_scale,
                               int group_size, int8_t* X_q, float* X_scale, uint16_t* out,
                               int n_tokens, int dim, void* stream);

/* fish::kernels::silu_forward / mul_forward / residual_add
 * (src/kernels/kernels.h:111-140, ffn_activations.cu:139-161), in place on x/a. */
int fa_silu(uint16_t* x, int64_t n, void* stream);
int fa_mul(uint16_t* a, const uint16_t* b, int64_t n, void* stream);
int fa_residual_add(uint16_t* a, const uint16_t* b, int64_t n, void* stream);

/* silu(gate) * up (each rounded to fp16, as silu_forward then mul_forward)
 * fused with the activation quantizer that feeds w2
 * (dual_ar_engine.cc:640-646).  gate/up fp16 [n_tokens, dim]; out (the fp16
 * product) may be NULL. */
int fa_silu_mul_quant(const uint16_t* gate, const uint16_t* up,
                      const uint16_t* smooth_inv, const uint16_t* act_scale, int group_size,
                      int8_t* X_q, float* X_scale, uint16_t* out,
                      int n_tokens, int dim, void* stream);

/* Group-wise symmetric weight quantizer, tools/quant_utils.py:171-194
 * quantize_groupwise, on the device: fp16 w [rows, K] -> int8 q [rows, K],
 * fp16 scale [rows, G] (G = ceil(K / group_size), group_size > 0). */
int fa_quantize_weights_groupwise(const uint16_t* w, int64_t rows, int64_t K, int group_size,
                                  int8_t* q, uint16_t* scale, void* stream);

/* ------------------------------------------------------------------------ */
/* Prefill attention side: the neighbours of the wqkv and wo linears.        */
/* ------------------------------------------------------------------------ */

/* fish::kernels::qkv_split_heads_gqa (src/kernels/kernels.h:338-341,
 * prefill_attention.cu:38-66): fused QKV fp16 [T, (n_q + 2 n_kv) head_dim]
 * (the wqkv output) -> head-major q [n_q, T, head_dim], k / v
 * [n_kv, T, head_dim]. */
int fa_qkv_split_heads_gqa(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                           int n_q, int n_kv, int head_dim, void* stream);
/* fish::kernels::qkv_split_heads (kernels.h:335-336, prefill_attention.cu:14-36):
 * the n_kv == n_heads case. */
int fa_qkv_split_heads(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                       int n_heads, int head_dim, void* stream);
/* fish::kernels::merge_heads (kernels.h:343-344, prefill_attention.cu:68-86):
 * head-major [n_heads, T, head_dim] -> token-major [T, n_heads head_dim]
 * (the wo input). */
int fa_merge_heads(const uint16_t* heads, uint16_t* out, int T, int n_heads, int head_dim,
                   void* stream);
/* fish::kernels::prefill_attention_gpu (kernels.h:324-333,
 * prefill_attention.cu:226-349): causal GQA attention, query head h reading
 * KV head h / (n_q / n_kv); window_size > 0 limits query i to keys
 * i - window_size + 1 .. i.  q / out [n_q, T, D], k / v [n_kv, T, D], fp16,
 * head-major; n_q % n_kv == 0; D <= 512; any finite sm_scale.  The fused
 * kernel serves D % 8 == 0, D <= 128, sm_scale > 0 and 16-byte aligned
 * buffers; anything else runs an exact-order any-shape kernel (slower).
 * Either way the T x T scores stay on chip, so `workspace` is not used (it may be NULL; the reference's cuBLAS handle has no
 * counterpart).  Results agree with the reference within the order of fp32
 * sums (scores are rounded to fp16 before scaling, probabilities enter the V
 * product as fp16). */
int fa_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out,
                         void* workspace, int n_q, int n_kv, int T, int D, float sm_scale,
                         void* stream, int window_size);
/* prefill_attention_gpu followed by merge_heads (dual_ar_engine.cc:499-502),
 * as one launch: the same attention, written token-major, out [T, n_q D]
 * (bit-identical to fa_prefill_attention then fa_merge_heads).  Additive: no
 * single reference counterpart. */
int fa_prefill_attention_merged(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                                void* stream, int window_size);

/* ------------------------------------------------------------------------ */
/* Decode chain: a sequence of one-token W8A8 linears as one launch.          */
/* ------------------------------------------------------------------------ */

/* One linear of a chain.  Step s reads what step s - 1 (and earlier steps)
 * wrote; the device runs the steps in order, but each step's weight loads
 * start before the previous step has finished.  Results are bit-identical to
 * the per-linear entry points:
 *   prologue 0 = fa_w8a8_gemm at N = 1 (dynamic per-group quantization);
 *   prologue 2 = fa_w8a8_gemm_rms at N = 1 (h = x + x2 when x2 is given,
 *                RMSNorm with gamma and eps, quantization; h goes to h_out
 *                when given);
 *   epilogue 1 = fa_w8a8_gemm_swiglu's pair epilogue (rows 2i / 2i + 1 are the
 *                interleaved w1 / w3 rows; y[i] = silu(gate) * up, m / 2
 *                values).
 * No act_scale / smooth_inv: the chain serves the dynamic-quantization
 * decode path.  x, x2, gamma, h_out and w must be 16-byte aligned, y 4-byte
 * aligned; k a multiple of 16, at least group_size, at most 12288 (4096 with
 * prologue 2); y and h_out must not overlap the same step's inputs. */
typedef struct {
    const int8_t* w;            /* [m, k] int8, row-major                        */
    const uint16_t* w_scale;    /* [m, ceil(k / group_size)] fp16                */
    const uint16_t* x;          /* [k] fp16 input (prologue 2: residual stream)  */
    const uint16_t* x2;         /* prologue 2: residual addend [k], or NULL      */
    const uint16_t* gamma;      /* prologue 2: RMSNorm weight [k]                */
    uint16_t* h_out;            /* prologue 2: h = x + x2 written here, or NULL  */
    uint16_t* y;                /* [m] fp16 (epilogue 0) or [m / 2] (epilogue 1)  */
    int m, k;
    int prologue;               /* 0 or 2 (see above)                            */
    int epilogue;               /* 0 or 1 (see above)                            */
    float eps;                  /* prologue 2: RMSNorm epsilon                   */
} fa_chain_step;

typedef struct fa_chain fa_chain;

/* The per-layer launch sequence of DualAREngine::decode_step
 * (dual_ar_engine.cc:576-648) -- rms_norm + quantize + int8 GEMV per
 * projection, launch by launch -- as a device-ordered chain.  Validates the
 * steps and uploads the step table (allocates device memory: call once,
 * outside a capture).  All steps share group_size (64, 128 or 256). */
int fa_chain_create(const fa_chain_step* steps, int n_steps, int group_size, fa_chain** out);
/* Run the chain on `stream`: a small kernel that zeroes the step counters,
 * then one ordinary launch of one workgroup per CU (576 threads, one per CU
 * by its LDS use).  No allocation, no host sync.
 * The launch is not cooperative: the steps order themselves through device
 * counters, which assumes every workgroup of the grid is resident at once.
 * That holds on an otherwise idle device; kernels running concurrently on
 * other streams can keep workgroups from starting.  Every wait is bounded
 * (fa_chain_set_spin_limit), so the kernel always finishes; when a wait gave
 * up, fa_chain_status reports FA_ERR_HIP and the outputs of that run are
 * incomplete (run it again, or take the per-linear entry points).
 * Runs on one stream at a time: overlapping runs of one chain race.
 * Experimental: measured slower than the four fused launches per layer
 * (fa_w8a8_gemm_rms / _swiglu / fa_w8a8_gemm) and limited to dynamic
 * quantization, so the engine path is those entry points. */
int fa_chain_run(fa_chain* chain, void* stream);
/* Wait for `stream`, then report whether the last run finished: FA_ERR_HIP
 * when a step's wait for its predecessor gave up (spin limit reached), in
 * which case the outputs are incomplete. */
int fa_chain_status(fa_chain* chain, void* stream);
/* Upper bound on the polls of one wait (default 1 << 21); testing hook. */
int fa_chain_set_spin_limit(fa_chain* chain, int polls);
int fa_chain_destroy(fa_chain* chain);

/* ------------------------------------------------------------------------ */
/* Scratch.                                                                  */
/* ------------------------------------------------------------------------ */

/* Pre-size this thread's scratch on the current device for calls up to the
 * given shape, so later calls never allocate (the reference grows its
 * thread_local workspace with cudaMalloc inside the call,
 * int8_gemm.cu:31-44, 97-102, 405-413).  Calls on one thread share the
 * scratch: calls from one thread on two streams that overlap in time race. */
int fa_workspace_reserve(int max_tokens, int max_M, int max_K, int min_group_size,
                         void* stream);
/* (max_M counts rows as the linears see them: 2F for fa_w8a8_gemm_swiglu.) */
/* Release this thread's scratch on the current device (waits for the device). */
int fa_workspace_release(void);

/* ------------------------------------------------------------------------ */
/* Per-shape timing (src/kernels/int8_gemm.cu:45-145, FISH_INT8_PROFILE).    */
/* ------------------------------------------------------------------------ */

/* With FISH_INT8_PROFILE set to a non-empty value other than "0", or after
 * fa_profile_enable(1), each call of fa_w8a8_gemm, fa_w8a8_gemm_rms,
 * fa_w8a8_gemm_swiglu and fa_w8a8_gemm_silu_mul is timed with events on its
 * stream and waited for (so profiling serialises the caller, as the
 * reference's does); times accumulate per (entry, M, N, K, group size,
 * static / dynamic activation scales, smooth_inv) and are printed to stderr
 * at process exit, as "quant" (a separate quantization launch) and "gemm"
 * (everything else).  Calls on a stream under graph capture are not timed.
 * fa_profile_enable returns the previous setting. */
int fa_profile_enable(int on);
/* Copies the summary text (at most n - 1 bytes and a NUL) into buf and
 * returns its full length; buf may be NULL to query the length. */
size_t fa_profile_summary(char* buf, size_t n);
/* Clears the accumulated times. */
void fa_profile_reset(void);

/* ------------------------------------------------------------------------ */
/* dual_ar.bin container (src/model/tensor.h:8-67, src/model/loader.cc).     */
/* ------------------------------------------------------------------------ */

typedef struct fa_bin fa_bin;

typedef struct {
    char name[256];
    uint32_t dtype;      /* 0 FP32, 1 FP16, 2 BF16, 3 INT8 (tensor.h:8-13) */
    uint32_t ndim;
    int64_t shape[8];
    uint64_t offset;     /* byte offset of the data in the file */
    uint64_t size;       /* byte count of the data */
    const void* data;    /* host pointer into the read-only mapping */
} fa_tensor_info;

/* Companions of one int8 weight, as DualAREngine::init finds them
 * (src/engine/dual_ar_engine.cc:231-275): <w>_scale, <w>_smooth_inv and
 * <w>_act_scale; group_size inferred from the scale shape (:17-24). */
typedef struct {
    int has_scale, has_smooth_inv, has_act_scale;
    int group_size;      /* 0 when the weight has no scale (fp16 weight) */
    int64_t M, K;        /* weight rows and row length */
    int64_t groups;      /* G as stored in the scale tensor */
} fa_quant_meta;

/* ModelLoader::load (loader.cc:50-152): mmap + header parse.  Also checks that
 * every tensor's data lies inside the file. */
int fa_bin_open(const char* path, fa_bin** out);
void fa_bin_close(fa_bin* bin);
int fa_bin_num_tensors(const fa_bin* bin);
int fa_bin_tensor_at(const fa_bin* bin, int index, fa_tensor_info* info);
/* ModelLoader::get / has (loader.cc:155-170); FA_ERR_NOT_FOUND if absent. */
int fa_bin_find(const fa_bin* bin, const char* name, fa_tensor_info* info);
int fa_bin_quant_meta(const fa_bin* bin, const char* weight_name, fa_quant_meta* meta);
/* The FFN's w1 and w3 (feed_forward.w1 / .w3, with their _scale companions)
 * as one row-interleaved int8 weight for fa_w8a8_gemm_swiglu: row 2i = w1 row
 * i, row 2i+1 = w3 row i, scales likewise ([2F] or [2F, G]), on the host.
 * Replaces the two separate uploads DualAREngine::init makes
 * (dual_ar_engine.cc:194-278) when both halves share one input quantization:
 * FA_ERR_INVALID_ARG when only one has a _smooth_inv / _act_scale or theirs
 * differ (then the reference's two quantized_gemm calls see different int8
 * inputs and cannot be fused).  w13 (2F * K bytes) and s13 may be NULL to
 * only check and fill meta (M = 2F). */
int fa_bin_gate_up(const fa_bin* bin, const char* w1_name, const char* w3_name, int8_t* w13,
                   uint16_t* s13, fa_quant_meta* meta);
/* infer_group_size_from_scale (dual_ar_engine.cc:17-24). */
int fa_infer_group_size(int64_t K, int scale_ndim, int64_t scale_groups);

#ifdef __cplusplus
}
#endif
#endif

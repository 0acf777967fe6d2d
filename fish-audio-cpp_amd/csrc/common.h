// common.h -- shared device helpers and launcher declarations for the W8A8 path.
//
// Conventions (kept from the reference kernel API, src/kernels/kernels.h:242-259):
//   M = output features (rows of the int8 weight W [M, K], row-major),
//   N = tokens (X [N, K] row-major fp16), Y is col-major [M, N] = row-major
//   [N tokens, M].  Weight scales are fp16 [M] (one group) or [M, G] row-major.
//   Activation scales are fp32 [N, G] row-major, X_q int8 [N, K] row-major.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace fa {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
// Round-to-nearest-even fp32 -> fp16 (v_cvt_f16_f32 under the default mode).
// The empty asm pins `f` as an fp32 register value: without it the backend
// folds `f2h(a * b)` into v_fma_mixlo_f16, which rounds the product once,
// straight to fp16, instead of to fp32 and then to fp16 as the reference's
// `__float2half(a * b)` does.
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __half_as_ushort(__float2half(f));
}

// Activation quantization of one value given 1/scale, as the reference
// quantizer does it (src/kernels/int8_gemm.cu:202-209): RN-even, clamp +-127.
__device__ __forceinline__ int quant_rn(float v, float inv) {
    float t = __builtin_rintf(v * inv);
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    return (int)t;
}

// Dynamic scale from a group max (int8_gemm.cu:197-198) or a static scale
// (:185-186): both clamped below at 1e-8.
__device__ __forceinline__ float act_scale_from_amax(float amax) {
    float s = amax / 127.0f;
    return s < 1e-8f ? 1e-8f : s;
}

// Wave64 max/sum over lane subgroups of width W (a power of two <= 64).
template <int W>
__device__ __forceinline__ float subgroup_max(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// DPP move of a float within 16-lane rows (bound_ctrl off: lanes with no
// source read 0).
template <int CTL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTL, 0xF, 0xF, false));
}

// The shuffle-down sum tree of a 32-lane CUDA warp (offsets 16, 8, 4, 2, 1,
// `v += __shfl_down(v, off)`), on each 32-lane half of the wave.  Lane 0 of
// each half gets exactly the reference's pairing (rms_norm.cu:29-41): the
// cross-row step is a shuffle, the in-row steps are DPP row_shl (lane i reads
// lane i + off; lanes past the row end read 0, and their sums are never used).
__device__ __forceinline__ float warp32_sum_down(float v) {
    v += __shfl_down(v, 16, 32);
    v += dpp_f<0x108>(v);   // row_shl:8
    v += dpp_f<0x104>(v);   // row_shl:4
    v += dpp_f<0x102>(v);   // row_shl:2
    v += dpp_f<0x101>(v);   // row_shl:1
    return v;
}

// Reference SiLU (src/kernels/ffn_activations.cu:15) with expf replaced by a
// double-precision exp rounded to float; the division is IEEE.
__device__ __forceinline__ float silu_f(float v) {
    float e = (float)exp(-(double)v);
    return v / (1.0f + e);
}

// RMSNorm scale 1/sqrt(sum_sq / dim + eps) (rms_norm.cu:44), rsqrtf replaced
// by a double-precision 1/sqrt rounded to float.
__device__ __forceinline__ float rms_inv(float sum_sq, int dim, float eps) {
    const float t = sum_sq / (float)dim + eps;
    return (float)(1.0 / sqrt((double)t));
}

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace fa

// ---------------------------------------------------------------------------
// Launchers (host functions, one per kernel family).  They validate nothing:
// the C-ABI layer (api.cpp) checks shapes and alignment before calling them.
// Each returns the hipError_t of the launch.
// ---------------------------------------------------------------------------
namespace fa {

// Prologue kinds for the activation quantizer.
enum class Prologue : int { kPlain = 0, kSiluMul = 1 };

hipError_t launch_quantize_activations(const uint16_t* X, const uint16_t* up, Prologue kind,
                                       const uint16_t* act_scale, const uint16_t* smooth_inv,
                                       int8_t* x_q, float* x_scale, uint16_t* out_f16,
                                       int N, int K, int g, int G, hipStream_t stream);

// Normalises h = fp16(x + resid) (resid non-null; h_out required) or h = x,
// storing h to h_out when non-null (h_out == x updates x in place).
hipError_t launch_rms_norm_quant(const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                                 const uint16_t* weight,
                                 float eps,
                                 const uint16_t* smooth_inv, const uint16_t* act_scale,
                                 int g, int G, int8_t* x_q, float* x_scale, uint16_t* out_f16,
                                 int n_tokens, int dim, hipStream_t stream);

hipError_t launch_elementwise(int op, uint16_t* a, const uint16_t* b, int64_t n,
                              hipStream_t stream);

// act[i] = fp16(fp16(silu(y[2i])) * y[2i + 1]) for i < n (interleaved pairs).
hipError_t launch_swiglu_pairs(const uint16_t* y, uint16_t* act, int64_t n, hipStream_t stream);

hipError_t launch_quantize_weights(const uint16_t* w, int64_t rows, int64_t K, int g,
                                   int8_t* q, uint16_t* scale, hipStream_t stream);

// Decode GEMV (N <= 16 tokens): a v_dot4 kernel for N == 1 and an int8 MFMA
// kernel for 2 <= N <= 16.  kind == 0 means "shape not taken".
// Compute units of the current device (0 if the query fails); cached per
// device.
int device_cus();

struct GemvPlan {
    int kind = 0;    // 1, 2: dot kernel with 1 or 2 rows per wave; 3: MFMA kernel
                     // (dot: grid = row blocks)
    int kd = 0;      // dot: passes in flight per wave
    int lg = 0;      // dot: log2(group size)
    int passes = 0;  // dot: passes per row
    int spg = 0;     // mfma: 64-byte K steps per group
    int maxg = 0;    // mfma: groups per wave
    bool lc = false; // mfma: all terms in LDS, one chain lane per output
    int pro = 0;     // dot with in-kernel quantization: fused prologue (0 plain,
                     // 1 SiLU*mul, 2 residual + RMSNorm)
    int epi = 0;     // 1 = SwiGLU pair epilogue (rows interleaved w1 / w3; dot and
                     // mfma), 2 = the same on separate w1 / w3 quantized apart (dot)
    int qx = 0;      // mfma: quantizes the fp16 tokens in-kernel (1; 2 with smooth_inv)
    int grid = 0, block = 0;
    size_t lds = 0;
};
// qx: the kernel quantizes the fp16 tokens itself (N == 1: the dot kernel;
// 2 <= N <= 16: the MFMA kernel when the wave's K range fits its registers,
// `smooth` telling whether a smooth_inv vector comes along), else the plan is
// empty; pro != 0 adds a fused prologue in front of that quantizer (N == 1,
// K <= 12288, K % 8 == 0).
// epi == 1 plans the SwiGLU pair epilogue (M even; N == 1: two rows per
// wave, pro 0 or 2; N > 1: staged or in-kernel quantized tokens): Y [N][M / 2]
// gets fp16(fp16(silu(row 2i)) * row 2i+1).
// A plan that fails gemv_plan_valid is never returned: plan_gemv counts it
// (gemv_plan_rejects) and returns kind 0, so the caller takes its other path.
GemvPlan plan_gemv(int M, int N, int K, int g, int G, bool qx, int pro = 0, int epi = 0,
                   bool smooth = false);
// The planner itself, before that check (the planning query reports its
// plan and whether the check passes).
GemvPlan plan_gemv_raw(int M, int N, int K, int g, int G, bool qx, int pro = 0, int epi = 0,
                       bool smooth = false);
int gemv_plan_rejects();
// The grid and shape assumptions of the decode kernels, checked by
// plan_gemv on every plan and again by launch_gemv before every launch.
bool gemv_plan_valid(const GemvPlan& p, int M, int N, int K, int g, int G);
// Debug window: when dbg_partials is non-null the kernels also write the exact
// int32 partial of every (token, row, group) inside
// [dbg_tok0, +dbg_toks) x [dbg_row0, +dbg_rows) to
// dbg_partials[((tok - dbg_tok0) * dbg_rows + (row - dbg_row0)) * G + group].
// With X non-null (dot kernel only) the kernel quantizes the fp16 token X
// itself (act_scale / smooth_inv as in launch_quantize_activations) and
// ignores x_q / x_scale.  With p.pro == 1, X is the gate and x2 the up
// projection (SiLU * mul first); with p.pro == 2, X is the residual stream, x2
// the residual addend (nullable), gamma / eps the RMSNorm, and h_out
// (nullable; must not overlap X or x2) receives fp16(X + x2).
hipError_t launch_gemv(const GemvPlan& p, const int8_t* W, const uint16_t* w_scale,
                       const int8_t* x_q, const float* x_scale, const uint16_t* X,
                       const uint16_t* act_scale, const uint16_t* smooth_inv, uint16_t* Y,
                       int32_t* dbg_partials, int dbg_row0, int dbg_rows, int dbg_tok0,
                       int dbg_toks, int M, int N, int K, int g, int G, hipStream_t stream,
                       const uint16_t* x2 = nullptr, const uint16_t* gamma = nullptr,
                       float eps = 0.0f, uint16_t* h_out = nullptr,
                       const int8_t* w3 = nullptr, const uint16_t* w3_scale = nullptr,
                       const uint16_t* act_scale3 = nullptr,
                       const uint16_t* smooth_inv3 = nullptr);

// Prefill GEMM on int8 MFMA with LDS-staged tiles.
hipError_t launch_gemm(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                       const float* x_scale, uint16_t* Y, int32_t* dbg_partials, int dbg_row0,
                       int dbg_rows, int dbg_tok0, int dbg_toks, int M, int N, int K, int g, int G,
                       hipStream_t stream);

// Prefill GEMM with a direct-to-LDS multi-stage pipeline (K % 256 == 0,
// g % 64 == 0).
bool gemm_pipe_ok(int M, int N, int K, int g);
// Scratch the pipelined GEMM needs for its group-major scale tables.
size_t gemm_pipe_tables_bytes(int M, int N, int G);
// Two launches: the scale tables into `tables`, then the GEMM.
hipError_t launch_gemm_pipe(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                            const float* x_scale, float* tables, uint16_t* Y, int32_t* dbg_partials,
                            int dbg_row0, int dbg_rows, int dbg_tok0, int dbg_toks, int M, int N,
                            int K, int g, int G, hipStream_t stream);

// Prefill tile kernel: g in {64, 128, 256}, K % 256 == 0; same scale tables
// (gemm_pipe_tables_bytes) and the same two launches as launch_gemm_pipe.
bool gemm_tile_ok(int M, int N, int K, int g);
// variant: 0 = by shape (gemm_tile_choice), 1 = 256 x 128 tiles, 2 = 128 x 128.
// scales: -1 = by group size, 0 = group-major tables (extra launch), 1 = gathered
// in-kernel from the given layouts.
int gemm_tile_choice(int M, int N, int K, int g);
// K split over nsplit workgroups per tile (1 = none) for grids with few tiles;
// the split needs gemm_tile_split_bytes of partial sums plus one zeroed int
// counter per tile (left zeroed by every launch).
int gemm_tile_split(int M, int N, int K, int g, int variant = 0);
int set_k_split(int max_splits);   // process-wide cap; returns the previous one
size_t gemm_tile_split_bytes(int M, int N, int variant, int nsplit);
hipError_t launch_gemm_tile(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                            const float* x_scale, float* tables, uint16_t* Y, int32_t* dbg_partials,
                            int dbg_row0, int dbg_rows, int dbg_tok0, int dbg_toks, int M, int N,
                            int K, int g, int G, hipStream_t stream, int variant = 0,
                            int scales = -1, int nsplit = 1, float* part = nullptr,
                            int* tile_cnt = nullptr);

// fp16 x fp16 -> fp16 linear with fp32 accumulation (the FP16 weight path):
// a streaming GEMV for K % 8 == 0, K <= 4096 and 16-byte aligned W / X
// (tokens in chunks of up to 8, each chunk reads W once), and an any-shape
// kernel (N <= 65535).
bool gemv_f16_ok(int M, int N, int K);
hipError_t launch_gemv_f16(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N, int K,
                           hipStream_t stream);
hipError_t launch_gemm_f16_generic(const uint16_t* W, const uint16_t* X, uint16_t* Y, int M, int N,
                                   int K, hipStream_t stream);

// Prefill attention side (attn.hip).  attention_padded_dim gives the head dim
// the fused attention kernel is instantiated for (32, 64 or 128), 0 if D > 128.
int attention_padded_dim(int D);
int attention_max_dim();   // head dims above it are rejected
hipError_t launch_prefill_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                    uint16_t* out, int n_q, int n_kv, int T, int D, float sm_scale,
                                    int window, bool token_major,
                                    hipStream_t stream);
hipError_t launch_qkv_split(const uint16_t* qkv, uint16_t* q, uint16_t* k, uint16_t* v, int T,
                            int n_q, int n_kv, int D, bool vec, hipStream_t stream);
hipError_t launch_merge_heads(const uint16_t* heads, uint16_t* out, int T, int H, int D, bool vec,
                              hipStream_t stream);

// Any-shape fallback (any K, any group size, unaligned pointers).
hipError_t launch_gemm_generic(const int8_t* W, const uint16_t* w_scale, const int8_t* x_q,
                               const float* x_scale, uint16_t* Y, int32_t* dbg_partials,
                               int dbg_row0, int dbg_rows, int dbg_tok0, int dbg_toks, int M,
                               int N, int K, int g, int G, hipStream_t stream);

}  // namespace fa

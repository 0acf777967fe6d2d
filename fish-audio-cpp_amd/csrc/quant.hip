// quant.hip -- activation quantizer (plain / SiLU*mul prologue), fused
// RMSNorm+quant, fp16 elementwise ops and the group-wise weight quantizer.
//
// All of these are HBM-bound byte/halfword streams: one pass over the input,
// 16-byte loads per lane where the shape allows, group maxima reduced inside
// lane subgroups with cross-lane shuffles (max is order-independent, so the
// reductions are exact), no LDS round trip except in the fused RMSNorm, whose
// normalised row is staged in LDS between the norm and the quantizer.
#include "common.h"

namespace fa {
namespace {

constexpr int kThreads = 256;


// Load VEC consecutive fp16 values (16-byte load when VEC == 8).
template <int VEC>
__device__ __forceinline__ void load_h(const uint16_t* p, uint16_t (&h)[VEC]) {
    if constexpr (VEC == 8) {
        uint4 u = *reinterpret_cast<const uint4*>(p);
        const uint16_t* s = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
        for (int i = 0; i < 8; ++i) h[i] = s[i];
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) h[i] = p[i];
    }
}

template <int VEC>
__device__ __forceinline__ void store_q(int8_t* p, const int (&q)[VEC]) {
    if constexpr (VEC == 8) {
        uint2 u;
        u.x = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
              ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
        u.y = (uint32_t)(q[4] & 0xff) | ((uint32_t)(q[5] & 0xff) << 8) |
              ((uint32_t)(q[6] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24);
        *reinterpret_cast<uint2*>(p) = u;
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) p[i] = (int8_t)q[i];
    }
}

template <int VEC>
__device__ __forceinline__ void store_h(uint16_t* p, const uint16_t (&h)[VEC]) {
    if constexpr (VEC == 8) {
        uint4 u;
        uint16_t* d = reinterpret_cast<uint16_t*>(&u);
#pragma unroll
        for (int i = 0; i < 8; ++i) d[i] = h[i];
        *reinterpret_cast<uint4*>(p) = u;
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) p[i] = h[i];
    }
}


// Runtime-width subgroup max (width = 1 << lg, lg <= 6; all lanes get it);
// every lane of the wave must call it.  Within 16-lane rows one DPP op per
// step, across rows xor shuffles.  The max is exact in any order.
__device__ __forceinline__ float subgroup_max_rt(float v, int lg) {
    if (lg >= 1) v = fmaxf(v, dpp_f<0xB1>(v));    // quad_perm [1,0,3,2]
    if (lg >= 2) v = fmaxf(v, dpp_f<0x4E>(v));    // quad_perm [2,3,0,1]
    if (lg >= 3) v = fmaxf(v, dpp_f<0x141>(v));   // row_half_mirror
    if (lg >= 4) v = fmaxf(v, dpp_f<0x140>(v));   // row_mirror
    if (lg >= 5) v = fmaxf(v, __shfl_xor(v, 16, 64));
    if (lg >= 6) v = fmaxf(v, __shfl_xor(v, 32, 64));
    return v;
}


// Values entering the quantizer for elements [k, k+VEC) of token row `n`:
// the prologue output rounded to fp16 (what the reference writes to memory
// before its quantizer reads it back), times smooth_inv when present.
template <int VEC, Prologue P>
__device__ __forceinline__ void prologue_values(const uint16_t* X, const uint16_t* up,
                                                const uint16_t* smooth_inv, size_t off, int k,
                                                float (&v)[VEC], uint16_t (&h)[VEC]) {
    load_h<VEC>(X + off, h);
    if constexpr (P == Prologue::kSiluMul) {
        uint16_t u[VEC];
        load_h<VEC>(up + off, u);
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            // silu_forward (ffn_activations.cu:12-17) then mul_forward (:35-39),
            // each rounding to fp16.
            uint16_t s = f2h(silu_f(h2f(h[i])));
            h[i] = f2h(h2f(s) * h2f(u[i]));
        }
    }
    if (smooth_inv) {
        uint16_t sm[VEC];
        load_h<VEC>(smooth_inv + k, sm);
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] = h2f(h[i]) * h2f(sm[i]);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] = h2f(h[i]);
    }
}

// One lane subgroup of width 2^lg quantizes one (token, group) pair; a lane
// handles VEC consecutive elements per iteration.  Restates
// quantize_activation_groups_kernel (src/kernels/int8_gemm.cu:147-211).
template <int VEC, Prologue P>
__global__ __launch_bounds__(kThreads) void quantize_act_kernel(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ act_scale, const uint16_t* __restrict__ smooth_inv,
    int8_t* __restrict__ x_q, float* __restrict__ x_scale, uint16_t* __restrict__ out_f16,
    int N, int K, int g, int G, int lg) {
    const int lanes = 1 << lg;
    const long slot = ((long)blockIdx.x * kThreads + threadIdx.x) >> lg;
    const int sub = threadIdx.x & (lanes - 1);
    const bool active = slot < (long)N * G;
    const int n = active ? (int)(slot / G) : 0;
    const int gi = active ? (int)(slot % G) : 0;
    const int k0 = gi * g;
    const int k1 = active ? min(k0 + g, K) : k0;
    const size_t row = (size_t)n * K;

    if (g <= lanes * VEC) {
        // one VEC chunk per lane covers the group: the prologue values are
        // formed once and kept in registers for the max and the codes
        const int k = k0 + sub * VEC;
        const bool ok = k < k1;
        float v[VEC];
        uint16_t h[VEC];
        if (ok) {
            prologue_values<VEC, P>(X, up, smooth_inv, row + k, k, v, h);
        } else {
#pragma unroll
            for (int i = 0; i < VEC; ++i) v[i] = 0.0f;
        }
        float s;
        if (act_scale) {
            s = h2f(act_scale[gi]);
            s = s < 1e-8f ? 1e-8f : s;
        } else {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(v[i]));
            amax = subgroup_max_rt(amax, lg);
            s = act_scale_from_amax(amax);
        }
        if (active && sub == 0) x_scale[(size_t)n * G + gi] = s;
        if (ok) {
            const float inv = 1.0f / s;
            int q[VEC];
#pragma unroll
            for (int i = 0; i < VEC; ++i) q[i] = quant_rn(v[i], inv);
            store_q<VEC>(x_q + row + k, q);
            if (P == Prologue::kSiluMul && out_f16) store_h<VEC>(out_f16 + row + k, h);
        }
        return;
    }

    float s;
    if (act_scale) {
        s = h2f(act_scale[gi]);
        s = s < 1e-8f ? 1e-8f : s;
    } else {
        float amax = 0.0f;
        for (int k = k0 + sub * VEC; k < k1; k += lanes * VEC) {
            float v[VEC];
            uint16_t h[VEC];
            prologue_values<VEC, P>(X, up, smooth_inv, row + k, k, v, h);
#pragma unroll
            for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(v[i]));
        }
        amax = subgroup_max_rt(amax, lg);
        s = act_scale_from_amax(amax);
    }
    if (active && sub == 0) x_scale[(size_t)n * G + gi] = s;
    const float inv = 1.0f / s;
    for (int k = k0 + sub * VEC; k < k1; k += lanes * VEC) {
        float v[VEC];
        uint16_t h[VEC];
        prologue_values<VEC, P>(X, up, smooth_inv, row + k, k, v, h);
        int q[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) q[i] = quant_rn(v[i], inv);
        store_q<VEC>(x_q + row + k, q);
        if (P == Prologue::kSiluMul && out_f16) store_h<VEC>(out_f16 + row + k, h);
    }
}

int lanes_log2_for(int g, int vec) {
    int need = (g + vec - 1) / vec;
    int lg = 0;
    while ((1 << lg) < need && lg < 6) ++lg;
    return lg;
}

// ------------------------------------------------------------ RMSNorm ----

// rms_norm_kernel (src/kernels/rms_norm.cu:10-58) with the same reduction
// order: thread t < T (T = min(next_pow2(dim), 1024), rms_norm.cu:69-70) sums
// x[t], x[t+T], ... with FMAs (nvcc contracts `local_sum += val * val`); each
// 32-lane half-wave reduces by the shuffle-down tree of a CUDA warp; the warp
// sums are reduced by the same tree.  rsqrtf is replaced by a double 1/sqrt.
// The normalised fp16 row is then quantized per K-group straight from LDS.
__global__ __launch_bounds__(1024) void rms_norm_quant_kernel(
    const uint16_t* x, const uint16_t* __restrict__ resid, uint16_t* h_out,
    const uint16_t* __restrict__ weight, float eps,
    const uint16_t* __restrict__ smooth_inv, const uint16_t* __restrict__ act_scale,
    int8_t* __restrict__ x_q, float* __restrict__ x_scale, uint16_t* __restrict__ out_f16,
    int dim, int T, int g, int G, int lg, int vec8) {
    extern __shared__ __align__(16) uint16_t s_row[];  // dim fp16 values
    __shared__ float s_warp[32];
    __shared__ float s_rms;
    const int tid = threadIdx.x;
    const size_t base = (size_t)blockIdx.x * dim;

    // Thread t holds x[t], x[t + T], ... (at most kNV of them when
    // dim <= kNV * T, else the loop re-reads x); all its loads, gamma's
    // included, go out before the first use, so the row costs one memory
    // latency.  With `resid` the row normalised is h = fp16(x + resid)
    // (residual_add, ffn_activations.cu:41-45), else h = x; h is stored to
    // h_out when h_out is non-null (required with resid; h_out may equal x,
    // an in-place update).
    constexpr int kNV = 8;
    const bool regs = dim <= kNV * T;
    float xv[kNV], gv[kNV];
    if (regs) {
        uint16_t xr[kNV], rr[kNV], gr[kNV];
#pragma unroll
        for (int j = 0; j < kNV; ++j) {
            const int i = min(tid + j * T, dim - 1);
            xr[j] = x[base + i];
            gr[j] = weight[i];
            if (resid) rr[j] = resid[base + i];
        }
#pragma unroll
        for (int j = 0; j < kNV; ++j) {
            xv[j] = h2f(xr[j]);
            uint16_t hs = xr[j];
            if (resid) {
                hs = f2h(xv[j] + h2f(rr[j]));
                xv[j] = h2f(hs);
            }
            if (h_out && tid < T && tid + j * T < dim) h_out[base + tid + j * T] = hs;
            gv[j] = h2f(gr[j]);
        }
    } else if (h_out) {
        for (int i = tid; i < dim; i += blockDim.x)
            h_out[base + i] = resid ? f2h(h2f(x[base + i]) + h2f(resid[base + i])) : x[base + i];
        __syncthreads();
    }
    const uint16_t* hrow = resid ? h_out : x;  // h, where the re-reading paths find it

    float local = 0.0f;
    if (tid < T) {
        if (regs) {
#pragma unroll
            for (int j = 0; j < kNV; ++j)
                if (tid + j * T < dim) local = __builtin_fmaf(xv[j], xv[j], local);
        } else {
            for (int i = tid; i < dim; i += T) {
                float v = h2f(hrow[base + i]);
                local = __builtin_fmaf(v, v, local);
            }
        }
    }
    local = warp32_sum_down(local);
    if ((tid & 31) == 0) s_warp[tid >> 5] = local;
    __syncthreads();
    if (tid < 32) {
        const int nw = (T + 31) >> 5;
        float v = tid < nw ? s_warp[tid] : 0.0f;
        v = warp32_sum_down(v);
        if (tid == 0) {
            s_rms = rms_inv(v, dim, eps);
        }
    }
    __syncthreads();
    const float r = s_rms;
    if (regs && blockDim.x == T) {
#pragma unroll
        for (int j = 0; j < kNV; ++j) {
            const int i = tid + j * T;
            if (i < dim) {
                const uint16_t h = f2h((xv[j] * r) * gv[j]);
                s_row[i] = h;
                if (out_f16) out_f16[base + i] = h;
            }
        }
    } else {
        for (int i = tid; i < dim; i += blockDim.x) {
            uint16_t h = f2h((h2f(hrow[base + i]) * r) * h2f(weight[i]));
            s_row[i] = h;
            if (out_f16) out_f16[base + i] = h;
        }
    }
    if (!x_q) return;
    __syncthreads();

    // Group quantization of the fp16 row: subgroups of 2^lg lanes, one group
    // each, VEC elements per lane per iteration.
    const int lanes = 1 << lg;
    const int sub = tid & (lanes - 1);
    const int slots = blockDim.x >> lg;
    const int vec = vec8 ? 8 : 1;
    for (int gbase = 0; gbase < G; gbase += slots) {
        const int gi = gbase + (tid >> lg);
        const bool active = gi < G;
        const int k0 = gi * g;
        const int k1 = active ? min(k0 + g, dim) : k0;
        float s;
        if (act_scale) {
            s = active ? h2f(act_scale[gi]) : 1.0f;
            s = s < 1e-8f ? 1e-8f : s;
        } else {
            float amax = 0.0f;
            for (int k = k0 + sub * vec; k < k1; k += lanes * vec)
                for (int i = 0; i < vec; ++i) {
                    float v = h2f(s_row[k + i]);
                    if (smooth_inv) v *= h2f(smooth_inv[k + i]);
                    amax = fmaxf(amax, fabsf(v));
                }
            amax = subgroup_max_rt(amax, lg);
            s = act_scale_from_amax(amax);
        }
        if (active && sub == 0) x_scale[(size_t)blockIdx.x * G + gi] = s;
        const float inv = 1.0f / s;
        for (int k = k0 + sub * vec; k < k1; k += lanes * vec) {
            if (vec == 8) {
                int q[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float v = h2f(s_row[k + i]);
                    if (smooth_inv) v *= h2f(smooth_inv[k + i]);
                    q[i] = quant_rn(v, inv);
                }
                store_q<8>(x_q + base + k, q);
            } else {
                float v = h2f(s_row[k]);
                if (smooth_inv) v *= h2f(smooth_inv[k]);
                x_q[base + k] = (int8_t)quant_rn(v, inv);
            }
        }
    }
}

// --------------------------------------------------------- elementwise ----

// ffn_activations.cu:12-17 (silu), :35-39 (mul), :41-45 (residual add).
__global__ __launch_bounds__(kThreads) void elementwise_kernel(int op, uint16_t* __restrict__ a,
                                                               const uint16_t* __restrict__ b,
                                                               int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride) {
        float va = h2f(a[i]);
        float r;
        if (op == 0) r = silu_f(va);
        else if (op == 1) r = va * h2f(b[i]);
        else r = va + h2f(b[i]);
        a[i] = f2h(r);
    }
}

// SwiGLU on interleaved pairs: act[i] = fp16(fp16(silu(y[2i])) * y[2i + 1])
// (silu_forward then mul_forward, ffn_activations.cu:12-17, 35-39).
__global__ __launch_bounds__(kThreads) void swiglu_pairs_kernel(const uint16_t* __restrict__ y,
                                                                uint16_t* __restrict__ act,
                                                                int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n; i += stride)
        act[i] = f2h(h2f(f2h(silu_f(h2f(y[2 * i])))) * h2f(y[2 * i + 1]));
}

// ------------------------------------------------------ weight quantizer ----

// tools/quant_utils.py:171-194 quantize_groupwise on the device: per (row,
// group) amax = max(max|w|, 1e-8); s = fp16(amax / 127); q = clip(rint(w / s)).
// A NaN quotient (all-zero group, s == 0) becomes 0, as numpy's float->int8
// cast does on x86.
template <int VEC>
__global__ __launch_bounds__(kThreads) void quantize_weights_kernel(
    const uint16_t* __restrict__ w, int8_t* __restrict__ q, uint16_t* __restrict__ scale,
    int64_t rows, int64_t K, int g, int64_t G, int lg) {
    const int lanes = 1 << lg;
    const int64_t slot = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> lg;
    const int sub = threadIdx.x & (lanes - 1);
    const bool active = slot < rows * G;
    const int64_t r = active ? slot / G : 0;
    const int64_t gi = active ? slot % G : 0;
    const int64_t k0 = gi * g;
    const int64_t k1 = active ? (k0 + g < K ? k0 + g : K) : k0;
    const size_t row = (size_t)r * K;
    float amax = 0.0f;
    for (int64_t k = k0 + sub * VEC; k < k1; k += lanes * VEC) {
        uint16_t h[VEC];
        load_h<VEC>(w + row + k, h);
#pragma unroll
        for (int i = 0; i < VEC; ++i) amax = fmaxf(amax, fabsf(h2f(h[i])));
    }
    amax = subgroup_max_rt(amax, lg);
    if (!(amax > 1e-8f)) amax = 1e-8f;
    const uint16_t sh = f2h(amax / 127.0f);
    if (active && sub == 0) scale[(size_t)r * G + gi] = sh;
    const float s = h2f(sh);
    for (int64_t k = k0 + sub * VEC; k < k1; k += lanes * VEC) {
        uint16_t h[VEC];
        load_h<VEC>(w + row + k, h);
        int qv[VEC];
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
            float v = h2f(h[i]) / s;
            if (__builtin_isnan(v)) {
                qv[i] = 0;
            } else {
                float t = __builtin_rintf(v);
                qv[i] = (int)fminf(fmaxf(t, -127.0f), 127.0f);
            }
        }
        store_q<VEC>(q + row + k, qv);
    }
}

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; }

}  // namespace

hipError_t launch_quantize_activations(const uint16_t* X, const uint16_t* up, Prologue kind,
                                       const uint16_t* act_scale, const uint16_t* smooth_inv,
                                       int8_t* x_q, float* x_scale, uint16_t* out_f16,
                                       int N, int K, int g, int G, hipStream_t stream) {
    if (N <= 0 || K <= 0) return hipSuccess;
    const bool vec8 = (K % 8 == 0) && (g % 8 == 0) && aligned16(X) && aligned16(up) &&
                      aligned16(smooth_inv) && aligned16(out_f16) && ((uintptr_t)x_q & 7) == 0;
    const int vec = vec8 ? 8 : 1;
    const int lg = lanes_log2_for(g, vec);
    const long slots = (long)N * G;
    const long threads = slots << lg;
    const int blocks = (int)((threads + kThreads - 1) / kThreads);
    if (vec8) {
        if (kind == Prologue::kSiluMul)
            hipLaunchKernelGGL((quantize_act_kernel<8, Prologue::kSiluMul>), dim3(blocks),
                               dim3(kThreads), 0, stream, X, up, act_scale, smooth_inv, x_q,
                               x_scale, out_f16, N, K, g, G, lg);
        else
            hipLaunchKernelGGL((quantize_act_kernel<8, Prologue::kPlain>), dim3(blocks),
                               dim3(kThreads), 0, stream, X, up, act_scale, smooth_inv, x_q,
                               x_scale, out_f16, N, K, g, G, lg);
    } else {
        if (kind == Prologue::kSiluMul)
            hipLaunchKernelGGL((quantize_act_kernel<1, Prologue::kSiluMul>), dim3(blocks),
                               dim3(kThreads), 0, stream, X, up, act_scale, smooth_inv, x_q,
                               x_scale, out_f16, N, K, g, G, lg);
        else
            hipLaunchKernelGGL((quantize_act_kernel<1, Prologue::kPlain>), dim3(blocks),
                               dim3(kThreads), 0, stream, X, up, act_scale, smooth_inv, x_q,
                               x_scale, out_f16, N, K, g, G, lg);
    }
    return hipGetLastError();
}

hipError_t launch_rms_norm_quant(const uint16_t* x, const uint16_t* resid, uint16_t* h_out,
                                 const uint16_t* weight,
                                 float eps,
                                 const uint16_t* smooth_inv, const uint16_t* act_scale,
                                 int g, int G, int8_t* x_q, float* x_scale, uint16_t* out_f16,
                                 int n_tokens, int dim, hipStream_t stream) {
    if (n_tokens <= 0 || dim <= 0) return hipSuccess;
    int T = 1;
    while (T < dim && T < 1024) T <<= 1;
    const int block = T < 64 ? 64 : T;
    const bool vec8 = (dim % 8 == 0) && (g % 8 == 0) && aligned16(smooth_inv) &&
                      ((uintptr_t)x_q & 7) == 0;
    const int lg = x_q ? lanes_log2_for(g, vec8 ? 8 : 1) : 0;
    const size_t lds = ((size_t)dim * 2 + 15) & ~(size_t)15;
    if (resid && !h_out) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_norm_quant_kernel, dim3(n_tokens), dim3(block), lds, stream, x, resid,
                       h_out, weight, eps, smooth_inv, act_scale, x_q, x_scale, out_f16, dim, T, g, G, lg,
                       vec8 ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_swiglu_pairs(const uint16_t* y, uint16_t* act, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(swiglu_pairs_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, y,
                       act, n);
    return hipGetLastError();
}

hipError_t launch_elementwise(int op, uint16_t* a, const uint16_t* b, int64_t n,
                              hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(elementwise_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, op,
                       a, b, n);
    return hipGetLastError();
}

hipError_t launch_quantize_weights(const uint16_t* w, int64_t rows, int64_t K, int g,
                                   int8_t* q, uint16_t* scale, hipStream_t stream) {
    if (rows <= 0 || K <= 0) return hipSuccess;
    const int64_t G = (K + g - 1) / g;
    const bool vec8 = (K % 8 == 0) && (g % 8 == 0) && aligned16(w) && ((uintptr_t)q & 7) == 0;
    const int vec = vec8 ? 8 : 1;
    const int lg = lanes_log2_for(g, vec);
    const int64_t threads = (rows * G) << lg;
    const int64_t blocks = (threads + kThreads - 1) / kThreads;
    if (vec8)
        hipLaunchKernelGGL((quantize_weights_kernel<8>), dim3((unsigned)blocks), dim3(kThreads), 0,
                           stream, w, q, scale, rows, K, g, G, lg);
    else
        hipLaunchKernelGGL((quantize_weights_kernel<1>), dim3((unsigned)blocks), dim3(kThreads), 0,
                           stream, w, q, scale, rows, K, g, G, lg);
    return hipGetLastError();
}

}  // namespace fa

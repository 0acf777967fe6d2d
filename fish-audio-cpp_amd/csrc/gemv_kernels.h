// gemv_kernels.h -- decode-shaped W8A8 linear (N <= 16 tokens) for CDNA4:
// the kernel templates, shared by the translation units that instantiate them
// (gemv.hip: plan, launch and the MFMA GEMV; gemv_dot*.hip: the N == 1
// kernel families).
//
// Replaces the reference's int8_matvec_dequant_kernel (N == 1), its
// small-batch kernel (2 <= N <= 4) and, for 5 <= N <= 16, its per-group
// cuBLAS loop (src/kernels/int8_gemm.cu:245-380, 439-498).
//
// Both kernels below form every int32 per-group partial P_g exactly and then
// sum the groups in the reference accumulate kernel's order
// (int8_gemm.cu:213-234, nvcc contracting `acc += float(P) * ws * xs` into
// fma(float(P) * ws, xs, acc)), sequentially over g = 0, 1, ..., so the fp16
// output is bit-identical to the host oracle.  Splitting K across waves only
// changes who computes the terms float(P_g) * ws; the fma chain over the terms
// runs in group order on one lane per output.
//
// gemv_dot_kernel (N == 1): one wave streams R = 1 or 2 weight rows.  A row's
// 64/R lanes each load 16 bytes per pass (128-bit loads, a pass covers
// 1024/R contiguous bytes of the row) and form 4 v_dot4_i32_i8 products with
// the activation bytes; lanes holding the same K-group (g/16 of them) add
// their partials with cross-lane shuffles.  Up to KD passes are in flight per
// wave (a register ring refilled as it drains); no split-K, so every CU keeps
// dozens of independent row streams.
//
// gemv_mfma_kernel (2 <= N <= 16): a workgroup owns 16 weight rows; its NW
// waves split the K-groups into contiguous ranges.  Lane l streams 16 bytes of
// row l&15 at byte offset 16*(l>>4) of each 64-byte K step, the tokens' int8
// activations ride in the second MFMA operand with the same byte mapping, so
// v_mfma_i32_16x16x64_i8 yields the exact int32 dot of every (row, token) pair
// over 64 bytes; g/64 chained MFMAs make P_g.  Terms are kept in registers;
// afterwards the waves pass the running fp32 sums along in group order
// through LDS.
//
// With QX the MFMA kernel quantizes the fp16 tokens itself: lane l loads the
// 16 fp16 values of token l&15 that its B fragment covers at every step of
// the wave's K range, the group maximum comes from its own values and the
// three other lanes of the same token (xor 16, 32), and the codes go straight
// into the hoisted B fragments; no int8 copy of the tokens is written.  With
// EPI 1 rows 2i / 2i+1 are a SwiGLU pair (gate, up) and Y [N][M / 2] gets
// fp16(fp16(silu(fp16(gate))) * fp16(up)).
#pragma once

#include "common.h"

namespace fa {
namespace gv {


struct DbgWindow {
    int32_t* p;
    int row0, rows, tok0, toks;
    __device__ bool in(int row, int tok) const {
        return p && row >= row0 && row < row0 + rows && tok >= tok0 && tok < tok0 + toks;
    }
    __device__ int32_t& at(int row, int tok, int gi, int G) const {
        return p[((size_t)(tok - tok0) * rows + (row - row0)) * G + gi];
    }
};

__device__ __forceinline__ v4i ld16(const int8_t* p) { return *reinterpret_cast<const v4i*>(p); }

// Fused prologue of the N == 1 kernel with in-kernel quantization (QX):
//   PRO 0: quantize X itself (int8_dequant_gemm_fp16's own quantizer);
//   PRO 1: X = gate, x2 = up; the quantizer sees fp16(fp16(silu(gate)) * up)
//          (silu_forward then mul_forward, ffn_activations.cu:12-17, 35-39);
//   PRO 2: X = residual stream, x2 = residual addend or null, gamma, eps; the
//          quantizer sees rms_norm(h, gamma) with h = fp16(X + x2) (residual_add,
//          ffn_activations.cu:41-45, then rms_norm.cu:10-58), and workgroup 0
//          writes h to h_out.
struct ProArgs {
    const uint16_t* x2;
    const uint16_t* gamma;
    uint16_t* h_out;
    float eps;
    // EPI 2: the up weight (w3), its scales and its own quantization
    // companions (the gate weight w1 comes as W / w_scale)
    const int8_t* w3;
    const uint16_t* w3_scale;
    const uint16_t* act_scale3;
    const uint16_t* smooth_inv3;
};

// ------------------------------------------------------------ N == 1 ----

constexpr int kDotWaves = 4;     // waves per workgroup, staged int8 codes
constexpr int kDotWavesQx = 8;   // waves per workgroup, in-kernel quantization

// Sum of an int over aligned blocks of LG lanes (all lanes get the block sum).
// LG <= 16 stays inside a 16-lane DPP row: quad_perm swaps, then half-row and
// row mirrors, one v_add_*_dpp each.  Integer sums are exact in any order.
template <int LG>
__device__ __forceinline__ int group_sum(int p, int lg_rt) {
    if constexpr (LG == 0) {
        for (int off = 1; off < (1 << lg_rt); off <<= 1) p += __shfl_xor(p, off, 64);
        return p;
    } else {
        if constexpr (LG >= 2) p += __builtin_amdgcn_update_dpp(0, p, 0xB1, 0xF, 0xF, false);
        if constexpr (LG >= 4) p += __builtin_amdgcn_update_dpp(0, p, 0x4E, 0xF, 0xF, false);
        if constexpr (LG >= 8) p += __builtin_amdgcn_update_dpp(0, p, 0x141, 0xF, 0xF, false);
        if constexpr (LG >= 16) p += __builtin_amdgcn_update_dpp(0, p, 0x140, 0xF, 0xF, false);
        if constexpr (LG >= 32) p += __shfl_xor(p, 16, 64);
        if constexpr (LG >= 64) p += __shfl_xor(p, 32, 64);
        return p;
    }
}

// Max of a non-negative float over aligned blocks of 2^lgl lanes (runtime
// width; all lanes get the block max).  Within 16-lane DPP rows one
// v_max_f32_dpp per step; wider blocks add xor shuffles across rows.  The
// max is exact in any order.
__device__ __forceinline__ float block_max(float m, int lgl) {
    if (lgl >= 1) m = fmaxf(m, dpp_f<0xB1>(m));    // quad_perm [1,0,3,2]
    if (lgl >= 2) m = fmaxf(m, dpp_f<0x4E>(m));    // quad_perm [2,3,0,1]
    if (lgl >= 3) m = fmaxf(m, dpp_f<0x141>(m));   // row_half_mirror
    if (lgl >= 4) m = fmaxf(m, dpp_f<0x140>(m));   // row_mirror
    if (lgl >= 5) m = fmaxf(m, __shfl_xor(m, 16, 64));
    if (lgl >= 6) m = fmaxf(m, __shfl_xor(m, 32, 64));
    return m;
}

// ---------------------------------------------------- in-kernel quant ----
//
// The fp16 token a one-token kernel quantizes itself (QX), in two halves so
// the caller can put its weight loads in between: qx_load issues the
// activation loads (XV 16-byte chunks of 8 fp16 values per thread, chunk c =
// tid + i * NT), qx_stage applies the fused prologue and writes the int8
// codes to xq_s [K] and the group scales to xs_s [G] (int8_gemm.cu:147-211
// semantics: per-group amax/127 or a static scale, optional smooth_inv).
template <int XV, int PRO>
struct QxIn {
    v4i xr[XV];
    v4i x2r[PRO != 0 ? XV : 1];
    v4i gmr[PRO == 2 ? XV : 1];
    v4i smr[XV], sm2r[XV];   // smooth_inv chunks of the first / second companions
};

template <int XV, int NT, int PRO, bool SM2 = false>
__device__ __forceinline__ void qx_load(QxIn<XV, PRO>& in, const uint16_t* __restrict__ X, int K,
                                        const ProArgs& pro, int tid,
                                        const uint16_t* __restrict__ smooth_inv = nullptr,
                                        const uint16_t* __restrict__ smooth_inv2 = nullptr) {
    // unconditional loads from clamped addresses (a load under a branch
    // makes the compiler wait for it on the spot); without a smooth_inv
    // vector its chunks re-read X and are not used
    const uint16_t* sm1 = smooth_inv ? smooth_inv : X;
    const uint16_t* sm2 = smooth_inv2 ? smooth_inv2 : X;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
        const int k = (tid + i * NT) * 8;
        const int kc = k < K ? k : K - 8;
        in.xr[i] = *reinterpret_cast<const v4i*>(X + kc);
        in.smr[i] = *reinterpret_cast<const v4i*>(sm1 + kc);
        if constexpr (SM2) in.sm2r[i] = *reinterpret_cast<const v4i*>(sm2 + kc);
    }
    // prologue operands: up (PRO 1) or the residual addend (PRO 2; X again
    // when there is none) and gamma
    if constexpr (PRO != 0) {
        const uint16_t* x2 = pro.x2 ? pro.x2 : X;
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int k = (tid + i * NT) * 8;
            const int kc = k < K ? k : K - 8;
            in.x2r[i] = *reinterpret_cast<const v4i*>(x2 + kc);
            if constexpr (PRO == 2) in.gmr[i] = *reinterpret_cast<const v4i*>(pro.gamma + kc);
        }
    }
}

// write_h: this workgroup writes h to pro.h_out (PRO 2).  Contains workgroup
// barriers (PRO 2): every thread of the workgroup must call it.  The caller
// synchronises before reading xq_s / xs_s.
template <int XV, int NT, int PRO>
__device__ __forceinline__ void qx_stage(QxIn<XV, PRO>& in, const uint16_t* __restrict__ X,
                                         const uint16_t* __restrict__ act_scale,
                                         const uint16_t* __restrict__ smooth_inv, int K, int lg_g,
                                         int G, const ProArgs& pro, int tid, bool write_h,
                                         int8_t* xq_s, float* xs_s, uint16_t* h_s, float* red_s,
                                         int8_t* xq2_s = nullptr, float* xs2_s = nullptr,
                                         const uint16_t* __restrict__ act_scale2 = nullptr,
                                         const uint16_t* __restrict__ smooth_inv2 = nullptr) {
    // Chunk c holds x[8c, 8c + 8); chunk c of thread tid is tid + i * NT,
    // so a K-group (g / 8 chunks) lies in g / 8 consecutive lanes of one
    // wave.  Its |v| maximum (exact in any order) comes from xor shuffles,
    // then scale and int8 codes are formed in registers: no atomics and a
    // single barrier (the caller's) before the codes are read.
    const int glanes = 1 << (lg_g - 3);
    // smv: this chunk's smooth_inv values when loaded ahead (qx_load), else
    // they are read here
    auto chunk = [&](int c, const v4i& raw, const uint16_t* __restrict__ act_scale,
                     const uint16_t* __restrict__ smooth_inv, int8_t* xq_s, float* xs_s,
                     const v4i* smv) {
        const int k = c * 8;
        const bool ok = k < K;
        const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw);
        const uint16_t* sh = reinterpret_cast<const uint16_t*>(smv);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            v[e] = h2f(h[e]);
            if (smooth_inv) v[e] *= h2f(smv ? sh[e] : smooth_inv[ok ? k + e : e]);
        }
        const int gi = ok ? k >> lg_g : G - 1;
        float sc_;
        if (act_scale) {
            sc_ = h2f(act_scale[gi]);
            sc_ = sc_ < 1e-8f ? 1e-8f : sc_;
        } else {
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
            if (!ok) m = 0.0f;
            m = block_max(m, lg_g - 3);
            sc_ = act_scale_from_amax(m);
        }
        if (ok) {
            const float inv = 1.0f / sc_;
            int q[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) q[e] = quant_rn(v[e], inv);
            uint2 u;
            u.x = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                  ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
            u.y = (uint32_t)(q[4] & 0xff) | ((uint32_t)(q[5] & 0xff) << 8) |
                  ((uint32_t)(q[6] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24);
            *reinterpret_cast<uint2*>(xq_s + k) = u;
            if ((c & (glanes - 1)) == 0) xs_s[gi] = sc_;
        }
    };
    if constexpr (PRO == 1) {
        // silu_forward then mul_forward, each rounded to fp16
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            uint16_t* h = reinterpret_cast<uint16_t*>(&in.xr[i]);
            const uint16_t* u = reinterpret_cast<const uint16_t*>(&in.x2r[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(f2h(silu_f(h2f(h[e])))) * h2f(u[e]));
        }
    } else if constexpr (PRO == 2) {
        // h = fp16(x + resid) into LDS (and to h_out from one workgroup)
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int k = (tid + i * NT) * 8;
            uint16_t* h = reinterpret_cast<uint16_t*>(&in.xr[i]);
            if (pro.x2) {
                const uint16_t* r = reinterpret_cast<const uint16_t*>(&in.x2r[i]);
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(h[e]) + h2f(r[e]));
            }
            if (k < K) {
                *reinterpret_cast<v4i*>(h_s + k) = in.xr[i];
                if (pro.h_out && write_h) *reinterpret_cast<v4i*>(pro.h_out + k) = in.xr[i];
            }
        }
        __syncthreads();
        // Sum of squares in the reference's order (rms_norm.cu:22-41):
        // T = min(next_pow2(K), 1024) threads, thread t sums h[t],
        // h[t + T], ... with FMAs, each 32-thread warp reduces by the
        // shuffle-down tree, then the warp sums by the same tree.  Thread
        // tid plays threads tid, tid + NT, ...
        int T = 1;
        while (T < K) T <<= 1;
        if (T > 1024) T = 1024;
        const int lanes = T < 32 ? 32 : T;
        for (int t0 = 0; t0 < lanes; t0 += NT) {      // uniform trip count
            const int t = t0 + tid;
            float loc = 0.0f;
            if (t < T)
                for (int k = t; k < K; k += T) {
                    const float v = h2f(h_s[k]);
                    loc = __builtin_fmaf(v, v, loc);
                }
            loc = warp32_sum_down(loc);
            if (t < lanes && (t & 31) == 0) red_s[t >> 5] = loc;
        }
        __syncthreads();
        if (tid < 32) {
            const int nw = (T + 31) >> 5;
            float v = tid < nw ? red_s[tid] : 0.0f;
            v = warp32_sum_down(v);
            if (tid == 0) red_s[32] = rms_inv(v, K, pro.eps);
        }
        __syncthreads();
        const float rr = red_s[32];
        // normalised fp16 row (rms_norm.cu:52-56)
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            uint16_t* h = reinterpret_cast<uint16_t*>(&in.xr[i]);
            const uint16_t* gm = reinterpret_cast<const uint16_t*>(&in.gmr[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = f2h((h2f(h[e]) * rr) * h2f(gm[e]));
        }
    }
#pragma unroll
    for (int i = 0; i < XV; ++i)
        chunk(tid + i * NT, in.xr[i], act_scale, smooth_inv, xq_s, xs_s, &in.smr[i]);
    if (xq2_s) {   // a second weight's own companions (wave-uniform)
#pragma unroll
        for (int i = 0; i < XV; ++i)
            chunk(tid + i * NT, in.xr[i], act_scale2, smooth_inv2, xq2_s, xs2_s, &in.sm2r[i]);
    }
    if constexpr (PRO == 0) {
        for (int c0 = XV * NT; c0 * 8 < K; c0 += NT) {   // K beyond XV * NT * 8 (uniform trip count)
            const int c = c0 + tid;
            const v4i raw = *reinterpret_cast<const v4i*>(X + (c * 8 < K ? c * 8 : K - 8));
            chunk(c, raw, act_scale, smooth_inv, xq_s, xs_s, nullptr);
            if (xq2_s) chunk(c, raw, act_scale2, smooth_inv2, xq2_s, xs2_s, nullptr);
        }
    }
}

// One wave streams R rows (R = 1, 2 or 4; 64/R lanes per row, 16 bytes per
// lane per pass).  After 4 v_dot4 per lane, lanes of one K-group (LG = g/16
// of them) sum their partials with DPP, so every lane of a group holds the
// exact int32 P_g.  The groups of a pass are then in known lanes: group slot j
// of row r sits in lane r * 64/R + j * LG.  Each of those terms
// float(P_g) * ws is broadcast with v_readlane, and every lane advances its
// rows' fp32 sums in group order, acc = fma(term, x_scale[g], acc) -- the
// reference's accumulate order (int8_gemm.cu:231), so the result is the
// oracle's bit for bit without any per-row serial tail.
//
// QX: the kernel quantizes the fp16 token itself (int8_gemm.cu:147-211
// semantics: per-group amax/127 or a static scale, optional smooth_inv) while
// the first weight loads are in flight; otherwise it stages the given int8
// activations and fp32 scales.  Either way x_q [K] and x_scale [G] sit in LDS.
//
// Work: row blocks of NWV * R rows (NWV waves per workgroup); block b,
// b + gridDim.x, ... belong to workgroup b.  A uniform cursor (row block,
// pass) walks the wave's passes in order and the weight ring is KD passes
// ahead of the consumer.  g is a power of two (lg_g = log2 g) with
// 16 <= g <= 16 * 64/R.  With QX every workgroup quantizes the whole token,
// so QX launches use 8-wave workgroups (half as many copies of that work).
//
// PRO (QX only, see ProArgs): the quantizer's input comes from a fused
// prologue; then every chunk of the token is held in registers
// (K <= XV * NWV * 512), and for PRO 2 the fp16 row h goes through LDS once
// for the sum of squares.
//
// EPI 1 (R == 2): SwiGLU pair epilogue.  Rows 2i and 2i+1 are the gate (w1)
// and up (w3) rows of FFN column i, interleaved at load time; the wave holds
// both chains, rounds each to fp16 (the reference's two GEMMs output fp16)
// and stores act[i] = fp16(fp16(silu(gate)) * up) (silu_forward then
// mul_forward, ffn_activations.cu:12-17, 35-39) into Y [M / 2].
template <int R, int KD, int LG, bool QX, int XV, int NWV = kDotWaves, int PRO = 0,
          int EPI = 0>
__global__ __launch_bounds__(NWV * 64) void gemv_dot_kernel(
    const int8_t* __restrict__ W, const uint16_t* __restrict__ w_scale,
    const int8_t* __restrict__ x_q, const float* __restrict__ x_scale,
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ act_scale,
    const uint16_t* __restrict__ smooth_inv,
    uint16_t* __restrict__ Y, DbgWindow dbg, int M, int K, int lg_g, int G, int passes,
    int nblocks, ProArgs pro) {
    static_assert(PRO == 0 || QX, "prologues need in-kernel quantization");
    static_assert(EPI == 0 || R == 2, "the SwiGLU pair needs two rows per wave");
    static_assert(EPI != 2 || QX, "separate w1 / w3 quantize in-kernel");
    constexpr int RL = 64 / R;            // lanes per row
    constexpr int PB = RL * 16;           // bytes of a row per pass
    constexpr int GPP = RL / LG;          // groups per row per pass
    constexpr int NT = NWV * 64;
    static_assert(LG >= 1 && LG <= RL, "group must fit a row's lanes");
    extern __shared__ __align__(16) float lds[];
    const int Kp = (K + 15) & ~15;
    int8_t* xq_s = reinterpret_cast<int8_t*>(lds);                  // [Kp]
    float* xs_s = lds + Kp / 4;                                      // [G], padded to 4
    // PRO 2: the fp16 row [Kp] and 32 warp sums + the scale after xs_s
    uint16_t* h_s = reinterpret_cast<uint16_t*>(xs_s + ((G + 3) & ~3));
    float* red_s = reinterpret_cast<float*>(h_s + Kp);
    // EPI 2: the up weight's codes [Kp] and scales [G] after the PRO 2 area
    int8_t* xq3_s = reinterpret_cast<int8_t*>(lds) + (((size_t)Kp + 4 * ((G + 3) & ~3) + 2 * Kp +
                                                        33 * 4 + 15) & ~(size_t)15);
    float* xs3_s = reinterpret_cast<float*>(xq3_s + Kp);
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;

    const int rsub = lane / RL;
    const int li = lane % RL;
    const int lane_k = li * 16;

    // ---- activation loads first: their wait then does not cover the ring.
    // XV 16-byte chunks per thread (int8 codes, or 8 fp16 values with QX);
    // unconditional loads from clamped addresses (a load under a branch makes
    // the compiler wait for it on the spot).
    v4i xr[XV];
    float xsr = 0.0f;
    QxIn<XV, PRO> qin;
    if constexpr (!QX) {
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int k = (tid + i * NT) * 16;
            xr[i] = ld16(x_q + (k < Kp ? k : Kp - 16));
        }
        xsr = x_scale[tid < G ? tid : G - 1];
    } else {
        qx_load<XV, NT, PRO, EPI == 2>(qin, X, K, pro, tid, smooth_inv,
                                       EPI == 2 ? pro.smooth_inv3 : nullptr);
    }

    // ---- weight ring
    int l_blk = blockIdx.x, l_pass = 0;     // load cursor (uniform)
    const int8_t* const wlast = W + (size_t)(M - 1) * K;
    v4i a[KD];
    uint16_t sc[KD];
    const v4i zero = {0, 0, 0, 0};
    auto row_of_blk = [&](int blk) { return (blk * NWV + wave) * R + rsub; };
    auto load = [&](int slot) {
        const bool live = l_blk < nblocks;
        const int row = row_of_blk(live ? l_blk : blockIdx.x);
        const int rowc = row < M ? row : M - 1;
        const int k = l_pass * PB + lane_k;
        const bool ok = live && k < K;
        const int kk = ok ? k : 0;
        // no select on the loaded value (that would wait for the load here):
        // bytes past K meet zero activations in consume()
        if constexpr (EPI == 2) {
            // row 2i: gate weight row i, row 2i + 1: up weight row i
            const int8_t* wb = (rowc & 1) ? pro.w3 : W;
            const uint16_t* sb = (rowc & 1) ? pro.w3_scale : w_scale;
            const int pr = rowc >> 1;
            a[slot] = ld16(wb + (size_t)pr * K + kk);
            sc[slot] = sb[G == 1 ? (size_t)pr : (size_t)pr * G + (kk >> lg_g)];
        } else {
            const int8_t* wrow = row < M ? W + (size_t)row * K : wlast;
            const v4i wa = ld16(wrow + kk);
            sc[slot] = w_scale[G == 1 ? (size_t)rowc : (size_t)rowc * G + (kk >> lg_g)];
            a[slot] = wa;
        }
        if (++l_pass == passes) {
            l_pass = 0;
            l_blk += gridDim.x;
        }
    };
#pragma unroll
    for (int s = 0; s < KD; ++s) load(s);

    // ---- stage activations into LDS
    if constexpr (!QX) {
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int k = (tid + i * NT) * 16;
            if (k < Kp) *reinterpret_cast<v4i*>(xq_s + k) = xr[i];
        }
        if (tid < G) xs_s[tid] = xsr;
        for (int k = (tid + XV * NT) * 16; k < Kp; k += NT * 16)   // K > 16 KB
            *reinterpret_cast<v4i*>(xq_s + k) = ld16(x_q + k);
        for (int i = tid + NT; i < G; i += NT) xs_s[i] = x_scale[i];
    } else {
        if constexpr (EPI == 2)
            qx_stage<XV, NT, PRO>(qin, X, act_scale, smooth_inv, K, lg_g, G, pro, tid,
                                  blockIdx.x == 0, xq_s, xs_s, h_s, red_s, xq3_s, xs3_s,
                                  pro.act_scale3, pro.smooth_inv3);
        else
            qx_stage<XV, NT, PRO>(qin, X, act_scale, smooth_inv, K, lg_g, G, pro, tid,
                                  blockIdx.x == 0, xq_s, xs_s, h_s, red_s);
    }
    __syncthreads();

    // ---- consume
    int c_blk = blockIdx.x, c_pass = 0;     // consume cursor (uniform)
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    auto consume = [&](int slot) {
        const int kbase = c_pass * PB;                 // row offset of this pass (uniform)
        const int k = kbase + lane_k;
        const int8_t* xqr = (EPI == 2 && rsub == 1) ? xq3_s : xq_s;   // EPI 2: the row's codes
        v4i b = *reinterpret_cast<const v4i*>(xqr + (k < K ? k : 0));
        if (k >= K) b = zero;
        int p = __builtin_amdgcn_sdot4(a[slot].x, b.x, 0, false);
        p = __builtin_amdgcn_sdot4(a[slot].y, b.y, p, false);
        p = __builtin_amdgcn_sdot4(a[slot].z, b.z, p, false);
        p = __builtin_amdgcn_sdot4(a[slot].w, b.w, p, false);
        p = group_sum<LG>(p, 0);
        const float term = (float)p * h2f(sc[slot]);
        if (dbg.p) {
            const int row = row_of_blk(c_blk);
            if (k < K && (li & (LG - 1)) == 0 && row < M && dbg.in(row, 0))
                dbg.at(row, 0, k >> lg_g, G) = p;
        }
        // group order within the pass: slot j of every row; the pass's
        // GPP scales come in one LDS read (kbase / g is a multiple of GPP)
        // (EPI 2: row slot 1 takes the up weight's token scales)
        constexpr int NXS = EPI == 2 ? 2 : 1;
        float xsv[NXS][GPP];
#pragma unroll
        for (int q = 0; q < NXS; ++q) {
            const float* xp = (q ? xs3_s : xs_s) + (kbase >> lg_g);
            if constexpr (GPP == 4) {
                const float4 v = *reinterpret_cast<const float4*>(xp);
                xsv[q][0] = v.x; xsv[q][1] = v.y; xsv[q][2] = v.z; xsv[q][3] = v.w;
            } else if constexpr (GPP == 2) {
                const float2 v = *reinterpret_cast<const float2*>(xp);
                xsv[q][0] = v.x; xsv[q][1] = v.y;
            } else {
#pragma unroll
                for (int j = 0; j < GPP; ++j) xsv[q][j] = xp[j];
            }
        }
#pragma unroll
        for (int j = 0; j < GPP; ++j) {
            const int kg = kbase + j * LG * 16;        // first byte of slot j (uniform)
            if (kg < K) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float tj = __builtin_bit_cast(
                        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, term),
                                                         r * RL + j * LG));
                    acc[r] = __builtin_fmaf(tj, xsv[NXS == 2 ? r : 0][j], acc[r]);
                }
            }
        }
        if (++c_pass == passes) {
            const int row = row_of_blk(c_blk);
            if constexpr (EPI != 0) {
                // every lane holds both chains; lane 0 (row slot 0: the even
                // gate row) stores the pair's activation
                if (lane == 0 && row + 1 < M) {
                    const uint16_t gh = f2h(acc[0]), uh = f2h(acc[R - 1]);
                    Y[row >> 1] = f2h(h2f(f2h(silu_f(h2f(gh)))) * h2f(uh));
                }
            } else {
                // lane r*RL (li == 0) of row slot r stores that row
#pragma unroll
                for (int r = 0; r < R; ++r)
                    if (rsub == r && li == 0 && row < M) Y[row] = f2h(acc[r]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = 0.0f;
            c_pass = 0;
            c_blk += gridDim.x;
        }
    };
    // Rounds that refill the ring, then a last round that only drains it (so
    // every load is unconditional and the wait counts stay exact).
    const int my_blocks = (nblocks - 1 - (int)blockIdx.x) / (int)gridDim.x + 1;
    const int items = my_blocks * passes;
    int base = 0;
    for (; base + KD < items; base += KD) {
#pragma unroll
        for (int s = 0; s < KD; ++s) {
            consume(s);
            load(s);
        }
    }
#pragma unroll
    for (int s = 0; s < KD; ++s)
        if (base + s < items) consume(s);
}

// ------------------------------------------------------ 2 <= N <= 16 ----

constexpr int kTile = 16;

__device__ __forceinline__ uint16_t swiglu_h(uint16_t gate, uint16_t up) {
    return f2h(h2f(f2h(silu_f(h2f(gate)))) * h2f(up));
}

// QX: 0 = staged int8 codes (x_q, x_scale), 1 = quantize X in-kernel,
// 2 = the same times smooth_inv.  EPI 1: SwiGLU pairs (M even).
template <int SPG, int MAXG, bool LC, bool kDbg, int kKD = 12, int QX = 0,
          int EPI = 0>
__global__ __launch_bounds__(512) void gemv_mfma_kernel(
    const int8_t* __restrict__ W, const uint16_t* __restrict__ w_scale,
    const int8_t* __restrict__ x_q, const float* __restrict__ x_scale,
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ act_scale,
    const uint16_t* __restrict__ smooth_inv,
    uint16_t* __restrict__ Y, DbgWindow dbg, int M, int N, int K, int G) {
    constexpr int NSTEP = SPG * MAXG;
    static_assert(QX == 0 || NSTEP <= 32, "in-kernel quantization fills the hoisted codes");
    // ring depth: kKD steps, 8 when 16+ groups' terms are held in registers
    constexpr int KDM = (!LC && MAXG >= 16) ? 8 : kKD;
    constexpr int KD = NSTEP < KDM ? NSTEP : KDM;
    extern __shared__ float lds[];
    float* ws_s = lds;                   // [16 rows][G]
    float* xs_s = lds + kTile * G;       // [16 tokens][G]
    float* chain = lds + 2 * kTile * G;  // [16 tokens][16 rows] (!LC)
    // LC: every term float(P_g) * ws in LDS, [G][ns tokens][16 rows]
    const int ns = N <= 8 ? 8 : 16;
    float* tl = lds + 2 * kTile * G;

    const int NW = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * kTile;
    const int gb = (wave * G) / NW;
    const int ng = ((wave + 1) * G) / NW - gb;
    const int nsteps = ng * SPG;
    // steps of the wave's range that lie inside the row: when K % g != 0 the
    // last group is short (K % 64 == 0 here); later steps re-load step 0
    // (in bounds) and skip their MFMA
    const int nvalid = min(nsteps, (K - gb * SPG * 64) / 64);

    const int lr = lane & 15;            // A: weight row in tile; B: token
    const int kq = (lane >> 4) * 16;
    const int row_ld = min(row0 + lr, M - 1);
    const size_t kbase = (size_t)gb * SPG * 64 + kq;
    const int8_t* wp = W + (size_t)row_ld * K + kbase;
    // token lanes past N read token N-1: their MFMA columns are never stored
    const int8_t* xp = QX ? nullptr : x_q + (size_t)min(lr, N - 1) * K + kbase;

    // The wave's B fragments (the tokens' codes of its K range) are loaded
    // once, ahead of the weight ring, when they fit in registers (measured
    // on MI355X at 8 tokens, g64: qkv 8.47 -> 7.32 us, gate_up 16.7 -> 15.2,
    // down 15.6 -> 13.8, o unchanged; g256: qkv 7.63 -> 7.20, o 6.63 ->
    // 6.04); the ring then carries weights only.
    constexpr bool BH = NSTEP <= 32;
    v4i a[KD], b[BH ? 1 : KD];
    v4i bh[BH ? NSTEP : 1];
    const v4i zero = {0, 0, 0, 0};
    // QX: the 16 fp16 values per step (two 16-byte chunks), the smooth_inv
    // chunks (QX 2) and the static group scales, loaded first
    v4i xf[QX ? NSTEP : 1][2], sf[QX == 2 ? NSTEP : 1][2];
    uint16_t asr[QX ? MAXG : 1];
    if constexpr (QX) {
        const uint16_t* xh = X + (size_t)min(lr, N - 1) * K + kbase;
#pragma unroll
        for (int st = 0; st < NSTEP; ++st) {
            const size_t off = (size_t)(st < nvalid ? st : 0) * 64;
            xf[st][0] = *reinterpret_cast<const v4i*>(xh + off);
            xf[st][1] = *reinterpret_cast<const v4i*>(xh + off + 8);
            if constexpr (QX == 2) {
                sf[st][0] = *reinterpret_cast<const v4i*>(smooth_inv + kbase + off);
                sf[st][1] = *reinterpret_cast<const v4i*>(smooth_inv + kbase + off + 8);
            }
        }
        // without static scales these loads re-read w_scale (not used)
        const uint16_t* asp = act_scale ? act_scale : w_scale;
#pragma unroll
        for (int j = 0; j < MAXG; ++j) asr[j] = asp[gb + (j < ng ? j : 0)];
    } else if constexpr (BH) {
#pragma unroll
        for (int st = 0; st < NSTEP; ++st)
            bh[st] = ld16(xp + (size_t)(st < nvalid ? st : 0) * 64);
    }
    // unconditional loads, no select on the loaded data: a select would make
    // the compiler wait for each load right where it is issued
    auto load = [&](int slot, int step) {
        const size_t off = (size_t)(step < nvalid ? step : 0) * 64;
        a[slot] = ld16(wp + off);
        if constexpr (!BH) b[slot] = ld16(xp + off);
    };
    // Scales of the tile's 16 rows and of the tokens, all groups: at most 5
    // per thread (the plan keeps G <= 20 * NW).  Their loads go out before
    // the weight ring's, so the wait before the LDS stores covers only them.
    // Token rows past N repeat token N-1 (their outputs are never stored).
    constexpr int kSt = 5;
    uint16_t wsr[kSt];
    float xsr[kSt];
#pragma unroll
    for (int q = 0; q < kSt; ++q) {
        const int i = min((int)threadIdx.x + q * (int)blockDim.x, kTile * G - 1);
        const int r = i / G, gi = i - r * G;
        const int row = min(row0 + r, M - 1);
        wsr[q] = w_scale[G == 1 ? (size_t)row : (size_t)row * G + gi];
        if constexpr (!QX) xsr[q] = x_scale[(size_t)min(r, N - 1) * G + gi];
    }
#pragma unroll
    for (int s = 0; s < KD; ++s) load(s, s);
    // QX: per (token lr, group) scale (int8_gemm.cu:147-211 semantics: the
    // group's |v| maximum / 127 or the static scale, clamped at 1e-8) and the
    // codes rint(v / s) clipped to +-127, packed in memory byte order
    float qsv[QX ? MAXG : 1];
    if constexpr (QX) {
        // value e of step st, formed from the packed halves where it is used
        // (no float copy of the wave's values stays live)
        auto val = [&](int st, int e) {
            const int w = xf[st][e >> 3][(e >> 1) & 3];
            float x = h2f((uint16_t)((e & 1) ? ((unsigned)w >> 16) : ((unsigned)w & 0xffffu)));
            if constexpr (QX == 2) {
                const int sw = sf[st][e >> 3][(e >> 1) & 3];
                x *= h2f((uint16_t)((e & 1) ? ((unsigned)sw >> 16) : ((unsigned)sw & 0xffffu)));
            }
            return x;
        };
#pragma unroll
        for (int j = 0; j < MAXG; ++j) {
            float amax = 0.0f;
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                const int st = j * SPG + s;
                float m = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) m = fmaxf(m, fabsf(val(st, e)));
                amax = st < nvalid ? fmaxf(amax, m) : amax;
            }
            amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
            float sc;
            if (act_scale) {
                sc = h2f(asr[j]);
                sc = sc < 1e-8f ? 1e-8f : sc;
            } else {
                sc = act_scale_from_amax(amax);
            }
            qsv[j] = sc;
            const float inv = 1.0f / sc;
#pragma unroll
            for (int s = 0; s < SPG; ++s) {
                const int st = j * SPG + s;
                v4i c;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    unsigned u = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b)
                        u |= ((unsigned)quant_rn(val(st, 4 * d + b), inv) & 0xffu) << (8 * b);
                    c[d] = (int)u;
                }
                bh[st] = c;
            }
            if (LC && lane < 16 && j < ng) xs_s[lr * G + gb + j] = sc;
        }
    }
#pragma unroll
    for (int q = 0; q < kSt; ++q) {
        const int i = threadIdx.x + q * blockDim.x;
        if (i < kTile * G) {
            ws_s[i] = h2f(wsr[q]);
            if constexpr (!QX) xs_s[i] = xsr[q];
        }
    }
    __syncthreads();

    const int orow = 4 * (lane >> 4);    // this lane's 4 output rows: orow .. orow+3
    float terms[LC ? 1 : MAXG][4];
#pragma unroll
    for (int j = 0; j < MAXG; ++j) {
        v4i P = zero;
#pragma unroll
        for (int s = 0; s < SPG; ++s) {
            const int step = j * SPG + s;
            const int slot = step % KD;
            if (step < nvalid) {   // wave-uniform
                if constexpr (BH)
                    P = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[slot], bh[step], P, 0, 0, 0);
                else
                    P = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[slot], b[slot], P, 0, 0, 0);
            }
            load(slot, step + KD);
        }
        const int gi = gb + (j < ng ? j : 0);
        if constexpr (LC) {
            if (j < ng && lr < ns) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    tl[(gi * ns + lr) * kTile + orow + r] = (float)P[r] * ws_s[(orow + r) * G + gi];
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) terms[j][r] = (float)P[r] * ws_s[(orow + r) * G + gi];
        }
        if constexpr (kDbg) {
            if (j < ng && lr < N) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = row0 + orow + r;
                    if (row < M && dbg.in(row, lr)) dbg.at(row, lr, gb + j, G) = P[r];
                }
            }
        }
    }

    if constexpr (LC) {
        // one lane per output runs the whole chain in group order
        __syncthreads();
        // (EPI 1: one lane per SwiGLU pair runs both rows' chains)
        constexpr int RPL = EPI == 1 ? 2 : 1;   // rows per lane
        for (int t = threadIdx.x; t < kTile / RPL * N; t += blockDim.x) {
            const int r = (t & (kTile / RPL - 1)) * RPL, tok = t / (kTile / RPL);
            const float* tp = tl + tok * kTile + r;      // term of group gi at gi * ns * kTile
            const float* xp = xs_s + tok * G;
            float acc[RPL] = {};
            // eight groups' operands read before their eight fmas, so the
            // chain waits on LDS once per eight groups, not once per group
            int gi = 0;
            for (; gi + 8 <= G; gi += 8) {
                float tv[8][RPL], xv[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
#pragma unroll
                    for (int q = 0; q < RPL; ++q) tv[u][q] = tp[(gi + u) * ns * kTile + q];
                    xv[u] = xp[gi + u];
                }
#pragma unroll
                for (int u = 0; u < 8; ++u)
#pragma unroll
                    for (int q = 0; q < RPL; ++q) acc[q] = __builtin_fmaf(tv[u][q], xv[u], acc[q]);
            }
            for (; gi < G; ++gi)
#pragma unroll
                for (int q = 0; q < RPL; ++q)
                    acc[q] = __builtin_fmaf(tp[gi * ns * kTile + q], xp[gi], acc[q]);
            if (row0 + r < M) {
                if constexpr (EPI == 1)
                    Y[(size_t)tok * (M >> 1) + ((row0 + r) >> 1)] = swiglu_h(f2h(acc[0]), f2h(acc[1]));
                else
                    Y[(size_t)tok * M + row0 + r] = f2h(acc[0]);
            }
        }
    } else {
        // this lane's token scales for the wave's groups, read before the chain
        // (the chain's LDS writes would otherwise keep these reads inside it)
        float xsv[MAXG];
#pragma unroll
        for (int j = 0; j < MAXG; ++j) {
            if constexpr (QX) xsv[j] = qsv[j];
            else xsv[j] = xs_s[lr * G + gb + (j < ng ? j : 0)];
        }

        // Group-ordered fp32 chain: wave 0 starts from zero, each wave continues
        // the previous wave's sums over its own groups.
        for (int w = 0; w < NW; ++w) {
            if (wave == w) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float acc = w == 0 ? 0.0f : chain[lr * kTile + orow + r];
#pragma unroll
                    for (int j = 0; j < MAXG; ++j)
                        if (j < ng) acc = __builtin_fmaf(terms[j][r], xsv[j], acc);
                    chain[lr * kTile + orow + r] = acc;
                }
            }
            __syncthreads();
        }
        if constexpr (EPI == 1) {
            for (int i = threadIdx.x; i < kTile / 2 * N; i += blockDim.x) {
                const int t = i / (kTile / 2), r = 2 * (i - t * (kTile / 2));
                if (row0 + r < M)
                    Y[(size_t)t * (M >> 1) + ((row0 + r) >> 1)] =
                        swiglu_h(f2h(chain[t * kTile + r]), f2h(chain[t * kTile + r + 1]));
            }
        } else {
            for (int i = threadIdx.x; i < kTile * N; i += blockDim.x) {
                const int t = i / kTile, r = i - t * kTile;
                if (row0 + r < M) Y[(size_t)t * M + row0 + r] = f2h(chain[t * kTile + r]);
            }
        }
    }
}

template <bool D>
using MfmaFn = void (*)(const int8_t*, const uint16_t*, const int8_t*, const float*,
                        const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, DbgWindow,
                        int, int, int, int);

// Steps (64 bytes of K) a wave may hold as fp16 for in-kernel quantization
// (the largest counts that compile without scratch spills for gfx950).
constexpr int kMfmaQxSteps = 16;
constexpr int kMfmaQxStepsSmooth = 8;

// The MFMA kernel with in-kernel quantization (qx 1 plain, 2 smooth_inv)
// and / or the SwiGLU pair epilogue (epi 1); null for a shape outside the
// instantiated set (gemv_mfma_fused.hip).
MfmaFn<false> mfma_fused(int qx, int epi, bool lc, int spg, int maxg);

using DotFn = void (*)(const int8_t*, const uint16_t*, const int8_t*, const float*,
                       const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, DbgWindow,
                       int, int, int, int, int, int, ProArgs);


// The N == 1 kernel families, each instantiated in its own translation unit
// (kd: ring depth 3..5; lgl: log2 of the lanes per group, 2..5).
DotFn dot_plain(int R, bool qx, int K, int kd, int lgl);        // gemv_dot.hip
DotFn dot_pro(int R, int pro, int K, int kd, int lgl);          // gemv_dot_pro.hip
DotFn dot_swiglu(int pro, int K, int kd, int lgl, bool sep = false);  // gemv_dot_swiglu.hip

// Instantiation helpers for those units.
template <int R, int KD, bool QX, int XV, int NWV, int PRO, int EPI>
DotFn dot_for_lg(int lg) {
    switch (lg) {
        case 2: return gemv_dot_kernel<R, KD, 4, QX, XV, NWV, PRO, EPI>;     // g64
        case 3: return gemv_dot_kernel<R, KD, 8, QX, XV, NWV, PRO, EPI>;     // g128
        case 4: return gemv_dot_kernel<R, KD, 16, QX, XV, NWV, PRO, EPI>;    // g256
        default: return gemv_dot_kernel<R, KD, 32, QX, XV, NWV, PRO, EPI>;   // g512
    }
}

template <int R, bool QX, int XV, int NWV, int PRO, int EPI>
DotFn dot_for_kd(int kd, int lg) {
    switch (kd) {
        case 3: return dot_for_lg<R, 3, QX, XV, NWV, PRO, EPI>(lg);
        case 4: return dot_for_lg<R, 4, QX, XV, NWV, PRO, EPI>(lg);
        default: return dot_for_lg<R, 5, QX, XV, NWV, PRO, EPI>(lg);
    }
}

// Staged int8 codes: 4 waves, XV = 1 or 3 16-byte chunks per thread
// (K <= 4096 / 12288).  In-kernel quantization: 8 waves, XV = 1 or 3 chunks of
// 8 fp16 values per thread (K <= 4096 / 12288).  Larger K use a tail loop
// (plain quantization only: a fused prologue needs K <= 12288).
template <int R, bool QX, int NWV, int PRO, int EPI>
DotFn dot_for_xv(int K, int kd, int lg) {
    return K <= (QX ? 8 : 16) * 64 * NWV ? dot_for_kd<R, QX, 1, NWV, PRO, EPI>(kd, lg)
                                         : dot_for_kd<R, QX, 3, NWV, PRO, EPI>(kd, lg);
}

}  // namespace gv
}  // namespace fa

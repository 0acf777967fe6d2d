// chain.hip -- a decode step's W8A8 linears (one token) as ONE persistent
// launch: the device orders the linears, and the weight stream of linear
// s + 1 is already in flight while linear s finishes.
//
// Replaces the per-linear launch sequence of DualAREngine::decode_step
// (src/engine/dual_ar_engine.cc:576-648: rms_norm -> quantize -> int8 GEMV ->
// ... per projection) for the int8 projections; each step computes exactly
// what the fused N == 1 GEMV kernels compute (gemv_kernels.h, R = 2):
//   prologue 0: x -> per-group dynamic int8 codes (int8_gemm.cu:147-211);
//   prologue 2: h = fp16(x + x2) (residual_add, ffn_activations.cu:41-45),
//               rms_norm(h, gamma) (rms_norm.cu:10-58), then the quantizer; the
//               step's first row block writes h to h_out;
//   epilogue 0: y[row] = fp16 of the group-ordered fp32 sum (int8_gemm.cu:
//               213-234, acc = fma(float(P_g) * ws, xs, acc) over g in order);
//   epilogue 1: rows 2i / 2i + 1 are the interleaved w1 / w3 rows of FFN
//               column i: y[i] = fp16(fp16(silu(gate)) * up)
//               (silu_forward then mul_forward, ffn_activations.cu:12-17, 35-39).
// Every int32 group partial is exact and every fp32 operation happens in the
// reference order, so each step's output is bit-identical to the oracle's.
//
// Work.  Step s has nblocks row blocks of ROWS rows; workgroup b owns blocks
// b, b + grid, ... of every step.  Its work list -- (step, block, 512-byte
// pass) in order -- is walked by two uniform cursors: a load cursor KD passes
// ahead fills a register ring of 16-byte weight loads, a consume cursor
// drains it.  The weight loads never depend on activations, so the ring runs
// ahead across block and step boundaries: the next step's weights are in
// flight while the workgroup waits for the previous step to finish.
//
// Ordering.  When the consumer reaches its first block of step s it waits
// until every block of step s - 1 is done (a per-step counter that each
// workgroup bumps once, by its block count, after its last block of the
// step), then forms the step's activation codes in LDS.  The grid is
// launched cooperatively (all workgroups resident), so every awaited block
// has a running owner.  Each wait is bounded: past `spin_limit` polls the
// workgroup raises the error word and every waiting workgroup gives up.
//
// Signals.  A workgroup adds its block count to the step's counter once,
// after its last block of the step; the one whose add completes the count
// writes the launch's epoch into the step's flag, one copy per XCD (128 bytes
// apart), and waiters poll the copy of their own XCD -- so no line is hit by
// every workgroup at once.  The epoch changes every launch, so flags are
// never cleared.
//
// Memory.  Outputs (y, h_out) are written and activation inputs read with
// agent-scope accesses (sc1: coherent across the XCDs' L2s, no whole-cache
// write-back or invalidation), and a writer waits for its stores to complete
// (s_waitcnt vmcnt(0)) before its counter add.
//
// sync[s]: finished blocks of step s (0 .. nsteps - 1); sync[nsteps]: error
// word; both zero before a launch.  flags[(s * 8 + x) * 32]: step s done, for
// XCD x.
#include "common.h"
#include "chain.h"

namespace fa {
namespace {

using ch::ChainStepDev;

constexpr int R = 2;              // rows per wave
constexpr int RL = 64 / R;        // lanes per row
constexpr int PB = RL * 16;       // bytes of a row per pass
constexpr int KD = kChainRing;    // passes in flight per wave

// Global-address-space loads: the ring selects between two row pointers,
// which would otherwise leave generic pointers and flat loads (counted by
// lgkmcnt as well, so every LDS wait would drain the ring).
typedef __attribute__((address_space(1))) const v4i gv4i;
typedef __attribute__((address_space(1))) const uint16_t gu16;
__device__ __forceinline__ v4i ld16c(const int8_t* p) {
    return *(gv4i*)(__builtin_bit_cast(uintptr_t, p));
}
__device__ __forceinline__ uint16_t ldu16g(const uint16_t* p) {
    return *(gu16*)(__builtin_bit_cast(uintptr_t, p));
}

// Agent-scope (sc1) accesses: outputs and signals, coherent across the XCDs.
typedef __attribute__((address_space(1))) uint32_t gu32;
__device__ __forceinline__ gu32* g32(const void* p) {
    return (gu32*)(__builtin_bit_cast(uintptr_t, p));
}
__device__ __forceinline__ v4i ld16_coh(const uint16_t* p) {
    gu32* q = g32(p);
    v4i r;
    r.x = (int)__hip_atomic_load(q + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    r.y = (int)__hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    r.z = (int)__hip_atomic_load(q + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    r.w = (int)__hip_atomic_load(q + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return r;
}
// a step's activation input (written by an earlier step of this launch)
__device__ __forceinline__ v4i ld16_act(const uint16_t* p) {
#ifdef FA_CHAIN_X_CACHED
    return ld16c(reinterpret_cast<const int8_t*>(p));
#else
    return ld16_coh(p);
#endif
}
__device__ __forceinline__ void st16_coh(uint16_t* p, const v4i& v) {
    gu32* q = g32(p);
    __hip_atomic_store(q + 0, (uint32_t)v.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 1, (uint32_t)v.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 2, (uint32_t)v.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(q + 3, (uint32_t)v.w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st2_coh(uint16_t* p, uint16_t v) {
    asm volatile("global_store_short %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
// every store this wave issued has completed
__device__ __forceinline__ void stores_done() { asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); }

// Max of a non-negative float over aligned blocks of 2^lgl lanes.
__device__ __forceinline__ float lane_block_max(float m, int lgl) {
    if (lgl >= 1) m = fmaxf(m, dpp_f<0xB1>(m));
    if (lgl >= 2) m = fmaxf(m, dpp_f<0x4E>(m));
    if (lgl >= 3) m = fmaxf(m, dpp_f<0x141>(m));
    if (lgl >= 4) m = fmaxf(m, dpp_f<0x140>(m));
    if (lgl >= 5) m = fmaxf(m, __shfl_xor(m, 16, 64));
    if (lgl >= 6) m = fmaxf(m, __shfl_xor(m, 32, 64));
    return m;
}

// Exact int32 sum over aligned blocks of LG lanes (LG <= 16: DPP in a row).
template <int LG>
__device__ __forceinline__ int lane_group_sum(int p) {
    if constexpr (LG >= 2) p += __builtin_amdgcn_update_dpp(0, p, 0xB1, 0xF, 0xF, false);
    if constexpr (LG >= 4) p += __builtin_amdgcn_update_dpp(0, p, 0x4E, 0xF, 0xF, false);
    if constexpr (LG >= 8) p += __builtin_amdgcn_update_dpp(0, p, 0x141, 0xF, 0xF, false);
    if constexpr (LG >= 16) p += __builtin_amdgcn_update_dpp(0, p, 0x140, 0xF, 0xF, false);
    return p;
}

// One row block of a step, as the ring needs it (uniform values).
struct Blk {
    int s, blk, P;                // step, block, passes padded to a multiple of KD
};

// LG = g / 16 lanes per K-group (g = 64, 128 or 256), NWV waves per workgroup.
template <int LG, int NWV>
__global__ __launch_bounds__(NWV * 64) void chain_kernel(const ChainStepDev* __restrict__ steps,
                                                         int nsteps, int* __restrict__ sync,
                                                         int* __restrict__ flags, int epoch,
                                                         int spin_limit, int kp_max, int g_pad,
                                                         int kh) {
    constexpr int NT = NWV * 64;
    constexpr int GPP = RL / LG;            // groups per row per pass
    constexpr int ROWS = NWV * R;           // rows per block
    constexpr int XV = kChainMaxK / (NT * 8);          // activation chunks per thread
    constexpr int XV2 = kChainMaxKPro / (NT * 8);      // ... with prologue 2
    static_assert(XV * NT * 8 == kChainMaxK && XV2 * NT * 8 == kChainMaxKPro, "chunking");
    extern __shared__ __align__(16) float lds[];
    int8_t* xq_s = reinterpret_cast<int8_t*>(lds);                // [kp_max]
    float* xs_s = lds + kp_max / 4;                               // [g_pad]
    uint16_t* h_s = reinterpret_cast<uint16_t*>(xs_s + g_pad);    // [kh] (prologue 2)
    float* red_s = reinterpret_cast<float*>(h_s + kh);            // [33]
    int* ctl_s = reinterpret_cast<int*>(red_s + 34);              // [2]
    uint16_t* y_s0 = reinterpret_cast<uint16_t*>(ctl_s + 2);      // [2][ROWS]

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int rsub = lane / RL;
    const int li = lane % RL;
    const int lane_k = li * 16;
    const int b = blockIdx.x;
    const int grid = gridDim.x;
    int* const err = sync + nsteps;
    const v4i zero = {0, 0, 0, 0};

    // this workgroup's first block at or after step s (s == nsteps: none)
    auto first_from = [&](int s) {
        while (s < nsteps && b >= steps[s].nblocks) ++s;
        Blk r;
        r.s = s;
        r.blk = b;
        r.P = s < nsteps ? (steps[s].passes + KD - 1) / KD * KD : KD;
        return r;
    };
    auto next_of = [&](const Blk& c) {
        if (c.blk + grid < steps[c.s].nblocks) {
            Blk r = c;
            r.blk += grid;
            return r;
        }
        return first_from(c.s + 1);
    };
    // Per-lane weight-row and scale-row pointers of a block (row clamped;
    // past the end of the list: row 0 of step 0, never consumed).
    struct RowPtr {
        const int8_t* w;
        const uint16_t* ws;
        int K, lg_g;
    };
    auto row_ptr = [&](const Blk& c) {
        const bool live = c.s < nsteps;
        const ChainStepDev& st = steps[live ? c.s : 0];
        const int row = (c.blk * NWV + wave) * R + rsub;
        const int rowc = live ? (row < st.M ? row : st.M - 1) : 0;
        RowPtr r;
        r.w = st.W + (size_t)rowc * st.K;
        r.ws = st.w_scale + (size_t)rowc * st.G;
        r.K = st.K;
        r.lg_g = st.lg_g;
        return r;
    };

    Blk cur = first_from(0);
    if (cur.s >= nsteps) return;

    v4i a[KD];
    uint16_t sc[KD];
    // pass p of a block: bytes past K (padding passes) re-read the row start
    auto load = [&](int slot, const RowPtr& rp, int pass) {
        const int k = pass * PB + lane_k;
        const int kk = k < rp.K ? k : 0;
        a[slot] = ld16c(rp.w + kk);
        sc[slot] = ldu16g(rp.ws + (kk >> rp.lg_g));
    };
    {
        const RowPtr rp = row_ptr(cur);
#pragma unroll
        for (int q = 0; q < KD; ++q) load(q, rp, q);
    }

    int done_here = 0;        // blocks of `prepared` finished by this workgroup
    int fin = 0;              // blocks finished (parity picks the output staging half)
    int prepared = -1;        // step whose activation codes are in LDS

    auto signal = [&](int s) {
        stores_done();
        __syncthreads();
        if (tid == 0) {
            const int old = (int)__hip_atomic_fetch_add(g32(sync + s), (uint32_t)done_here,
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // every other owner's add (each after its own stores completed)
            // is performed: the step is done
            if (old + done_here == steps[s].nblocks) {
#pragma unroll
                for (int x = 0; x < 8; ++x)
                    __hip_atomic_store(g32(flags + (s * 8 + x) * 32), (uint32_t)epoch,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        done_here = 0;
    };

    for (;;) {
        const ChainStepDev& st = steps[cur.s];
        const int K = st.K, lg_g = st.lg_g, M = st.M;
        // ---- a new step: signal the last one, wait for s - 1, prologue
        if (cur.s != prepared) {
            if (prepared >= 0) signal(prepared);
            const int s = cur.s;
            if (tid == 0) {
                int status = 0;
                if (s > 0) {
                    gu32* const flag = g32(flags + ((s - 1) * 8 + (b & 7)) * 32);
                    int polls = 0;
                    while ((int)__hip_atomic_load(flag, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) != epoch) {
                        if (++polls > spin_limit ||
                            ((polls & 63) == 0 &&
                             __hip_atomic_load(g32(err), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
                            status = 1;
                            __hip_atomic_store(g32(err), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                asm volatile("" : : : "memory");
                ctl_s[1] = status;
            }
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(ctl_s[1]) != 0) break;
            const uint16_t* const X = st.X;
            v4i xr[XV];
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const int k = (tid + i * NT) * 8;
                xr[i] = ld16_act(X + (k < K ? k : K - 8));
            }
            if (st.pro == 2) {
                v4i x2r[XV2], gmr[XV2];
                const uint16_t* const x2 = st.x2 ? st.x2 : X;
#pragma unroll
                for (int i = 0; i < XV2; ++i) {
                    const int k = (tid + i * NT) * 8;
                    const int kc = k < K ? k : K - 8;
                    x2r[i] = ld16_act(x2 + kc);
                    gmr[i] = ld16c(reinterpret_cast<const int8_t*>(st.gamma + kc));
                }
                // h = fp16(x + x2) into LDS (and to h_out from the owner of block 0)
#pragma unroll
                for (int i = 0; i < XV2; ++i) {
                    const int k = (tid + i * NT) * 8;
                    uint16_t* h = reinterpret_cast<uint16_t*>(&xr[i]);
                    if (st.x2) {
                        const uint16_t* r = reinterpret_cast<const uint16_t*>(&x2r[i]);
#pragma unroll
                        for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(h[e]) + h2f(r[e]));
                    }
                    if (k < K) {
                        *reinterpret_cast<v4i*>(h_s + k) = xr[i];
                        if (st.h_out && b == 0) st16_coh(st.h_out + k, xr[i]);
                    }
                }
                __syncthreads();
                // Sum of squares in the reference's order (rms_norm.cu:22-41):
                // T = min(next_pow2(K), 1024) threads, thread t sums h[t],
                // h[t + T], ... with FMAs, each 32-thread warp reduces by the
                // shuffle-down tree, then the warp sums by the same tree.
                int T = 1;
                while (T < K) T <<= 1;
                if (T > 1024) T = 1024;
                const int lanes = T < 32 ? 32 : T;
                for (int t0 = 0; t0 < lanes; t0 += NT) {
                    const int tt = t0 + tid;
                    float loc = 0.0f;
                    if (tt < T)
                        for (int k = tt; k < K; k += T) {
                            const float v = h2f(h_s[k]);
                            loc = __builtin_fmaf(v, v, loc);
                        }
                    loc = warp32_sum_down(loc);
                    if (tt < lanes && (tt & 31) == 0) red_s[tt >> 5] = loc;
                }
                __syncthreads();
                if (tid < 32) {
                    const int nw = (T + 31) >> 5;
                    float v = tid < nw ? red_s[tid] : 0.0f;
                    v = warp32_sum_down(v);
                    if (tid == 0) red_s[32] = rms_inv(v, K, st.eps);
                }
                __syncthreads();
                const float rr = red_s[32];
#pragma unroll
                for (int i = 0; i < XV2; ++i) {
                    uint16_t* h = reinterpret_cast<uint16_t*>(&xr[i]);
                    const uint16_t* gm = reinterpret_cast<const uint16_t*>(&gmr[i]);
#pragma unroll
                    for (int e = 0; e < 8; ++e) h[e] = f2h((h2f(h[e]) * rr) * h2f(gm[e]));
                }
            }
            // Per-group dynamic quantization: chunk c = x[8c, 8c + 8) sits in
            // thread c % NT, so a group's g / 8 chunks are consecutive lanes of
            // one wave; their |v| max comes from DPP / shuffles.
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const int c = tid + i * NT;
                const int k = c * 8;
                const bool ok = k < K;
                const uint16_t* h = reinterpret_cast<const uint16_t*>(&xr[i]);
                float v[8];
                float m = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    v[e] = h2f(h[e]);
                    m = fmaxf(m, fabsf(v[e]));
                }
                if (!ok) m = 0.0f;
                m = lane_block_max(m, lg_g - 3);
                const float scl = act_scale_from_amax(m);
                if (ok) {
                    const float inv = 1.0f / scl;
                    int q[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) q[e] = quant_rn(v[e], inv);
                    uint2 u;
                    u.x = (uint32_t)(q[0] & 0xff) | ((uint32_t)(q[1] & 0xff) << 8) |
                          ((uint32_t)(q[2] & 0xff) << 16) | ((uint32_t)(q[3] & 0xff) << 24);
                    u.y = (uint32_t)(q[4] & 0xff) | ((uint32_t)(q[5] & 0xff) << 8) |
                          ((uint32_t)(q[6] & 0xff) << 16) | ((uint32_t)(q[7] & 0xff) << 24);
                    *reinterpret_cast<uint2*>(xq_s + k) = u;
                    if ((c & ((1 << (lg_g - 3)) - 1)) == 0) xs_s[k >> lg_g] = scl;
                }
            }
            __syncthreads();
            prepared = s;
        }

        // ---- the block's passes, KD per round; each consumed slot is
        // refilled with pass + KD of this block or, past its padded end,
        // with the next block's first passes (selected, not branched)
        const Blk nxt = next_of(cur);
        const RowPtr rc = row_ptr(cur), rn = row_ptr(nxt);
        float acc[R] = {0.0f, 0.0f};
        for (int base = 0; base < cur.P; base += KD) {
#pragma unroll
            for (int q = 0; q < KD; ++q) {
                const int kbase = (base + q) * PB;
                const int k = kbase + lane_k;
                v4i bq = *reinterpret_cast<const v4i*>(xq_s + (k < K ? k : 0));
                if (k >= K) bq = zero;
                int p = __builtin_amdgcn_sdot4(a[q].x, bq.x, 0, false);
                p = __builtin_amdgcn_sdot4(a[q].y, bq.y, p, false);
                p = __builtin_amdgcn_sdot4(a[q].z, bq.z, p, false);
                p = __builtin_amdgcn_sdot4(a[q].w, bq.w, p, false);
                p = lane_group_sum<LG>(p);
                const float term = (float)p * h2f(sc[q]);
                float xsv[GPP];
                const float* xp = xs_s + (kbase >> lg_g);
#pragma unroll
                for (int j = 0; j < GPP; ++j) xsv[j] = xp[j];
#pragma unroll
                for (int j = 0; j < GPP; ++j) {
                    if (kbase + j * LG * 16 < K) {
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            const float tj = __builtin_bit_cast(
                                float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, term),
                                                                 r * RL + j * LG));
                            acc[r] = __builtin_fmaf(tj, xsv[j], acc[r]);
                        }
                    }
                }
                const int np = base + q + KD;
                const bool here = np < cur.P;
                RowPtr rp;
                rp.w = here ? rc.w : rn.w;
                rp.ws = here ? rc.ws : rn.ws;
                rp.K = here ? rc.K : rn.K;
                rp.lg_g = here ? rc.lg_g : rn.lg_g;
                load(q, rp, here ? np : np - cur.P);
            }
        }

        // ---- outputs: staged in LDS, stored by wave 0 (agent-coherent)
        {
            uint16_t* const y_s = y_s0 + (fin & 1) * ROWS;
            ++fin;
            if (lane == 0) {
                if (st.epi == 1) {
                    y_s[wave] = f2h(h2f(f2h(silu_f(h2f(f2h(acc[0]))))) * h2f(f2h(acc[1])));
                } else {
                    y_s[2 * wave] = f2h(acc[0]);
                    y_s[2 * wave + 1] = f2h(acc[1]);
                }
            }
            __syncthreads();
            const int per = st.epi == 1 ? ROWS / 2 : ROWS;
            const int total_out = st.epi == 1 ? M / 2 : M;
            const int ob = cur.blk * per;
            const int cnt = min(per, total_out - ob);
            if (tid < (cnt + 1) / 2) {
                uint16_t* dst = st.Y + ob + 2 * tid;
                if (2 * tid + 1 < cnt)
                    __hip_atomic_store(g32(dst),
                                       (uint32_t)y_s[2 * tid] | ((uint32_t)y_s[2 * tid + 1] << 16),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                else
                    st2_coh(dst, y_s[2 * tid]);
            }
            ++done_here;
        }
        if (nxt.s >= nsteps) {
            signal(cur.s);
            break;
        }
        cur = nxt;
    }
    stores_done();
}

__global__ void chain_zero_kernel(int* p, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0;
}

template <int LG>
hipError_t launch_lg(const ChainPlan& p, hipStream_t stream) {
    hipLaunchKernelGGL(chain_zero_kernel, dim3(1), dim3(256), 0, stream, p.sync, p.nsteps + 1);
    const ChainStepDev* steps = p.steps;
    int nsteps = p.nsteps, spin = p.spin_limit, kp = p.kp_max, gp = p.g_pad, kh = p.kh;
    int* sync = p.sync;
    int* flags = p.flags;
    int epoch = p.epoch;
    void* args[] = {&steps, &nsteps, &sync, &flags, &epoch, &spin, &kp, &gp, &kh};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(chain_kernel<LG, kChainWaves>),
                                      dim3((unsigned)p.grid), dim3(kChainWaves * 64), args, p.lds,
                                      stream);
}

template <int LG>
int grid_lg(size_t lds) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, chain_kernel<LG, kChainWaves>,
                                                     kChainWaves * 64, lds) != hipSuccess)
        return 0;
    return cus * per_cu;
}

}  // namespace

size_t chain_lds_bytes(int kp_max, int g_pad, int kh) {
    return (size_t)kp_max + (size_t)g_pad * 4 + (size_t)kh * 2 + 36 * 4 +
           (size_t)2 * kChainWaves * R * 2;
}

int chain_rows_per_task() { return kChainWaves * R; }
int chain_max_k() { return kChainMaxK; }
int chain_max_k_pro() { return kChainMaxKPro; }

int chain_grid(int lg, size_t lds) {
    if (lg == 6) return grid_lg<4>(lds);
    if (lg == 7) return grid_lg<8>(lds);
    if (lg == 8) return grid_lg<16>(lds);
    return 0;
}

hipError_t launch_chain(const ChainPlan& p, hipStream_t stream) {
    if (p.lg == 6) return launch_lg<4>(p, stream);
    if (p.lg == 7) return launch_lg<8>(p, stream);
    if (p.lg == 8) return launch_lg<16>(p, stream);
    return hipErrorInvalidValue;
}

}  // namespace fa

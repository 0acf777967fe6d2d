// chain.hip -- a decode step's W8A8 linears (one token) as ONE persistent
// launch: the device orders the linears, and every workgroup keeps the next
// linear's weights streaming into LDS while the previous one finishes.
//
// Replaces the per-linear launch sequence of DualAREngine::decode_step
// (src/engine/dual_ar_engine.cc:576-648: rms_norm -> quantize -> int8 GEMV ->
// ... per projection) for the int8 projections; each step computes exactly
// what the fused N == 1 GEMV kernels compute (gemv_kernels.h):
//   prologue 0: x -> per-group dynamic int8 codes (int8_gemm.cu:147-211);
//   prologue 2: h = fp16(x + x2) (residual_add, ffn_activations.cu:41-45),
//               rms_norm(h, gamma) (rms_norm.cu:10-58), then the quantizer;
//               workgroup 0 writes h to h_out;
//   epilogue 0: y[row] = fp16 of the group-ordered fp32 sum (int8_gemm.cu:
//               213-234, acc = fma(float(P_g) * ws, xs, acc) over g in order);
//   epilogue 1: rows 2i / 2i + 1 are the interleaved w1 / w3 rows of FFN
//               column i: y[i] = fp16(fp16(silu(gate)) * up)
//               (silu_forward then mul_forward, ffn_activations.cu:12-17, 35-39).
// Every int32 group partial is exact and every fp32 operation happens in the
// reference order, so each step's output is bit-identical to the oracle's.
//
// Work.  One workgroup per CU: 8 streaming waves and one control wave.  Step
// s's rows, in pairs, are split evenly over the workgroups (contiguous pair
// ranges); a workgroup's (pair, 512-byte pass) items are split evenly over
// its streaming waves (contiguous item ranges, which may cut a row between
// two waves).  An item is one pass of a row pair: each of the 64 lanes
// multiplies 16 weight bytes with 16 activation codes (4 v_dot4), lanes of
// one K-group add their partials with DPP, and the group's leader lane
// writes the exact term float(P_g) * ws to an LDS term table [row][group].
// At the step's end the control wave runs each row's fp32 chain over the
// terms in group order -- so splitting a row between waves changes nothing.
//
// Ring.  Each streaming wave owns an LDS ring of DEPTH slots.  A slot holds
// one item's weights (64 lanes x 16 bytes) and the fp16 scale pair of each
// lane's group (64 x 4 bytes), both loaded straight into LDS by
// global_load_lds (no registers held).  The wave's item list runs across
// steps, and the ring is refilled DEPTH items ahead of the consumer as soon
// as a slot is read, so while the workgroup waits for step s - 1 to finish
// everywhere, DEPTH items of step s are already landing (8 x DEPTH KB per CU).
// The streaming waves issue no other global memory operation: every wait
// is `s_waitcnt vmcnt(2 * (DEPTH - 1))`, exactly one item old.
//
// Control wave.  Between steps (three workgroup barriers): it turns the
// terms of step s - 1 into outputs and stores them (agent-scope sc1 stores),
// waits for its stores, counts the workgroup into the step's counter (8
// copies, one per XCD, 128 bytes apart; adds whose result is not awaited),
// polls its XCD's copy until every workgroup is counted, and loads step s's
// inputs into LDS with sc1 direct-to-LDS loads; then all waves form the
// step's int8 codes in LDS (the prologue), and the streaming waves go on.
// Each wait is bounded: past `spin_limit` polls the wave raises the error
// word and every workgroup leaves.  The launch is an ordinary one whose grid
// is the number of workgroups the device holds at once, so every awaited
// workgroup is running (a missing one would only make the bounded waits
// give up).
//
// flags[(s * 8 + x) * 32]: workgroups done with step s, copy x; sync[nsteps]:
// error word.  A small kernel zeroes both before each launch.
#include "common.h"
#include "chain.h"

namespace fa {
namespace {

using ch::ChainLds;
using ch::ChainStepDev;

#ifdef FA_CHAIN_TRACE
constexpr bool kTrace = true;    // measurement build: per-step timestamps
#else
constexpr bool kTrace = false;
#endif
#ifdef FA_CHAIN_SIG_FLAGS
constexpr bool kSigCopies = false;  // measurement builds: one counter, last adder raises flags
#else
constexpr bool kSigCopies = true;   // 8 counter copies, adds not awaited (measured faster)
#endif
#ifdef FA_CHAIN_SLEEP
constexpr int kSleep = FA_CHAIN_SLEEP;
#else
constexpr int kSleep = 1;
#endif
#ifdef FA_CHAIN_PREFETCH
constexpr bool kPrefetch = true;    // measurement builds: cache prefetch ahead of the ring
#else
constexpr bool kPrefetch = false;   // measured slower: the prefetched lines do not survive in L2
#endif

constexpr int NS = kChainWaves;          // streaming waves
constexpr int NTS = NS * 64;             // streaming threads
constexpr int NTH = NTS + 64;            // plus the control wave
constexpr int PB = 512;                  // bytes of a row per item (32 lanes x 16)
constexpr int kSlot = 1024 + 256;        // ring slot: weights, then scale pairs
constexpr int XV = kChainMaxK / (NTS * 8);   // 8-value chunks per streaming thread
static_assert(XV * NTS * 8 == kChainMaxK, "chunking");

typedef __attribute__((address_space(1))) uint32_t gu32;
__device__ __forceinline__ gu32* g32(const void* p) {
    return (gu32*)(__builtin_bit_cast(uintptr_t, p));
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const void*)p);
}

// Direct-to-LDS loads: lane i's bytes land at lds + i * size (m0 = the
// wave-uniform LDS base).
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :: "v"(g), "s"(lds) : "memory");
}
// ... agent-coherent (sc1): data written by other workgroups of this launch
__device__ __forceinline__ void dma16_coh(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off sc1"
                 :: "v"(g), "s"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkm0() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void st2_coh(uint16_t* p, uint16_t v) {
    asm volatile("global_store_short %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st16_coh(uint16_t* p, const v4i& v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

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

// The step fields a cursor needs (wave-uniform).
struct StepC {
    const int8_t* W;
    const uint16_t* ws;
    int M, K, G, lg, passes, mg2;
};
__device__ __forceinline__ StepC step_c(const ChainStepDev& st) {
    StepC c;
    c.W = st.W;
    c.ws = st.w_scale;
    c.M = st.M;
    c.K = st.K;
    c.G = st.G;
    c.lg = st.lg_g;
    c.passes = st.passes;
    c.mg2 = (int)st.MG - 2;
    return c;
}

__device__ __forceinline__ int ufirst(int v) { return __builtin_amdgcn_readfirstlane(v); }

// A wave's walk through its items: step s, pair pl (within the workgroup's
// pairs pa + ...), pass; `rem` items of the step left.  All wave-uniform.
struct Cursor {
    int s, pa, pl, pass, rem;
    StepC c;
};

// LG = g / 16 lanes per K-group (g = 64, 128 or 256); DEPTH ring slots; PF:
// each item issue also touches the weight lines of the item DEPTH + PFD
// ahead (cache prefetch); TR: per-step timestamps (measurement builds).
template <int LG, int DEPTH, bool PF, bool TR>
__global__ __launch_bounds__(NTH, 1) void chain_kernel(const ChainStepDev* __restrict__ steps,
                                                      int nsteps, int* __restrict__ sync,
                                                      int* __restrict__ flags,
                                                      int spin_limit, ChainLds lay,
                                                      unsigned long long* __restrict__ trace) {
    constexpr int NOPS = PF ? 3 : 2;   // global ops per item issue
#ifdef FA_CHAIN_PFD
    constexpr int PFD = FA_CHAIN_PFD;    // measurement builds: other prefetch distances
#else
    constexpr int PFD = 2 * DEPTH;       // prefetch distance beyond the ring
#endif
    extern __shared__ __align__(16) unsigned char smem[];
    const int tid = threadIdx.x;
    const int wave = ufirst(tid >> 6);
    const int lane = tid & 63;
    const bool ctrl = wave == NS;
    const int b = blockIdx.x;
    const int grid = gridDim.x;
    int8_t* const xq_s = reinterpret_cast<int8_t*>(smem + lay.xq);
    float* const xs_s = reinterpret_cast<float*>(smem + lay.xs);
    unsigned char* const stage = smem + lay.stage;       // inputs, then the step's terms
    float* const terms = reinterpret_cast<float*>(stage);   // [group][row of the workgroup]
    float* const red_s = reinterpret_cast<float*>(smem + lay.red);   // [33] + status
    int* const ctl_s = reinterpret_cast<int*>(red_s + 34);
    int* const err = sync + nsteps;
    const v4i zero = {0, 0, 0, 0};
    const int rsub = lane >> 5;              // row of the pair this lane reads
    const int lk = (lane & 31) * 16;         // byte of the pass this lane reads
    auto tr = [&](int s, int e) {
        if constexpr (TR) {
            if (ctrl && lane == 0)
                trace[((size_t)s * grid + b) * 8 + e] = __builtin_amdgcn_s_memrealtime();
        }
    };

    // pairs [pa, pb) of a step with M rows owned by this workgroup
    auto wg_pairs = [&](int M, int& pa, int& pb) {
        const int64_t P = (M + 1) >> 1;
        pa = (int)(P * b / grid);
        pb = (int)(P * (b + 1) / grid);
    };
    // this wave's first item of step s: cursor fields
    auto start = [&](Cursor& u, int s) {
        u.s = s;
        if (s >= nsteps) return;
        u.c = step_c(steps[s]);
        int pa, pb;
        wg_pairs(u.c.M, pa, pb);
        const int n = (pb - pa) * u.c.passes;
        const int i0 = (int)((int64_t)n * wave / NS);
        const int i1 = (int)((int64_t)n * (wave + 1) / NS);
        u.pa = pa;
        u.pl = i0 / u.c.passes;
        u.pass = i0 - u.pl * u.c.passes;
        u.rem = i1 - i0;
    };
    // next item (skipping steps where this wave has none)
    auto advance = [&](Cursor& u) {
        if (++u.pass == u.c.passes) {
            u.pass = 0;
            ++u.pl;
        }
        if (--u.rem == 0) {
            start(u, u.s + 1);
            while (u.s < nsteps && u.rem == 0) start(u, u.s + 1);
        }
    };
    auto first = [&](Cursor& u) {
        start(u, 0);
        while (u.s < nsteps && u.rem == 0) start(u, u.s + 1);
    };
    // this lane's weight and scale-pair addresses of item u (rows past M
    // read row M - 1, bytes past K the row start; such rows are never
    // stored and such bytes' products are dropped)
    auto item_addr = [&](const Cursor& u, const int8_t*& wp, const uint16_t*& sp) {
        int row = 2 * (u.pa + u.pl) + rsub;
        row = row < u.c.M ? row : u.c.M - 1;
        int k = u.pass * PB + lk;
        k = k < u.c.K ? k : 0;
        wp = u.c.W + (uint32_t)(row * u.c.K + k);
        int lo = (row * u.c.G + (k >> u.c.lg)) & ~1;
        lo = lo < u.c.mg2 ? lo : u.c.mg2;
        sp = u.c.ws + lo;
    };

    const uint32_t ring = lds_addr(smem) + (uint32_t)(ctrl ? 0 : wave) * DEPTH * kSlot;
    const uint32_t junk = lds_addr(smem + lay.red) + 64 * 4;   // prefetch landing (256 B)
    Cursor ld{}, pf{}, cs{};
    auto issue = [&](int slot) {
        const int8_t* wp = steps[0].W;
        const uint16_t* sp = steps[0].w_scale;
        if (ld.s < nsteps) {
            item_addr(ld, wp, sp);
            advance(ld);
        }
        // past the end of the list: re-read a valid address (keeps every
        // wave's wait counts exact); those slots are never consumed
        const uint32_t base = ufirst(ring + (uint32_t)slot * kSlot);
        dma16(wp, base);
        dma4(sp, base + 1024);
        if constexpr (PF) {
            const int8_t* pw = steps[0].W;
            const uint16_t* ps;
            if (pf.s < nsteps) {
                item_addr(pf, pw, ps);
                advance(pf);
            }
            // every 64-byte line of the item, from 16 lanes
            if ((lane & 3) == 0) dma4(pw, junk);
        }
    };
    int slot = 0;
    if (!ctrl) {
        first(ld);
        first(pf);
        for (int q = 0; q < PFD; ++q)
            if (pf.s < nsteps) advance(pf);
#pragma unroll 1
        for (int q = 0; q < DEPTH; ++q) issue(q);
    }

    for (int s = 0; s <= nsteps; ++s) {
        // ---- between steps s - 1 and s
        __syncthreads();   // A: every term of step s - 1 is in LDS
        tr(s, 0);
        if (ctrl) {
            int status = 0;
            if (s > 0) {
                // outputs of step s - 1 from its terms, in group order
                const ChainStepDev& st = steps[s - 1];
                int pa, pb;
                wg_pairs(st.M, pa, pb);
                const int np = pb - pa, G = st.G, nr = 2 * np;
                if (st.epi == 1) {
                    for (int pl = lane; pl < np; pl += 64) {
                        float a0 = 0.0f, a1 = 0.0f;
                        const float* t = terms + 2 * pl;
                        int g = 0;
                        for (; g + 4 <= G; g += 4) {
                            float u0[4], u1[4];
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                u0[j] = t[(g + j) * nr];
                                u1[j] = t[(g + j) * nr + 1];
                            }
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                a0 = __builtin_fmaf(u0[j], xs_s[g + j], a0);
                                a1 = __builtin_fmaf(u1[j], xs_s[g + j], a1);
                            }
                        }
                        for (; g < G; ++g) {
                            a0 = __builtin_fmaf(t[g * nr], xs_s[g], a0);
                            a1 = __builtin_fmaf(t[g * nr + 1], xs_s[g], a1);
                        }
                        const uint16_t gh = f2h(a0), uh = f2h(a1);
                        st2_coh(st.Y + pa + pl, f2h(h2f(f2h(silu_f(h2f(gh)))) * h2f(uh)));
                    }
                } else {
                    for (int r = lane; r < nr; r += 64) {
                        const int row = 2 * pa + r;
                        float a = 0.0f;
                        const float* t = terms + r;
                        int g = 0;
                        for (; g + 8 <= G; g += 8) {
                            float u[8];
#pragma unroll
                            for (int j = 0; j < 8; ++j) u[j] = t[(g + j) * nr];
#pragma unroll
                            for (int j = 0; j < 8; ++j) a = __builtin_fmaf(u[j], xs_s[g + j], a);
                        }
                        for (; g < G; ++g) a = __builtin_fmaf(t[g * nr], xs_s[g], a);
                        if (row < st.M) st2_coh(st.Y + row, f2h(a));
                    }
                }
                wait_vm<0>();   // this wave's stores (outputs, h_out) are done
                if constexpr (kSigCopies) {
                    // count the workgroup into the step's 8 counter copies (one
                    // per XCD); no returned value is awaited
                    if (lane < 8)
                        (void)__hip_atomic_fetch_add(g32(flags + ((s - 1) * 8 + lane) * 32), 1u,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else if (lane == 0) {
                    // count the workgroup; the last one raises the step's 8
                    // per-XCD flag lines
                    const int old = (int)__hip_atomic_fetch_add(
                        g32(sync + s - 1), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old + 1 == grid) {
#pragma unroll
                        for (int x = 0; x < 8; ++x)
                            __hip_atomic_store(g32(flags + ((s - 1) * 8 + x) * 32), (uint32_t)grid,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
                tr(s, 1);
            }
            if (s < nsteps) {
                if (s > 0) {
                    // every workgroup has finished step s - 1
                    gu32* const cnt = g32(flags + ((s - 1) * 8 + (b & 7)) * 32);
                    int polls = 0;
                    while ((int)__hip_atomic_load(cnt, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) < grid) {
                        if (++polls > spin_limit ||
                            ((polls & 63) == 0 &&
                             __hip_atomic_load(g32(err), __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT))) {
                            status = 1;
                            __hip_atomic_store(g32(err), 1u, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                            break;
                        }
                        __builtin_amdgcn_s_sleep(kSleep);
                    }
                }
                tr(s, 2);
                if (status == 0) {
                    // step s's inputs into LDS: x, and for the RMSNorm
                    // prologue x2 and gamma (1 KB per instruction; lanes past
                    // the end re-read the last 16 bytes)
                    const ChainStepDev& st = steps[s];
                    const int nb = st.K * 2;
                    const int kpb = (nb + 1023) & ~1023;
                    const uint32_t sb = lds_addr(stage);
                    for (int c = 0; c < kpb; c += 1024) {
                        const int off = min(c + lane * 16, nb - 16);
                        dma16_coh(reinterpret_cast<const char*>(st.X) + off, sb + c);
                    }
                    if (st.pro == 2) {
                        const uint16_t* x2 = st.x2 ? st.x2 : st.X;
                        for (int c = 0; c < kpb; c += 1024) {
                            const int off = min(c + lane * 16, nb - 16);
                            dma16_coh(reinterpret_cast<const char*>(x2) + off, sb + kpb + c);
                            dma16(reinterpret_cast<const char*>(st.gamma) + off, sb + 2 * kpb + c);
                        }
                    }
                    wait_vm<0>();
                }
                tr(s, 3);
            }
            if (lane == 0) ctl_s[0] = status;
        }
        __syncthreads();   // B: inputs of step s in LDS (or a wait gave up)
        if (s == nsteps || ufirst(ctl_s[0]) != 0) break;

        // ---- prologue of step s: its int8 codes and group scales in LDS
        const ChainStepDev& st = steps[s];
        const int K = st.K, lg_g = st.lg_g;
        const int kpb = (K * 2 + 1023) & ~1023;
        uint16_t* const xst = reinterpret_cast<uint16_t*>(stage);
        // chunk round i of this wave holds any of x[0, K) (wave-uniform)
        auto live_chunks = [&](int i) { return (i * NTS + wave * 64) * 8 < K; };
        v4i xr[XV];
        if (!ctrl) {
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                const int k = (tid + i * NTS) * 8;
                xr[i] = k < K ? *reinterpret_cast<const v4i*>(xst + k) : zero;
            }
        }
        if (st.pro == 2) {
            const uint16_t* const x2s = reinterpret_cast<const uint16_t*>(stage + kpb);
            const uint16_t* const gms = reinterpret_cast<const uint16_t*>(stage + 2 * kpb);
            if (!ctrl && st.x2) {
                // h = fp16(x + x2), written back in place
#pragma unroll
                for (int i = 0; i < XV; ++i) {
                    const int k = (tid + i * NTS) * 8;
                    if (live_chunks(i) && k < K) {
                        uint16_t* h = reinterpret_cast<uint16_t*>(&xr[i]);
                        const v4i rv = *reinterpret_cast<const v4i*>(x2s + k);
                        const uint16_t* r = reinterpret_cast<const uint16_t*>(&rv);
#pragma unroll
                        for (int e = 0; e < 8; ++e) h[e] = f2h(h2f(h[e]) + h2f(r[e]));
                        *reinterpret_cast<v4i*>(xst + k) = xr[i];
                    }
                }
            }
            __syncthreads();
            if (ctrl && b == 0 && st.h_out) {
                for (int k = lane * 8; k < K; k += 64 * 8)
                    st16_coh(st.h_out + k, *reinterpret_cast<const v4i*>(xst + k));
            }
            // Sum of squares in the reference's order (rms_norm.cu:22-41):
            // T = min(next_pow2(K), 1024) threads, thread t sums h[t],
            // h[t + T], ... with FMAs, each 32-thread warp reduces by the
            // shuffle-down tree, then the warp sums by the same tree.
            int T = 1;
            while (T < K) T <<= 1;
            if (T > 1024) T = 1024;
            const int lanes = T < 32 ? 32 : T;
            if (!ctrl) {
                for (int t0 = 0; t0 < lanes; t0 += NTS) {
                    const int tt = t0 + tid;
                    float loc = 0.0f;
                    if (tt < T)
                        for (int k = tt; k < K; k += T) {
                            const float v = h2f(xst[k]);
                            loc = __builtin_fmaf(v, v, loc);
                        }
                    loc = warp32_sum_down(loc);
                    if (tt < lanes && (tt & 31) == 0) red_s[tt >> 5] = loc;
                }
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
            if (!ctrl) {
#pragma unroll
                for (int i = 0; i < XV; ++i) {
                    const int k = (tid + i * NTS) * 8;
                    if (live_chunks(i) && k < K) {
                        uint16_t* h = reinterpret_cast<uint16_t*>(&xr[i]);
                        const v4i gv = *reinterpret_cast<const v4i*>(gms + k);
                        const uint16_t* gm = reinterpret_cast<const uint16_t*>(&gv);
#pragma unroll
                        for (int e = 0; e < 8; ++e) h[e] = f2h((h2f(h[e]) * rr) * h2f(gm[e]));
                    }
                }
            }
        }
        if (!ctrl) {
            // Per-group dynamic quantization: chunk c = x[8c, 8c + 8) sits in
            // thread c % NTS, so a group's g / 8 chunks are consecutive lanes
            // of one wave; their |v| max comes from DPP / shuffles.
#pragma unroll
            for (int i = 0; i < XV; ++i) {
                if (!live_chunks(i)) continue;   // no chunk of this wave reaches K
                const int c = tid + i * NTS;
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
        }
        __syncthreads();   // C: codes ready; the input staging is free for terms
        tr(s, 4);

        // ---- the wave's items of step s, UB at a time (independent LDS
        // reads and dot products in flight together), then one by one
        if (!ctrl) {
            start(cs, s);
            int pa, pb;
            wg_pairs(cs.c.M, pa, pb);
            const int nr = 2 * (pb - pa);     // term table row stride
            auto item = [&](int sl, int pl, int pass, float& term, int& tix) {
                const uint32_t base = (uint32_t)(wave * DEPTH + sl) * kSlot;
                const v4i wv = *reinterpret_cast<const v4i*>(smem + base + lane * 16);
                const uint32_t sw =
                    *reinterpret_cast<const uint32_t*>(smem + base + 1024 + lane * 4);
                const int k = pass * PB + lk;
                const bool live = k < cs.c.K;
                const v4i xq = *reinterpret_cast<const v4i*>(xq_s + (live ? k : 0));
                int p = __builtin_amdgcn_sdot4(wv.x, xq.x, 0, false);
                p = __builtin_amdgcn_sdot4(wv.y, xq.y, p, false);
                p = __builtin_amdgcn_sdot4(wv.z, xq.z, p, false);
                p = __builtin_amdgcn_sdot4(wv.w, xq.w, p, false);
                // bytes past K (a short last group) add nothing to its sum
                p = live ? p : 0;
                p = lane_group_sum<LG>(p);
                int row = 2 * (cs.pa + pl) + rsub;
                row = row < cs.c.M ? row : cs.c.M - 1;
                const int kk = live ? k : 0;
                const int idx = row * cs.c.G + (kk >> cs.c.lg);
                int lo = idx & ~1;
                lo = lo < cs.c.mg2 ? lo : cs.c.mg2;
                const uint16_t ws = (uint16_t)(idx != lo ? sw >> 16 : sw & 0xffffu);
                term = (float)p * h2f(ws);
                // only the group leader of a live group stores its term
                tix = (live && (lane & (LG - 1)) == 0) ? (k >> cs.c.lg) * nr + 2 * pl + rsub : -1;
            };
            auto step_pos = [&](int& pl, int& pass) {
                if (++pass == cs.c.passes) {
                    pass = 0;
                    ++pl;
                }
            };
            constexpr int UB = 4;
            while (cs.rem >= UB) {
                wait_vm<NOPS * (DEPTH - UB)>();   // items it .. it + 3 landed
                float t[UB];
                int ti[UB];
                int pl = cs.pl, pass = cs.pass, sl = slot;
#pragma unroll
                for (int u = 0; u < UB; ++u) {
                    item(sl, pl, pass, t[u], ti[u]);
                    step_pos(pl, pass);
                    sl = sl + 1 == DEPTH ? 0 : sl + 1;
                }
#pragma unroll
                for (int u = 0; u < UB; ++u)
                    if (ti[u] >= 0) terms[ti[u]] = t[u];
                wait_lgkm0();   // the slots' reads are done before they are refilled
#pragma unroll 1
                for (int u = 0; u < UB; ++u) {
                    issue(slot);
                    slot = slot + 1 == DEPTH ? 0 : slot + 1;
                }
                cs.pl = ufirst(pl);
                cs.pass = ufirst(pass);
                cs.rem -= UB;
            }
            while (cs.rem > 0) {
                wait_vm<NOPS * (DEPTH - 1)>();   // the item has landed
                float t0;
                int ti0;
                item(slot, cs.pl, cs.pass, t0, ti0);
                if (ti0 >= 0) terms[ti0] = t0;
                wait_lgkm0();
                issue(slot);
                slot = slot + 1 == DEPTH ? 0 : slot + 1;
                step_pos(cs.pl, cs.pass);
                --cs.rem;
            }
        }
    }
    wait_vm<0>();   // no direct-to-LDS write may outlive the workgroup
}

__global__ void chain_zero_kernel(int* a, int na, int* c, int nc) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < na; i += gridDim.x * blockDim.x)
        a[i] = 0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nc; i += gridDim.x * blockDim.x)
        c[i] = 0;
}

template <int LG, int DEPTH>
void* kernel_ptr() {
    return reinterpret_cast<void*>(chain_kernel<LG, DEPTH, kPrefetch, kTrace>);
}
template <int DEPTH>
void* kernel_for(int lg) {
    if (lg == 6) return kernel_ptr<4, DEPTH>();
    if (lg == 7) return kernel_ptr<8, DEPTH>();
    if (lg == 8) return kernel_ptr<16, DEPTH>();
    return nullptr;
}
void* kernel_for(int lg, int depth) {
    if (depth == 12) return kernel_for<12>(lg);
    if (depth == 8) return kernel_for<8>(lg);
    return nullptr;
}

}  // namespace

ch::ChainLds chain_lds(int depth, int kp_max, int kh, int g_pad, int term_floats) {
    ch::ChainLds l{};
    int off = NS * depth * kSlot;
    l.xq = off;
    off += (kp_max + 15) & ~15;
    l.xs = off;
    off += ((g_pad + 3) & ~3) * 4;
    l.stage = off;
    const int kpb = (kp_max * 2 + 1023) & ~1023;
    const int kpbh = (kh * 2 + 1023) & ~1023;
    int st = kpb;
    if (3 * kpbh > st) st = 3 * kpbh;
    if (term_floats * 4 > st) st = term_floats * 4;
    off += (st + 15) & ~15;
    l.red = off;
    off += 64 * 4 + 256;   // reduction words, status, prefetch landing
    l.total = off;
    return l;
}

int chain_depth_for(int lds_total_at_depth8) {
    // the deeper ring when its 8 * 4 extra slots per wave still fit in 160 KB
    return lds_total_at_depth8 + NS * 4 * kSlot <= 160 * 1024 ? 12 : 8;
}

int chain_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return cus;
}

int chain_grid(int lg, int depth, size_t lds) {
    void* k = kernel_for(lg, depth);
    if (!k) return 0;
    // raise the dynamic LDS limit where the runtime keeps one (the result is
    // checked through the occupancy query below)
    (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NTH, lds) != hipSuccess) return 0;
    return chain_cus() * per_cu;
}

int chain_max_k() { return kChainMaxK; }
int chain_max_k_pro() { return kChainMaxKPro; }

hipError_t launch_chain(const ChainPlan& p, hipStream_t stream) {
    void* k = kernel_for(p.lg, p.depth);
    if (!k) return hipErrorInvalidValue;
    hipLaunchKernelGGL(chain_zero_kernel, dim3(64), dim3(256), 0, stream, p.flags,
                       p.nsteps * 8 * 32, p.sync, p.nsteps + 1);
    const ChainStepDev* steps = p.steps;
    int nsteps = p.nsteps, spin = p.spin_limit;
    int* sync = p.sync;
    int* flags = p.flags;
    ch::ChainLds lay = p.lay;
    unsigned long long* trace = p.trace;
    void* args[] = {&steps, &nsteps, &sync, &flags, &spin, &lay, &trace};
    return hipLaunchKernel(k, dim3((unsigned)p.grid), dim3(NTH), args, (size_t)p.lay.total,
                           stream);
}

}  // namespace fa

// chain.h -- device-side step table and launch plan of the persistent decode
// chain kernel (chain.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace fa {

constexpr int kChainWaves = 8;      // waves per workgroup; a row block is 2 * kChainWaves rows
constexpr int kChainMaxK = 12288;   // longest input of a step
constexpr int kChainMaxKPro = 4096; // ... with the RMSNorm prologue
constexpr int kChainMaxSteps = 4096;
constexpr int kChainRing = 5;       // 512-byte passes in flight per wave; blocks pad to a multiple

namespace ch {
// One linear of the chain, as the kernel reads it (built by the host from
// the public step description).  Tasks task0 .. task0 + nblocks - 1 are its
// row blocks.
struct ChainStepDev {
    const int8_t* W;
    const uint16_t* w_scale;
    const uint16_t* X;
    const uint16_t* x2;
    const uint16_t* gamma;
    uint16_t* h_out;
    uint16_t* Y;
    int M, K, lg_g, G, passes, nblocks, task0, pro, epi;
    float eps;
};
}  // namespace ch

struct ChainPlan {
    const ch::ChainStepDev* steps;   // device array [nsteps]
    int* sync;                       // device [nsteps + 1]: per-step counters, error word
    int* flags;                      // device [nsteps * 8 * 32]: per-step, per-XCD done flags
    int nsteps, total, lg, grid, spin_limit, kp_max, g_pad, kh;
    int epoch;                       // this launch's flag value (never 0)
    size_t lds;
};

size_t chain_lds_bytes(int kp_max, int g_pad, int kh);
int chain_rows_per_task();
int chain_max_k();
int chain_max_k_pro();
int chain_grid(int lg, size_t lds);
hipError_t launch_chain(const ChainPlan& p, hipStream_t stream);

}  // namespace fa

// chain.h -- device-side step table and launch plan of the persistent decode
// chain kernel (chain.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace fa {

constexpr int kChainWaves = 8;      // streaming waves per workgroup (plus one control wave)
constexpr int kChainMaxK = 12288;   // longest input of a step
constexpr int kChainMaxKPro = 4096; // ... with the RMSNorm prologue
constexpr int kChainMaxSteps = 4096;

namespace ch {
// One linear of the chain, as the kernel reads it (built by the host from
// the public step description).
struct ChainStepDev {
    const int8_t* W;
    const uint16_t* w_scale;
    const uint16_t* X;
    const uint16_t* x2;
    const uint16_t* gamma;
    uint16_t* h_out;
    uint16_t* Y;
    int64_t MG;                      // M * G: scale elements
    int M, K, lg_g, G, passes, pro, epi;
    float eps;
};

// Byte offsets of the kernel's LDS regions.
struct ChainLds {
    int xq, xs, stage, red, total;
};
}  // namespace ch

struct ChainPlan {
    const ch::ChainStepDev* steps;   // device array [nsteps]
    int* sync;                       // device [nsteps + 1]: sync[nsteps] is the error word
    int* flags;                      // device [nsteps * 8 * 32]: per-step counters, 8 copies
    int nsteps, lg, grid, spin_limit, depth;
    ch::ChainLds lay;
    unsigned long long* trace;       // measurement builds: [nsteps + 1][grid][8] timestamps
};

// LDS layout for a ring of `depth` slots per streaming wave, inputs up to
// kp_max values (kh with the RMSNorm prologue), g_pad group scales and
// term_floats per-step terms.
ch::ChainLds chain_lds(int depth, int kp_max, int kh, int g_pad, int term_floats);
int chain_depth_for(int lds_total);           // ring depths the kernel is built for
int chain_grid(int lg, int depth, size_t lds);  // resident workgroups (all must be resident)
int chain_max_k();
int chain_max_k_pro();
int chain_cus();
hipError_t launch_chain(const ChainPlan& p, hipStream_t stream);

}  // namespace fa

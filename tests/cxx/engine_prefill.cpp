// engine_prefill.cpp -- test driver: the DualAR engine's prefill attention
// block (src/engine/dual_ar_engine.cc:442-505: wqkv linear, QKV head split,
// prefill attention, head merge) written against the C++ mirror of the
// reference API (fish_amd/loader.h, fish_amd/kernels.h), as a maintainer
// would write it after switching the engine to this library.
//
// usage: engine_prefill <weights.bin> <out.raw> <n_q> <n_kv> <head_dim> <window>
//   weights.bin holds "wqkv" (int8 [M, K]) with "wqkv_scale" (fp16 [M] or
//   [M, G]) and "x" (fp16 [T, K]); M = (n_q + 2 n_kv) head_dim.
//   out.raw receives the fp16 wqkv output [T, M], then the fp16 merged
//   attention output [T, n_q head_dim].
// Exit status 0 on success; any failure prints a message and returns 1.
#include "fish_amd/kernels.h"
#include "fish_amd/loader.h"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <vector>

#define HIP_OK(call)                                                                  \
    do {                                                                              \
        hipError_t e_ = (call);                                                       \
        if (e_ != hipSuccess) throw std::runtime_error(hipGetErrorString(e_));        \
    } while (0)

template <typename T>
static T* upload(const fish::TensorView& t) {
    T* d = nullptr;
    HIP_OK(hipMalloc(&d, t.nbytes()));
    HIP_OK(hipMemcpy(d, t.data, t.nbytes(), hipMemcpyHostToDevice));
    return d;
}

int main(int argc, char** argv) {
    if (argc != 7) {
        std::fprintf(stderr, "usage: %s weights.bin out.raw n_q n_kv head_dim window\n", argv[0]);
        return 1;
    }
    try {
        const int n_q = std::atoi(argv[3]), n_kv = std::atoi(argv[4]), D = std::atoi(argv[5]);
        const int window = std::atoi(argv[6]);
        fish::ModelLoader loader;
        if (!loader.load(argv[1])) throw std::runtime_error(loader.last_error());
        const fish::TensorView w = loader.get("wqkv"), s = loader.get("wqkv_scale");
        const fish::TensorView x = loader.get("x");
        const fish::QuantMetaHost meta = fish::quant_meta_for(loader, "wqkv");
        const int M = (int)w.shape[0], K = (int)w.shape[1], T = (int)x.shape[0];
        if (M != (n_q + 2 * n_kv) * D || x.shape[1] != K)
            throw std::runtime_error("shape mismatch");

        hipStream_t stream;
        HIP_OK(hipStreamCreate(&stream));
        const int8_t* dW = upload<int8_t>(w);
        const __half* dS = upload<__half>(s);
        const __half* dX = upload<__half>(x);
        __half *qkv, *q, *k, *v, *heads, *merged;
        HIP_OK(hipMalloc(&qkv, (size_t)T * M * 2));
        HIP_OK(hipMalloc(&q, (size_t)n_q * T * D * 2));
        HIP_OK(hipMalloc(&k, (size_t)n_kv * T * D * 2));
        HIP_OK(hipMalloc(&v, (size_t)n_kv * T * D * 2));
        HIP_OK(hipMalloc(&heads, (size_t)n_q * T * D * 2));
        HIP_OK(hipMalloc(&merged, (size_t)T * n_q * D * 2));

        // dual_ar_engine.cc:448-453 (quantized_gemm -> int8_dequant_gemm_fp16,
        // then the GQA split), :499-502 (attention, merge)
        fish::kernels::int8_dequant_gemm_fp16(dW, dS, meta.group_size, nullptr, nullptr, dX, qkv,
                                              M, T, K, nullptr, stream);
        fish::kernels::qkv_split_heads_gqa(qkv, q, k, v, T, n_q, n_kv, D, stream);
        fish::kernels::prefill_attention_gpu(q, k, v, heads, nullptr, n_q, n_kv, T, D,
                                             1.0f / std::sqrt((float)D), nullptr, stream, window);
        fish::kernels::merge_heads(heads, merged, T, n_q, D, stream);
        HIP_OK(hipStreamSynchronize(stream));

        std::vector<uint16_t> h((size_t)T * M + (size_t)T * n_q * D);
        HIP_OK(hipMemcpy(h.data(), qkv, (size_t)T * M * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(h.data() + (size_t)T * M, merged, (size_t)T * n_q * D * 2,
                         hipMemcpyDeviceToHost));
        FILE* f = std::fopen(argv[2], "wb");
        if (!f || std::fwrite(h.data(), 2, h.size(), f) != h.size())
            throw std::runtime_error("cannot write output");
        std::fclose(f);
        for (void* p : {(void*)dW, (void*)dS, (void*)dX, (void*)qkv, (void*)q, (void*)k,
                        (void*)v, (void*)heads, (void*)merged})
            HIP_OK(hipFree(p));
        HIP_OK(hipStreamDestroy(stream));
    } catch (const std::exception& e) {
        std::fprintf(stderr, "engine_prefill: %s\n", e.what());
        return 1;
    }
    return 0;
}

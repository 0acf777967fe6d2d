"""Synthetic inputs for the W8A8 path (no checkpoints exist offline).

Distributions: W fp16 ~ N(0, 0.02); X fp16 ~ N(0, 1) with
ceil(1% of K) channels, chosen without replacement, scaled x20 as outliers;
RMSNorm gamma fp16 ~ 1 + N(0, 0.1).  numpy PCG64 with the given seed.
"""
import math

import numpy as np

# Qwen3-4B-class DualAR layer linears (src/model/dual_ar_config.h:9-30):
# name -> (K, N_out).  gate_up is w1 and w3 stacked (2 x 9728 rows).
LAYER_SHAPES = {
    "qkv": (2560, 6144),
    "o": (4096, 2560),
    "gate_up": (2560, 19456),
    "down": (9728, 2560),
}


def outlier_channels(K, seed=0):
    rng = np.random.default_rng(seed + 7919)
    n = int(math.ceil(0.01 * K))
    return np.sort(rng.choice(K, size=n, replace=False))


def weights_f16(rows, K, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, K), dtype=np.float32) * 0.02).astype(np.float16)


def activations_f16(N, K, seed=0):
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((N, K), dtype=np.float32)
    x[:, outlier_channels(K, seed)] *= 20.0
    return x.astype(np.float16)


def gamma_f16(dim, seed=0):
    rng = np.random.default_rng(seed + 2)
    return (1.0 + 0.1 * rng.standard_normal(dim, dtype=np.float32)).astype(np.float16)

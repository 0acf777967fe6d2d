"""Decode planning on the CPU (no device calls): every plan the library makes
for N <= 16 tokens meets the grid and shape assumptions its kernels take for
granted (the same check every launch makes), over a seeded sweep of shapes
and all prologue / epilogue / quantization modes, and the configs[1] /
configs[2] layer shapes take the paths the design names."""
import ctypes

import numpy as np
import pytest

from fish_amd import _lib

LAYER = {"qkv": (2560, 6144), "o": (4096, 2560), "gate_up": (2560, 19456), "down": (9728, 2560)}


def plan(M, N, K, g, qx=0, pro=0, epi=0, smooth=0):
    out = (ctypes.c_int * 10)()
    kind = _lib.lib().fa_debug_gemv_plan(M, N, K, g, qx, pro, epi, smooth,
                                         ctypes.cast(out, ctypes.c_void_p))
    d = dict(zip(["kind", "grid", "block", "lds", "spg", "maxg", "lc", "qx", "epi", "valid"],
                 list(out)))
    assert d["kind"] == kind
    return d


def _shapes(n=4000, seed=11):
    rng = np.random.default_rng(seed)
    for _ in range(n):
        N = int(rng.integers(1, 17))
        M = int(rng.integers(1, 40000))
        if rng.random() < 0.7:
            K = int(rng.integers(1, 512)) * 64
        else:
            K = int(rng.integers(1, 4000)) * 16
        g = int(rng.choice([64, 128, 256, 512, 0, 32, 1000]))
        yield N, M, K, g


def test_every_plan_meets_the_kernel_assumptions():
    seen = {1: 0, 2: 0, 3: 0}
    modes = [(0, 0, 0, 0), (1, 0, 0, 0), (1, 0, 0, 1), (1, 2, 0, 0), (1, 1, 0, 0),
             (1, 0, 1, 0), (1, 2, 1, 0), (0, 0, 1, 0), (1, 0, 1, 1), (1, 2, 2, 0)]
    for N, M, K, g in _shapes():
        for qx, pro, epi, sm in modes:
            if epi:
                M2 = M + (M & 1)
            else:
                M2 = M
            d = plan(M2, N, K, g, qx, pro, epi, sm)
            if d["kind"] == 0:
                continue
            seen[d["kind"]] += 1
            assert d["valid"] == 1, (N, M2, K, g, qx, pro, epi, sm, d)
            if d["kind"] == 3:
                assert d["grid"] * 16 >= M2 and d["block"] <= 512
                if qx:
                    assert d["qx"] == (2 if sm else 1)
                    assert d["spg"] * d["maxg"] <= (8 if sm else 16)
                assert d["epi"] == epi
            else:
                assert N == 1
    assert all(v > 100 for v in seen.values()), seen


@pytest.mark.parametrize("name", list(LAYER))
def test_layer_shapes_take_the_named_paths(name):
    K, M = LAYER[name]
    # one token, g256, in-kernel quantization -> the dot GEMV
    d = plan(M, 1, K, 256, qx=1)
    assert d["kind"] in (1, 2) and d["valid"] == 1
    # 8 tokens, g64, staged codes -> the MFMA GEMV
    d = plan(M, 8, K, 64)
    assert d["kind"] == 3 and d["valid"] == 1 and d["qx"] == 0
    # in-kernel quantization at 8 tokens where each wave's range fits
    d = plan(M, 8, K, 64, qx=1)
    if name == "down":     # 152 groups over at most 8 waves: 19 steps > 16
        assert d["kind"] == 0
    else:
        assert d["kind"] == 3 and d["qx"] == 1 and d["spg"] * d["maxg"] <= 16
    # the SwiGLU epilogue at 8 tokens on the interleaved gate_up weight
    if name == "gate_up":
        d = plan(M, 8, K, 64, epi=1)
        assert d["kind"] == 3 and d["epi"] == 1


def test_plans_refused_where_the_kernels_do_not_go():
    assert plan(100, 17, 512, 64)["kind"] == 0          # N > 16: the GEMM paths
    assert plan(101, 8, 512, 64, epi=1)["kind"] == 0    # odd rows cannot pair
    assert plan(100, 8, 512, 64, epi=2)["kind"] == 0    # separate w1 / w3: one token only
    assert plan(100, 2, 512, 64, qx=1, pro=2)["kind"] == 0   # fused prologue: one token only
    assert plan(100, 1, 40000, 64, qx=1)["kind"] == 0   # K beyond the one-token kernels


TP8 = {"qkv": (2560, 768), "o": (512, 2560), "gate_up": (2560, 2432), "down": (1216, 2560)}


@pytest.mark.parametrize("name", list(TP8))
@pytest.mark.parametrize("g", [256, 64])
def test_tp8_shard_shapes_plan(name, g):
    """One GPU's share under 8-way tensor parallelism (o and down split K:
    2 groups of 256, or 4.75 -- a short last group for down at g256): the
    decode paths plan them and every plan meets the kernel assumptions."""
    K, M = TP8[name]
    for N in (1, 2, 8, 16):
        for qx, pro, epi, sm in [(0, 0, 0, 0), (1, 0, 0, 0), (1, 0, 0, 1), (1, 2, 0, 0),
                                 (1, 1, 0, 0), (1, 0, 1, 0), (1, 2, 1, 0)]:
            d = plan(M, N, K, g, qx, pro, epi, sm)
            if d["kind"]:
                assert d["valid"] == 1, (name, g, N, qx, pro, epi, sm, d)
    assert plan(M, 1, K, g, qx=1)["kind"] in (1, 2)
    assert plan(M, 8, K, g)["kind"] == 3


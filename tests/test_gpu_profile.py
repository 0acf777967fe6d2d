"""GPU: per-shape timing of the linear entry points (the reference's
FISH_INT8_PROFILE, src/kernels/int8_gemm.cu:45-145): calls are counted per
(entry, shape, group size, quantization mode), the separate quantization
launch is timed apart, nested entry points count once, calls under graph
capture are not timed, and results are unchanged."""
import ctypes
import re

import numpy as np
import pytest
import torch

from fish_amd import _lib, ops, synth
from oracle import ref

pytestmark = pytest.mark.gpu


def summary():
    l = _lib.lib()
    n = l.fa_profile_summary(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    assert l.fa_profile_summary(buf, n + 1) == n
    return buf.value.decode()


def bucket(text, entry, M, N, K, g):
    pat = r"%s M=%d N=%d K=%d group=%d act=dynamic smooth=no calls=(\d+) .*?" \
          r"avg=([0-9.]+)ms \(quant=([0-9.]+) gemm=([0-9.]+)\)" % (entry, M, N, K, g)
    m = re.search(pat, text)
    assert m, (entry, M, N, K, g, text)
    return int(m.group(1)), float(m.group(2)), float(m.group(3)), float(m.group(4))


def dev(a):
    return torch.from_numpy(np.array(a, copy=True, order="C")).cuda()


def test_profile_buckets():
    l = _lib.lib()
    prev = l.fa_profile_enable(1)
    try:
        l.fa_profile_reset()
        M, K, g = 2560, 4096, 256
        q, s = ref.quantize_weights(synth.weights_f16(M, K, seed=3), g)
        Wd, Sd = dev(q), dev(s)
        x1 = dev(synth.activations_f16(1, K, seed=4))
        x64 = dev(synth.activations_f16(64, K, seed=5))
        ys = [ops.w8a8_gemm(Wd, Sd, x1, g) for _ in range(3)]
        for _ in range(2):
            ops.w8a8_gemm(Wd, Sd, x64, g)
        # nested: the SwiGLU entry at 3 tokens runs fa_w8a8_gemm_rms inside
        F = 512
        q13, s13 = ref.quantize_weights(synth.weights_f16(2 * F, K, seed=6), g)
        x3 = dev(synth.activations_f16(3, K, seed=7))
        gamma = dev(synth.gamma_f16(K, seed=8))
        act = torch.empty((3, F), dtype=torch.float16, device="cuda")
        W13, S13 = dev(q13), dev(s13)
        _lib.check(l.fa_w8a8_gemm_swiglu(W13.data_ptr(), S13.data_ptr(), g, None, None,
                                         x3.data_ptr(), None, None, gamma.data_ptr(), 1e-6,
                                         act.data_ptr(), F, 3, K, ops._stream()))
        # graph capture: not timed
        y = torch.empty((1, M), dtype=torch.float16, device="cuda")
        gr = torch.cuda.CUDAGraph()
        ops.w8a8_gemm(Wd, Sd, x1, g, out=y)
        torch.cuda.synchronize()
        before = bucket(summary(), "fa_w8a8_gemm", M, 1, K, g)[0]
        with torch.cuda.graph(gr):
            ops.w8a8_gemm(Wd, Sd, x1, g, out=y)
        gr.replay()
        torch.cuda.synchronize()
        text = summary()
        print(text, flush=True)
        c1, avg1, qt1, gm1 = bucket(text, "fa_w8a8_gemm", M, 1, K, g)
        assert c1 == before == 4 and avg1 > 0 and qt1 == 0.0
        c64, avg64, qt64, gm64 = bucket(text, "fa_w8a8_gemm", M, 64, K, g)
        assert c64 == 2 and qt64 > 0 and gm64 > 0
        csw = bucket(text, "fa_w8a8_gemm_swiglu", 2 * F, 3, K, g)[0]
        assert csw == 1
        assert "fa_w8a8_gemm_rms" not in text
        # results are the oracle's with timing on
        want = ref.w8a8_gemm(q, s, g, x1.cpu().numpy())
        for yy in ys + [y]:
            assert np.array_equal(yy.cpu().numpy().view(np.uint16), want.view(np.uint16))
        l.fa_profile_reset()
        assert summary() == ""
    finally:
        l.fa_profile_enable(prev)
        l.fa_profile_reset()

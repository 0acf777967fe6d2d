"""GPU: the engine's prefill attention block in C++ through the mirror of the
reference API (tests/cxx/engine_prefill.cpp, built by build()): a .bin file
read with fish::ModelLoader, the wqkv linear (int8_dequant_gemm_fp16), the
GQA head split, prefill_attention_gpu and merge_heads, as
dual_ar_engine.cc:442-505 calls them.  The linear and the split / merge are
checked bit for bit against the oracle; attention within the tolerance of
tests/test_gpu_attention.py."""
import os
import subprocess

import numpy as np
import pytest

from oracle import ref
from fish_amd import binfile, build

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,n_q,n_kv,D,g,window", [(50, 8, 2, 64, 128, 0), (96, 4, 4, 32, 64, 17)])
def test_engine_prefill_block_cxx(tmp_path, T, n_q, n_kv, D, g, window):
    assert os.path.exists(build.TEST_DRIVER), "run __graft_entry__.build() first"
    print("engine_prefill T=%d n_q=%d n_kv=%d D=%d g=%d window=%d" % (T, n_q, n_kv, D, g, window),
          flush=True)
    rng = np.random.default_rng(T + D)
    K, M = 256, (n_q + 2 * n_kv) * D
    w = (rng.standard_normal((M, K)) * 0.05).astype(np.float16)
    W, S = ref.quantize_weights(w, g)
    x = rng.standard_normal((T, K)).astype(np.float16)
    path = str(tmp_path / "w.bin")
    binfile.write_bin(path, [("wqkv", W), ("wqkv_scale", S), ("x", x)])
    out = str(tmp_path / "out.raw")
    res = subprocess.run([build.TEST_DRIVER, path, out, str(n_q), str(n_kv), str(D), str(window)],
                         stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert res.returncode == 0, res.stdout
    h = np.fromfile(out, dtype=np.float16)
    y, merged = h[:T * M].reshape(T, M), h[T * M:].reshape(T, n_q * D)

    want_y = ref.w8a8_gemm(W, S, g, x)
    assert np.array_equal(y.view(np.uint16), want_y.view(np.uint16))

    q, k, v = ref.qkv_split_gqa(y, n_q, n_kv, D)
    o, aw = ref.prefill_attention(q, k, v, 1.0 / np.sqrt(np.float32(D)), window)
    want = ref.merge_heads(o).astype(np.float64)
    tol = ref.attention_tolerance(o, aw).transpose(1, 0, 2).reshape(T, n_q * D)
    err = np.abs(merged.astype(np.float64) - want)
    assert np.all(err <= tol), float((err / tol).max())

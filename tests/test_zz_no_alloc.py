"""fa_w8a8_gemm_noalloc (scratch in a static per-device array, no allocation
in the call) against fa_w8a8_gemm, bit for bit, on consecutive calls whose
second input is smaller (the array keeps the first call's contents), plus
the size limit.  Where fa_w8a8_gemm splits K (fa_w8a8_gemm_k_splits > 1) the
no-alloc entry, which never splits, equals the oracle bit for bit and the
two agree within the split tolerance."""
import numpy as np
import pytest
import torch

from fish_amd import _lib, ops, synth
from oracle import ref

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.array(a, copy=True, order="C")).cuda()


def run_pair(N, M, K, g, seed, act=None, sm=None):
    q, s = ref.quantize_weights(synth.weights_f16(M, K, seed=seed), g)
    x = dev(synth.activations_f16(N, K, seed=seed + 1))
    Wd, Sd = dev(q), dev(s)
    a = ops.w8a8_gemm(Wd, Sd, x, g, act_scale=act, smooth_inv=sm)
    b = ops.w8a8_gemm_noalloc(Wd, Sd, x, g, act_scale=act, smooth_inv=sm)
    torch.cuda.synchronize()
    if ops.k_splits(M, N, K, g) == 1:
        assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (N, M, K, g)
    else:
        hx = x.cpu().numpy()
        ha = None if act is None else act.cpu().numpy()
        hs = None if sm is None else sm.cpu().numpy()
        rY = ref.w8a8_gemm(q, s, g, hx, act_scale=ha, smooth_inv=hs)
        assert np.array_equal(b.cpu().numpy().view(np.uint16), rY.view(np.uint16))
        rq, rs = ref.quantize_activations(hx, g, act_scale=ha, smooth_inv=hs)
        bound = ref.split_chain_tolerance(q, s, g, rq, rs, rY)
        err = np.abs(a.cpu().numpy().astype(np.float64) - rY.astype(np.float64))
        assert np.all(err <= bound), (N, M, K, g)
    return b


@pytest.mark.parametrize("first,second", [
    ((2048, 2560, 9728, 256), (512, 6144, 2560, 256)),   # prefill tile kernel, then smaller
    ((64, 512, 2560, 64), (8, 256, 2560, 64)),           # tile kernel, then the MFMA GEMV
    ((8, 2560, 4096, 64), (1, 2560, 4096, 256)),         # GEMV, then one token (no scratch)
    ((300, 260, 512, 256), (3, 40, 100, 48)),            # ragged tiles, then the generic kernel
    ((512, 2560, 4096, 256), (200, 640, 1024, 128)),     # K split in fa_w8a8_gemm, then smaller
])
def test_noalloc_matches_entry_point(first, second):
    N, M, K, g = first
    assert _lib.lib().fa_noalloc_scratch_bytes(M, N, K, g) <= _lib.FA_NOALLOC_SCRATCH_BYTES
    run_pair(*first, seed=1)
    run_pair(*second, seed=2)


def test_noalloc_static_and_smooth_companions():
    K, g = 2560, 64
    G = K // g
    act = dev(np.full(G, 0.05, np.float16))
    sm = dev(synth.gamma_f16(K, seed=3))
    run_pair(16, 1024, K, g, seed=4, act=act, sm=sm)
    run_pair(4, 512, K, g, seed=5, sm=sm)


def test_noalloc_rejects_oversized_shape():
    # 8192 tokens x K 9728 codes alone exceed the 32 MiB array
    N, M, K, g = 8192, 256, 9728, 256
    assert _lib.lib().fa_noalloc_scratch_bytes(M, N, K, g) > _lib.FA_NOALLOC_SCRATCH_BYTES
    W = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    S = torch.ones((M, K // g), dtype=torch.float16, device="cuda")
    X = torch.zeros((N, K), dtype=torch.float16, device="cuda")
    with pytest.raises(_lib.FaError) as e:
        ops.w8a8_gemm_noalloc(W, S, X, g)
    assert e.value.code == _lib.FA_ERR_INVALID_ARG
    assert "maximum" in str(e.value)
    # the library still works afterwards
    run_pair(4, 64, 512, 64, seed=6)


def _noalloc_sweep(n=10, seed=55):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        N = int(rng.choice([1, int(rng.integers(2, 17)), int(rng.integers(17, 700))]))
        M = int(rng.integers(1, 3000 if N <= 16 else 1000))
        K = int(rng.integers(1, 300 if N <= 16 else 120)) * 16
        g = int(rng.choice([64, 128, 256, 512]))
        if N * M * K > 1.2e9:
            continue
        if _lib.lib().fa_noalloc_scratch_bytes(M, N, K, g) > _lib.FA_NOALLOC_SCRATCH_BYTES:
            continue
        out.append((N, M, K, g))
    return out


@pytest.mark.parametrize("N,M,K,g", _noalloc_sweep())
def test_noalloc_random_shapes(N, M, K, g):
    """Seeded random shapes, each against fa_w8a8_gemm (or, where that
    splits K, the oracle), one call after another on the shared array."""
    print("noalloc sweep N=%d M=%d K=%d g=%d" % (N, M, K, g), flush=True)
    run_pair(N, M, K, g, seed=N + M + K)

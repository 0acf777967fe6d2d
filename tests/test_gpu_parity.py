"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bar: bit-exact everywhere.  int8 activations, activation scales, weight
quantization, RMSNorm and the elementwise ops match the oracle bit for bit;
every int32 per-group partial matches exactly; and every linear-layer path
(decode GEMV, prefill GEMM, any-shape kernel) sums the K-groups in the
oracle's order, so its fp16 output matches bit for bit as well -- stricter
than the path's stated output tolerance of 1 fp16 ulp or rtol 1e-3, which
the oracle itself is held to against float64 in test_oracle.py.
"""
import os
import tempfile

import numpy as np
import pytest
import torch

from oracle import ref
from fish_amd import ops, synth
from fish_amd.binfile import BinFile, write_bin

pytestmark = pytest.mark.gpu

LAYER = synth.LAYER_SHAPES


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a device"
    from fish_amd import _lib
    _lib.lib()   # fails loudly when the HIP library is missing
    ref.lib()
    yield
    torch.cuda.synchronize()


def dev(a):
    # a copy: arrays viewing a read-only memory map are not writable
    return torch.from_numpy(np.array(a, copy=True, order="C")).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    return np.array_equal(a.view(np.uint8), b.view(np.uint8))


def make_linear(M, K, g, seed=0):
    """W fp16 ~ N(0, 0.02) quantized group-wise by the oracle -> (q, scale)."""
    w = synth.weights_f16(M, K, seed=seed)
    ge = K if g <= 0 or g > K else g
    return ref.quantize_weights(w, ge)


# ------------------------------------------------------- quantizers ----

@pytest.mark.parametrize("N,K,g", [(1, 2560, 256), (8, 2560, 64), (16, 512, 64), (5, 100, 48),
                                   (3, 96, 0), (2, 4096, 5000), (7, 9728, 64), (4, 24, 8)])
@pytest.mark.parametrize("variant", ["dynamic", "static", "smooth"])
def test_quantize_activations_bitexact(N, K, g, variant):
    x = synth.activations_f16(N, K, seed=K + N)
    G = ref.groups(K, g)
    act = np.abs(synth.activations_f16(1, G, seed=9)[0]) * np.float16(0.05) if variant == "static" else None
    sm = synth.gamma_f16(K, seed=5) if variant == "smooth" else None
    xq, xs = ops.quantize_activations(dev(x), g, act_scale=None if act is None else dev(act),
                                      smooth_inv=None if sm is None else dev(sm))
    rq, rs = ref.quantize_activations(x, g, act_scale=act, smooth_inv=sm)
    assert same(host(xq), rq)
    assert same(host(xs), rs)


@pytest.mark.parametrize("rows,K,g", [(64, 512, 64), (37, 100, 48), (128, 2560, 256), (5, 64, 1000)])
def test_quantize_weights_bitexact(rows, K, g):
    w = synth.weights_f16(rows, K, seed=rows)
    w[1] = 0
    q, s = ops.quantize_weights_groupwise(dev(w), g)
    rq, rs = ref.quantize_weights(w, g)
    assert same(host(q), rq) and same(host(s), rs)


@pytest.mark.parametrize("n,dim", [(4, 8), (1, 4), (3, 16), (2, 100), (3, 1000), (5, 2560),
                                   (2, 4096), (1, 9728)])
def test_rms_norm_bitexact(n, dim):
    x = synth.activations_f16(n, dim, seed=dim)
    w = synth.gamma_f16(dim)
    out = ops.rms_norm(dev(x), dev(w), 1e-6)
    assert same(host(out), ref.rms_norm(x, w, 1e-6))


def test_rms_norm_reference_closed_forms():
    # tests/test_kernels.cu:121-210 through the device kernel
    out = host(ops.rms_norm(dev(np.ones((4, 8), np.float16)), dev(np.ones(8, np.float16)), 1e-6))
    assert np.all(np.abs(out.astype(np.float32) - 1) <= 1e-3)
    out = host(ops.rms_norm(dev(np.zeros((2, 4), np.float16)), dev(np.ones(4, np.float16)), 1e-5))
    assert np.all(np.isfinite(out.astype(np.float32)))
    x = np.array([[1, 3, 1, 3]], np.float16)
    out = host(ops.rms_norm(dev(x), dev(np.full(4, 2, np.float16)), 1e-6)).astype(np.float64)
    assert np.all(np.abs(out - 2 * x / np.sqrt(5 + 1e-6)) <= 1e-2)


@pytest.mark.parametrize("n,dim,g", [(8, 2560, 64), (1, 2560, 256), (3, 100, 48), (2, 4096, 0),
                                     (2, 9000, 128)])
@pytest.mark.parametrize("variant", ["dynamic", "static", "smooth"])
def test_rms_norm_quant_bitexact(n, dim, g, variant):
    x = synth.activations_f16(n, dim, seed=n)
    w = synth.gamma_f16(dim)
    G = ref.groups(dim, g)
    act = np.full(G, 0.03, np.float16) if variant == "static" else None
    sm = synth.gamma_f16(dim, seed=4) if variant == "smooth" else None
    xq, xs, out = ops.rms_norm_quant(dev(x), dev(w), 1e-6, g, smooth_inv=None if sm is None else dev(sm),
                                     act_scale=None if act is None else dev(act), want_out=True)
    rq, rs, rout = ref.rms_norm_quant(x, w, 1e-6, g, smooth_inv=sm, act_scale=act)
    assert same(host(out), rout)
    assert same(host(xq), rq)
    assert same(host(xs), rs)


@pytest.mark.parametrize("n,dim,g", [(1, 2560, 256), (8, 2560, 64), (3, 100, 48), (2, 9000, 128)])
def test_residual_rms_norm_quant_bitexact(n, dim, g):
    """h <- fp16(h + r) in place, then RMSNorm + group quant of the new h; the
    fused kernel equals residual_add followed by rms_norm_quant.  dim = 9000
    exceeds the register path (8 values per thread) and takes the loop."""
    h = synth.activations_f16(n, dim, seed=n + 7)
    r = (synth.activations_f16(n, dim, seed=n + 8) * np.float16(0.5)).astype(np.float16)
    w = synth.gamma_f16(dim)
    hd = dev(h)
    xq, xs, out = ops.residual_rms_norm_quant_(hd, dev(r), dev(w), 1e-6, g, want_out=True)
    rh = ref.residual_add(h, r)
    rq, rs, rout = ref.rms_norm_quant(rh, w, 1e-6, g)
    assert same(host(hd), rh)
    assert same(host(out), rout)
    assert same(host(xq), rq)
    assert same(host(xs), rs)


def test_elementwise_bitexact():
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(100003) * 4).astype(np.float16)
    b = rng.standard_normal(100003).astype(np.float16)
    assert same(host(ops.silu_(dev(a))), ref.silu(a))
    assert same(host(ops.mul_(dev(a), dev(b))), ref.mul(a, b))
    assert same(host(ops.residual_add_(dev(a), dev(b))), ref.residual_add(a, b))
    # tests/test_kernels.cu:355-379, 432-481 closed forms
    x = np.arange(-8, 8).astype(np.float16)
    got = host(ops.silu_(dev(x))).astype(np.float64)
    assert np.all(np.abs(got - x / (1 + np.exp(-x.astype(np.float64)))) <= 1e-2)


@pytest.mark.parametrize("n,dim,g", [(8, 9728, 64), (1, 9728, 256), (2, 100, 48)])
def test_silu_mul_quant_bitexact(n, dim, g):
    rng = np.random.default_rng(dim)
    gate = (rng.standard_normal((n, dim)) * 3).astype(np.float16)
    up = rng.standard_normal((n, dim)).astype(np.float16)
    xq, xs, out = ops.silu_mul_quant(dev(gate), dev(up), g, want_out=True)
    rq, rs, rout = ref.silu_mul_quant(gate, up, g)
    assert same(host(out), rout)
    assert same(host(xq), rq)
    assert same(host(xs), rs)


# --------------------------------------------------------- linear ----

def check_linear(N, M, K, g, seed=0, full_entry=True):
    """Partials bit-exact, Y within the path's tolerance (bit-exact on the
    GEMM path).  Returns the device Y."""
    q, s = make_linear(M, K, g, seed=seed)
    if s.shape[1] == 1:
        s = s[:, 0]
    x = synth.activations_f16(N, K, seed=seed + 1)
    rq, rs = ref.quantize_activations(x, g)
    Wd, Sd = dev(q), dev(s)
    Y, P = ops.w8a8_gemm_partials(Wd, Sd, g, dev(rq), dev(rs))
    rP = ref.group_partials(q, rq, g)
    assert same(host(P), rP), "int32 partials differ"
    rY = ref.gemm_quantized(q, s, g, rq, rs)
    check_y(host(Y), rY, q, s, g, rq, rs, ops.k_splits(M, N, K, g))
    if full_entry:
        Y2 = ops.w8a8_gemm(Wd, Sd, dev(x), g)
        check_y(host(Y2), ref.w8a8_gemm(q, s, g, x), q, s, g, rq, rs, ops.k_splits(M, N, K, g))
        # the whole entry point runs the same kernels as the partials hook
        assert same(host(Y2), host(Y))
    return Y


def check_y(Y, rY, q, s, g, rq, rs, splits):
    """Y bit-identical to the oracle when the linear keeps one group chain
    (fa_w8a8_gemm_k_splits == 1, the default); with K split over several
    workgroups (opted in with fa_w8a8_set_k_split), within
    ref.split_chain_tolerance (1 fp16 ulp + the fp32 reassociation bound of
    the partial chains) and within north_star's 1 fp16 ulp or rtol 1e-3."""
    if splits == 1:
        assert same(Y, rY), "Y differs from the oracle"
        return
    bound = ref.split_chain_tolerance(q, s, g, rq, rs, rY)
    err = np.abs(Y.astype(np.float64) - rY.astype(np.float64))
    assert np.all(err <= bound), float((err / bound).max())
    ns = ref.north_star_tolerance(rY)
    assert np.all(err <= ns), "outside 1 ulp / rtol 1e-3: %d outputs" % int((err > ns).sum())
    # the reassociation moves only rounding-boundary outputs
    assert np.mean(Y.view(np.uint16) == rY.view(np.uint16)) > 0.99


def test_config0_plumbing_m16_k512_n512_g64():
    """16 tokens, K=512, 512 outputs, g64, seed 0."""
    check_linear(16, 512, 512, 64, seed=0)


@pytest.mark.parametrize("name", list(LAYER))
def test_config1_decode_m1_g256(name):
    K, Nout = LAYER[name]
    check_linear(1, Nout, K, 256, seed=1)


@pytest.mark.parametrize("name", list(LAYER))
def test_config2_decode_m8_g64_fused_prologue(name):
    """8 tokens, g64, activation quant fused with RMSNorm (qkv,
    gate_up), SiLU*mul (down) or plain (o)."""
    K, Nout = LAYER[name]
    g, n = 64, 8
    q, s = make_linear(Nout, K, g, seed=2)
    if name in ("qkv", "gate_up"):
        x = synth.activations_f16(n, K, seed=3)
        gam = synth.gamma_f16(K)
        xq, xs = ops.rms_norm_quant(dev(x), dev(gam), 1e-6, g)
        rq, rs, _ = ref.rms_norm_quant(x, gam, 1e-6, g)
    elif name == "down":
        rng = np.random.default_rng(4)
        gate = (rng.standard_normal((n, K)) * 2).astype(np.float16)
        up = rng.standard_normal((n, K)).astype(np.float16)
        xq, xs = ops.silu_mul_quant(dev(gate), dev(up), g)
        rq, rs, _ = ref.silu_mul_quant(gate, up, g)
    else:
        x = synth.activations_f16(n, K, seed=5)
        xq, xs = ops.quantize_activations(dev(x), g)
        rq, rs = ref.quantize_activations(x, g)
    assert same(host(xq), rq) and same(host(xs), rs)
    Y, P = ops.w8a8_gemm_partials(dev(q), dev(s), g, xq, xs)
    assert same(host(P), ref.group_partials(q, rq, g))
    check_y(host(Y), ref.gemm_quantized(q, s, g, rq, rs), q, s, g, rq, rs,
            ops.k_splits(Nout, n, K, g))


@pytest.mark.parametrize("name", list(LAYER))
@pytest.mark.parametrize("n,g", [(8, 64), (8, 256), (5, 64), (16, 128), (2, 256)])
def test_small_batch_linear(name, n, g):
    """2 <= N <= 16 through fa_w8a8_gemm_quantized (the MFMA GEMV without
    the partials hook): Y bit-identical to the oracle at the configs[2] layer
    shapes (check_y: the GEMV keeps one group chain, k_splits == 1)."""
    K, Nout = LAYER[name]
    q, s = make_linear(Nout, K, g, seed=n + g)
    x = synth.activations_f16(n, K, seed=n + 3)
    rq, rs = ref.quantize_activations(x, g)
    Y = ops.w8a8_gemm_quantized(dev(q), dev(s), g, dev(rq), dev(rs))
    check_y(host(Y), ref.gemm_quantized(q, s, g, rq, rs), q, s, g, rq, rs,
            ops.k_splits(Nout, n, K, g))


def test_config3_prefill_m512_qkv_bitexact():
    K, Nout = LAYER["qkv"]
    check_linear(512, Nout, K, 256, seed=6, full_entry=False)


@pytest.mark.parametrize("N,g", [(512, 256), (2048, 256), (2048, 64)])
@pytest.mark.parametrize("name", list(LAYER))
def test_config3_prefill_subblock(name, N, g):
    """configs[3] at M=512 and M=2048 (plus g64): int32 per-group partials
    bit-exact on a 64x64 output sub-block, fp16 outputs bit-exact on sampled
    rows x tokens.  M=512 runs the 64-token tiles for qkv, o and down."""
    K, Nout = LAYER[name]
    torch.manual_seed(0)
    w = (torch.randn(Nout, K, device="cuda") * 0.02).half()
    Wd, Sd = ops.quantize_weights_groupwise(w, g)
    x = (torch.randn(N, K, device="cuda")).half()
    xq, xs = ops.quantize_activations(x, g)
    r0, t0 = (Nout // 3) // 16 * 16 + 5, N // 2 - 21
    Y, P = ops.w8a8_gemm_partials(Wd, Sd, g, xq, xs, row0=r0, rows=64, tok0=t0, toks=64)
    q, s, hq, hs, hY, hP = (host(t) for t in (Wd, Sd, xq, xs, Y, P))
    rP = ref.group_partials(q[r0:r0 + 64], hq[t0:t0 + 64], g)
    assert same(hP, rP)
    rows = np.unique(np.concatenate([np.arange(0, Nout, 97), [Nout - 1]]))
    toks = np.unique(np.concatenate([np.arange(0, N, 61), [N - 1]]))
    rY = ref.gemm_quantized(q[rows], s[rows], g, hq[toks], hs[toks])
    check_y(hY[np.ix_(toks, rows)], rY, q[rows], s[rows], g, hq[toks], hs[toks],
            ops.k_splits(Nout, N, K, g))


@pytest.mark.parametrize("name", ["o", "down"])
def test_prefill_k_split_512_tokens(name):
    """configs[3] at 512 tokens, o and down, with the opt-in K split: 80
    tiles of 128 x 128 split K over several workgroups.  The int32 partials
    are exact (64 x 64 block), every fp16 output of the full [512, 2560]
    result lies within the split tolerance of the oracle's single chain and
    within 1 fp16 ulp or rtol 1e-3, repeated calls give identical results,
    and with the split off (the default) the same call is bit-exact."""
    K, Nout = LAYER[name]
    N, g = 512, 256
    assert ops.k_splits(Nout, N, K, g) == 1
    torch.manual_seed(7)
    w = (torch.randn(Nout, K, device="cuda") * 0.02).half()
    Wd, Sd = ops.quantize_weights_groupwise(w, g)
    xq, xs = ops.quantize_activations((torch.randn(N, K, device="cuda")).half(), g)
    with ops.k_split(8):
        splits = ops.k_splits(Nout, N, K, g)
        assert splits > 1
        Y, P = ops.w8a8_gemm_partials(Wd, Sd, g, xq, xs, row0=640, rows=64, tok0=200, toks=64)
        Y2 = ops.w8a8_gemm_quantized(Wd, Sd, g, xq, xs)
        Y3 = ops.w8a8_gemm_quantized(Wd, Sd, g, xq, xs)
    q, s, hq, hs, hY, hP = (host(t) for t in (Wd, Sd, xq, xs, Y, P))
    assert same(hP, ref.group_partials(q[640:704], hq[200:264], g))
    rY = ref.gemm_quantized(q, s, g, hq, hs)
    check_y(hY, rY, q, s, g, hq, hs, splits)
    assert same(host(Y2), hY) and same(host(Y3), hY)
    Y4 = ops.w8a8_gemm_quantized(Wd, Sd, g, xq, xs)
    assert same(host(Y4), rY)


@pytest.mark.parametrize("N,M,K,g", [
    (1, 100, 512, 64),      # partial 16-row tile
    (1, 70, 2560, 256),     # N = 1, rows split over wave pairs, odd pass count
    (1, 33, 9728, 64),      # N = 1 split, ragged last pass, g64
    (1, 4100, 1536, 128),   # N = 1, two rows per wave and split
    (16, 48, 64, 64),       # one K step
    (3, 16, 4096, 4096),    # g == K (one group, 1-D scale)
    (2, 40, 128, 0),        # group_size <= 0 -> K
    (1, 40, 128, 1000),     # group_size > K  -> K
    (4, 64, 1024, 128),     # g128: two MFMA steps per group
    (17, 130, 256, 128),    # first GEMM size, ragged tiles
    (300, 200, 512, 512),   # GEMM, ragged tokens
    (300, 260, 512, 256),   # tile kernel, ragged tokens and rows
    (40, 300, 768, 64),     # tile kernel, g64 (two groups per stage)
    (129, 520, 1280, 128),  # tile kernel, g128
    (33, 64, 384, 128),     # K % 256 == 128: pipelined kernel, odd stage count
    (70, 259, 768, 256),    # tile kernel, in-kernel scale gather, M * G odd (last pair clamped)
    (40, 333, 256, 256),    # one group: 1-D scales, M odd
    (9, 389, 3392, 128),    # MFMA GEMV, K % g != 0: the last group one 64-byte step
    (5, 100, 192, 128),     # MFMA GEMV, two groups, the second short
    (16, 77, 1344, 256),    # MFMA GEMV, g256, last group 64 of 256 bytes
    (40, 300, 640, 512),    # pipelined kernel, g512, last group 128 bytes
    (3, 40, 100, 48),       # K, g not multiples of 64: generic kernel
    (20, 33, 96, 32),       # generic kernel, N > 16
])
def test_edge_shapes(N, M, K, g):
    check_linear(N, M, K, g, seed=N + M)


def _sweep_shapes(n=28, seed=2024):
    """Seeded random (N, M, K, g): one-token, small-batch and GEMM token
    counts, row counts that leave every tile ragged, K a multiple of 16 (and
    a few that are not), every group size the paths take."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        N = int(rng.choice([1, int(rng.integers(2, 17)), int(rng.integers(17, 129)),
                            int(rng.integers(129, 700))]))
        M = int(rng.integers(1, 3000))
        g = int(rng.choice([64, 128, 256, 512, 0]))
        K = int(rng.integers(1, 257)) * 16 if rng.random() < 0.85 else int(rng.integers(8, 2500))
        if N * M * K > 1.5e9:
            continue
        out.append((N, M, K, g))
    return out


@pytest.mark.parametrize("N,M,K,g", _sweep_shapes())
def test_random_shape_sweep(N, M, K, g):
    """Partials bit-exact and Y as the oracle's on seeded random shapes,
    through the partials hook and the full entry point."""
    print("sweep N=%d M=%d K=%d g=%d" % (N, M, K, g), flush=True)
    check_linear(N, M, K, g, seed=(N * 7 + M * 3 + K) % 1000)


def test_unaligned_weight_uses_exact_path():
    M, K, g, N = 24, 256, 64, 2
    q, s = make_linear(M, K, g, seed=11)
    x = synth.activations_f16(N, K, seed=12)
    buf = torch.zeros(M * K + 16, dtype=torch.int8, device="cuda")
    Wd = buf[1:1 + M * K].view(M, K)
    Wd.copy_(dev(q))
    Y = ops.w8a8_gemm(Wd, dev(s), dev(x), g)
    assert same(host(Y), ref.w8a8_gemm(q, s, g, x)), "unaligned"


def test_static_and_smooth_through_entry_point():
    M, K, g, N = 256, 512, 64, 4
    q, s = make_linear(M, K, g, seed=13)
    x = synth.activations_f16(N, K, seed=14)
    act = np.full(K // g, 0.04, np.float16)
    sm = synth.gamma_f16(K, seed=15)
    Y = ops.w8a8_gemm(dev(q), dev(s), dev(x), g, act_scale=dev(act), smooth_inv=dev(sm))
    assert same(host(Y), ref.w8a8_gemm(q, s, g, x, act_scale=act, smooth_inv=sm)), "static"


@pytest.mark.parametrize("N,M,K,g", [
    (8, 2560, 4096, 64),    # configs[2] o: in-kernel quantization, terms in LDS
    (8, 6144, 2560, 64),    # configs[2] qkv: more waves per tile so the range fits
    (8, 2560, 9728, 64),    # configs[2] down: range too long, separate quantizer
    (3, 333, 1344, 256),    # K % g != 0: the last group one 64-byte step
    (16, 48, 512, 512),     # one group of eight steps
    (2, 100, 192, 128),     # two groups, the second short
    (13, 1000, 2560, 256),
])
@pytest.mark.parametrize("mode", ["dynamic", "static", "smooth", "static_smooth"])
def test_small_batch_entry_quantization(N, M, K, g, mode):
    """fa_w8a8_gemm at 2 <= N <= 16, where the MFMA GEMV quantizes the fp16
    tokens itself (or the separate quantizer runs when the wave's K range is
    too long): Y equals the oracle's quantize-then-linear for dynamic and
    static scales, with and without smooth_inv."""
    print("qx N=%d M=%d K=%d g=%d %s" % (N, M, K, g, mode), flush=True)
    q, s = make_linear(M, K, g, seed=M + K)
    x = synth.activations_f16(N, K, seed=N + K)
    G = (K + g - 1) // g
    act = np.full(G, 0.03, np.float16) if "static" in mode else None
    sm = synth.gamma_f16(K, seed=K + 1) if "smooth" in mode else None
    Y = ops.w8a8_gemm(dev(q), dev(s), dev(x), g,
                      act_scale=None if act is None else dev(act),
                      smooth_inv=None if sm is None else dev(sm))
    assert same(host(Y), ref.w8a8_gemm(q, s, g, x, act_scale=act, smooth_inv=sm)), mode


def test_gemv_deterministic_across_calls():
    """Repeated calls with other shapes in between give identical Y."""
    K, Nout = LAYER["down"]
    q, s = make_linear(Nout, K, 256, seed=21)
    x = synth.activations_f16(1, K, seed=22)
    Wd, Sd, Xd = dev(q), dev(s), dev(x)
    first = host(ops.w8a8_gemm(Wd, Sd, Xd, 256))
    for _ in range(3):
        check_linear(2, 48, 512, 64, seed=3, full_entry=False)
        again = host(ops.w8a8_gemm(Wd, Sd, Xd, 256))
        assert same(first, again)


def test_bin_file_end_to_end():
    """int8 weight + fp16 scale written in the dual_ar.bin layout, read back by
    the library's loader, group size inferred from the scale shape, run."""
    K, Nout, g = 2560, 512, 64
    q, s = make_linear(Nout, K, g, seed=31)
    name = "text_model.model.layers.0.attention.wqkv.weight"
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "dual_ar.bin")
        write_bin(path, [(name, q), (name + "_scale", s)])
        with BinFile(path) as b:
            meta = b.quant_meta(name)
            assert meta.group_size == g and meta.has_scale
            Wd, Sd = dev(b.array(name)), dev(b.array(name + "_scale"))
    x = synth.activations_f16(1, K, seed=32)
    Y = ops.w8a8_gemm(Wd, Sd, dev(x), meta.group_size)
    assert same(host(Y), ref.w8a8_gemm(q, s, g, x)), "bin"


def test_bin_gate_up_swiglu_end_to_end():
    """feed_forward.w1 / .w3 written separately in the dual_ar.bin layout,
    interleaved by the loader (fa_bin_gate_up), run through the SwiGLU GEMV:
    the activation equals the oracle's two linears + silu_mul."""
    K, F, g = 2560, 1024, 256
    q1, s1 = make_linear(F, K, g, seed=61)
    q3, s3 = make_linear(F, K, g, seed=62)
    w1 = "text_model.model.layers.0.feed_forward.w1.weight"
    w3 = "text_model.model.layers.0.feed_forward.w3.weight"
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "dual_ar.bin")
        write_bin(path, [(w1, q1), (w1 + "_scale", s1), (w3, q3), (w3 + "_scale", s3)])
        with BinFile(path) as b:
            w13, s13, meta = b.gate_up(w1, w3)
    x = synth.activations_f16(1, K, seed=63)
    gam = synth.gamma_f16(K, seed=64)
    act = ops.w8a8_gemm_swiglu(dev(w13), dev(s13), dev(x), meta.group_size, gamma=dev(gam))
    rq, rs, _ = ref.rms_norm_quant(x, gam, 1e-6, g)
    _, _, ract = ref.silu_mul_quant(ref.gemm_quantized(q1, s1, g, rq, rs),
                                    ref.gemm_quantized(q3, s3, g, rq, rs), g)
    assert same(host(act), ract)


# ------------------------------------------------------- fp16 linear ----

def check_fp16_linear(W, X, Y, rows=None):
    """|Y - exact| within ref.fp16_linear_tolerance (1 fp16 ulp or 1e-3 rel.,
    plus 2^-18 * sum |w x| for fp32 accumulation in any order)."""
    Wh, Xh, Yh = host(W), host(X), host(Y)
    if rows is not None:
        Wh, Yh = Wh[rows], Yh[:, rows]
    ye, ab = ref.gemm_fp16_exact(Wh, Xh)
    err = np.abs(Yh.astype(np.float64) - ye)
    assert np.all(err <= ref.fp16_linear_tolerance(ye, ab)), float(err.max())


@pytest.mark.parametrize("N,M,K", [(1, 1000, 2560), (3, 777, 2560), (8, 512, 4096), (11, 300, 512),
                                   (2, 64, 100), (1, 40, 8192)])
def test_gemm_fp16(N, M, K):
    """fa_gemm_fp16 (gemm_fp16's cublasGemmEx fp16 / COMPUTE_32F semantics):
    streaming GEMV (K % 8 == 0, K <= 4096; token chunks 8/4/2/1) and the
    any-shape kernel (K = 100, K = 8192)."""
    torch.manual_seed(N * M + K)
    W = (torch.randn(M, K, device="cuda") * 0.05).half()
    X = torch.randn(N, K, device="cuda").half()
    check_fp16_linear(W, X, ops.gemm_fp16(W, X))


def test_gemm_fp16_logits_head():
    """The tied-embedding logits head at full size (155776 x 2560, 0.8 GB of
    fp16 weight, one token), checked on every 97th row and the last."""
    torch.manual_seed(9)
    W = (torch.randn(155776, 2560, device="cuda") * 0.02).half()
    X = torch.randn(1, 2560, device="cuda").half()
    Y = ops.gemm_fp16(W, X)
    rows = np.unique(np.concatenate([np.arange(0, 155776, 97), [155775]]))
    check_fp16_linear(W, X, Y, rows=rows)


# -------------------------------------------- fused prologue entries ----

@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("name,g", [("qkv", 256), ("gate_up", 64), ("qkv", 128)])
@pytest.mark.parametrize("with_resid", [True, False])
def test_gemm_rms_bitexact(name, g, T, with_resid):
    """fa_w8a8_gemm_rms = residual_add + rms_norm + quant + linear: Y and the
    residual output h_out bit-identical to the oracle chain (one fused GEMV
    launch at T == 1, separate launches otherwise)."""
    K, Nout = LAYER[name]
    q, s_ = make_linear(Nout, K, g, seed=31)
    x = synth.activations_f16(T, K, seed=32)
    gam = synth.gamma_f16(K, seed=33)
    res = synth.activations_f16(T, K, seed=34) if with_resid else None
    h_out = torch.empty((T, K), dtype=torch.float16, device="cuda")
    xd = dev(x)
    Y = ops.w8a8_gemm_rms(dev(q), dev(s_), xd, dev(gam), 1e-6, g,
                          resid=dev(res) if with_resid else None, h_out=h_out)
    h = ref.residual_add(x, res) if with_resid else x
    rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g)
    assert same(host(Y), ref.gemm_quantized(q, s_, g, rq, rs))
    assert same(host(h_out), h)
    assert same(host(xd), x)   # the input stream is not written


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("g", [256, 64])
def test_gemm_silu_mul_bitexact(g, T):
    K, Nout = LAYER["down"]
    q, s_ = make_linear(Nout, K, g, seed=41)
    rng = np.random.default_rng(42)
    gate = (rng.standard_normal((T, K)) * 2).astype(np.float16)
    up = rng.standard_normal((T, K)).astype(np.float16)
    Y = ops.w8a8_gemm_silu_mul(dev(q), dev(s_), dev(gate), dev(up), g)
    rq, rs, _ = ref.silu_mul_quant(gate, up, g)
    assert same(host(Y), ref.gemm_quantized(q, s_, g, rq, rs))


def test_gemm_rms_small_and_odd_dims():
    """RMS prologue where the reference reduction has fewer than 1024 threads
    (dim 384 -> 512 threads, 16 warps; dim 64 -> 64 threads, 2 warps)."""
    for K, g in ((384, 128), (64, 64)):
        q, s_ = make_linear(48, K, g, seed=K)
        x = synth.activations_f16(1, K, seed=K + 1)
        gam = synth.gamma_f16(K, seed=K + 2)
        Y = ops.w8a8_gemm_rms(dev(q), dev(s_), dev(x), dev(gam), 1e-6, g)
        rq, rs, _ = ref.rms_norm_quant(x, gam, 1e-6, g)
        assert same(host(Y), ref.gemm_quantized(q, s_, g, rq, rs)), K


@pytest.mark.parametrize("T", [1, 3, 8, 16])
@pytest.mark.parametrize("g", [256, 64])
@pytest.mark.parametrize("mode", ["rms_resid", "rms", "plain"])
def test_gemm_swiglu_bitexact(g, T, mode):
    """fa_w8a8_gemm_swiglu on a row-interleaved w1 / w3 weight: act equals
    the oracle's two linears + silu_mul (fp16 roundings included), h_out the
    residual add."""
    K, F = 2560, 1536
    q1, s1 = make_linear(F, K, g, seed=51)
    q3, s3 = make_linear(F, K, g, seed=52)
    q13 = np.stack((q1, q3), axis=1).reshape(2 * F, K)
    s13 = np.stack((s1, s3), axis=1).reshape(2 * F, -1)
    x = synth.activations_f16(T, K, seed=53)
    gam = synth.gamma_f16(K, seed=54)
    res = synth.activations_f16(T, K, seed=55)
    h_out = torch.empty((T, K), dtype=torch.float16, device="cuda")
    if mode == "plain":
        act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g)
        rq, rs = ref.quantize_activations(x, g)
    else:
        r = dev(res) if mode == "rms_resid" else None
        act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g, gamma=dev(gam), eps=1e-6,
                                   resid=r, h_out=h_out)
        h = ref.residual_add(x, res) if mode == "rms_resid" else x
        rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g)
        assert same(host(h_out), h)
    gate = ref.gemm_quantized(q1, s1, g, rq, rs)
    up = ref.gemm_quantized(q3, s3, g, rq, rs)
    _, _, ract = ref.silu_mul_quant(gate, up, g)
    assert same(host(act), ract)


def _fused_sweep(n=18, seed=77):
    """Seeded random cases for the fused entry points: (entry, T, M, K, g)."""
    rng = np.random.default_rng(seed)
    entries = ["rms", "rms_resid", "silu_mul", "swiglu", "swiglu_rms"]
    out = []
    for i in range(n):
        e = entries[i % len(entries)]
        T = int(rng.choice([1, 1, 2, int(rng.integers(3, 40))]))
        M = int(rng.integers(1, 1500)) * (2 if e.startswith("swiglu") else 1)
        K = int(rng.integers(1, 400)) * 16
        g = int(rng.choice([64, 128, 256, 512]))
        out.append((e, T, M, K, g))
    return out


@pytest.mark.parametrize("entry,T,M,K,g", _fused_sweep())
def test_fused_entry_sweep(entry, T, M, K, g):
    """The fused entry points on seeded random shapes (K % g often nonzero,
    odd row counts), against the oracle's chain of separate functions."""
    print("fused %s T=%d M=%d K=%d g=%d" % (entry, T, M, K, g), flush=True)
    rng = np.random.default_rng(M * 31 + K)
    x = synth.activations_f16(T, K, seed=M)
    gam = synth.gamma_f16(K, seed=K)
    res = synth.activations_f16(T, K, seed=M + 1)
    if entry.startswith("swiglu"):
        F = M // 2
        q1, s1 = make_linear(F, K, g, seed=M + 2)
        q3, s3 = make_linear(F, K, g, seed=M + 3)
        q13 = np.stack((q1, q3), axis=1).reshape(2 * F, K)
        s13 = np.stack((s1, s3), axis=1).reshape(2 * F, -1)
        if entry == "swiglu":
            act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g)
            rq, rs = ref.quantize_activations(x, g)
        else:
            h_out = torch.empty((T, K), dtype=torch.float16, device="cuda")
            act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g, gamma=dev(gam), eps=1e-6,
                                       resid=dev(res), h_out=h_out)
            h = ref.residual_add(x, res)
            rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g)
            assert same(host(h_out), h)
        _, _, ract = ref.silu_mul_quant(ref.gemm_quantized(q1, s1, g, rq, rs),
                                        ref.gemm_quantized(q3, s3, g, rq, rs), g)
        assert same(host(act), ract)
        return
    q, s_ = make_linear(M, K, g, seed=M + 4)
    if entry == "silu_mul":
        gate = (rng.standard_normal((T, K)) * 2).astype(np.float16)
        up = rng.standard_normal((T, K)).astype(np.float16)
        Y = ops.w8a8_gemm_silu_mul(dev(q), dev(s_), dev(gate), dev(up), g)
        rq, rs, _ = ref.silu_mul_quant(gate, up, g)
    else:
        resid = entry == "rms_resid"
        h_out = torch.empty((T, K), dtype=torch.float16, device="cuda")
        Y = ops.w8a8_gemm_rms(dev(q), dev(s_), dev(x), dev(gam), 1e-6, g,
                              resid=dev(res) if resid else None, h_out=h_out)
        h = ref.residual_add(x, res) if resid else x
        rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g)
        assert same(host(h_out), h)
    assert same(host(Y), ref.gemm_quantized(q, s_, g, rq, rs))


# ------------------------------------------------------- decode stack ----

@pytest.mark.parametrize("g,T", [(256, 1), (64, 2)])
def test_decode_stack_bitexact(g, T):
    """configs[4] pipeline (fish_amd.decode_stack.run_stack, fused residual +
    RMSNorm + quant included) over two layers, against the same sequence of
    oracle functions: the final residual stream is bit-identical."""
    from fish_amd.decode_stack import DecodeStack, FFN, Q_DIM
    st = DecodeStack(n_layers=2, g=g, tokens=T, seed=5)
    st.h.copy_(st.h0)
    st.run_stack()
    torch.cuda.synchronize()
    h = host(st.h0)
    for lay in st.layers:
        def lin(name, xq, xs):
            return ref.gemm_quantized(host(lay[name].W), host(lay[name].scale), g, xq, xs)
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["attn_norm"]), 1e-6, g)
        y = lin("qkv", xq, xs)
        xq, xs = ref.quantize_activations(np.ascontiguousarray(y[:, :Q_DIM]), g)
        h = ref.residual_add(h, lin("o", xq, xs))
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["ffn_norm"]), 1e-6, g)
        y = lin("gate_up", xq, xs)      # rows interleaved: gate 2i, up 2i + 1
        xq, xs, _ = ref.silu_mul_quant(np.ascontiguousarray(y[:, 0::2]),
                                       np.ascontiguousarray(y[:, 1::2]), g)
        h = ref.residual_add(h, lin("down", xq, xs))
    assert same(host(st.h), h)


# One GPU's share under 8-way tensor parallelism: qkv and gate_up split
# their output rows, o and down their K (down's 1216 leaves a short last
# group at g256; o's 512 is two groups).
TP8 = {"qkv": (2560, 768), "o": (512, 2560), "gate_up": (2560, 2432), "down": (1216, 2560)}


@pytest.mark.parametrize("name", list(TP8))
@pytest.mark.parametrize("N,g", [(1, 256), (8, 64), (8, 256), (16, 256), (512, 256),
                                 (2048, 256)])
def test_tp8_shard_shapes(name, N, g):
    """TP=8 shard shapes through fa_w8a8_gemm_partials (every int32 group
    partial up to 16 tokens, a 64 x 64 window beyond) and fa_w8a8_gemm:
    bit-exact against the oracle."""
    K, Nout = TP8[name]
    if N <= 16:
        check_linear(N, Nout, K, g, seed=50 + N)
        return
    q, s = make_linear(Nout, K, g, seed=60)
    x = synth.activations_f16(N, K, seed=61)
    rq, rs = ref.quantize_activations(x, g)
    r0, t0 = Nout // 2 - 32, N // 3
    Y, P = ops.w8a8_gemm_partials(dev(q), dev(s), g, dev(rq), dev(rs), row0=r0, rows=64,
                                  tok0=t0, toks=64)
    assert same(host(P), ref.group_partials(q[r0:r0 + 64], rq[t0:t0 + 64], g))
    assert same(host(Y), ref.gemm_quantized(q, s, g, rq, rs))
    Y2 = ops.w8a8_gemm(dev(q), dev(s), dev(x), g)
    assert same(host(Y2), host(Y))

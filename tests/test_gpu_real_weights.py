"""GPU parity of the calibrated-weight (AWQ / static-scale) decode branches.

A calibrated dual_ar.bin gives every wqkv / w1 / w3 its own `_smooth_inv`
(/root/reference/tools/step2_export_w8a8.py:477, uploaded per weight at
src/engine/dual_ar_engine.cc:253-261) and, with FISH_INT8_STATIC_ACT_SCALE=1,
an `_act_scale` (:262-269); the quantizer applies them at
src/kernels/int8_gemm.cu:178 and :206.  At one token the entry points
quantize inside the GEMV (no separate launch), so these tests drive exactly
that in-kernel branch at the configs[1] / configs[2] layer shapes and
compare bit for bit with the oracle: fa_w8a8_gemm, fa_w8a8_gemm_rms (with and
without the residual), fa_w8a8_gemm_silu_mul and fa_w8a8_gemm_swiglu, each
with a per-weight smooth_inv and, separately, a static act_scale, including
K that is not a multiple of the group size.
"""
import numpy as np
import pytest
import torch

from oracle import ref
from fish_amd import ops, synth

pytestmark = pytest.mark.gpu

LAYER = synth.LAYER_SHAPES


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a device"
    from fish_amd import _lib
    _lib.lib()
    yield
    torch.cuda.synchronize()


def dev(a):
    return torch.from_numpy(np.array(a, copy=True, order="C")).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    return np.array_equal(a.view(np.uint8), b.view(np.uint8))


def make_linear(M, K, g, seed):
    return ref.quantize_weights(synth.weights_f16(M, K, seed=seed), g)


def smooth_inv_f16(K, seed):
    """AWQ-style per-channel factors: log-normal around 1 (0.2 .. 5)."""
    rng = np.random.default_rng(seed)
    return np.exp(np.clip(rng.standard_normal(K) * 0.5, -1.6, 1.6)).astype(np.float16)


def act_scale_f16(K, g, seed, amax=40.0):
    """Static per-group scales as compute_group_act_scales makes them
    (step2_export_w8a8.py:194-204: calibration amax / 127 per group); some
    groups get a small scale so their codes saturate at +-127."""
    G = ref.groups(K, g)
    rng = np.random.default_rng(seed)
    s = (amax * (0.2 + rng.random(G)) / 127.0).astype(np.float16)
    s[::5] = np.float16(0.004)
    return s


def companions(variant, K, g, seed):
    if variant == "smooth":
        return None, smooth_inv_f16(K, seed)
    if variant == "static":
        return act_scale_f16(K, g, seed), None
    return act_scale_f16(K, g, seed), smooth_inv_f16(K, seed + 1)   # both


def opt(a):
    return None if a is None else dev(a)


# (name, K, M, g): the configs[1] and configs[2] layer shapes at one token,
# plus K = 2576 (not a multiple of 64 or 256: a 16-wide last group)
SHAPES = [(n, K, M, 256) for n, (K, M) in LAYER.items()] + \
         [(n, K, M, 64) for n, (K, M) in LAYER.items()] + \
         [("k2576", 2576, 1000, 256), ("k2576", 2576, 700, 64), ("k2576", 2576, 300, 128)]


@pytest.mark.parametrize("variant", ["smooth", "static", "both"])
@pytest.mark.parametrize("name,K,M,g", SHAPES)
def test_gemm_one_token(name, K, M, g, variant):
    q, s = make_linear(M, K, g, seed=K + M)
    x = synth.activations_f16(1, K, seed=M)
    act, sm = companions(variant, K, g, seed=K)
    Y = ops.w8a8_gemm(dev(q), dev(s), dev(x), g, act_scale=opt(act), smooth_inv=opt(sm))
    assert same(host(Y), ref.w8a8_gemm(q, s, g, x, act_scale=act, smooth_inv=sm)), \
        (name, K, M, g, variant)


RMS_SHAPES = [("qkv", 2560, 6144, 256), ("gate_up", 2560, 19456, 256), ("qkv", 2560, 6144, 64),
              ("k2576", 2576, 520, 256), ("k2576", 2576, 520, 64)]


@pytest.mark.parametrize("with_resid", [True, False])
@pytest.mark.parametrize("variant", ["smooth", "static"])
@pytest.mark.parametrize("name,K,M,g", RMS_SHAPES)
def test_gemm_rms_one_token(name, K, M, g, variant, with_resid):
    q, s = make_linear(M, K, g, seed=K + 3)
    x = synth.activations_f16(1, K, seed=7)
    gam = synth.gamma_f16(K, seed=8)
    res = synth.activations_f16(1, K, seed=9) if with_resid else None
    act, sm = companions(variant, K, g, seed=K + 5)
    h_out = torch.empty((1, K), dtype=torch.float16, device="cuda")
    xd = dev(x)
    Y = ops.w8a8_gemm_rms(dev(q), dev(s), xd, dev(gam), 1e-6, g, resid=opt(res), h_out=h_out,
                          act_scale=opt(act), smooth_inv=opt(sm))
    h = ref.residual_add(x, res) if with_resid else x
    rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g, smooth_inv=sm, act_scale=act)
    assert same(host(Y), ref.gemm_quantized(q, s, g, rq, rs)), (name, g, variant)
    assert same(host(h_out), h)
    assert same(host(xd), x)


@pytest.mark.parametrize("variant", ["smooth", "static"])
@pytest.mark.parametrize("K,M,g", [(9728, 2560, 256), (9728, 2560, 64), (2576, 640, 256)])
def test_gemm_silu_mul_one_token(K, M, g, variant):
    q, s = make_linear(M, K, g, seed=K + 11)
    rng = np.random.default_rng(K)
    gate = (rng.standard_normal((1, K)) * 2).astype(np.float16)
    up = rng.standard_normal((1, K)).astype(np.float16)
    act, sm = companions(variant, K, g, seed=K + 12)
    Y = ops.w8a8_gemm_silu_mul(dev(q), dev(s), dev(gate), dev(up), g, act_scale=opt(act),
                               smooth_inv=opt(sm))
    rq, rs, _ = ref.silu_mul_quant(gate, up, g, smooth_inv=sm, act_scale=act)
    assert same(host(Y), ref.gemm_quantized(q, s, g, rq, rs)), (K, g, variant)


@pytest.mark.parametrize("variant", ["smooth", "static"])
@pytest.mark.parametrize("mode", ["rms_resid", "plain"])
@pytest.mark.parametrize("g", [256, 64])
def test_gemm_swiglu_one_token_shared_companions(g, mode, variant):
    """w1 and w3 sharing one smooth_inv / act_scale (the case the fused
    pair serves): act = silu(gate) * up of the oracle's two linears."""
    K, F = 2560, 1536
    q1, s1 = make_linear(F, K, g, seed=71)
    q3, s3 = make_linear(F, K, g, seed=72)
    q13 = np.stack((q1, q3), axis=1).reshape(2 * F, K)
    s13 = np.stack((s1, s3), axis=1).reshape(2 * F, -1)
    x = synth.activations_f16(1, K, seed=73)
    gam = synth.gamma_f16(K, seed=74)
    res = synth.activations_f16(1, K, seed=75)
    act_s, sm = companions(variant, K, g, seed=76)
    if mode == "plain":
        act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g, act_scale=opt(act_s),
                                   smooth_inv=opt(sm))
        rq, rs = ref.quantize_activations(x, g, act_scale=act_s, smooth_inv=sm)
    else:
        h_out = torch.empty((1, K), dtype=torch.float16, device="cuda")
        act = ops.w8a8_gemm_swiglu(dev(q13), dev(s13), dev(x), g, gamma=dev(gam), eps=1e-6,
                                   resid=dev(res), h_out=h_out, act_scale=opt(act_s),
                                   smooth_inv=opt(sm))
        h = ref.residual_add(x, res)
        rq, rs, _ = ref.rms_norm_quant(h, gam, 1e-6, g, smooth_inv=sm, act_scale=act_s)
        assert same(host(h_out), h)
    _, _, ract = ref.silu_mul_quant(ref.gemm_quantized(q1, s1, g, rq, rs),
                                    ref.gemm_quantized(q3, s3, g, rq, rs), g)
    assert same(host(act), ract)


# ------------------------------------------------- calibrated decode stack ----

@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("g,T,layers", [(256, 1, 3), (64, 1, 2), (256, 2, 2)])
def test_awq_decode_stack_bitexact(g, T, layers, fused):
    """DecodeStack(awq=True): wqkv, w1 and w3 each carry their own
    smooth_inv (the calibrated dual_ar.bin layout), so w1 and w3 see
    differently quantized inputs -- one fa_w8a8_gemm_swiglu_sep launch
    (run_stack_awq) or two RMS-fused linears and silu_mul
    (run_stack_awq_unfused).  The final residual stream equals the oracle's
    sequence of separate functions bit for bit."""
    from fish_amd.decode_stack import DecodeStack, Q_DIM
    st = DecodeStack(n_layers=layers, g=g, tokens=T, seed=9, awq=True)
    st.h.copy_(st.h0)
    (st.run_stack_awq if fused else st.run_stack_awq_unfused)()
    torch.cuda.synchronize()
    h = host(st.h0)
    for lay in st.layers:
        def lin(name, xq, xs):
            return ref.gemm_quantized(host(lay[name].W), host(lay[name].scale), g, xq, xs)
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["attn_norm"]), 1e-6, g,
                                       smooth_inv=host(lay["qkv_smooth"]))
        y = lin("qkv", xq, xs)
        xq, xs = ref.quantize_activations(np.ascontiguousarray(y[:, :Q_DIM]), g)
        h = ref.residual_add(h, lin("o", xq, xs))
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["ffn_norm"]), 1e-6, g,
                                       smooth_inv=host(lay["w1_smooth"]))
        gate = lin("w1", xq, xs)
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["ffn_norm"]), 1e-6, g,
                                       smooth_inv=host(lay["w3_smooth"]))
        up = lin("w3", xq, xs)
        xq, xs, _ = ref.silu_mul_quant(gate, up, g)
        h = ref.residual_add(h, lin("down", xq, xs))
    assert same(host(st.h), h)


# ------------------------------------------- separate w1 / w3 SwiGLU ----

@pytest.mark.parametrize("T", [1, 3])
@pytest.mark.parametrize("mode", ["plain", "rms", "rms_resid"])
@pytest.mark.parametrize("comp", ["smooth", "static", "mixed"])
@pytest.mark.parametrize("F,K,g", [(9728, 2560, 256), (1531, 2560, 64), (700, 2576, 128)])
def test_swiglu_sep(F, K, g, comp, mode, T):
    """fa_w8a8_gemm_swiglu_sep: act = fp16(silu(gate)) * up with gate and up
    from separate weights whose inputs quantize with their own companions,
    bit for bit against the oracle's two linears and silu_mul; h_out is the
    residual stream.  One launch at T == 1, separate launches otherwise."""
    print("swiglu_sep F=%d K=%d g=%d %s %s T=%d" % (F, K, g, comp, mode, T), flush=True)
    q1, s1 = make_linear(F, K, g, seed=61)
    q3, s3 = make_linear(F, K, g, seed=62)
    x = synth.activations_f16(T, K, seed=63)
    gam = synth.gamma_f16(K, seed=64)
    res = synth.activations_f16(T, K, seed=65)
    if comp == "smooth":
        a1, m1, a3, m3 = None, smooth_inv_f16(K, 66), None, smooth_inv_f16(K, 67)
    elif comp == "static":
        a1, m1, a3, m3 = act_scale_f16(K, g, 68), None, act_scale_f16(K, g, 69, amax=20.0), None
    else:
        a1, m1, a3, m3 = None, smooth_inv_f16(K, 70), act_scale_f16(K, g, 71), None
    h_out = torch.empty((T, K), dtype=torch.float16, device="cuda") if mode != "plain" else None
    d = dict(W1=dev(q1), s1=dev(s1), W3=dev(q3), s3=dev(s3), x=dev(x), gam=dev(gam), res=dev(res))
    act = ops.w8a8_gemm_swiglu_sep(
        d["W1"], d["s1"], d["W3"], d["s3"], d["x"], g,
        gamma=None if mode == "plain" else d["gam"], eps=1e-6,
        resid=d["res"] if mode == "rms_resid" else None, h_out=h_out,
        act_scale1=opt(a1), smooth_inv1=opt(m1), act_scale3=opt(a3), smooth_inv3=opt(m3))
    h = ref.residual_add(x, res) if mode == "rms_resid" else x
    def quant(a, m):
        if mode == "plain":
            return ref.quantize_activations(h, g, act_scale=a, smooth_inv=m)
        xq, xs, _ = ref.rms_norm_quant(h, gam, 1e-6, g, act_scale=a, smooth_inv=m)
        return xq, xs
    gate = ref.gemm_quantized(q1, s1, g, *quant(a1, m1))
    up = ref.gemm_quantized(q3, s3, g, *quant(a3, m3))
    _, _, want = ref.silu_mul_quant(gate, up, g)
    assert same(host(act), want)
    if h_out is not None:
        assert same(host(h_out), h)
    assert same(host(d["x"]), x)


# ------------------------------------------------------- fast decoder ----

def test_fast_decoder_pass_bitexact():
    """One codebook pass of the fast decoder (dual_ar_engine.cc:794-838): the
    4-layer stack at the slow layer's shapes, then RMSNorm + the int8 output
    head (4096 x 2560, one token) -- hidden state and logits bit-identical to
    the oracle's sequence; a second pass repeats the first exactly."""
    from fish_amd.decode_stack import FastDecoder, Q_DIM
    g = 256
    fd = FastDecoder(g=g, seed=21)
    fd.run_pass()
    torch.cuda.synchronize()
    h = host(fd.h0)
    for lay in fd.layers:
        def lin(name, xq, xs):
            return ref.gemm_quantized(host(lay[name].W), host(lay[name].scale), g, xq, xs)
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["attn_norm"]), 1e-6, g)
        y = lin("qkv", xq, xs)
        xq, xs = ref.quantize_activations(np.ascontiguousarray(y[:, :Q_DIM]), g)
        h = ref.residual_add(h, lin("o", xq, xs))
        xq, xs, _ = ref.rms_norm_quant(h, host(lay["ffn_norm"]), 1e-6, g)
        y = lin("gate_up", xq, xs)
        xq, xs, _ = ref.silu_mul_quant(np.ascontiguousarray(y[:, 0::2]),
                                       np.ascontiguousarray(y[:, 1::2]), g)
        h = ref.residual_add(h, lin("down", xq, xs))
    assert same(host(fd.h), h)
    xq, xs, _ = ref.rms_norm_quant(h, host(fd.fast_norm), 1e-6, g)
    rl = ref.gemm_quantized(host(fd.head.W), host(fd.head.scale), g, xq, xs)
    first = host(fd.logits).copy()
    assert same(first, rl)
    fd.run_pass()
    assert same(host(fd.logits), first)

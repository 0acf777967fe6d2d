"""GPU: the decode chain (fa_chain, every linear of a decode step in one
persistent launch) against the oracle and against the four-launch-per-layer
stack -- bit-exact, like every other linear-layer path."""
import numpy as np
import pytest
import torch

from oracle import ref
from fish_amd import _lib, ops, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    assert torch.cuda.is_available(), "GPU tests need a device"
    _lib.lib()
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


def stack_oracle(st, h, g):
    """The decode_stack oracle sequence over st's layers from residual h."""
    from fish_amd.decode_stack import Q_DIM
    for lay in st.layers:
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
    return h


@pytest.mark.parametrize("g", [256, 64])
def test_chain_stack_bitexact(g):
    """configs[4]'s linears as one chain launch: the final residual stream is
    bit-identical to the four-launch stack and to the oracle, and a second
    run (counters reset by the launch itself) repeats it."""
    from fish_amd.decode_stack import DecodeStack
    st = DecodeStack(n_layers=3, g=g, tokens=1, seed=11)
    st.h.copy_(st.h0)
    st.run_stack()
    h_stack = host(st.h).copy()
    for rep in range(2):
        st.h.copy_(st.h0)
        st.run_chain()
        assert st.chain.status() == 0, _lib.lib().fa_last_error()
        assert same(host(st.h), h_stack), ("chain != stack", rep)
    assert same(h_stack, stack_oracle(st, host(st.h0), g))


def test_stack_and_chain_36_layers():
    """configs[4] at its full size: 36 layers of distinct weights, one token,
    g256 -- the four-launch stack, the chain launch and the oracle's chain
    of separate functions end in the same residual stream, bit for bit."""
    from fish_amd.decode_stack import DecodeStack
    st = DecodeStack(n_layers=36, g=256, tokens=1, seed=23)
    st.h.copy_(st.h0)
    st.run_stack()
    h_stack = host(st.h).copy()
    st.h.copy_(st.h0)
    st.run_chain()
    assert same(host(st.h), h_stack), "chain != stack at 36 layers"
    st.chain.close()
    h_ref = stack_oracle(st, host(st.h0), 256)
    assert same(h_stack, h_ref), "stack != oracle at 36 layers"
    assert np.isfinite(h_ref.astype(np.float32)).all()


@pytest.mark.parametrize("ks", [(512, 768, 1024), (528, 784, 1040)])
@pytest.mark.parametrize("g", [64, 128, 256])
def test_chain_step_kinds_bitexact(g, ks):
    """Every step kind, odd row counts, and a step reading what an earlier
    step's prologue wrote (h_out), against the oracle; the second K set
    leaves every step's last group short (K % g != 0)."""
    rng = np.random.default_rng(100 + g)
    K0, K1, K2 = ks
    W0, s0 = ref.quantize_weights(synth.weights_f16(37, K0, seed=1), g)
    W1, s1 = ref.quantize_weights(synth.weights_f16(70, K1, seed=2), g)
    W2, s2 = ref.quantize_weights(synth.weights_f16(2 * 33, K2, seed=3), g)
    W3, s3 = ref.quantize_weights(synth.weights_f16(50, K1, seed=4), g)
    xa = synth.activations_f16(1, K0, seed=5)
    xb = synth.activations_f16(1, K1, seed=6)
    xr = (rng.standard_normal((1, K1)) * 0.5).astype(np.float16)
    gm = (1 + 0.1 * rng.standard_normal(K1)).astype(np.float16)
    xc = synth.activations_f16(1, K2, seed=7)
    d = {k: dev(v) for k, v in dict(W0=W0, s0=s0, W1=W1, s1=s1, W2=W2, s2=s2, W3=W3, s3=s3,
                                    xa=xa, xb=xb, xr=xr, gm=gm, xc=xc).items()}
    y0 = torch.empty(37, dtype=torch.float16, device="cuda")
    y1 = torch.empty(70, dtype=torch.float16, device="cuda")
    act = torch.empty(33, dtype=torch.float16, device="cuda")
    y3 = torch.empty(50, dtype=torch.float16, device="cuda")
    hb = torch.empty(K1, dtype=torch.float16, device="cuda")
    steps = [
        dict(w=d["W0"], w_scale=d["s0"], x=d["xa"], y=y0),
        dict(w=d["W1"], w_scale=d["s1"], x=d["xb"], x2=d["xr"], gamma=d["gm"], h_out=hb,
             y=y1, prologue=2, eps=1e-6),
        dict(w=d["W2"], w_scale=d["s2"], x=d["xc"], y=act, epilogue=1),
        dict(w=d["W3"], w_scale=d["s3"], x=hb, y=y3),
    ]
    ch = ops.Chain(steps, g)
    for rep in range(2):
        for t in (y0, y1, act, y3, hb):
            t.fill_(0)
        ch.run()
        assert ch.status() == 0
        xq, xs = ref.quantize_activations(xa, g)
        assert same(host(y0), ref.gemm_quantized(W0, s0, g, xq, xs)[0])
        h = ref.residual_add(xb, xr)
        assert same(host(hb), h[0])
        xq, xs, _ = ref.rms_norm_quant(h, gm, 1e-6, g)
        assert same(host(y1), ref.gemm_quantized(W1, s1, g, xq, xs)[0])
        xq, xs = ref.quantize_activations(xc, g)
        y = ref.gemm_quantized(W2, s2, g, xq, xs)
        _, _, ract = ref.silu_mul_quant(np.ascontiguousarray(y[:, 0::2]),
                                        np.ascontiguousarray(y[:, 1::2]), g)
        assert same(host(act), ract[0])
        xq, xs = ref.quantize_activations(h, g)
        assert same(host(y3), ref.gemm_quantized(W3, s3, g, xq, xs)[0])
    ch.close()


@pytest.mark.parametrize("case", range(4))
def test_chain_random_steps(case):
    """Seeded random step lists (row counts, K, prologue and epilogue kinds,
    K % g often nonzero), every step against the oracle."""
    rng = np.random.default_rng(900 + case)
    g = int(rng.choice([64, 128, 256]))
    steps, checks, keep = [], [], []
    for i in range(int(rng.integers(3, 7))):
        pro = int(rng.choice([0, 2]))
        epi = int(rng.choice([0, 0, 1]))
        K = int(rng.integers(max(1, g // 16), (4096 if pro else 8192) // 16 + 1)) * 16
        M = int(rng.integers(2, 1200)) * (2 if epi else 1)
        q, s_ = ref.quantize_weights(synth.weights_f16(M, K, seed=case * 10 + i), g)
        x = synth.activations_f16(1, K, seed=case * 10 + i + 100)
        st = dict(w=dev(q), w_scale=dev(s_), x=dev(x))
        if pro == 2:
            x2 = synth.activations_f16(1, K, seed=case * 10 + i + 200)
            gm = synth.gamma_f16(K, seed=case * 10 + i)
            h_out = torch.empty(K, dtype=torch.float16, device="cuda")
            st.update(x2=dev(x2), gamma=dev(gm), h_out=h_out, prologue=2, eps=1e-6)
            h = ref.residual_add(x, x2)
            xq, xs, _ = ref.rms_norm_quant(h, gm, 1e-6, g)
        else:
            h = None
            xq, xs = ref.quantize_activations(x, g)
        y = ref.gemm_quantized(q, s_, g, xq, xs)
        if epi:
            st["epilogue"] = 1
            _, _, y = ref.silu_mul_quant(np.ascontiguousarray(y[:, 0::2]),
                                         np.ascontiguousarray(y[:, 1::2]), g)
        out = torch.empty(y.shape[1], dtype=torch.float16, device="cuda")
        st["y"] = out
        steps.append(st)
        checks.append((out, y[0], st.get("h_out"), None if h is None else h[0]))
    ch = ops.Chain(steps, g)
    try:
        for rep in range(2):
            for out, _, ho, _ in checks:
                out.fill_(0)
                if ho is not None:
                    ho.fill_(0)
            ch.run()
            assert ch.status() == 0
            for i, (out, want, ho, hw) in enumerate(checks):
                assert same(host(out), want), (case, rep, i)
                if ho is not None:
                    assert same(host(ho), hw), (case, rep, i, "h_out")
    finally:
        ch.close()


def test_chain_gives_up_and_recovers():
    """With no polls allowed, a step that has to wait for its predecessor
    gives up: every workgroup leaves, the status reports it, and the next run
    with the default limit is complete and exact.  (The kernels always exit;
    only the bounded wait is shortened, from the host.)"""
    from fish_amd.decode_stack import DecodeStack
    st = DecodeStack(n_layers=2, g=256, tokens=1, seed=3)
    st.h.copy_(st.h0)
    st.run_stack()
    h_stack = host(st.h).copy()
    st.build_chain()
    st.chain.set_spin_limit(0)
    st.h.copy_(st.h0)
    st.run_chain(check=False)
    assert st.chain.status() == _lib.FA_ERR_HIP
    st.chain.set_spin_limit(1 << 21)
    st.h.copy_(st.h0)
    st.run_chain()
    assert st.chain.status() == 0
    assert same(host(st.h), h_stack)

"""Pins the CPU oracle (oracle/w8a8_ref.c) before it is trusted as a checker.

The reference ships no golden vectors or numeric fixtures for this path (it
has no INT8 test at all), so every check here is one of: numpy's independent
float16 conversion, a hand-computed known answer, the reference's own
closed-form tests (tests/test_kernels.cu:121-247, 354-481), an invariant the
mathematics fixes, or a float64 / exact-integer evaluation of the same sum.
"""
import numpy as np
import pytest

from oracle import ref
from helpers import assert_fp16_close, fp16_ulp


@pytest.fixture(scope="module", autouse=True)
def _built():
    from fish_amd.build import build_oracle
    build_oracle()


# ------------------------------------------------------------------ fp16 ----

def test_h2f_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    got = ref.h2f(h)
    want = h.astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_matches_numpy_incl_ties():
    rng = np.random.default_rng(0)
    halves = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16)
    hv = halves.astype(np.float64)
    mids = ((hv[:-1] + hv[1:]) / 2).astype(np.float32)          # exact ties
    assert np.array_equal(mids.astype(np.float64), (hv[:-1] + hv[1:]) / 2)
    near = np.concatenate([np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(0))])
    rand = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * s for s in (1e-7, 1e-5, 1e-2, 1, 100, 3e4)])
    special = np.array([0.0, -0.0, 65504, 65519.996, 65520, 65536, 1e30, np.inf, -np.inf,
                        5.96e-8, 2.98e-8, 2.99e-8, 1e-10, 6.1e-5, 6.103515625e-05], np.float32)
    x = np.concatenate([halves.astype(np.float32), mids, near, rand, special])
    x = np.concatenate([x, -x])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16)
    got = ref.f2h(x)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    nan = ref.f2h(np.array([np.nan], np.float32))
    assert np.isnan(nan.astype(np.float32)[0])


# ---------------------------------------------------------- weight quant ----

def test_weight_quant_known_answers():
    # amax = 127 * 2^-7 -> s = amax / 127 = 2^-7 exactly; 0.5 and 1.5 steps
    # are exact ties and round to even (np.round semantics).
    w = np.array([[0.9921875, -0.4921875, 0.00390625, 0.01171875]], np.float16)
    q, s = ref.quantize_weights(w, 4)
    assert s.shape == (1, 1)
    assert s[0, 0] == np.float16(2.0 ** -7)
    assert q.tolist() == [[127, -63, 0, 2]]
    # amax = 1.27 (fp16 1.26953125): amax/127 = 0.0099963 -> fp16 0.0099945068
    w = np.array([[1.27, -0.635, 0.0, 0.005]], np.float16)
    q, s = ref.quantize_weights(w, 4)
    assert s[0, 0] == np.float16(0.0099945068359375)
    assert q.tolist() == [[127, -64, 0, 1]]     # -63.511 -> -64, 0.50038 -> 1
    # all-zero group: s = fp16(1e-8/127) = 0, q = 0 (numpy's NaN -> int8 on x86)
    q0, s0 = ref.quantize_weights(np.zeros((2, 8), np.float16), 4)
    assert np.all(q0 == 0) and np.all(s0 == 0)


@pytest.mark.parametrize("K,g", [(512, 64), (256, 256), (100, 64), (100, 48), (64, 1000)])
def test_weight_quant_invariants(K, g):
    rng = np.random.default_rng(K + g)
    w = (rng.standard_normal((37, K)) * 0.02).astype(np.float16)
    w[3, :] = 0
    q, s = ref.quantize_weights(w, g)
    gg = min(g, K) if g <= K else g
    G = (K + g - 1) // g
    assert s.shape == (37, G)
    wf = w.astype(np.float32)
    for gi in range(G):
        k0, k1 = gi * g, min(gi * g + g, K)
        amax = np.abs(wf[:, k0:k1]).max(axis=1)
        sg = s[:, gi].astype(np.float64)
        nz = amax > 1e-8
        # s is amax/127 rounded to fp16: within half an fp16 ulp
        assert np.all(np.abs(sg[nz] - amax[nz] / 127.0) <= 0.5 * fp16_ulp(amax[nz] / 127.0) + 1e-12)
        qa = np.abs(q[:, k0:k1].astype(np.int32)).max(axis=1)
        assert np.all(qa[nz] == 127)
        err = np.abs(wf[nz, k0:k1] - q[nz, k0:k1] * sg[nz, None])
        assert np.all(err <= 0.5 * sg[nz, None] * (1 + 1e-6) + 1e-12)
    assert np.all(q[3] == 0)
    del gg


# ------------------------------------------------------ activation quant ----

def test_act_quant_known_answers():
    K = 8
    x = np.zeros((3, K), np.float16)
    x[1, 5] = 5.0                                      # one-hot group
    x[2, :] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5]   # s = 1 exactly: ties to even
    q, s = ref.quantize_activations(x, 8)
    assert s[0, 0] == np.float32(1e-8) and np.all(q[0] == 0)
    assert s[1, 0] == np.float32(5.0) / np.float32(127.0)
    assert q[1].tolist() == [0, 0, 0, 0, 0, 127, 0, 0]
    assert s[2, 0] == 1.0
    assert q[2].tolist() == [127, 2, 4, -2, -4, 0, 2, 0]


def test_act_quant_static_and_smooth():
    K, g = 16, 8
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, K)).astype(np.float16)
    # static scale 0.5 -> q = clamp(rint(2 v)); a zero static scale clamps to 1e-8
    act = np.array([0.5, 0.0], np.float16)
    q, s = ref.quantize_activations(x, g, act_scale=act)
    assert np.all(s[:, 0] == 0.5) and np.all(s[:, 1] == np.float32(1e-8))
    want0 = np.clip(np.rint(x[:, :8].astype(np.float32) * 2.0), -127, 127)
    assert np.array_equal(q[:, :8], want0.astype(np.int8))
    assert np.all(np.abs(q[:, 8:]) == np.where(x[:, 8:] == 0, 0, 127))
    # smooth_inv by powers of two is exact: same as quantizing x * smooth
    sm = (2.0 ** rng.integers(-2, 3, K)).astype(np.float16)
    q1, s1 = ref.quantize_activations(x, g, smooth_inv=sm)
    q2, s2 = ref.quantize_activations((x.astype(np.float32) * sm).astype(np.float16), g)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


@pytest.mark.parametrize("K,g", [(512, 64), (2560, 256), (100, 48), (96, 0), (96, 500)])
def test_act_quant_invariants(K, g):
    rng = np.random.default_rng(K)
    x = rng.standard_normal((5, K)).astype(np.float32)
    x[:, ::37] *= 20
    x = x.astype(np.float16)
    q, s = ref.quantize_activations(x, g)
    ge = K if g <= 0 or g > K else g
    G = (K + ge - 1) // ge
    assert s.shape == (5, G)
    xf = x.astype(np.float32)
    for gi in range(G):
        k0, k1 = gi * ge, min(gi * ge + ge, K)
        amax = np.abs(xf[:, k0:k1]).max(axis=1)
        assert np.array_equal(s[:, gi], np.maximum(amax / np.float32(127), np.float32(1e-8)))
        assert np.all(np.abs(q[:, k0:k1].astype(int)).max(axis=1) == 127)
        err = np.abs(xf[:, k0:k1] - q[:, k0:k1] * s[:, gi:gi + 1].astype(np.float64))
        assert np.all(err <= 0.5 * s[:, gi:gi + 1] * (1 + 1e-5))


# ------------------------------------------------------- int32 partials ----

@pytest.mark.parametrize("M,N,K,g", [(16, 3, 512, 64), (5, 2, 100, 48), (7, 1, 256, 256)])
def test_partials_brute_force(M, N, K, g):
    rng = np.random.default_rng(M * N)
    W = rng.integers(-127, 128, (M, K), dtype=np.int8)
    X = rng.integers(-127, 128, (N, K), dtype=np.int8)
    P = ref.group_partials(W, X, g)
    G = (K + g - 1) // g
    for gi in range(G):
        k0, k1 = gi * g, min(gi * g + g, K)
        want = X[:, k0:k1].astype(np.int64) @ W[:, k0:k1].astype(np.int64).T
        assert np.array_equal(P[:, :, gi], want)


def test_partials_closed_forms():
    W = np.ones((4, 256), np.int8)
    X = np.ones((2, 256), np.int8)
    assert np.all(ref.group_partials(W, X, 64) == 64)
    Wm = np.full((1, 256), 127, np.int8)
    Xm = np.full((1, 256), -127, np.int8)
    assert np.all(ref.group_partials(Wm, Xm, 256) == -256 * 127 * 127)


# -------------------------------------------------------------- epilogue ----

def _float64_gemm(W, ws, xq, xs, g):
    M, K = W.shape
    G = xs.shape[1]
    acc = np.zeros((xq.shape[0], M))
    for gi in range(G):
        k0, k1 = gi * g, min(gi * g + g, K)
        P = xq[:, k0:k1].astype(np.int64) @ W[:, k0:k1].astype(np.int64).T
        wsg = (ws if ws.ndim == 1 else ws[:, gi]).astype(np.float64)
        acc += P * wsg[None, :] * xs[:, gi:gi + 1].astype(np.float64)
    return acc


@pytest.mark.parametrize("M,N,K,g", [(512, 16, 512, 64), (96, 3, 2560, 256), (33, 5, 100, 48),
                                     (40, 2, 128, 0)])
def test_gemm_against_float64(M, N, K, g):
    from fish_amd import synth
    w = synth.weights_f16(M, K, seed=M)
    x = synth.activations_f16(N, K, seed=N)
    ge = K if g <= 0 or g > K else g
    q, s = ref.quantize_weights(w, ge)
    if s.shape[1] == 1:
        s = s[:, 0]                                  # 1-D scale when G == 1
    xq, xs = ref.quantize_activations(x, g)
    Y = ref.gemm_quantized(q, s, g, xq, xs)
    exact = _float64_gemm(q, s, xq, xs, ge)
    assert_fp16_close(Y, exact.astype(np.float16), "oracle vs float64", max_ulp=1)
    # whole entry point == quantizer + dequant GEMM
    assert np.array_equal(ref.w8a8_gemm(q, s, g, x).view(np.uint16), Y.view(np.uint16))


def test_gemm_detects_scale_swap():
    """A swapped (row, group) scale index must be caught by the float64 check."""
    from fish_amd import synth
    M, N, K, g = 64, 4, 512, 64
    q, s = ref.quantize_weights(synth.weights_f16(M, K, seed=1), g)
    xq, xs = ref.quantize_activations(synth.activations_f16(N, K, seed=2), g)
    exact = _float64_gemm(q, s, xq, xs, g)
    wrong = ref.gemm_quantized(q, s[:, ::-1].copy(), g, xq, xs)
    with pytest.raises(AssertionError):
        assert_fp16_close(wrong, exact.astype(np.float16), "swapped")


@pytest.mark.parametrize("splits", [3, 6, 8])
def test_split_chain_tolerance(splits):
    """ref.split_chain_tolerance bounds a K-split group chain: per-split fp32
    chains (emulated here one rounding per fma in float64 -> float32, over
    consecutive whole groups), added in split order and rounded to fp16,
    stay within it of the oracle's single chain; outputs that drop a group
    or use a neighbouring group's scale fail it."""
    from fish_amd import synth
    M, N, K, g = 96, 12, 4096, 256
    G = K // g
    q, s = ref.quantize_weights(synth.weights_f16(M, K, seed=5), g)
    xq, xs = ref.quantize_activations(synth.activations_f16(N, K, seed=6), g)
    Y = ref.gemm_quantized(q, s, g, xq, xs)
    P = ref.group_partials(q, xq, g).astype(np.float64)            # [N, M, G]
    ws = s.astype(np.float32)

    def chain(gs, ge, scale=ws):
        acc = np.zeros((N, M), np.float32)
        for gi in range(gs, ge):
            t = (P[:, :, gi].astype(np.float32) * scale[None, :, gi]).astype(np.float32)
            acc = (t.astype(np.float64) * xs[:, None, gi] + acc).astype(np.float32)
        return acc

    bounds = [(G * i) // splits for i in range(splits + 1)]
    tot = np.zeros((N, M), np.float32)
    for i in range(splits):
        tot = (tot + chain(bounds[i], bounds[i + 1])).astype(np.float32)
    Ys = tot.astype(np.float16)
    bound = ref.split_chain_tolerance(q, s, g, xq, xs, Y)
    err = np.abs(Ys.astype(np.float64) - Y.astype(np.float64))
    assert np.all(err <= bound)
    assert bound.max() < 0.05 * np.abs(Y.astype(np.float64)).max()
    # north_star's own bound (1 fp16 ulp or rtol 1e-3) holds here too, and
    # catches what the reassociation bound lets through: a 2-ulp error on
    # the output nearest zero
    ns = ref.north_star_tolerance(Y)
    assert np.all(err <= ns)
    i = np.unravel_index(np.argmin(np.abs(Y.astype(np.float64)) + (Y == 0)), Y.shape)
    off = Y.copy()
    off[i] = np.nextafter(np.nextafter(Y[i], np.float16(np.inf)), np.float16(np.inf))
    e2 = np.abs(off.astype(np.float64) - Y.astype(np.float64))
    assert e2[i] > ns[i]
    # plausible mistakes exceed it
    dropped = chain(0, G - 1).astype(np.float16)
    assert np.mean(np.abs(dropped.astype(np.float64) - Y) > bound) > 0.5
    shifted = chain(0, G, np.roll(ws, 1, axis=1)).astype(np.float16)
    assert np.mean(np.abs(shifted.astype(np.float64) - Y) > bound) > 0.5


# --------------------------------------------------------------- RMSNorm ----

def test_rms_norm_reference_closed_forms():
    # tests/test_kernels.cu:121-152 -- x = w = 1 -> 1
    out = ref.rms_norm(np.ones((4, 8), np.float16), np.ones(8, np.float16), 1e-6)
    assert np.all(np.abs(out.astype(np.float32) - 1.0) <= 1e-3)
    # :154-180 -- zero input -> finite
    out = ref.rms_norm(np.zeros((2, 4), np.float16), np.ones(4, np.float16), 1e-5)
    assert np.all(np.isfinite(out.astype(np.float32)))
    # :181-210 -- [1,3,1,3], w = 2 -> 2 x / sqrt(5 + eps)
    x = np.array([[1, 3, 1, 3]], np.float16)
    out = ref.rms_norm(x, np.full(4, 2, np.float16), 1e-6)
    want = 2 * x.astype(np.float64) / np.sqrt(5 + 1e-6)
    assert np.all(np.abs(out.astype(np.float64) - want) <= 1e-2)
    assert np.array_equal(out, want.astype(np.float16))
    # :212-247 -- output rms ~ 1 with unit weights
    rng = np.random.default_rng(42)
    x = rng.standard_normal((3, 16)).astype(np.float16)
    out = ref.rms_norm(x, np.ones(16, np.float16), 1e-6).astype(np.float64)
    assert np.all(np.abs(np.sqrt((out ** 2).mean(axis=1)) - 1) <= 1e-3)


@pytest.mark.parametrize("dim", [4, 100, 1000, 2560, 4096, 9728])
def test_rms_norm_against_float64(dim):
    from fish_amd import synth
    x = synth.activations_f16(4, dim, seed=dim)
    w = synth.gamma_f16(dim)
    out = ref.rms_norm(x, w, 1e-6)
    xf = x.astype(np.float64)
    r = 1 / np.sqrt((xf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    want = (xf * r * w.astype(np.float64)).astype(np.float16)
    assert_fp16_close(out, want, "rms_norm", max_ulp=1, rtol=0)
    # fused variant == rms_norm then quantizer
    xq, xs, h = ref.rms_norm_quant(x, w, 1e-6, 64)
    assert np.array_equal(h.view(np.uint16), out.view(np.uint16))
    xq2, xs2 = ref.quantize_activations(out, 64)
    assert np.array_equal(xq, xq2) and np.array_equal(xs, xs2)


# ------------------------------------------------------------ elementwise ----

def test_silu_mul_residual_closed_forms():
    # tests/test_kernels.cu:355-379: silu(-8..7) vs x*sigmoid(x), tol 1e-2
    x = np.arange(-8, 8).astype(np.float16)
    out = ref.silu(x).astype(np.float64)
    xf = x.astype(np.float64)
    want = xf / (1 + np.exp(-xf))
    assert np.all(np.abs(out - want) <= 1e-2)
    assert np.array_equal(ref.silu(x), want.astype(np.float16))
    # :432-455 mul, :457-481 residual
    a = np.arange(1, 9).astype(np.float16)
    b = np.array([2, 3, 4, 5, 1, 1, 1, 1], np.float16)
    assert ref.mul(a, b).tolist() == [2, 6, 12, 20, 5, 6, 7, 8]
    b2 = np.array([10, 20, 30, 40, 0, -1, -2, -3], np.float16)
    assert ref.residual_add(a, b2).tolist() == [11, 22, 33, 44, 5, 5, 5, 5]


def test_silu_against_float64():
    rng = np.random.default_rng(123)
    x = (rng.standard_normal(100000) * 4).astype(np.float16)
    xf = x.astype(np.float64)
    want = (xf / (1 + np.exp(-xf))).astype(np.float16)
    assert_fp16_close(ref.silu(x), want, "silu", max_ulp=1, rtol=0)
    gate = x.reshape(10, -1)
    up = (rng.standard_normal(gate.shape)).astype(np.float16)
    xq, xs, h = ref.silu_mul_quant(gate, up, 256)
    assert np.array_equal(h, ref.mul(ref.silu(gate), up))
    xq2, xs2 = ref.quantize_activations(h, 256)
    assert np.array_equal(xq, xq2) and np.array_equal(xs, xs2)


def test_group_helpers():
    # int8_gemm.cu:396-397 and dual_ar_engine.cc:17-24
    assert ref.eff_group(512, 0) == 512 and ref.eff_group(512, 1000) == 512
    assert ref.groups(512, 64) == 8 and ref.groups(100, 48) == 3
    l = ref.lib()
    assert l.orc_infer_group_size(2560, 1, 1) == 2560
    assert l.orc_infer_group_size(2560, 2, 1) == 2560
    assert l.orc_infer_group_size(2560, 2, 10) == 256
    assert l.orc_infer_group_size(100, 2, 3) == 34


# ----------------------------------------------------------- fp16 linear ----

def test_gemm_fp16_exact_rational():
    """The double-precision fp16 linear equals the exact rational sum (Python
    fractions over the fp16 values) on small random inputs, and one-hot rows
    select single products exactly."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((5, 37)) * 0.3).astype(np.float16)
    X = (rng.standard_normal((3, 37)) * 2).astype(np.float16)
    Y, A = ref.gemm_fp16_exact(W, X)
    for n in range(3):
        for m in range(5):
            s = sum(Fraction(float(W[m, k])) * Fraction(float(X[n, k])) for k in range(37))
            a = sum(abs(Fraction(float(W[m, k])) * Fraction(float(X[n, k]))) for k in range(37))
            assert Y[n, m] == float(s) and A[n, m] == float(a)
    # one-hot weight rows: row m picks X[:, m] (times 1) exactly
    W1 = np.zeros((4, 8), np.float16)
    for m in range(4):
        W1[m, 2 * m] = 1.0
    Y1, _ = ref.gemm_fp16_exact(W1, X[:, :8])
    assert np.array_equal(Y1, X[:, [0, 2, 4, 6]].astype(np.float64))
    # a transposed operand or a swapped output index fails
    assert not np.allclose(ref.gemm_fp16_exact(W, X)[0], ref.gemm_fp16_exact(W, X)[0][:, ::-1])


# ------------------------------------------------------- prefill attention ---

def _qkv(rng, T, n_q, n_kv, D, scale=1.0):
    return (rng.standard_normal((T, (n_q + 2 * n_kv) * D)) * scale).astype(np.float16)


def test_qkv_split_and_merge_index_algebra():
    rng = np.random.default_rng(11)
    n_q, n_kv, T, D = 6, 2, 19, 32
    qkv = _qkv(rng, T, n_q, n_kv, D)
    q, k, v = ref.qkv_split_gqa(qkv, n_q, n_kv, D)
    heads = qkv.reshape(T, n_q + 2 * n_kv, D).transpose(1, 0, 2)
    assert np.array_equal(q, heads[:n_q])
    assert np.array_equal(k, heads[n_q:n_q + n_kv])
    assert np.array_equal(v, heads[n_q + n_kv:])
    # merge_heads inverts the q split; swapping T and H in merge would fail this
    assert np.array_equal(ref.merge_heads(q), qkv[:, :n_q * D])


def _attention_f64(q, k, v, sm_scale, window):
    n_q, T, D = q.shape
    rep = n_q // k.shape[0]
    kk = np.repeat(k, rep, 0).astype(np.float64)
    vv = np.repeat(v, rep, 0).astype(np.float64)
    S = np.einsum("htd,hsd->hts", q.astype(np.float64), kk) * sm_scale
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    mask = j <= i
    if window > 0:
        mask &= j >= i - window + 1
    S = np.where(mask, S, -np.inf)
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    return P @ vv


def test_attention_closed_forms():
    rng = np.random.default_rng(12)
    n_q, n_kv, T, D = 4, 2, 23, 64
    q, k, v = ref.qkv_split_gqa(_qkv(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    rep = n_q // n_kv
    vq = np.repeat(v, rep, 0)
    # T = 1: the only key is row 0, P = 1 exactly
    o1, _ = ref.prefill_attention(q[:, :1], k[:, :1], v[:, :1], 0.125)
    assert np.array_equal(o1, vq[:, :1])
    # window 1: every query sees only itself
    ow, _ = ref.prefill_attention(q, k, v, 0.125, window=1)
    assert np.array_equal(ow, vq)
    # Q = 0: uniform weights over the causal prefix (window 4: the last 4)
    z = np.zeros_like(q)
    for win in (0, 4):
        oz, _ = ref.prefill_attention(z, k, v, 0.125, window=win)
        want = np.empty(oz.shape)
        for i in range(T):
            lo = max(0, i - win + 1) if win else 0
            want[:, i] = vq[:, lo:i + 1].astype(np.float64).mean(1)
        # P = half(1/n) carries up to 2^-11 relative error per weight
        assert np.all(np.abs(oz - want) <= 2 * fp16_ulp(want) + 1e-3 * np.abs(vq).max())


@pytest.mark.parametrize("n_q,n_kv,T,D,win", [(4, 2, 37, 64, 0), (8, 2, 64, 128, 0),
                                               (4, 4, 50, 64, 7), (2, 1, 130, 32, 0)])
def test_attention_against_float64(n_q, n_kv, T, D, win):
    rng = np.random.default_rng(13 + T)
    q, k, v = ref.qkv_split_gqa(_qkv(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    s = 1.0 / np.sqrt(D)
    o, aw = ref.prefill_attention(q, k, v, s, window=win)
    want = _attention_f64(q, k, v, s, win)
    assert np.all(np.abs(o - want) <= ref.attention_tolerance(want, aw))


def test_attention_tolerance_rejects_plausible_mistakes():
    rng = np.random.default_rng(14)
    n_q, n_kv, T, D = 4, 2, 40, 64
    q, k, v = ref.qkv_split_gqa(_qkv(rng, T, n_q, n_kv, D, 2.0), n_q, n_kv, D)
    s = 1.0 / np.sqrt(D)
    want = _attention_f64(q, k, v, s, 0)
    _, aw = ref.prefill_attention(q, k, v, s)
    tol = ref.attention_tolerance(want, aw)
    # K and V swapped, a non-causal mask, a wrong kv head mapping, no scale
    nc = np.einsum("htd,hsd->hts", q.astype(np.float64), np.repeat(k, 2, 0).astype(np.float64)) * s
    P = np.exp(nc - nc.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    bad = [ref.prefill_attention(q, v, k, s)[0],
           (P @ np.repeat(v, 2, 0).astype(np.float64)).astype(np.float16),
           ref.prefill_attention(q, k[::-1].copy(), v[::-1].copy(), s)[0],
           ref.prefill_attention(q, k, v, 1.0)[0]]
    for b in bad:
        assert np.any(np.abs(b - want) > tol)

"""GPU: the prefill attention side (fused QKV split, head merge, fused causal
GQA attention) against the oracle.

The split and merge are copies: bit-exact.  Attention is floating point; the
kernel sums in a different order than the reference (matrix-core tiles, and
weights normalised after the V product, not before), so outputs are compared
with the oracle within

    |o - o_ref| <= 2 ulp_fp16(o_ref) + 1e-3 |o_ref| + 4e-3 sum_j P_ij |V_jd|

(oracle.ref.attention_tolerance; the oracle itself is pinned against float64
attention with the same bound).  The reference's own test
(tests/test_kernels.cu:53-118) checks its kernel against a float reference with
|err| <= 2e-3 on sin / cos inputs; that case is repeated here with its bound."""
import numpy as np
import pytest
import torch

from oracle import ref
from fish_amd import _lib, ops

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


def qkv_rand(rng, T, n_q, n_kv, D, scale=1.0):
    return (rng.standard_normal((T, (n_q + 2 * n_kv) * D)) * scale).astype(np.float16)


@pytest.mark.parametrize("T,n_q,n_kv,D", [(1, 4, 2, 64), (37, 32, 8, 128), (129, 8, 8, 64),
                                          (5, 3, 1, 12)])
def test_qkv_split_and_merge_bit_exact(T, n_q, n_kv, D):
    print("qkv split/merge T=%d n_q=%d n_kv=%d D=%d" % (T, n_q, n_kv, D), flush=True)
    rng = np.random.default_rng(T + D)
    qkv = qkv_rand(rng, T, n_q, n_kv, D)
    q, k, v = ops.qkv_split_heads_gqa(dev(qkv), n_q, n_kv, D)
    rq, rk, rv = ref.qkv_split_gqa(qkv, n_q, n_kv, D)
    for got, want in ((q, rq), (k, rk), (v, rv)):
        assert np.array_equal(host(got).view(np.uint16), want.view(np.uint16))
    m = ops.merge_heads(q)
    assert np.array_equal(host(m).view(np.uint16), ref.merge_heads(rq).view(np.uint16))


def test_qkv_split_heads_mha_entry():
    rng = np.random.default_rng(3)
    T, H, D = 9, 4, 64
    qkv = dev(qkv_rand(rng, T, H, H, D))
    q = torch.empty((H, T, D), dtype=torch.float16, device="cuda")
    k, v = torch.empty_like(q), torch.empty_like(q)
    _lib.check(_lib.lib().fa_qkv_split_heads(qkv.data_ptr(), q.data_ptr(), k.data_ptr(),
                                             v.data_ptr(), T, H, D, None))
    rq, rk, rv = ref.qkv_split_gqa(host(qkv), H, H, D)
    assert np.array_equal(host(q), rq) and np.array_equal(host(k), rk)
    assert np.array_equal(host(v), rv)


def check_attention(q, k, v, sm_scale, window, what):
    got = host(ops.prefill_attention(dev(q), dev(k), dev(v), sm_scale, window))
    want, aw = ref.prefill_attention(q, k, v, sm_scale, window)
    assert np.all(np.isfinite(got.astype(np.float64))), what
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = ref.attention_tolerance(want, aw)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError("%s: %d/%d outside tolerance; worst at %s: got %r want %r tol %r"
                             % (what, int(bad.sum()), bad.size, i, got[i], want[i], tol[i]))
    return float((err / tol).max())


CASES = [
    # T, n_q, n_kv, D, window, input scale
    (1, 4, 1, 64, 0, 1.0),
    (32, 4, 4, 64, 0, 1.0),
    (77, 32, 8, 128, 0, 1.0),       # the DualAR head layout, ragged T
    (200, 8, 8, 64, 0, 2.0),        # the DAC transformer layout (dac_config.h:12-16)
    (150, 8, 2, 128, 33, 1.0),      # sliding window
    (64, 6, 2, 32, 1, 1.0),         # window 1: each query sees itself; 3 heads per group
    (40, 2, 1, 40, 0, 1.0),         # D padded to 64
    (300, 4, 1, 128, 0, 3.0),       # large scores (sharp softmax)
    (70, 16, 2, 64, 0, 1.0),        # 8 heads per group: two workgroups per tile
    (45, 12, 2, 128, 0, 1.0),       # 6 heads per group: the second one half idle
    (1000, 8, 2, 128, 256, 1.0),    # long window, many fully visible blocks
    # grids large enough that a workgroup packs several query tiles:
    (1024, 32, 32, 64, 128, 1.0),   # DAC-style MHA, window 128: 1 head x 4 tiles
    (512, 64, 32, 64, 0, 1.0),      # 2 heads per group: 2 heads x 2 tiles
]


@pytest.mark.parametrize("T,n_q,n_kv,D,window,scale", CASES)
def test_prefill_attention_vs_oracle(T, n_q, n_kv, D, window, scale):
    what = "attention T=%d n_q=%d n_kv=%d D=%d window=%d scale=%g" % (T, n_q, n_kv, D, window,
                                                                      scale)
    print(what, flush=True)
    rng = np.random.default_rng(T * 7 + D)
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D, scale), n_q, n_kv, D)
    r = check_attention(q, k, v, 1.0 / np.sqrt(D), window, what)
    print("  max err / tol = %.3f" % r, flush=True)


def test_prefill_attention_reference_case():
    """tests/test_kernels.cu:53-118: H = 2, T = 4, D = 8, window 3, inputs
    sin(0.13 i) 0.7, cos(0.11 i) 0.6, sin(0.17 i) 0.5, |err| <= 2e-3 against
    float attention."""
    H, T, D, window = 2, 4, 8, 3
    i = np.arange(H * T * D, dtype=np.float32)
    q = (np.sin(i * np.float32(0.13)) * np.float32(0.7)).astype(np.float16).reshape(H, T, D)
    k = (np.cos(i * np.float32(0.11)) * np.float32(0.6)).astype(np.float16).reshape(H, T, D)
    v = (np.sin(i * np.float32(0.17)) * np.float32(0.5)).astype(np.float16).reshape(H, T, D)
    scale = np.float32(1.0 / np.sqrt(np.float32(D)))
    got = host(ops.prefill_attention(dev(q), dev(k), dev(v), scale, window)).astype(np.float64)
    S = np.einsum("htd,hsd->hts", q.astype(np.float64), k.astype(np.float64)) * float(scale)
    a = np.arange(T)
    mask = (a[None, :] <= a[:, None]) & (a[None, :] >= a[:, None] - window + 1)
    S = np.where(mask, S, -np.inf)
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    assert np.abs(got - P @ v.astype(np.float64)).max() <= 2e-3
    check_attention(q, k, v, scale, window, "reference case")


def test_prefill_attention_dualar_2048():
    """The DualAR prefill shape at full length: n_q 32, n_kv 8, D 128, T 2048.
    The oracle runs on a sample of query rows (every head, 64 rows spread over
    the sequence, including the first and last); every output is checked
    finite and, through Q = 0 rows, against the uniform-average closed form."""
    T, n_q, n_kv, D = 2048, 32, 8, 128
    rng = np.random.default_rng(2048)
    qkv = qkv_rand(rng, T, n_q, n_kv, D)
    q, k, v = ops.qkv_split_heads_gqa(dev(qkv), n_q, n_kv, D)
    q[:, 5, :] = 0       # closed form rows
    q[:, T - 1, :] = 0
    out = host(ops.prefill_attention(q, k, v, 1.0 / np.sqrt(D)))
    assert np.all(np.isfinite(out.astype(np.float32)))
    hq, hk, hv = host(q), host(k), host(v)
    rows = np.unique(np.concatenate([[0, 5, 31, 32, T - 1], rng.integers(0, T, 59)]))
    for h in range(0, n_q, 5):
        g = h // (n_q // n_kv)
        for i in rows:
            # oracle on the causal prefix of row i only (rows are independent)
            qi = hq[h:h + 1, i:i + 1]
            kk, vv = hk[g:g + 1, :i + 1], hv[g:g + 1, :i + 1]
            qpad = np.zeros((1, i + 1, D), np.float16)
            qpad[0, i] = qi[0, 0]
            want, aw = ref.prefill_attention(qpad, kk, vv, 1.0 / np.sqrt(D))
            tol = ref.attention_tolerance(want[0, i], aw[0, i])
            err = np.abs(out[h, i].astype(np.float64) - want[0, i].astype(np.float64))
            assert np.all(err <= tol), (h, i, err.max())
    for i in (5, T - 1):
        mean = hv[:, :i + 1].astype(np.float64).mean(1)           # [n_kv, D]
        got = out[:, i].astype(np.float64).reshape(n_kv, n_q // n_kv, D)
        assert np.all(np.abs(got - mean[:, None]) <= 2 * ref.attention_tolerance(
            mean[:, None], np.abs(hv[:, :i + 1]).astype(np.float64).mean(1)[:, None]))


def test_prefill_attention_stream_and_repeat():
    """Two runs on a side stream give identical bits (the kernel has no
    cross-workgroup state)."""
    rng = np.random.default_rng(9)
    T, n_q, n_kv, D = 96, 8, 2, 128
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    dq, dk, dvv = dev(q), dev(k), dev(v)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a = ops.prefill_attention(dq, dk, dvv, 0.088)
        b = ops.prefill_attention(dq, dk, dvv, 0.088)
    s.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("T,n_q,n_kv,D,window", [(77, 32, 8, 128, 0), (300, 8, 8, 64, 128),
                                                 (40, 6, 2, 40, 0)])
def test_prefill_attention_merged_equals_attention_then_merge(T, n_q, n_kv, D, window):
    """The fused token-major store gives exactly merge_heads(attention)."""
    rng = np.random.default_rng(T + 5)
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    dq, dk, dvv = dev(q), dev(k), dev(v)
    sep = ops.merge_heads(ops.prefill_attention(dq, dk, dvv, 1.0 / np.sqrt(D), window))
    fused = ops.prefill_attention_merged(dq, dk, dvv, 1.0 / np.sqrt(D), window)
    torch.cuda.synchronize()
    assert torch.equal(sep, fused)


@pytest.mark.parametrize("T,n_q,n_kv,D,window,sm", [
    (37, 4, 2, 12, 0, None),       # D % 8 != 0
    (60, 4, 1, 136, 0, None),      # D > 128
    (45, 2, 2, 256, 9, None),      # D 256, window
    (50, 4, 2, 64, 0, -0.125),     # negative scale (max taken after scaling)
    (33, 2, 1, 64, 0, 0.0),        # zero scale: uniform weights
])
def test_prefill_attention_any_shape(T, n_q, n_kv, D, window, sm):
    """Shapes outside the fused kernel (head dim not a multiple of 8 or above
    128, a non-positive scale) run the any-shape kernel, against the oracle
    within the same bound."""
    what = "generic T=%d n_q=%d n_kv=%d D=%d window=%d sm=%r" % (T, n_q, n_kv, D, window, sm)
    print(what, flush=True)
    rng = np.random.default_rng(T * 3 + D)
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    check_attention(q, k, v, 1.0 / np.sqrt(D) if sm is None else sm, window, what)


def test_prefill_attention_unaligned_buffers():
    """Buffers offset by one fp16 element (2-byte aligned only) take the
    any-shape kernel and give the same result within the bound."""
    rng = np.random.default_rng(77)
    T, n_q, n_kv, D = 40, 4, 2, 64
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D), n_q, n_kv, D)
    def off(a):
        t = torch.empty(a.size + 1, dtype=torch.float16, device="cuda")
        t[1:] = dev(a.reshape(-1))
        return t
    dq, dk, dvv, do = off(q), off(k), off(v), torch.zeros(q.size + 1, dtype=torch.float16,
                                                          device="cuda")
    l = _lib.lib()
    sc = 1.0 / np.sqrt(D)
    _lib.check(l.fa_prefill_attention(dq.data_ptr() + 2, dk.data_ptr() + 2, dvv.data_ptr() + 2,
                                      do.data_ptr() + 2, None, n_q, n_kv, T, D, sc, None, 0))
    got = host(do)[1:].reshape(n_q, T, D).astype(np.float64)
    want, aw = ref.prefill_attention(q, k, v, sc)
    assert np.all(np.abs(got - want) <= ref.attention_tolerance(want, aw))


def _attn_sweep(n=10, seed=31):
    """Seeded random attention shapes: token counts, GQA ratios, head dims
    of the fused kernel and of the any-shape one, windows, input scales."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        n_kv = int(rng.choice([1, 2, 4]))
        n_q = n_kv * int(rng.choice([1, 2, 3, 4, 8]))
        D = int(rng.choice([32, 64, 128, 40, 96, 24, 160]))
        T = int(rng.integers(1, 400))
        window = int(rng.choice([0, 0, int(rng.integers(1, 300))]))
        scale = float(rng.choice([0.5, 1.0, 2.0]))
        out.append((T, n_q, n_kv, D, window, scale))
    return out


@pytest.mark.parametrize("T,n_q,n_kv,D,window,scale", _attn_sweep())
def test_prefill_attention_random_shapes(T, n_q, n_kv, D, window, scale):
    what = "attn sweep T=%d n_q=%d n_kv=%d D=%d window=%d scale=%g" % (T, n_q, n_kv, D, window,
                                                                       scale)
    print(what, flush=True)
    rng = np.random.default_rng(T * 13 + D)
    q, k, v = ref.qkv_split_gqa(qkv_rand(rng, T, n_q, n_kv, D, scale), n_q, n_kv, D)
    check_attention(q, k, v, 1.0 / np.sqrt(D), window, what)

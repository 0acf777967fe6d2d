"""numpy front end of the C oracle (oracle/w8a8_ref.c).  TEST INFRASTRUCTURE.

fp16 arrays are passed as numpy float16 (bit patterns are identical to the
uint16 the C code takes).  Index names follow the reference API: M = output
rows, N = tokens, K = input features; Y is returned as [N, M].
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle_w8a8.so")
LIB_V4_PATH = os.path.join(HERE, "_build", "liboracle_w8a8_v4.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_SIGS = {
    "orc_h2f": (_f, [ctypes.c_uint16]),
    "orc_f2h": (ctypes.c_uint16, [_f]),
    "orc_h2f_array": (None, [_p, _p, _i64]),
    "orc_f2h_array": (None, [_p, _p, _i64]),
    "orc_effective_group": (_i, [_i, _i]),
    "orc_num_groups": (_i, [_i, _i]),
    "orc_infer_group_size": (_i, [_i64, _i, _i64]),
    "orc_quantize_weights_groupwise": (None, [_p, _i64, _i64, _i, _p, _p]),
    "orc_quantize_activations": (None, [_p, _p, _p, _i, _i, _i, _p, _p]),
    "orc_group_partials": (None, [_p, _p, _i, _i, _i, _i, _p]),
    "orc_gemm_quantized": (None, [_p, _p, _i, _p, _p, _p, _i, _i, _i]),
    "orc_w8a8_gemm": (None, [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i]),
    "orc_rms_inv": (_f, [_f, _i, _f]),
    "orc_rms_norm": (None, [_p, _p, _p, _i, _i, _f]),
    "orc_rms_norm_quant": (None, [_p, _p, _f, _p, _p, _i, _p, _p, _p, _i, _i]),
    "orc_silu": (None, [_p, _i64]),
    "orc_mul": (None, [_p, _p, _i64]),
    "orc_residual_add": (None, [_p, _p, _i64]),
    "orc_silu_mul_quant": (None, [_p, _p, _p, _p, _i, _p, _p, _p, _i, _i]),
    "orc_gemm_fp16_exact": (None, [_p, _p, _p, _p, _i, _i, _i]),
    "orc_qkv_split_gqa": (None, [_p, _p, _p, _p, _i, _i, _i, _i]),
    "orc_merge_heads": (None, [_p, _p, _i, _i, _i]),
    "orc_prefill_attention": (None, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _i]),
    "orc_num_threads": (_i, []),
    "orc_set_num_threads": (None, [_i]),
}
_LIB = None


def host_cpu():
    """(model name, has AVX-512 F/BW/CD/DQ/VL) of this host, from /proc/cpuinfo."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    v4 = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    return model, v4


def host_cpu_id():
    """'<model name> (family F, model M, stepping S), <logical CPUs> logical
    CPUs' from /proc/cpuinfo: enough to tell two hosts whose model names
    read the same apart."""
    info = {}
    n = 0
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if ":" not in line:
                    continue
                k, v = (t.strip() for t in line.split(":", 1))
                if k == "processor":
                    n += 1
                elif k in ("model name", "cpu family", "model", "stepping") and k not in info:
                    info[k] = v
    except OSError:
        pass
    return "%s (family %s, model %s, stepping %s), %d logical CPUs" % (
        info.get("model name", "unknown"), info.get("cpu family", "?"), info.get("model", "?"),
        info.get("stepping", "?"), n)


def use_baseline_build():
    """For the CPU-baseline timing only: load the x86-64-v4 build when this
    host has AVX-512 (call before any other oracle function).  Returns the
    -march level in use."""
    global _LIB
    if _LIB is not None:
        return getattr(_LIB, "_march", "x86-64-v3")
    if host_cpu()[1] and os.path.exists(LIB_V4_PATH):
        _load(LIB_V4_PATH, "x86-64-v4")
    else:
        lib()
    return _LIB._march


def lib():
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        _load(LIB_PATH, "x86-64-v3")
    return _LIB


def _load(path, march):
    global _LIB
    l = ctypes.CDLL(path)
    l._march = march
    for k, (r, a) in _SIGS.items():
        fn = getattr(l, k)
        fn.restype = r
        fn.argtypes = a
    _LIB = l
    return _LIB


def _c(a, dtype):
    if a is None:
        return None
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


def _ptr(a):
    return None if a is None else a.ctypes.data


def groups(K, g):
    return lib().orc_num_groups(K, g)


def eff_group(K, g):
    return lib().orc_effective_group(K, g)


def f2h(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.float16)
    lib().orc_f2h_array(_ptr(x), _ptr(out), x.size)
    return out


def h2f(h):
    h = _c(h, np.float16)
    out = np.empty(h.shape, np.float32)
    lib().orc_h2f_array(_ptr(h), _ptr(out), h.size)
    return out


def quantize_weights(w, group_size):
    w = _c(w, np.float16)
    rows, K = w.shape
    G = (K + group_size - 1) // group_size
    q = np.empty((rows, K), np.int8)
    s = np.empty((rows, G), np.float16)
    lib().orc_quantize_weights_groupwise(_ptr(w), rows, K, group_size, _ptr(q), _ptr(s))
    return q, s


def quantize_activations(X, group_size, act_scale=None, smooth_inv=None):
    X = _c(X, np.float16)
    N, K = X.shape
    G = groups(K, group_size)
    xq = np.empty((N, K), np.int8)
    xs = np.empty((N, G), np.float32)
    act_scale = _c(act_scale, np.float16)
    smooth_inv = _c(smooth_inv, np.float16)
    lib().orc_quantize_activations(_ptr(X), _ptr(act_scale), _ptr(smooth_inv), N, K, group_size,
                                   _ptr(xq), _ptr(xs))
    return xq, xs


def group_partials(W, xq, group_size):
    W = _c(W, np.int8)
    xq = _c(xq, np.int8)
    M, K = W.shape
    N = xq.shape[0]
    G = groups(K, group_size)
    P = np.empty((N, M, G), np.int32)
    lib().orc_group_partials(_ptr(W), _ptr(xq), M, N, K, group_size, _ptr(P))
    return P


def gemm_quantized(W, w_scale, group_size, xq, xs):
    W = _c(W, np.int8)
    w_scale = _c(w_scale, np.float16)
    xq = _c(xq, np.int8)
    xs = _c(xs, np.float32)
    M, K = W.shape
    N = xq.shape[0]
    Y = np.empty((N, M), np.float16)
    lib().orc_gemm_quantized(_ptr(W), _ptr(w_scale), group_size, _ptr(xq), _ptr(xs), _ptr(Y), M, N, K)
    return Y


def split_chain_tolerance(W, w_scale, group_size, xq, xs, y_ref):
    """Bound on |y - y_ref| for a linear whose fp32 group chain was split into
    partial chains added afterwards (fa_w8a8_gemm_k_splits > 1): one fp16 ulp
    of y_ref plus 2^-20 * sum_g |float(P_g) * ws_g * xs_g| (fp32 reassociation
    of at most 8 partial sums; exact int32 partials).  Returns the bound,
    [N, M] float64."""
    W = _c(W, np.int8)
    P = group_partials(W, xq, group_size).astype(np.float64)        # [N, M, G]
    ws = np.asarray(w_scale, np.float16).astype(np.float64).reshape(W.shape[0], -1)
    t = P * ws[None, :, :] * np.asarray(xs, np.float64)[:, None, :]
    ulp = np.spacing(np.abs(np.asarray(y_ref, np.float16))).astype(np.float64)
    return ulp + 2.0 ** -20 * np.abs(t).sum(-1)


def north_star_tolerance(y_ref):
    """north_star's bound for fp16 outputs: one fp16 ulp of y_ref or 1e-3
    relative, whichever is larger.  Returns the bound, float64."""
    y = np.abs(np.asarray(y_ref, np.float16))
    return np.maximum(np.spacing(y).astype(np.float64), 1e-3 * y.astype(np.float64))


def w8a8_gemm(W, w_scale, group_size, X, act_scale=None, smooth_inv=None):
    W = _c(W, np.int8)
    w_scale = _c(w_scale, np.float16)
    X = _c(X, np.float16)
    act_scale = _c(act_scale, np.float16)
    smooth_inv = _c(smooth_inv, np.float16)
    M, K = W.shape
    N = X.shape[0]
    Y = np.empty((N, M), np.float16)
    lib().orc_w8a8_gemm(_ptr(W), _ptr(w_scale), group_size, _ptr(act_scale), _ptr(smooth_inv),
                        _ptr(X), _ptr(Y), M, N, K)
    return Y


def rms_norm(x, w, eps):
    x = _c(x, np.float16)
    w = _c(w, np.float16)
    n, d = x.shape
    out = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), _ptr(w), _ptr(out), n, d, eps)
    return out


def rms_norm_quant(x, w, eps, group_size, smooth_inv=None, act_scale=None):
    x = _c(x, np.float16)
    w = _c(w, np.float16)
    n, d = x.shape
    G = groups(d, group_size)
    xq = np.empty((n, d), np.int8)
    xs = np.empty((n, G), np.float32)
    out = np.empty_like(x)
    smooth_inv = _c(smooth_inv, np.float16)
    act_scale = _c(act_scale, np.float16)
    lib().orc_rms_norm_quant(_ptr(x), _ptr(w), eps, _ptr(smooth_inv), _ptr(act_scale), group_size,
                             _ptr(xq), _ptr(xs), _ptr(out), n, d)
    return xq, xs, out


def silu(x):
    x = np.array(x, dtype=np.float16, copy=True)
    lib().orc_silu(_ptr(x), x.size)
    return x


def mul(a, b):
    a = np.array(a, dtype=np.float16, copy=True)
    b = _c(b, np.float16)
    lib().orc_mul(_ptr(a), _ptr(b), a.size)
    return a


def residual_add(a, b):
    a = np.array(a, dtype=np.float16, copy=True)
    b = _c(b, np.float16)
    lib().orc_residual_add(_ptr(a), _ptr(b), a.size)
    return a


def silu_mul_quant(gate, up, group_size, smooth_inv=None, act_scale=None):
    gate = _c(gate, np.float16)
    up = _c(up, np.float16)
    n, d = gate.shape
    G = groups(d, group_size)
    xq = np.empty((n, d), np.int8)
    xs = np.empty((n, G), np.float32)
    out = np.empty_like(gate)
    smooth_inv = _c(smooth_inv, np.float16)
    act_scale = _c(act_scale, np.float16)
    lib().orc_silu_mul_quant(_ptr(gate), _ptr(up), _ptr(smooth_inv), _ptr(act_scale), group_size,
                             _ptr(xq), _ptr(xs), _ptr(out), n, d)
    return xq, xs, out


def gemm_fp16_exact(W, X):
    """(Y, sum |w x|) in float64, both [N, M], for fp16 W [M, K], X [N, K]."""
    W = _c(W, np.float16)
    X = _c(X, np.float16)
    M, K = W.shape
    N = X.shape[0]
    Y = np.empty((N, M), np.float64)
    A = np.empty((N, M), np.float64)
    lib().orc_gemm_fp16_exact(_ptr(W), _ptr(X), _ptr(Y), _ptr(A), M, N, K)
    return Y, A


def fp16_linear_tolerance(y_exact, abs_sum):
    """Allowed |y - y_exact| for an fp16 output of an fp32-accumulated sum:
    one fp16 ulp of the exact value (or 1e-3 relative), plus 2^-18 * sum |w x|
    for the fp32 accumulation: a lane chain of at most 4 * K / 512 + 4 fp32
    additions plus a 6-level tree, each rounding at most 2^-24 of a partial
    bounded by sum |w x| (fp16 products are exact in fp32)."""
    y16 = np.abs(y_exact).astype(np.float16)
    ulp = np.spacing(y16).astype(np.float64)
    return np.maximum(ulp, 1e-3 * np.abs(y_exact)) + abs_sum * 2.0 ** -18


def qkv_split_gqa(qkv, n_q, n_kv, D):
    """Token-major fused QKV [T, (n_q + 2 n_kv) D] -> q [n_q, T, D],
    k [n_kv, T, D], v [n_kv, T, D] (prefill_attention.cu:38-57)."""
    qkv = _c(qkv, np.float16)
    T = qkv.shape[0]
    q = np.empty((n_q, T, D), np.float16)
    k = np.empty((n_kv, T, D), np.float16)
    v = np.empty((n_kv, T, D), np.float16)
    lib().orc_qkv_split_gqa(_ptr(qkv), _ptr(q), _ptr(k), _ptr(v), T, n_q, n_kv, D)
    return q, k, v


def merge_heads(heads):
    """Head-major [H, T, D] -> token-major [T, H * D] (prefill_attention.cu:68-86)."""
    heads = _c(heads, np.float16)
    H, T, D = heads.shape
    out = np.empty((T, H * D), np.float16)
    lib().orc_merge_heads(_ptr(heads), _ptr(out), T, H, D)
    return out


def prefill_attention(q, k, v, sm_scale, window=0):
    """Causal GQA attention over head-major fp16 q [n_q, T, D], k / v
    [n_kv, T, D] (prefill_attention.cu:226-349).  Returns (out [n_q, T, D]
    fp16, sum_j P_ij |V_jd| float64) -- the second scales the tolerance."""
    q = _c(q, np.float16)
    k = _c(k, np.float16)
    v = _c(v, np.float16)
    n_q, T, D = q.shape
    n_kv = k.shape[0]
    assert k.shape == (n_kv, T, D) and v.shape == k.shape and n_q % n_kv == 0
    out = np.empty((n_q, T, D), np.float16)
    aw = np.empty((n_q, T, D), np.float64)
    lib().orc_prefill_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(aw), n_q, n_kv, T,
                                D, float(sm_scale), int(window))
    return out, aw


def attention_tolerance(o_ref, absw):
    """Allowed |o - o_ref| for a different (valid) evaluation order of the
    reference's attention: two fp16 ulps of the output (the reference rounds
    O once, a second evaluation may land one ulp away, plus one for the
    scores' and probabilities' own fp16 roundings reaching the output) and
    4e-3 of sum_j P_ij |V_jd| for the fp16 rounding of P (2^-11 relative,
    doubled for a one-ulp difference in a score feeding exp)."""
    o = np.abs(o_ref.astype(np.float64))
    ulp = np.spacing(np.abs(o_ref).astype(np.float16)).astype(np.float64)
    return 2.0 * ulp + 1e-3 * o + 4e-3 * absw


def rms_inv(sum_sq, dim, eps):
    return lib().orc_rms_inv(sum_sq, dim, eps)


def num_threads():
    return lib().orc_num_threads()


def set_num_threads(n):
    lib().orc_set_num_threads(n)

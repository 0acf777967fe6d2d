"""PyTorch-tensor front end of the C ABI.

torch supplies device memory and the current HIP stream; all arithmetic runs
in libfish_w8a8.so.  Shapes follow the reference kernel API
(src/kernels/kernels.h:242-259): W [M, K] int8, w_scale fp16 [M] or [M, G],
X [N, K] fp16, returned Y is [N, M] fp16 (= the reference's col-major [M, N]).
"""
import contextlib
import ctypes
import sys

import torch

from ._lib import ChainStep, FaError, check, lib


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _need(t, dtype, name):
    if t is None:
        return
    if not t.is_cuda:
        raise ValueError("%s must be a device tensor" % name)
    if t.dtype != dtype:
        raise ValueError("%s must be %s, got %s" % (name, dtype, t.dtype))
    if not t.is_contiguous():
        raise ValueError("%s must be contiguous" % name)


def num_groups(K, group_size):
    g = K if group_size <= 0 or group_size > K else group_size
    return (K + g - 1) // g


def w8a8_gemm(W, w_scale, X, group_size, act_scale=None, smooth_inv=None, out=None):
    """int8_dequant_gemm_fp16: Y[n, m] for X fp16 [N, K] and W int8 [M, K]."""
    _need(W, torch.int8, "W"); _need(w_scale, torch.float16, "w_scale"); _need(X, torch.float16, "X")
    _need(act_scale, torch.float16, "act_scale"); _need(smooth_inv, torch.float16, "smooth_inv")
    M, K = W.shape
    N = X.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=X.device)
    check(lib().fa_w8a8_gemm(_ptr(W), _ptr(w_scale), group_size, _ptr(act_scale), _ptr(smooth_inv),
                             _ptr(X), _ptr(Y), M, N, K, _stream()))
    return Y


def k_splits(M, N, K, group_size):
    """fa_w8a8_gemm_k_splits: 1 when the linear keeps the reference's single
    group-ordered fp32 chain (bit-exact; always, unless set_k_split opted in),
    else the number of K splits."""
    return lib().fa_w8a8_gemm_k_splits(M, N, K, group_size)


def set_k_split(max_splits):
    """fa_w8a8_set_k_split: opt in to (>= 3) or out of (<= 1) the K split of
    few-tile prefill grids; returns the previous setting."""
    return lib().fa_w8a8_set_k_split(max_splits)


@contextlib.contextmanager
def k_split(max_splits):
    """The K split opted in for the duration of a with-block."""
    prev = set_k_split(max_splits)
    try:
        yield
    finally:
        set_k_split(prev)


def w8a8_gemm_noalloc(W, w_scale, X, group_size, act_scale=None, smooth_inv=None, out=None):
    """fa_w8a8_gemm_noalloc: w8a8_gemm with its scratch in the library's
    static per-device array (no device allocation inside the call)."""
    _need(W, torch.int8, "W"); _need(w_scale, torch.float16, "w_scale"); _need(X, torch.float16, "X")
    _need(act_scale, torch.float16, "act_scale"); _need(smooth_inv, torch.float16, "smooth_inv")
    M, K = W.shape
    N = X.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=X.device)
    check(lib().fa_w8a8_gemm_noalloc(_ptr(W), _ptr(w_scale), group_size, _ptr(act_scale),
                                     _ptr(smooth_inv), _ptr(X), _ptr(Y), M, N, K, _stream()))
    return Y


def w8a8_gemm_rms(W, w_scale, x, gamma, eps, group_size, resid=None, h_out=None,
                  act_scale=None, smooth_inv=None, out=None):
    """RMSNorm (after an optional residual add written to h_out) + linear."""
    _need(W, torch.int8, "W"); _need(w_scale, torch.float16, "w_scale"); _need(x, torch.float16, "x")
    _need(gamma, torch.float16, "gamma"); _need(resid, torch.float16, "resid")
    _need(h_out, torch.float16, "h_out")
    M, K = W.shape
    N = x.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=x.device)
    check(lib().fa_w8a8_gemm_rms(_ptr(W), _ptr(w_scale), group_size, _ptr(act_scale),
                                 _ptr(smooth_inv), _ptr(x), _ptr(resid), _ptr(h_out), _ptr(gamma),
                                 eps, _ptr(Y), M, N, K, _stream()))
    return Y


def gemm_fp16(W, X, out=None):
    """gemm_fp16: Y[n, m] = fp16(sum_k W[m, k] X[n, k]) with fp32 accumulation."""
    _need(W, torch.float16, "W"); _need(X, torch.float16, "X")
    M, K = W.shape
    N = X.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=X.device)
    check(lib().fa_gemm_fp16(_ptr(W), _ptr(X), _ptr(Y), M, N, K, _stream()))
    return Y


def w8a8_gemm_swiglu(W13, w13_scale, x, group_size, gamma=None, eps=1e-6, resid=None,
                     h_out=None, act_scale=None, smooth_inv=None, out=None):
    """act [N, F] = fp16(silu(x @ w1.T)) * (x @ w3.T) on row-interleaved W13."""
    _need(W13, torch.int8, "W13"); _need(w13_scale, torch.float16, "w13_scale")
    _need(x, torch.float16, "x"); _need(gamma, torch.float16, "gamma")
    _need(resid, torch.float16, "resid"); _need(h_out, torch.float16, "h_out")
    M, K = W13.shape
    F = M // 2
    N = x.shape[0]
    Y = out if out is not None else torch.empty((N, F), dtype=torch.float16, device=x.device)
    check(lib().fa_w8a8_gemm_swiglu(_ptr(W13), _ptr(w13_scale), group_size, _ptr(act_scale),
                                    _ptr(smooth_inv), _ptr(x), _ptr(resid), _ptr(h_out),
                                    _ptr(gamma), eps, _ptr(Y), F, N, K, _stream()))
    return Y


def w8a8_gemm_swiglu_sep(W1, w1_scale, W3, w3_scale, x, group_size, gamma=None, eps=1e-6,
                         resid=None, h_out=None, act_scale1=None, smooth_inv1=None,
                         act_scale3=None, smooth_inv3=None, out=None):
    """act [N, F] = fp16(silu(x @ w1.T)) * (x @ w3.T) on separate w1 / w3, each
    input quantized with its weight's own companions."""
    for t, n in ((W1, "W1"), (W3, "W3")):
        _need(t, torch.int8, n)
    for t, n in ((w1_scale, "w1_scale"), (w3_scale, "w3_scale"), (x, "x"), (gamma, "gamma"),
                 (resid, "resid"), (h_out, "h_out")):
        _need(t, torch.float16, n)
    F, K = W1.shape
    if tuple(W3.shape) != (F, K):
        raise ValueError("W1 %s and W3 %s differ" % (tuple(W1.shape), tuple(W3.shape)))
    N = x.shape[0]
    Y = out if out is not None else torch.empty((N, F), dtype=torch.float16, device=x.device)
    check(lib().fa_w8a8_gemm_swiglu_sep(_ptr(W1), _ptr(w1_scale), _ptr(W3), _ptr(w3_scale),
                                        group_size, _ptr(act_scale1), _ptr(smooth_inv1),
                                        _ptr(act_scale3), _ptr(smooth_inv3), _ptr(x), _ptr(resid),
                                        _ptr(h_out), _ptr(gamma), eps, _ptr(Y), F, N, K,
                                        _stream()))
    return Y


def interleave_rows(a, b):
    """Rows of a and b interleaved: row 2i = a[i], row 2i + 1 = b[i]."""
    return torch.stack((a, b), dim=1).reshape(2 * a.shape[0], *a.shape[1:]).contiguous()


def w8a8_gemm_silu_mul(W, w_scale, gate, up, group_size, act_scale=None, smooth_inv=None,
                       out=None):
    """SiLU(gate) * up + linear."""
    _need(W, torch.int8, "W"); _need(w_scale, torch.float16, "w_scale")
    _need(gate, torch.float16, "gate"); _need(up, torch.float16, "up")
    M, K = W.shape
    N = gate.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=gate.device)
    check(lib().fa_w8a8_gemm_silu_mul(_ptr(W), _ptr(w_scale), group_size, _ptr(act_scale),
                                      _ptr(smooth_inv), _ptr(gate), _ptr(up), _ptr(Y), M, N, K,
                                      _stream()))
    return Y


def w8a8_gemm_quantized(W, w_scale, group_size, X_q, X_scale, out=None):
    _need(W, torch.int8, "W"); _need(w_scale, torch.float16, "w_scale")
    _need(X_q, torch.int8, "X_q"); _need(X_scale, torch.float32, "X_scale")
    M, K = W.shape
    N = X_q.shape[0]
    Y = out if out is not None else torch.empty((N, M), dtype=torch.float16, device=X_q.device)
    check(lib().fa_w8a8_gemm_quantized(_ptr(W), _ptr(w_scale), group_size, _ptr(X_q), _ptr(X_scale),
                                       _ptr(Y), M, N, K, _stream()))
    return Y


def w8a8_gemm_partials(W, w_scale, group_size, X_q, X_scale, row0=0, rows=None, tok0=0, toks=None):
    """Y plus the exact int32 partials [toks, rows, G] of the window."""
    M, K = W.shape
    N = X_q.shape[0]
    rows = M - row0 if rows is None else rows
    toks = N - tok0 if toks is None else toks
    G = num_groups(K, group_size)
    Y = torch.empty((N, M), dtype=torch.float16, device=X_q.device)
    P = torch.full((toks, rows, G), -2**31, dtype=torch.int32, device=X_q.device)
    check(lib().fa_w8a8_gemm_partials(_ptr(W), _ptr(w_scale), group_size, _ptr(X_q), _ptr(X_scale),
                                      _ptr(Y), _ptr(P), row0, rows, tok0, toks, M, N, K, _stream()))
    return Y, P


def quantize_activations(X, group_size, act_scale=None, smooth_inv=None):
    _need(X, torch.float16, "X")
    N, K = X.shape
    G = num_groups(K, group_size)
    X_q = torch.empty((N, K), dtype=torch.int8, device=X.device)
    X_s = torch.empty((N, G), dtype=torch.float32, device=X.device)
    check(lib().fa_quantize_activations(_ptr(X), _ptr(act_scale), _ptr(smooth_inv), _ptr(X_q),
                                        _ptr(X_s), N, K, group_size, _stream()))
    return X_q, X_s


def rms_norm(x, weight, eps):
    _need(x, torch.float16, "x"); _need(weight, torch.float16, "weight")
    n, d = x.shape
    out = torch.empty_like(x)
    check(lib().fa_rms_norm(_ptr(x), _ptr(weight), _ptr(out), n, d, eps, _stream()))
    return out


def rms_norm_quant(x, weight, eps, group_size, smooth_inv=None, act_scale=None, want_out=False):
    _need(x, torch.float16, "x"); _need(weight, torch.float16, "weight")
    n, d = x.shape
    G = num_groups(d, group_size)
    X_q = torch.empty((n, d), dtype=torch.int8, device=x.device)
    X_s = torch.empty((n, G), dtype=torch.float32, device=x.device)
    out = torch.empty_like(x) if want_out else None
    check(lib().fa_rms_norm_quant(_ptr(x), _ptr(weight), eps, _ptr(smooth_inv), _ptr(act_scale),
                                  group_size, _ptr(X_q), _ptr(X_s), _ptr(out), n, d, _stream()))
    return (X_q, X_s, out) if want_out else (X_q, X_s)


def residual_rms_norm_quant_(h, resid, weight, eps, group_size, smooth_inv=None, act_scale=None,
                             want_out=False):
    """h <- fp16(h + resid) in place, then rms_norm_quant of the new h."""
    _need(h, torch.float16, "h"); _need(resid, torch.float16, "resid")
    _need(weight, torch.float16, "weight")
    n, d = h.shape
    G = num_groups(d, group_size)
    X_q = torch.empty((n, d), dtype=torch.int8, device=h.device)
    X_s = torch.empty((n, G), dtype=torch.float32, device=h.device)
    out = torch.empty_like(h) if want_out else None
    check(lib().fa_residual_rms_norm_quant(_ptr(h), _ptr(resid), _ptr(weight), eps,
                                           _ptr(smooth_inv), _ptr(act_scale), group_size,
                                           _ptr(X_q), _ptr(X_s), _ptr(out), n, d, _stream()))
    return (X_q, X_s, out) if want_out else (X_q, X_s)


def silu_(x):
    _need(x, torch.float16, "x")
    check(lib().fa_silu(_ptr(x), x.numel(), _stream()))
    return x


def mul_(a, b):
    _need(a, torch.float16, "a"); _need(b, torch.float16, "b")
    check(lib().fa_mul(_ptr(a), _ptr(b), a.numel(), _stream()))
    return a


def residual_add_(a, b):
    _need(a, torch.float16, "a"); _need(b, torch.float16, "b")
    check(lib().fa_residual_add(_ptr(a), _ptr(b), a.numel(), _stream()))
    return a


def silu_mul_quant(gate, up, group_size, smooth_inv=None, act_scale=None, want_out=False):
    _need(gate, torch.float16, "gate"); _need(up, torch.float16, "up")
    n, d = gate.shape
    G = num_groups(d, group_size)
    X_q = torch.empty((n, d), dtype=torch.int8, device=gate.device)
    X_s = torch.empty((n, G), dtype=torch.float32, device=gate.device)
    out = torch.empty_like(gate) if want_out else None
    check(lib().fa_silu_mul_quant(_ptr(gate), _ptr(up), _ptr(smooth_inv), _ptr(act_scale),
                                  group_size, _ptr(X_q), _ptr(X_s), _ptr(out), n, d, _stream()))
    return (X_q, X_s, out) if want_out else (X_q, X_s)


def quantize_weights_groupwise(w, group_size):
    """tools/quant_utils.py quantize_groupwise on the device -> (q int8, scale fp16 [rows, G])."""
    _need(w, torch.float16, "w")
    rows, K = w.shape
    G = (K + group_size - 1) // group_size
    q = torch.empty((rows, K), dtype=torch.int8, device=w.device)
    s = torch.empty((rows, G), dtype=torch.float16, device=w.device)
    check(lib().fa_quantize_weights_groupwise(_ptr(w), rows, K, group_size, _ptr(q), _ptr(s),
                                              _stream()))
    return q, s


def qkv_split_heads_gqa(qkv, n_q, n_kv, head_dim):
    """qkv fp16 [T, (n_q + 2 n_kv) head_dim] -> head-major (q, k, v)
    (prefill_attention.cu:38-66)."""
    _need(qkv, torch.float16, "qkv")
    T = qkv.shape[0]
    assert qkv.shape[1] == (n_q + 2 * n_kv) * head_dim
    q = torch.empty((n_q, T, head_dim), dtype=torch.float16, device=qkv.device)
    k = torch.empty((n_kv, T, head_dim), dtype=torch.float16, device=qkv.device)
    v = torch.empty_like(k)
    check(lib().fa_qkv_split_heads_gqa(_ptr(qkv), _ptr(q), _ptr(k), _ptr(v), T, n_q, n_kv,
                                       head_dim, _stream()))
    return q, k, v


def prefill_attention_merged(q, k, v, sm_scale, window=0, out=None):
    """prefill_attention then merge_heads in one launch -> out [T, n_q D]."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, torch.float16, n)
    n_q, T, D = q.shape
    n_kv = k.shape[0]
    if out is None:
        out = torch.empty((T, n_q * D), dtype=torch.float16, device=q.device)
    check(lib().fa_prefill_attention_merged(_ptr(q), _ptr(k), _ptr(v), _ptr(out), n_q, n_kv, T, D,
                                            float(sm_scale), _stream(), int(window)))
    return out


def merge_heads(heads, out=None):
    """Head-major fp16 [H, T, D] -> token-major [T, H D] (prefill_attention.cu:68-86)."""
    _need(heads, torch.float16, "heads")
    H, T, D = heads.shape
    if out is None:
        out = torch.empty((T, H * D), dtype=torch.float16, device=heads.device)
    check(lib().fa_merge_heads(_ptr(heads), _ptr(out), T, H, D, _stream()))
    return out


def prefill_attention(q, k, v, sm_scale, window=0, out=None):
    """Causal GQA attention, head-major fp16 q [n_q, T, D], k / v [n_kv, T, D]
    (prefill_attention.cu:226-349) -> out [n_q, T, D]."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _need(t, torch.float16, n)
    n_q, T, D = q.shape
    n_kv = k.shape[0]
    if out is None:
        out = torch.empty_like(q)
    check(lib().fa_prefill_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), None, n_q, n_kv, T, D,
                                     float(sm_scale), _stream(), int(window)))
    return out


class Chain:
    """fa_chain: one-token W8A8 linears run as one device-ordered launch.

    `steps` is a list of dicts of device tensors: w (int8 [m, k]), w_scale
    (fp16 [m, G]), x (fp16, at least k values), y (fp16 output), and for
    prologue 2 gamma, optional x2 and h_out; `k` defaults to x.numel(),
    `prologue` / `epilogue` to 0, `eps` to 1e-6.  The tensors must outlive
    the chain (it keeps references)."""

    def __init__(self, steps, group_size):
        arr = (ChainStep * len(steps))()
        self._keep = []
        for i, st in enumerate(steps):
            w, ws, x, y = st["w"], st["w_scale"], st["x"], st["y"]
            _need(w, torch.int8, "w"); _need(ws, torch.float16, "w_scale")
            _need(x, torch.float16, "x"); _need(y, torch.float16, "y")
            for name in ("x2", "gamma", "h_out"):
                _need(st.get(name), torch.float16, name)
            c = arr[i]
            c.w, c.w_scale, c.x, c.y = w.data_ptr(), ws.data_ptr(), x.data_ptr(), y.data_ptr()
            c.x2, c.gamma, c.h_out = _ptr(st.get("x2")), _ptr(st.get("gamma")), _ptr(st.get("h_out"))
            c.m = w.shape[0]
            c.k = st.get("k", x.numel())
            if w.shape[1] != c.k:
                raise ValueError("step %d: w is [%d, %d] but k=%d" % (i, w.shape[0], w.shape[1], c.k))
            c.prologue = st.get("prologue", 0)
            c.epilogue = st.get("epilogue", 0)
            c.eps = st.get("eps", 1e-6)
            self._keep.append(st)
        h = ctypes.c_void_p()
        check(lib().fa_chain_create(arr, len(steps), group_size, ctypes.byref(h)))
        self._h = h

    def run(self):
        check(lib().fa_chain_run(self._h, _stream()))

    def status(self):
        """0 when the last run finished; waits for the current stream."""
        return lib().fa_chain_status(self._h, _stream())

    def set_spin_limit(self, polls):
        check(lib().fa_chain_set_spin_limit(self._h, polls))

    def close(self):
        if getattr(self, "_h", None):
            lib().fa_chain_destroy(self._h)
            self._h = None

    def __del__(self):
        # at interpreter exit the HIP runtime may already be gone: leave the
        # device memory to the process teardown
        # (module globals such as `sys` may already be None then)
        try:
            if sys.is_finalizing():
                return
            self.close()
        except Exception:
            pass

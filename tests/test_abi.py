"""The C-ABI library loads, exports every declared symbol, and rejects bad
arguments before touching the device (no GPU needed)."""
import ctypes
import os
import re
import subprocess

import pytest

from fish_amd import _lib
from fish_amd.build import LIB_PATH, REPO_ROOT

HEADER = os.path.join(REPO_ROOT, "include", "fish_w8a8.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


def test_library_exists_and_loads():
    assert os.path.exists(LIB_PATH), "run __graft_entry__.build() first"
    l = _lib.lib()
    assert l.fa_version().decode().startswith("fish-w8a8-mi355x")


def test_every_declared_symbol_is_exported():
    syms = declared_symbols()
    assert len(syms) >= 20
    l = ctypes.CDLL(LIB_PATH)
    missing = [s for s in syms if not hasattr(l, s)]
    assert not missing, missing
    # and the binding table covers exactly the header
    assert sorted(_lib.SIGNATURES) == syms


def test_cpp_mirror_symbols_exported():
    out = subprocess.run(["nm", "-D", "-C", "--defined-only", LIB_PATH], stdout=subprocess.PIPE,
                         text=True, check=True).stdout
    for name in ["fish::kernels::int8_dequant_gemm_fp16", "fish::kernels::rms_norm",
                 "fish::kernels::silu_forward", "fish::kernels::mul_forward",
                 "fish::kernels::residual_add", "fish::ModelLoader::load",
                 "fish::ModelLoader::get", "fish::infer_group_size_from_scale",
                 "fish::kernels::gemm_fp16", "fish::kernels::int8_rms_gemm_fp16",
                 "fish::kernels::int8_swiglu_gemm_fp16",
                 "fish::kernels::int8_silu_mul_gemm_fp16",
                 "fish::kernels::prefill_attention_gpu", "fish::kernels::qkv_split_heads",
                 "fish::kernels::qkv_split_heads_gqa", "fish::kernels::merge_heads",
                 "fish::kernels::prefill_attention_merged"]:
        assert name in out, name


def test_invalid_arguments_rejected_without_device():
    l = _lib.lib()
    dummy = ctypes.c_void_p(16)
    # null pointers
    rc = l.fa_w8a8_gemm(None, None, 64, None, None, None, None, 8, 1, 64, None)
    assert rc == _lib.FA_ERR_INVALID_ARG
    assert "null pointer" in l.fa_last_error().decode()
    # K must be positive, M/N non-negative
    assert l.fa_w8a8_gemm(dummy, dummy, 64, None, None, dummy, dummy, 8, 1, 0, None) == 1
    assert l.fa_w8a8_gemm(dummy, dummy, 64, None, None, dummy, dummy, -1, 1, 64, None) == 1
    assert l.fa_w8a8_gemm_quantized(dummy, dummy, 64, dummy, dummy, dummy, 8, -2, 64, None) == 1
    # empty batch is a no-op (nothing is launched)
    assert l.fa_w8a8_gemm(dummy, dummy, 64, None, None, dummy, dummy, 8, 0, 64, None) == 0
    # fused prologue entry points: a residual needs h_out, h_out must not alias
    x, r, h = ctypes.c_void_p(4096), ctypes.c_void_p(1 << 20), ctypes.c_void_p(4096 + 64)
    rc = l.fa_w8a8_gemm_rms(dummy, dummy, 64, None, None, x, r, None, dummy, 1e-6, dummy,
                            8, 1, 64, None)
    assert rc == _lib.FA_ERR_INVALID_ARG and "needs h_out" in l.fa_last_error().decode()
    rc = l.fa_w8a8_gemm_rms(dummy, dummy, 64, None, None, x, r, h, dummy, 1e-6, dummy,
                            8, 1, 64, None)
    assert rc == _lib.FA_ERR_INVALID_ARG and "overlaps" in l.fa_last_error().decode()
    rc = l.fa_w8a8_gemm_rms(dummy, dummy, 64, None, None, x, None, None, None, 1e-6, dummy,
                            8, 1, 64, None)
    assert rc == _lib.FA_ERR_INVALID_ARG   # gamma is required
    rc = l.fa_w8a8_gemm_silu_mul(dummy, dummy, 64, None, None, dummy, None, dummy, 8, 1, 64, None)
    assert rc == _lib.FA_ERR_INVALID_ARG
    assert l.fa_w8a8_gemm_silu_mul(dummy, dummy, 64, None, None, dummy, dummy, dummy, 8, 0, 64,
                                   None) == 0
    assert l.fa_w8a8_gemm_quantized(dummy, dummy, 64, dummy, dummy, dummy, 0, 4, 64, None) == 0
    # partials window outside the problem
    rc = l.fa_w8a8_gemm_partials(dummy, dummy, 64, dummy, dummy, dummy, dummy, 0, 9, 0, 1,
                                 8, 1, 64, None)
    assert rc == 1 and "window" in l.fa_last_error().decode()
    assert l.fa_rms_norm(dummy, dummy, dummy, 1, 0, 1e-6, None) == 1
    assert l.fa_rms_norm(dummy, dummy, dummy, 1, 70000, 1e-6, None) == 1
    assert l.fa_rms_norm_quant(dummy, dummy, 1e-6, None, None, 64, None, None, None, 1, 64,
                               None) == 1
    assert l.fa_silu(None, 4, None) == 1
    assert l.fa_silu(None, 0, None) == 0
    assert l.fa_mul(dummy, None, 4, None) == 1
    assert l.fa_quantize_weights_groupwise(dummy, 4, 64, 0, dummy, dummy, None) == 1
    assert l.fa_quantize_activations(None, None, None, None, None, 1, 64, 64, None) == 1
    # attention side: GQA ratio, head dim, alignment, empty sequence
    assert l.fa_prefill_attention(dummy, dummy, dummy, dummy, None, 6, 4, 8, 64, 0.1, None, 0) == 1
    assert "multiple" in l.fa_last_error().decode()
    assert l.fa_prefill_attention(dummy, dummy, dummy, dummy, None, 8, 4, 8, 520, 0.1, None,
                                  0) == 1
    assert "head dim" in l.fa_last_error().decode()
    odd = ctypes.c_void_p(17)
    assert l.fa_prefill_attention(odd, dummy, dummy, dummy, None, 8, 4, 8, 64, 0.1, None, 0) == 1
    assert "aligned" in l.fa_last_error().decode()
    assert l.fa_prefill_attention(None, None, None, None, None, 8, 4, 0, 64, 0.1, None, 0) == 0
    assert l.fa_prefill_attention(dummy, dummy, dummy, dummy, None, 8, 4, 8, 64, float("nan"),
                                  None, 0) == 1
    assert "sm_scale" in l.fa_last_error().decode()
    assert l.fa_qkv_split_heads_gqa(None, dummy, dummy, dummy, 4, 8, 4, 64, None) == 1
    assert l.fa_qkv_split_heads(None, None, None, None, 0, 8, 64, None) == 0
    assert l.fa_merge_heads(dummy, None, 4, 8, 64, None) == 1
    # a successful call clears the message
    assert l.fa_silu(None, 0, None) == 0
    assert l.fa_last_error().decode() == ""


def test_chain_rejects_bad_steps_without_device():
    """fa_chain_create validates every step before any device call (the
    pointers here are never dereferenced)."""
    l = _lib.lib()
    out = ctypes.c_void_p()

    def step(**kw):
        st = _lib.ChainStep()
        st.w, st.w_scale, st.x, st.y = 1 << 20, 1 << 21, 1 << 22, 1 << 23
        st.m, st.k, st.prologue, st.epilogue, st.eps = 64, 256, 0, 0, 1e-6
        for k, v in kw.items():
            setattr(st, k, v)
        return st

    def create(*steps, g=256):
        arr = (_lib.ChainStep * len(steps))(*steps)
        return l.fa_chain_create(arr, len(steps), g, ctypes.byref(out))

    bad = [
        (dict(w=None), "null pointer"),
        (dict(k=250), "k a multiple of 16"),
        (dict(k=16384), "k a multiple of 16"),
        (dict(k=128), "k a multiple of 16"),          # group larger than k
        (dict(m=0), "m=0"),
        (dict(prologue=1), "prologue 1"),
        (dict(epilogue=2), "epilogue 2"),
        (dict(epilogue=1, m=63), "even m"),
        (dict(prologue=2), "needs gamma"),
        (dict(gamma=1 << 24), "need prologue 2"),
        (dict(x=(1 << 22) + 8), "misaligned"),
        (dict(y=(1 << 22) + 64), "y overlaps"),
        (dict(prologue=2, gamma=1 << 24, h_out=(1 << 22) + 16), "h_out overlaps"),
    ]
    for kw, msg in bad:
        assert create(step(**kw)) == _lib.FA_ERR_INVALID_ARG, kw
        assert msg in l.fa_last_error().decode(), (kw, l.fa_last_error())
    assert create(step(), g=32) == _lib.FA_ERR_INVALID_ARG
    assert l.fa_chain_create(None, 1, 256, ctypes.byref(out)) == _lib.FA_ERR_INVALID_ARG
    arr = (_lib.ChainStep * 1)(step())
    assert l.fa_chain_create(arr, 0, 256, ctypes.byref(out)) == _lib.FA_ERR_INVALID_ARG
    assert l.fa_chain_run(None, None) == _lib.FA_ERR_INVALID_ARG
    assert l.fa_chain_status(None, None) == _lib.FA_ERR_INVALID_ARG
    assert l.fa_chain_set_spin_limit(None, 5) == _lib.FA_ERR_INVALID_ARG
    assert l.fa_chain_destroy(None) == 0


def test_infer_group_size():
    l = _lib.lib()
    # src/engine/dual_ar_engine.cc:17-24
    assert l.fa_infer_group_size(2560, 1, 1) == 2560
    assert l.fa_infer_group_size(2560, 2, 1) == 2560
    assert l.fa_infer_group_size(2560, 2, 10) == 256
    assert l.fa_infer_group_size(9728, 2, 152) == 64
    assert l.fa_infer_group_size(100, 2, 3) == 34

"""ctypes binding of libfish_w8a8.so (the C ABI in include/fish_w8a8.h).

Loading fails loudly: there is no CPU or PyTorch fallback for any entry point.
"""
import ctypes
import os
import sys

from .build import LIB_PATH as _BUILT_LIB

# FISH_W8A8_LIB selects another build of the library; by default the in-tree
# build is loaded.  A redirected load is announced on stderr with its path,
# so no test or benchmark output can silently come from another build.
LIB_PATH = os.environ.get("FISH_W8A8_LIB") or _BUILT_LIB

FA_OK = 0
FA_ERR_INVALID_ARG = 1
FA_ERR_HIP = 2
FA_ERR_IO = 3
FA_ERR_FORMAT = 4
FA_ERR_NOT_FOUND = 5
FA_NOALLOC_SCRATCH_BYTES = 32 << 20   # include/fish_w8a8.h

_c = ctypes
_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float


class TensorInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("dtype", ctypes.c_uint32),
        ("ndim", ctypes.c_uint32),
        ("shape", ctypes.c_int64 * 8),
        ("offset", ctypes.c_uint64),
        ("size", ctypes.c_uint64),
        ("data", ctypes.c_void_p),
    ]


class QuantMeta(ctypes.Structure):
    _fields_ = [
        ("has_scale", ctypes.c_int),
        ("has_smooth_inv", ctypes.c_int),
        ("has_act_scale", ctypes.c_int),
        ("group_size", ctypes.c_int),
        ("M", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("groups", ctypes.c_int64),
    ]


class ChainStep(ctypes.Structure):
    """fa_chain_step (include/fish_w8a8.h)."""
    _fields_ = [
        ("w", ctypes.c_void_p),
        ("w_scale", ctypes.c_void_p),
        ("x", ctypes.c_void_p),
        ("x2", ctypes.c_void_p),
        ("gamma", ctypes.c_void_p),
        ("h_out", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("m", ctypes.c_int),
        ("k", ctypes.c_int),
        ("prologue", ctypes.c_int),
        ("epilogue", ctypes.c_int),
        ("eps", ctypes.c_float),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "fa_last_error": (ctypes.c_char_p, []),
    "fa_version": (ctypes.c_char_p, []),
    "fa_w8a8_gemm": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fa_w8a8_gemm_noalloc": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fa_noalloc_scratch_bytes": (ctypes.c_size_t, [_i, _i, _i, _i]),
    "fa_w8a8_gemm_rms": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _f, _p, _i, _i, _i, _p]),
    "fa_w8a8_gemm_silu_mul": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fa_gemm_fp16": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "fa_w8a8_gemm_swiglu_sep": (_i, [_p, _p, _p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _p, _f, _p,
                                     _i, _i, _i, _p]),
    "fa_profile_enable": (_i, [_i]),
    "fa_profile_summary": (ctypes.c_size_t, [_p, ctypes.c_size_t]),
    "fa_profile_reset": (None, []),
    "fa_w8a8_gemm_swiglu": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _f, _p, _i, _i, _i, _p]),
    "fa_w8a8_gemm_quantized": (_i, [_p, _p, _i, _p, _p, _p, _i, _i, _i, _p]),
    "fa_w8a8_gemm_k_splits": (_i, [_i, _i, _i, _i]),
    "fa_w8a8_set_k_split": (_i, [_i]),
    "fa_debug_gemv_plan_rejects": (_i, []),
    "fa_debug_gemv_plan": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _p]),
    "fa_w8a8_gemm_partials": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p]),
    "fa_quantize_activations": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _p]),
    "fa_rms_norm": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "fa_rms_norm_quant": (_i, [_p, _p, _f, _p, _p, _i, _p, _p, _p, _i, _i, _p]),
    "fa_residual_rms_norm_quant": (_i, [_p, _p, _p, _f, _p, _p, _i, _p, _p, _p, _i, _i, _p]),
    "fa_silu": (_i, [_p, _i64, _p]),
    "fa_mul": (_i, [_p, _p, _i64, _p]),
    "fa_residual_add": (_i, [_p, _p, _i64, _p]),
    "fa_silu_mul_quant": (_i, [_p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _p]),
    "fa_quantize_weights_groupwise": (_i, [_p, _i64, _i64, _i, _p, _p, _p]),
    "fa_qkv_split_heads_gqa": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "fa_qkv_split_heads": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "fa_merge_heads": (_i, [_p, _p, _i, _i, _i, _p]),
    "fa_prefill_attention": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, ctypes.c_float, _p, _i]),
    "fa_prefill_attention_merged": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, ctypes.c_float, _p, _i]),
    "fa_workspace_reserve": (_i, [_i, _i, _i, _i, _p]),
    "fa_workspace_release": (_i, []),
    "fa_chain_create": (_i, [ctypes.POINTER(ChainStep), _i, _i, ctypes.POINTER(_p)]),
    "fa_chain_run": (_i, [_p, _p]),
    "fa_chain_status": (_i, [_p, _p]),
    "fa_chain_set_spin_limit": (_i, [_p, _i]),
    "fa_chain_destroy": (_i, [_p]),
    "fa_bin_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_p)]),
    "fa_bin_close": (None, [_p]),
    "fa_bin_num_tensors": (_i, [_p]),
    "fa_bin_tensor_at": (_i, [_p, _i, ctypes.POINTER(TensorInfo)]),
    "fa_bin_find": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(TensorInfo)]),
    "fa_bin_quant_meta": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(QuantMeta)]),
    "fa_bin_gate_up": (_i, [_p, ctypes.c_char_p, ctypes.c_char_p, _p, _p, ctypes.POINTER(QuantMeta)]),
    "fa_infer_group_size": (_i, [_i64, _i, _i64]),
}

_LIB = None


class FaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("fish_w8a8 error %d: %s" % (code, msg))
        self.code = code


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "libfish_w8a8.so is not built (%s); run __graft_entry__.build()" % LIB_PATH)
        if LIB_PATH != _BUILT_LIB:
            sys.stderr.write("fish_w8a8: FISH_W8A8_LIB is set; loading %s instead of %s\n"
                             % (os.path.abspath(LIB_PATH), _BUILT_LIB))
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = l
    return _LIB


def check(rc):
    if rc != FA_OK:
        raise FaError(rc, lib().fa_last_error().decode())
    return rc

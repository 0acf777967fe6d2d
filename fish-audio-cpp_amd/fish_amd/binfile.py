"""dual_ar.bin container: a writer (the layout tools/quant_utils.py:197-228
and tests/test_model_loader.cc:13-86 write) and a reader over the C ABI
(fa_bin_*, the ModelLoader of src/model/loader.cc).

File: u32 magic 0x46495348, u32 version 1, u32 n; n x 344-byte headers
{char name[256]; u32 dtype; u32 ndim; i64 shape[8]; u64 offset; u64 size};
data 256-byte aligned.  dtype: 0 FP32, 1 FP16, 2 BF16, 3 INT8.
"""
import ctypes
import struct

import numpy as np

from ._lib import FA_OK, FaError, QuantMeta, TensorInfo, check, lib

MAGIC = 0x46495348
FORMAT_VERSION = 1
HEADER_SIZE = 344
DTYPES = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int8): 3}
NP_OF = {0: np.float32, 1: np.float16, 2: np.uint16, 3: np.int8}


def _align256(x):
    return (x + 255) // 256 * 256


def write_bin(path, tensors):
    """tensors: list of (name, ndarray).  Returns the list of header dicts."""
    n = len(tensors)
    pos = _align256(12 + HEADER_SIZE * n)
    headers = []
    for name, arr in tensors:
        arr = np.ascontiguousarray(arr)
        headers.append({"name": name, "dtype": DTYPES[arr.dtype], "shape": list(arr.shape),
                        "offset": pos, "size": arr.nbytes, "arr": arr})
        pos = _align256(pos + arr.nbytes)
    with open(path, "wb") as f:
        f.write(struct.pack("<III", MAGIC, FORMAT_VERSION, n))
        for h in headers:
            name = h["name"].encode()
            if len(name) > 255:
                raise ValueError("tensor name too long: %s" % h["name"])
            shape = h["shape"] + [0] * (8 - len(h["shape"]))
            f.write(name + b"\0" * (256 - len(name)))
            f.write(struct.pack("<II", h["dtype"], len(h["shape"])))
            f.write(struct.pack("<8q", *shape))
            f.write(struct.pack("<QQ", h["offset"], h["size"]))
        for h in headers:
            f.seek(h["offset"])
            f.write(h["arr"].tobytes())
        end = headers[-1]["offset"] + headers[-1]["size"] if headers else f.tell()
        f.truncate(max(end, f.tell()))
    return headers


class BinFile:
    """Read-only view of a .bin file through the library's loader."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        rc = lib().fa_bin_open(path.encode(), ctypes.byref(h))
        if rc != FA_OK:
            raise FaError(rc, lib().fa_last_error().decode())
        self._h = h

    def close(self):
        if self._h:
            lib().fa_bin_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __len__(self):
        return lib().fa_bin_num_tensors(self._h)

    def info(self, name):
        ti = TensorInfo()
        rc = lib().fa_bin_find(self._h, name.encode(), ctypes.byref(ti))
        if rc != FA_OK:
            raise FaError(rc, "tensor not found: %s" % name)
        return ti

    def names(self):
        out = []
        for i in range(len(self)):
            ti = TensorInfo()
            lib().fa_bin_tensor_at(self._h, i, ctypes.byref(ti))
            out.append(ti.name.decode())
        return out

    def gate_up(self, w1, w3):
        """(W13 int8 [2F, K], S13 fp16 [2F] or [2F, G], QuantMeta): w1 and w3
        row-interleaved for fa_w8a8_gemm_swiglu."""
        meta = QuantMeta()
        rc = lib().fa_bin_gate_up(self._h, w1.encode(), w3.encode(), None, None,
                                  ctypes.byref(meta))
        check(rc)
        F2, K, G = meta.M, meta.K, meta.groups
        w13 = np.empty((F2, K), np.int8)
        s13 = np.empty((F2, G) if self.info(w1 + "_scale").ndim > 1 else (F2,), np.float16)
        check(lib().fa_bin_gate_up(self._h, w1.encode(), w3.encode(), w13.ctypes.data,
                                   s13.ctypes.data, None))
        return w13, s13, meta

    def array(self, name):
        ti = self.info(name)
        shape = tuple(ti.shape[i] for i in range(ti.ndim))
        dt = NP_OF[ti.dtype]
        buf = (ctypes.c_char * ti.size).from_address(ti.data)
        return np.frombuffer(bytes(buf), dtype=dt).reshape(shape)

    def quant_meta(self, weight_name):
        m = QuantMeta()
        rc = lib().fa_bin_quant_meta(self._h, weight_name.encode(), ctypes.byref(m))
        if rc != FA_OK:
            raise FaError(rc, "no weight %s" % weight_name)
        return m

"""dual_ar.bin container: writer -> library loader round trip, group-size
inference and QuantMeta discovery (src/model/tensor.h, loader.cc,
dual_ar_engine.cc:17-24, 231-275), error paths (no GPU needed).  The fixture
style follows the reference's BinFile helper (tests/test_model_loader.cc:13-86)."""
import os
import struct

import numpy as np
import pytest

from fish_amd import _lib
from fish_amd.binfile import BinFile, write_bin


@pytest.fixture
def tmpbin(tmp_path):
    return str(tmp_path / "model.bin")


def _layer(M=64, K=512, g=64, smooth=True, act=True):
    rng = np.random.default_rng(0)
    q = rng.integers(-127, 128, (M, K), dtype=np.int8)
    G = (K + g - 1) // g
    s = (rng.random((M, G)) * 1e-3 + 1e-4).astype(np.float16)
    t = [("layers.0.attention.wqkv.weight", q), ("layers.0.attention.wqkv.weight_scale", s)]
    if smooth:
        t.append(("layers.0.attention.wqkv.weight_smooth_inv", np.ones(K, np.float16)))
    if act:
        t.append(("layers.0.attention.wqkv.weight_act_scale", np.full(G, 0.05, np.float16)))
    t.append(("layers.0.attention_norm.weight", np.ones(K // 8, np.float16)))
    return t


def test_round_trip(tmpbin):
    tensors = _layer()
    headers = write_bin(tmpbin, tensors)
    assert all(h["offset"] % 256 == 0 for h in headers)
    raw = open(tmpbin, "rb").read()
    assert struct.unpack("<III", raw[:12]) == (0x46495348, 1, len(tensors))
    with BinFile(tmpbin) as b:
        assert len(b) == len(tensors)
        assert b.names() == [n for n, _ in tensors]
        for name, arr in tensors:
            got = b.array(name)
            assert got.dtype == arr.dtype and got.shape == arr.shape
            assert np.array_equal(got, arr)
        ti = b.info("layers.0.attention.wqkv.weight")
        assert ti.dtype == 3 and ti.ndim == 2 and list(ti.shape[:2]) == [64, 512]
        m = b.quant_meta("layers.0.attention.wqkv.weight")
        assert (m.has_scale, m.has_smooth_inv, m.has_act_scale) == (1, 1, 1)
        assert m.group_size == 64 and m.groups == 8 and m.M == 64 and m.K == 512
        m = b.quant_meta("layers.0.attention_norm.weight")
        assert m.has_scale == 0 and m.group_size == 0


@pytest.mark.parametrize("K,scale_shape,want", [
    (512, (64,), 512),            # 1-D (row-wise) scale -> g = K
    (512, (64, 1), 512),          # G == 1 -> K
    (2560, (64, 10), 256),
    (100, (64, 3), 34),           # K not a multiple of G: ceil(K / G)
])
def test_group_size_inference(tmpbin, K, scale_shape, want):
    q = np.zeros((64, K), np.int8)
    s = np.ones(scale_shape, np.float16)
    write_bin(tmpbin, [("w", q), ("w_scale", s)])
    with BinFile(tmpbin) as b:
        assert b.quant_meta("w").group_size == want


def test_missing_tensor(tmpbin):
    write_bin(tmpbin, _layer())
    with BinFile(tmpbin) as b:
        with pytest.raises(_lib.FaError) as e:
            b.info("nope")
        assert e.value.code == _lib.FA_ERR_NOT_FOUND


def test_bad_files(tmpbin, tmp_path):
    with pytest.raises(_lib.FaError) as e:
        BinFile(str(tmp_path / "does_not_exist.bin"))
    assert e.value.code == _lib.FA_ERR_IO
    write_bin(tmpbin, _layer())
    raw = bytearray(open(tmpbin, "rb").read())
    bad = str(tmp_path / "bad_magic.bin")
    open(bad, "wb").write(b"XXXX" + raw[4:])
    with pytest.raises(_lib.FaError) as e:
        BinFile(bad)
    assert e.value.code == _lib.FA_ERR_FORMAT
    badv = str(tmp_path / "bad_version.bin")
    open(badv, "wb").write(raw[:4] + struct.pack("<I", 2) + raw[8:])
    with pytest.raises(_lib.FaError) as e:
        BinFile(badv)
    assert e.value.code == _lib.FA_ERR_FORMAT
    for cut in (8, 12 + 100, len(raw) - 10):
        tr = str(tmp_path / ("trunc%d.bin" % cut))
        open(tr, "wb").write(raw[:cut])
        with pytest.raises(_lib.FaError) as e:
            BinFile(tr)
        assert e.value.code == _lib.FA_ERR_FORMAT, cut
        assert _lib.lib().fa_last_error().decode()

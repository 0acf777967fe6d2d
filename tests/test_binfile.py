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


def _ffn(F=48, K=512, g=64, smooth=(None, None), act=(None, None), seed=1):
    rng = np.random.default_rng(seed)
    G = K // g
    t = []
    for name, sm, ac in (("w1", smooth[0], act[0]), ("w3", smooth[1], act[1])):
        w = "layers.0.feed_forward.%s.weight" % name
        t.append((w, rng.integers(-127, 128, (F, K), dtype=np.int8)))
        t.append((w + "_scale", (rng.random((F, G)) * 1e-3 + 1e-4).astype(np.float16)))
        if sm is not None:
            t.append((w + "_smooth_inv", np.full(K, sm, np.float16)))
        if ac is not None:
            t.append((w + "_act_scale", np.full(G, ac, np.float16)))
    return t


W1, W3 = "layers.0.feed_forward.w1.weight", "layers.0.feed_forward.w3.weight"


def test_gate_up_interleave(tmpbin):
    """w1 / w3 -> one row-interleaved weight (row 2i = w1[i], 2i+1 = w3[i])."""
    tensors = _ffn(smooth=(0.5, 0.5), act=(0.04, 0.04))
    write_bin(tmpbin, tensors)
    d = dict(tensors)
    with BinFile(tmpbin) as b:
        w13, s13, meta = b.gate_up(W1, W3)
    assert meta.M == 96 and meta.K == 512 and meta.groups == 8 and meta.group_size == 64
    assert (meta.has_smooth_inv, meta.has_act_scale) == (1, 1)
    assert np.array_equal(w13[0::2], d[W1]) and np.array_equal(w13[1::2], d[W3])
    assert np.array_equal(s13[0::2], d[W1 + "_scale"]) and np.array_equal(s13[1::2], d[W3 + "_scale"])


@pytest.mark.parametrize("smooth,act", [((0.5, None), (None, None)),   # only one calibrated
                                        ((0.5, 0.25), (None, None)),   # different smooth_inv
                                        ((None, None), (0.04, 0.05))])  # different static scales
def test_gate_up_rejects_different_input_quantization(tmpbin, smooth, act):
    write_bin(tmpbin, _ffn(smooth=smooth, act=act))
    with BinFile(tmpbin) as b:
        with pytest.raises(_lib.FaError, match="fa_bin_gate_up"):
            b.gate_up(W1, W3)


def test_gate_up_shape_mismatch(tmpbin):
    t = _ffn()
    t[2] = (W3, np.zeros((40, 512), np.int8))
    t[3] = (W3 + "_scale", np.ones((40, 8), np.float16))
    write_bin(tmpbin, t)
    with BinFile(tmpbin) as b:
        with pytest.raises(_lib.FaError, match="differ in shape"):
            b.gate_up(W1, W3)

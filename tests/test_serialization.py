"""The .znn reader/writer against the format of src/serialization.zig (CPU).

The reference ships no .znn files, so the fixtures are built here byte by
byte from the layout its code writes: the packed FileHeader (:63-68, magic,
u32 version, u32 layer count), then per Dense layer writeLayer's fields
(:150-175: u32 type 1, u32 in, u32 out, u32 activation tag, f32 weights,
f32 bias), all little-endian; activation tags in declaration order of
Activation (src/activation.zig:14-22)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from zigneuron_amd import serialization as znn


def dense_bytes(n_in, n_out, tag, w, b, ltype=1):
    return struct.pack("<IIII", ltype, n_in, n_out, tag) + w.astype("<f4").tobytes() + b.astype("<f4").tobytes()


def model_bytes():
    rng = np.random.default_rng(0)
    w1, b1 = rng.standard_normal((5, 3)).astype(np.float32), rng.standard_normal(3).astype(np.float32)
    w2, b2 = rng.standard_normal((3, 2)).astype(np.float32), rng.standard_normal(2).astype(np.float32)
    data = b"ZNN\x00" + struct.pack("<II", 1, 2) + dense_bytes(5, 3, 0, w1, b1) + dense_bytes(3, 2, 4, w2, b2)
    return data, (w1, b1, w2, b2)


def test_parse_two_dense_layers():
    data, (w1, b1, w2, b2) = model_bytes()
    assert len(data) == 12 + (16 + 4 * (15 + 3)) + (16 + 4 * (6 + 2))
    l1, l2 = znn.parse(data)
    assert (l1.input_size, l1.output_size, l1.act) == (5, 3, "relu")
    assert (l2.input_size, l2.output_size, l2.act) == (3, 2, "linear")
    np.testing.assert_array_equal(l1.weights, w1)
    np.testing.assert_array_equal(l1.bias, b1)
    np.testing.assert_array_equal(l2.weights, w2)
    np.testing.assert_array_equal(l2.bias, b2)


def test_serialize_is_byte_identical():
    data, _ = model_bytes()
    assert znn.serialize(znn.parse(data)) == data


@pytest.mark.parametrize("tag,act", [(0, "relu"), (1, "sigmoid"), (2, "tanh"), (4, "linear")])
def test_activation_tags(tag, act):
    w, b = np.ones((2, 2), np.float32), np.zeros(2, np.float32)
    data = b"ZNN\x00" + struct.pack("<II", 1, 1) + dense_bytes(2, 2, tag, w, b)
    (layer,) = znn.parse(data)
    assert layer.act == act
    assert znn.serialize([layer]) == data


def test_empty_model():
    data = b"ZNN\x00" + struct.pack("<II", 1, 0)
    assert znn.parse(data) == []
    assert znn.serialize([]) == data


@pytest.mark.parametrize("mutate,error", [
    (lambda d: b"ZNX\x00" + d[4:], "InvalidMagic"),
    (lambda d: d[:4] + struct.pack("<I", 2) + d[8:], "UnsupportedVersion"),
    (lambda d: d[:12] + struct.pack("<I", 0) + d[16:], "UnknownLayerType"),
    (lambda d: d[:12] + struct.pack("<I", 13) + d[16:], "UnknownLayerType"),
    (lambda d: d[:12] + struct.pack("<I", 8) + d[16:], "UnsupportedLayerType"),
    (lambda d: d[:24] + struct.pack("<I", 8) + d[28:], "InvalidActivation"),
    (lambda d: d[:24] + struct.pack("<I", 3) + d[28:], "UnsupportedActivation"),
    (lambda d: d[:16] + struct.pack("<I", 0) + d[20:], "InvalidInputSize"),
    (lambda d: d[:20] + struct.pack("<I", 0) + d[24:], "InvalidOutputSize"),
    (lambda d: d[:-1], "EndOfStream"),
    (lambda d: d[:30], "EndOfStream"),
    (lambda d: d[:10], "EndOfStream"),
])
def test_malformed_files_are_rejected(mutate, error):
    data, _ = model_bytes()
    with pytest.raises(znn.ZnnError) as e:
        znn.parse(mutate(data))
    assert e.value.args[0] == error


def test_save_and_parse_specs(tmp_path):
    rng = np.random.default_rng(1)
    specs = [znn.DenseSpec(7, 4, "tanh", rng.standard_normal((7, 4)), rng.standard_normal(4)),
             znn.DenseSpec(4, 3, "sigmoid", rng.standard_normal((4, 3)), rng.standard_normal(3))]
    path = tmp_path / "m.znn"
    n = znn.save_model(specs, str(path))
    data = path.read_bytes()
    assert n == len(data) == 12 + 16 + 4 * (28 + 4) + 16 + 4 * (12 + 3)
    back = znn.parse(data)
    for s, t in zip(specs, back):
        assert (s.input_size, s.output_size, s.act) == (t.input_size, t.output_size, t.act)
        np.testing.assert_array_equal(s.weights, t.weights)
        np.testing.assert_array_equal(s.bias, t.bias)

"""``.znn`` model files (src/serialization.zig) for the Dense layers of this backend.

Format (little-endian, src/serialization.zig:1-10, 63-68, 150-175, 340-371):
  header  : b"ZNN\\0", u32 version (= 1), u32 layer count           (12 bytes)
  per layer: u32 layer type; for Dense (type 1):
             u32 input_size, u32 output_size, u32 activation tag,
             f32 weights[input_size * output_size]  ([in x out] row-major),
             f32 bias[output_size]
The activation tag is the declaration index of ``Activation``
(src/activation.zig:14-22): relu 0, sigmoid 1, tanh 2, softmax 3, linear 4,
gelu 5, leaky_relu 6, elu 7.  This backend runs linear, relu, sigmoid and
tanh; files with other activations or other layer types are rejected with the
reference's error names.

``load_model`` puts the weights straight into HBM (``DenseDevice``) or into the
host mirror (``Dense``); ``save_model`` writes the same bytes the reference's
``saveModel`` writes for Dense layers.
"""
from __future__ import annotations

import struct
from typing import List, Optional, Sequence, Union

import numpy as np

from . import _lib

MAGIC = b"ZNN\x00"
VERSION = 1
LAYER_DENSE = 1  # LayerType.dense (src/serialization.zig:51-64)
ACT_TAGS = ("relu", "sigmoid", "tanh", "softmax", "linear", "gelu", "leaky_relu", "elu")
SUPPORTED = ("linear", "relu", "sigmoid", "tanh")


class ZnnError(ValueError):
    """A malformed or unsupported .znn file; ``args[0]`` is the reference's error name."""


class DenseSpec:
    """One Dense layer as stored in a .znn file."""

    def __init__(self, input_size: int, output_size: int, act: str, weights: np.ndarray, bias: np.ndarray):
        self.input_size, self.output_size, self.act = input_size, output_size, act
        self.weights = np.ascontiguousarray(weights, dtype=np.float32).reshape(input_size, output_size)
        self.bias = np.ascontiguousarray(bias, dtype=np.float32).reshape(output_size)


def _take(buf: memoryview, pos: int, n: int) -> bytes:
    if pos + n > len(buf):
        raise ZnnError("EndOfStream")
    return bytes(buf[pos:pos + n])


def parse(data: bytes) -> List[DenseSpec]:
    """Parse the bytes of a .znn file (loadModel / readLayer, src/serialization.zig:104-143, 340-371)."""
    buf = memoryview(data)
    magic = _take(buf, 0, 4)
    version, count = struct.unpack("<II", _take(buf, 4, 8))
    if magic != MAGIC:
        raise ZnnError("InvalidMagic")
    if version != VERSION:
        raise ZnnError("UnsupportedVersion")
    pos, layers = 12, []
    for _ in range(count):
        (ltype,) = struct.unpack("<I", _take(buf, pos, 4))
        pos += 4
        if ltype != LAYER_DENSE:
            raise ZnnError("UnknownLayerType" if ltype == 0 or ltype > 12 else "UnsupportedLayerType")
        n_in, n_out, act_tag = struct.unpack("<III", _take(buf, pos, 12))
        pos += 12
        if act_tag >= len(ACT_TAGS):
            raise ZnnError("InvalidActivation")
        act = ACT_TAGS[act_tag]
        if act not in SUPPORTED:
            raise ZnnError("UnsupportedActivation")
        if n_in == 0:
            raise ZnnError("InvalidInputSize")  # Dense.init (src/layer.zig:306-307)
        if n_out == 0:
            raise ZnnError("InvalidOutputSize")
        wbytes = 4 * n_in * n_out
        w = np.frombuffer(_take(buf, pos, wbytes), dtype="<f4").astype(np.float32)
        pos += wbytes
        b = np.frombuffer(_take(buf, pos, 4 * n_out), dtype="<f4").astype(np.float32)
        pos += 4 * n_out
        layers.append(DenseSpec(n_in, n_out, act, w, b))
    return layers


def serialize(specs: Sequence[DenseSpec]) -> bytes:
    """The bytes saveModel / writeLayer write for Dense layers (src/serialization.zig:76-175)."""
    if len(specs) > 0xFFFFFFFF:
        raise ZnnError("LayerCountOverflow")
    out = [MAGIC, struct.pack("<II", VERSION, len(specs))]
    for s in specs:
        if s.act not in SUPPORTED:
            raise ZnnError("UnsupportedActivation")
        out.append(struct.pack("<IIII", LAYER_DENSE, s.input_size, s.output_size, ACT_TAGS.index(s.act)))
        out.append(np.ascontiguousarray(s.weights, dtype="<f4").tobytes())
        out.append(np.ascontiguousarray(s.bias, dtype="<f4").tobytes())
    return b"".join(out)


def _spec_of(layer) -> DenseSpec:
    """A DenseSpec from a Dense (host arrays) or a DenseDevice (downloads from HBM)."""
    from .layer import Dense, DenseDevice
    if isinstance(layer, DenseSpec):
        return layer
    if isinstance(layer, DenseDevice):
        return DenseSpec(layer.input_size, layer.output_size, layer.act, layer.weights.download(),
                         layer.bias.download())
    if isinstance(layer, Dense):
        return DenseSpec(layer.input_size, layer.output_size, layer.act, layer.weights, layer.bias)
    raise TypeError(f"not a Dense layer: {type(layer).__name__}")


def save_model(layers: Sequence, path: str) -> int:
    """Write layers to a .znn file; returns the byte count (saveModel's return value)."""
    data = serialize([_spec_of(l) for l in layers])
    with open(path, "wb") as f:
        f.write(data)
    return len(data)


def load_model(path: str, target, batch: Optional[int] = None) -> List[Union["Dense", "DenseDevice"]]:
    """Read a .znn file into layers of this backend.

    target: a ``Context`` -> ``DenseDevice`` layers with weights and bias in
    HBM (``batch`` sizes their activation buffers); a ``Backend`` -> host-mirror
    ``Dense`` layers."""
    from .backend import Backend, Context
    from .layer import Dense, DenseDevice
    with open(path, "rb") as f:
        specs = parse(f.read())
    layers = []
    for s in specs:
        if isinstance(target, Context):
            if batch is None:
                raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "load_model", "batch is required")
            layers.append(DenseDevice(target, s.input_size, s.output_size, s.act, batch, weights=s.weights,
                                      bias=s.bias))
        elif isinstance(target, Backend):
            d = Dense(target, s.input_size, s.output_size, s.act)
            d.weights = s.weights.ravel().copy()
            d.bias = s.bias.copy()
            layers.append(d)
        else:
            raise TypeError("target must be a Context or a Backend")
    return layers

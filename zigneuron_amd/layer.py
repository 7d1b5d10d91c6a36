"""Mirror of ZigNeuron's ``Dense`` layer (src/layer.zig:291-476) on the HIP arm.

Shapes and call sequence follow the reference:
  * weights [input_size x output_size] row-major, bias [output_size]
    (src/layer.zig:311-314), initialised U[-1,1) * scale with He / Xavier /
    linear scales (src/layer.zig:330-338); the bias starts at zero;
  * forward: NN GEMM + bias + activation (src/layer.zig:380-409).  On this
    backend the three steps run as one fused kernel through
    ``Backend.matMulBias{,Relu,Sigmoid,Tanh}`` (src/backend.zig:200-295);
  * backward: activationBackward -> NT GEMM for grad_input -> accumulateBias
    -> TN GEMM for grad_weights (src/layer.zig:411-475).

``DenseDevice`` is the same layer with every tensor resident in HBM (the
device-pointer C ABI), used for the MLP training-step workload.
"""
from __future__ import annotations

import math
from typing import Optional

import numpy as np

from . import _lib
from .backend import Backend, Context, DeviceBuffer, act_id

_FUSED = {"linear": "matMulBias", "relu": "matMulBiasRelu", "sigmoid": "matMulBiasSigmoid",
          "tanh": "matMulBiasTanh"}


def init_scale(act: str, input_size: int, output_size: int) -> float:
    """Weight scale of Dense.init (src/layer.zig:330-334)."""
    if act in ("relu", "leaky_relu"):
        return math.sqrt(2.0 / input_size)
    if act == "linear":
        return math.sqrt(1.0 / input_size)
    return math.sqrt(2.0 / (input_size + output_size))


def init_weights(input_size: int, output_size: int, act: str, seed: int) -> np.ndarray:
    """U[-1,1) * scale from a seeded PCG64 stream (the reference's Zig PRNG
    stream is not reproduced; parity tests feed the same arrays to both sides)."""
    rng = np.random.default_rng(seed)
    u = rng.random((input_size, output_size), dtype=np.float32)
    return ((u * np.float32(2.0) - np.float32(1.0)) * np.float32(init_scale(act, input_size, output_size))).astype(
        np.float32)


class Dense:
    def __init__(self, backend: Backend, input_size: int, output_size: int, act: str = "relu", seed: int = 1):
        if input_size == 0:
            raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "Dense.init", "InvalidInputSize")
        if output_size == 0:
            raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "Dense.init", "InvalidOutputSize")
        act_id(act)  # validates
        self.backend = backend
        self.input_size, self.output_size, self.act = input_size, output_size, act
        self.weights = init_weights(input_size, output_size, act, seed).ravel()
        self.bias = np.zeros(output_size, np.float32)
        self.grad_weights = np.zeros(input_size * output_size, np.float32)
        self.grad_bias = np.zeros(output_size, np.float32)

    def forward(self, inp, output) -> None:
        inp = np.ascontiguousarray(inp, dtype=np.float32)
        batch = inp.size // self.input_size
        if output.size != batch * self.output_size:
            raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "Dense.forward", "InvalidOutputSize")
        getattr(self.backend, _FUSED[self.act])(inp, self.weights, self.bias, output, batch, self.output_size,
                                                self.input_size)

    def backward(self, inp, grad_output, grad_input, activated_output) -> None:
        inp = np.ascontiguousarray(inp, dtype=np.float32)
        batch = inp.size // self.input_size if self.input_size > 0 else 1
        gaa = np.empty(batch * self.output_size, np.float32)
        self.backend.activationBackward(self.act, activated_output, grad_output, gaa)
        self.backend.matMulTransposeB(gaa, self.weights, grad_input, batch, self.input_size, self.output_size,
                                      False)
        self.backend.accumulateBias(self.grad_bias, gaa)
        self.backend.matMulTransposeA(inp, gaa, self.grad_weights, self.input_size, self.output_size, batch, False)


class DenseDevice:
    """Dense with weights, gradients and activations resident in HBM."""

    def __init__(self, ctx: Context, input_size: int, output_size: int, act: str, batch: int,
                 weights: Optional[np.ndarray] = None, bias: Optional[np.ndarray] = None, seed: int = 1):
        self.ctx, self.input_size, self.output_size, self.act, self.batch = ctx, input_size, output_size, act, batch
        w = init_weights(input_size, output_size, act, seed) if weights is None else weights
        b = np.zeros(output_size, np.float32) if bias is None else bias
        self.weights = ctx.to_device(w)
        self.bias = ctx.to_device(b)
        self.grad_weights = ctx.alloc(input_size * output_size).fill(0.0)
        self.grad_bias = ctx.alloc(output_size).fill(0.0)
        self.out = ctx.alloc(batch * output_size)
        self.gaa = ctx.alloc(batch * output_size)
        self.grad_input = ctx.alloc(batch * input_size)
        self._gaa_ready = False  # self.gaa was written by the layer above's chained backward

    def forward(self, x: DeviceBuffer) -> DeviceBuffer:
        """Fused NN + bias + activation into self.out (asynchronous).  A new forward
        starts a new step: a derivative left by an earlier chained backward is stale."""
        self._gaa_ready = False
        self.ctx.sgemm("nn", self.batch, self.output_size, self.input_size, x, self.input_size, self.weights,
                       self.output_size, self.out, self.output_size, False, self.bias, self.act)
        return self.out

    def backward(self, x: DeviceBuffer, grad_out: Optional[DeviceBuffer], fused: bool = True,
                 below: Optional["DenseDevice"] = None) -> DeviceBuffer:
        """activationBackward -> NT (grad_input) -> accumulateBias -> TN (grad_weights).

        fused: one zn_hip_dense_backward call (activation derivative and bias
        sums in one pass, bias summed over row splits); otherwise the
        reference's four calls, with the row-by-row bias sum.
        below: the layer whose output is x; this call then also writes that
        layer's activation derivative (zn_hip_dense_backward_chain), and that
        layer's own backward takes it as ready (its grad_out is not read).
        The results are the same bits as the unchained calls."""
        if fused:
            ready = self._gaa_ready
            if ready and grad_out is not None:
                raise _lib.InvalidArgumentError(
                    _lib.ZN_ERR_INVALID_ARG, "DenseDevice.backward",
                    "grad_out given, but the layer above's chained backward already wrote this layer's derivative")
            self._gaa_ready = False
            if below is None and not ready:
                self.ctx.dense_backward(self.act, x, self.weights, self.out, grad_out, self.gaa, self.grad_input,
                                        self.grad_weights, self.grad_bias, self.batch, self.input_size,
                                        self.output_size)
                return self.grad_input
            if below is not None and (below.output_size != self.input_size or below.batch != self.batch):
                raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "DenseDevice.backward", "below")
            self.ctx.dense_backward_chain(
                self.act, x, self.weights, None if ready else self.out, None if ready else grad_out, self.gaa,
                self.grad_input, self.grad_weights, self.grad_bias, self.batch, self.input_size, self.output_size,
                ready, below.act if below is not None else "linear", below.out if below is not None else None,
                below.gaa if below is not None else None)
            if below is not None:
                below._gaa_ready = True
            return self.grad_input
        if self._gaa_ready:
            raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "DenseDevice.backward",
                                            "the chained derivative needs fused=True")
        n_out = self.batch * self.output_size
        self.ctx.activation_backward(self.act, self.out, grad_out, self.gaa, n_out)
        self.ctx.sgemm("nt", self.batch, self.input_size, self.output_size, self.gaa, self.output_size,
                       self.weights, self.output_size, self.grad_input, self.input_size)
        self.ctx.accumulate_bias(self.grad_bias, self.gaa, self.batch, self.output_size)
        self.ctx.sgemm("tn", self.input_size, self.output_size, self.batch, x, self.input_size, self.gaa,
                       self.output_size, self.grad_weights, self.output_size)
        return self.grad_input


def _pair_check(lower: DenseDevice, upper: DenseDevice, where: str) -> None:
    if upper.input_size != lower.output_size or upper.batch != lower.batch or upper.ctx is not lower.ctx:
        raise _lib.InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, where, "upper must take lower's output")


def pair_forward(lower: DenseDevice, upper: DenseDevice, x: DeviceBuffer) -> DeviceBuffer:
    """Network.forward over two stacked layers (src/network.zig:309-360): lower.out =
    act(x.W + b) of the lower layer, then upper.out from it.  One launch when the upper layer
    has at most 16 outputs (zn_hip_dense_pair_forward), else one fused GEMM per layer."""
    _pair_check(lower, upper, "pair_forward")
    lower._gaa_ready = upper._gaa_ready = False
    lower.ctx.dense_pair_forward(lower.act, x, lower.weights, lower.bias, lower.out, upper.act, upper.weights,
                                 upper.bias, upper.out, lower.batch, lower.input_size, lower.output_size,
                                 upper.output_size)
    return upper.out


def pair_backward(lower: DenseDevice, upper: DenseDevice, x: DeviceBuffer, grad_out: DeviceBuffer,
                  grad_input: bool = True) -> Optional[DeviceBuffer]:
    """Network's backward loop over the same two layers (src/network.zig:455-477), upper first:
    every gradient, derivative and grad_input buffer of both layers, in one launch when the upper
    layer has at most 16 outputs (zn_hip_dense_pair_backward).  grad_input=False skips the lower
    layer's grad_input (the first layer of a network)."""
    _pair_check(lower, upper, "pair_backward")
    lower._gaa_ready = upper._gaa_ready = False
    lower.ctx.dense_pair_backward(
        lower.act, x, lower.weights, lower.out, lower.gaa, lower.grad_input if grad_input else None,
        lower.grad_weights, lower.grad_bias, upper.act, upper.weights, upper.out, grad_out, upper.gaa,
        upper.grad_input, upper.grad_weights, upper.grad_bias, lower.batch, lower.input_size, lower.output_size,
        upper.output_size)
    return lower.grad_input if grad_input else None

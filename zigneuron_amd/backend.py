"""Host-side mirror of ZigNeuron's ``Backend`` operator API for the GEMM path.

``Backend`` keeps the reference method names, argument order and meaning
(src/backend.zig:169-325, 367-399, 649-671): host ``float32`` arrays play the
role of Zig ``[]f32`` slices and outputs are written in place.  Every method
runs on the MI355X through the C ABI (include/zn_hip.h); errors surface as
``ZnError`` subclasses, the analogue of the reference's Zig error unions.

``Context``/``DeviceBuffer`` expose the device-pointer entry points
(``sgemm``, ``sgemm_strided_batched`` and the Dense helpers) for callers that
keep tensors resident in HBM.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional

import numpy as np

from . import _lib
from ._lib import (ACT_LINEAR, ACT_RELU, ACT_SIGMOID, ACT_TANH, LAYOUT_NN, LAYOUT_NT, LAYOUT_TN,
                   InvalidArgumentError, check)

ACTIVATIONS = {"linear": ACT_LINEAR, "relu": ACT_RELU, "sigmoid": ACT_SIGMOID, "tanh": ACT_TANH}
LAYOUTS = {"nn": LAYOUT_NN, "nt": LAYOUT_NT, "tn": LAYOUT_TN}


def act_id(act) -> int:
    """Map an activation name (src/activation.zig:14-22) to its C-ABI id."""
    if isinstance(act, int):
        return act
    try:
        return ACTIVATIONS[str(act)]
    except KeyError:
        raise InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "activation",
                                   f"{act!r} is not on the GEMM path (linear, relu, sigmoid, tanh)") from None


def layout_id(layout) -> int:
    if isinstance(layout, int):
        return layout
    return LAYOUTS[str(layout).lower()]


def available() -> bool:
    """zn_hip_available(): a HIP device is visible."""
    return bool(_lib.load().zn_hip_available())


def _f32_in(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _f32_out(x) -> np.ndarray:
    if not (isinstance(x, np.ndarray) and x.dtype == np.float32 and x.flags.c_contiguous and x.flags.writeable):
        raise InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "output",
                                   "outputs must be writable contiguous float32 arrays")
    return x


def _ptr(x: np.ndarray) -> int:
    return x.ctypes.data


class Graph:
    """A captured sequence of device calls, replayed with one launch (zn_hip_graph_*)."""

    def __init__(self, ctx: "Context", handle: ctypes.c_void_p):
        self._ctx, self.handle = ctx, handle
        ctx._graphs.add(self)

    def launch(self) -> None:
        if not self.handle or not self._ctx.handle:
            raise InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "zn_hip_graph_launch", "graph or context closed")
        check(_lib.load().zn_hip_graph_launch(self._ctx.handle, self.handle), "zn_hip_graph_launch")

    def close(self) -> None:
        """Release the graph (a no-op once it or its context is closed: the
        context's destruction releases its graphs)."""
        if self.handle and self._ctx.handle:
            _lib.load().zn_hip_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self, ctx: "Context"):
        self._ctx = ctx
        h = ctypes.c_void_p()
        check(_lib.load().zn_hip_event_create(ctx.handle, ctypes.byref(h)), "zn_hip_event_create")
        self.handle = h

    def record(self) -> None:
        check(_lib.load().zn_hip_event_record(self._ctx.handle, self.handle), "zn_hip_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(_lib.load().zn_hip_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)),
              "zn_hip_event_elapsed_ms")
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            _lib.load().zn_hip_event_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """A caller-owned float32 buffer in HBM (zn_hip_alloc / zn_hip_free)."""

    def __init__(self, ctx: "Context", count: int):
        self.ctx = ctx
        self.count = int(count)
        h = ctypes.c_void_p()
        check(_lib.load().zn_hip_alloc(ctx.handle, max(self.count, 1) * 4, ctypes.byref(h)), "zn_hip_alloc")
        self.ptr = int(h.value)

    def upload(self, host) -> "DeviceBuffer":
        h = _f32_in(host)
        if h.size > self.count:
            raise InvalidArgumentError(_lib.ZN_ERR_INVALID_ARG, "upload", "host array larger than buffer")
        check(_lib.load().zn_hip_h2d(self.ctx.handle, self.ptr, _ptr(h), h.size * 4), "zn_hip_h2d")
        return self

    def download(self, count: Optional[int] = None) -> np.ndarray:
        n = self.count if count is None else int(count)
        out = np.empty(n, np.float32)
        check(_lib.load().zn_hip_d2h(self.ctx.handle, _ptr(out), self.ptr, n * 4), "zn_hip_d2h")
        return out

    def fill(self, value: float) -> "DeviceBuffer":
        check(_lib.load().zn_hip_fill_f32(self.ctx.handle, self.ptr, float(value), self.count), "zn_hip_fill_f32")
        return self

    def offset(self, elements: int) -> int:
        return self.ptr + 4 * int(elements)

    def close(self) -> None:
        """Free the buffer; after its context is closed this only drops the pointer."""
        if self.ptr and self.ctx.handle:
            check(_lib.load().zn_hip_free(self.ctx.handle, self.ptr), "zn_hip_free")
        self.ptr = 0

    def __del__(self):  # pragma: no cover
        try:
            if self.ptr and self.ctx.handle:
                self.close()
        except Exception:
            pass


class Context:
    """One device, one stream, the loaded gfx950 code objects (zn_hip_create)."""

    def __init__(self, device: int = 0, code_object_dir: Optional[str] = None):
        h = ctypes.c_void_p()
        d = code_object_dir.encode() if code_object_dir else None
        check(_lib.load().zn_hip_create(int(device), d, ctypes.byref(h)), "zn_hip_create")
        self.handle = h.value
        self._graphs = weakref.WeakSet()
        info = _lib.DeviceInfo()
        check(_lib.load().zn_hip_device_info(self.handle, ctypes.byref(info)), "zn_hip_device_info")
        self.arch = info.name.decode()
        self.compute_units = int(info.compute_units)
        self.clock_khz = int(info.clock_khz)
        self.total_mem = int(info.total_mem)

    # --- memory / sync
    def alloc(self, count: int) -> DeviceBuffer:
        return DeviceBuffer(self, count)

    def to_device(self, host) -> DeviceBuffer:
        h = _f32_in(host)
        return DeviceBuffer(self, h.size).upload(h)

    def sync(self) -> None:
        check(_lib.load().zn_hip_sync(self.handle), "zn_hip_sync")

    def event(self) -> Event:
        return Event(self)

    def capture(self, fn) -> Graph:
        """Run fn() under stream capture and return the graph of its device calls.
        Run fn() once eagerly first (it sizes the split-K workspace)."""
        L = _lib.load()
        check(L.zn_hip_graph_begin(self.handle), "zn_hip_graph_begin")
        h = ctypes.c_void_p()
        try:
            fn()
        except BaseException:
            if L.zn_hip_graph_end(self.handle, ctypes.byref(h)) == _lib.ZN_OK and h:
                L.zn_hip_graph_destroy(h)
            raise
        check(L.zn_hip_graph_end(self.handle, ctypes.byref(h)), "zn_hip_graph_end")
        return Graph(self, h)

    def hold_stream(self, microseconds: float) -> None:
        """Keep the context stream busy for `microseconds` (a timing aid: launches queued behind it run back
        to back on the device)."""
        check(_lib.load().zn_hip_hold_stream(self.handle, float(microseconds)), "zn_hip_hold_stream")

    def copy(self, dst: int, src: int, count: int) -> None:
        check(_lib.load().zn_hip_copy_f32(self.handle, int(dst), int(src), int(count)), "zn_hip_copy_f32")

    def set_gemm_tile(self, tile="auto") -> None:
        """Force one macro tile ("256x128", "128x128", "128x64", "64x64", "32x32", "128x128k32", "64x64k16",
        "256x256") or "auto"."""
        check(_lib.load().zn_hip_set_gemm_tile(self.handle, _lib.TILES[tile] if isinstance(tile, str) else tile),
              "zn_hip_set_gemm_tile")

    def set_gemm_splits(self, splits: int = 0) -> None:
        """Force the number of split-K slices (1..256), or 0 for the policy."""
        check(_lib.load().zn_hip_set_gemm_splits(self.handle, int(splits)), "zn_hip_set_gemm_splits")

    def set_gemm_wave_split(self, waves: int = -1) -> None:
        """-1: the policy decides; 0: never; 4 or 8: every eligible GEMM splits K over that many waves of a workgroup."""
        check(_lib.load().zn_hip_set_gemm_wave_split(self.handle, int(waves)), "zn_hip_set_gemm_wave_split")

    def set_gemm_persistent(self, mode: int = -1) -> None:
        """-1: the policy decides; 0: never; 1: every eligible GEMM runs on the persistent kernels;
        2: the same, with deferred stores wherever they apply (bit-identical in every mode)."""
        check(_lib.load().zn_hip_set_gemm_persistent(self.handle, int(mode)), "zn_hip_set_gemm_persistent")

    # --- GEMM on device pointers (asynchronous on the context stream)
    def sgemm(self, layout, m, n, k, a, lda, b, ldb, c, ldc, accumulate=False, bias=None, act="linear") -> None:
        check(_lib.load().zn_hip_sgemm(self.handle, layout_id(layout), m, n, k, _dptr(a), lda, _dptr(b), ldb,
                                       _dptr(c), ldc, int(bool(accumulate)), _dptr(bias), act_id(act)),
              "zn_hip_sgemm")

    def sgemm_strided_batched(self, layout, m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c,
                              batch, accumulate=False, bias=None, act="linear") -> None:
        check(_lib.load().zn_hip_sgemm_strided_batched(
            self.handle, layout_id(layout), m, n, k, _dptr(a), lda, stride_a, _dptr(b), ldb, stride_b,
            _dptr(c), ldc, stride_c, batch, int(bool(accumulate)), _dptr(bias), act_id(act)),
            "zn_hip_sgemm_strided_batched")

    # --- Dense helpers on device pointers
    def add_bias(self, out, bias, rows, n) -> None:
        check(_lib.load().zn_hip_add_bias(self.handle, _dptr(out), _dptr(bias), rows, n), "zn_hip_add_bias")

    def activation_forward(self, act, inp, out, length) -> None:
        check(_lib.load().zn_hip_activation_forward(self.handle, act_id(act), _dptr(inp), _dptr(out), length),
              "zn_hip_activation_forward")

    def activation_backward(self, act, y, grad_out, grad_in, length) -> None:
        check(_lib.load().zn_hip_activation_backward(self.handle, act_id(act), _dptr(y), _dptr(grad_out),
                                                     _dptr(grad_in), length), "zn_hip_activation_backward")

    def accumulate_bias(self, grad_bias, gaa, rows, n) -> None:
        check(_lib.load().zn_hip_accumulate_bias(self.handle, _dptr(grad_bias), _dptr(gaa), rows, n),
              "zn_hip_accumulate_bias")

    def dense_backward(self, act, inp, weights, activated_output, grad_output, grad_after_act, grad_input,
                       grad_weights, grad_bias, batch, in_size, out_size) -> None:
        """Dense.backward in one call: fused activationBackward + bias-gradient pass, NT, TN
        (grad_input may be None)."""
        check(_lib.load().zn_hip_dense_backward(
            self.handle, act_id(act), _dptr(inp), _dptr(weights), _dptr(activated_output), _dptr(grad_output),
            _dptr(grad_after_act), _dptr(grad_input), _dptr(grad_weights), _dptr(grad_bias), batch, in_size, out_size),
            "zn_hip_dense_backward")

    def dense_backward_chain(self, act, inp, weights, activated_output, grad_output, grad_after_act, grad_input,
                             grad_weights, grad_bias, batch, in_size, out_size, gaa_ready=False, prev_act="linear",
                             prev_activated_output=None, prev_grad_after_act=None) -> None:
        """dense_backward for layers walked top-down: gaa_ready means grad_after_act already holds
        this layer's derivative (written by the layer above's call); prev_grad_after_act (with
        prev_act and prev_activated_output) receives the layer below's derivative from grad_input.
        Bit-identical to dense_backward layer by layer."""
        check(_lib.load().zn_hip_dense_backward_chain(
            self.handle, act_id(act), _dptr(inp), _dptr(weights), _dptr(activated_output), _dptr(grad_output),
            _dptr(grad_after_act), _dptr(grad_input), _dptr(grad_weights), _dptr(grad_bias), batch, in_size, out_size,
            int(bool(gaa_ready)), act_id(prev_act), _dptr(prev_activated_output), _dptr(prev_grad_after_act)),
            "zn_hip_dense_backward_chain")

    def dense_pair_forward(self, act1, x, w1, b1, h, act2, w2, b2, y, batch, in_size, hidden, out_size) -> None:
        """Two stacked Dense forwards, h = act1(x.W1 + b1) then y = act2(h.W2 + b2): one launch
        when the top layer has at most 16 outputs and the lower one is small."""
        check(_lib.load().zn_hip_dense_pair_forward(
            self.handle, act_id(act1), _dptr(x), _dptr(w1), _dptr(b1), _dptr(h), act_id(act2), _dptr(w2), _dptr(b2),
            _dptr(y), batch, in_size, hidden, out_size), "zn_hip_dense_pair_forward")

    def dense_pair_backward(self, act1, x, w1, h, gaa1, grad_x, grad_w1, grad_b1, act2, w2, y, grad_y, gaa2,
                            grad_h, grad_w2, grad_b2, batch, in_size, hidden, out_size) -> None:
        """The backward of the same pair (top layer first), in one launch under the same limits."""
        check(_lib.load().zn_hip_dense_pair_backward(
            self.handle, act_id(act1), _dptr(x), _dptr(w1), _dptr(h), _dptr(gaa1), _dptr(grad_x), _dptr(grad_w1),
            _dptr(grad_b1), act_id(act2), _dptr(w2), _dptr(y), _dptr(grad_y), _dptr(gaa2), _dptr(grad_h),
            _dptr(grad_w2), _dptr(grad_b2), batch, in_size, hidden, out_size), "zn_hip_dense_pair_backward")

    # --- convolution and attention on device pointers
    def im2col(self, inp, col, batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h=1, stride_w=1,
               pad_h=0, pad_w=0) -> None:
        check(_lib.load().zn_hip_im2col(self.handle, _dptr(inp), _dptr(col), batch, channels, in_h, in_w, k_h, k_w,
                                        out_h, out_w, stride_h, stride_w, pad_h, pad_w), "zn_hip_im2col")

    def conv2d_forward_im2col(self, inp, weights, bias, out, batch, in_channels, out_channels, k_h, k_w, in_h,
                              in_w, out_h, out_w, stride_h=1, stride_w=1, pad_h=0, pad_w=0) -> None:
        check(_lib.load().zn_hip_conv2d_forward_im2col(
            self.handle, _dptr(inp), _dptr(weights), _dptr(bias), _dptr(out), batch, in_channels, out_channels, k_h,
            k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w), "zn_hip_conv2d_forward_im2col")

    def conv2d_forward_direct(self, inp, weights, bias, out, batch, in_channels, out_channels, k_h, k_w, in_h,
                              in_w, out_h, out_w, stride_h=1, stride_w=1, pad_h=0, pad_w=0) -> None:
        """Implicit-GEMM convolution with W as [OC][C][kH][kW] (true NCHW convolution)."""
        check(_lib.load().zn_hip_conv2d_forward_direct(
            self.handle, _dptr(inp), _dptr(weights), _dptr(bias), _dptr(out), batch, in_channels, out_channels, k_h,
            k_w, in_h, in_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w), "zn_hip_conv2d_forward_direct")

    def col2im(self, col, out, batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, stride_h=1, stride_w=1,
               pad_h=0, pad_w=0) -> None:
        """Backend.col2im on device (bit-identical to the reference); `out` is overwritten."""
        check(_lib.load().zn_hip_col2im(self.handle, _dptr(col), _dptr(out), batch, channels, in_h, in_w, k_h, k_w,
                                        out_h, out_w, stride_h, stride_w, pad_h, pad_w), "zn_hip_col2im")

    def conv2d_backward_im2col(self, inp, weights, grad_output, grad_input, grad_weights, grad_bias, batch,
                               in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h=1, stride_w=1,
                               pad_h=0, pad_w=0) -> None:
        """cpuConv2dBackwardIm2col on device (grad_output read as [batch*OH*OW][OC] by the GEMMs)."""
        check(_lib.load().zn_hip_conv2d_backward_im2col(
            self.handle, _dptr(inp), _dptr(weights), _dptr(grad_output), _dptr(grad_input), _dptr(grad_weights),
            _dptr(grad_bias), batch, in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w,
            pad_h, pad_w), "zn_hip_conv2d_backward_im2col")

    def conv2d_backward_direct(self, inp, weights, grad_output, grad_input, grad_weights, grad_bias, batch,
                               in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h=1, stride_w=1,
                               pad_h=0, pad_w=0) -> None:
        """The direct branch of cpuConv2dBackward on device (NCHW, OIHW)."""
        check(_lib.load().zn_hip_conv2d_backward_direct(
            self.handle, _dptr(inp), _dptr(weights), _dptr(grad_output), _dptr(grad_input), _dptr(grad_weights),
            _dptr(grad_bias), batch, in_channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, stride_h, stride_w,
            pad_h, pad_w), "zn_hip_conv2d_backward_direct")

    def softmax_rows(self, inp, out, rows, n, scale=1.0) -> None:
        check(_lib.load().zn_hip_softmax_rows(self.handle, _dptr(inp), _dptr(out), rows, n, float(scale)),
              "zn_hip_softmax_rows")

    def attention_forward(self, q, k, v, out, batch, seq_len, d_k, scale) -> None:
        check(_lib.load().zn_hip_attention_forward(self.handle, _dptr(q), _dptr(k), _dptr(v), _dptr(out), batch,
                                                   seq_len, d_k, float(scale)), "zn_hip_attention_forward")

    def close(self) -> None:
        if self.handle:
            for g in list(self._graphs):  # zn_hip_destroy releases them
                g.handle = None
            _lib.load().zn_hip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


def _dptr(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


class Backend:
    """ZigNeuron ``Backend`` (src/backend.zig:15-325) with the HIP arm.

    Methods take host float32 arrays (the Zig slices) and write outputs in
    place; they return when the result is in host memory, like the
    reference's synchronous CUDA arms (src/cuda.zig:617).
    """

    def __init__(self, ctx: Context):
        self.ctx = ctx

    @classmethod
    def init(cls, device: int = 0) -> "Backend":
        """Backend.init + detect (src/backend.zig:43-94) with the HIP arm: raises
        NoDeviceError when no gfx950 device is present (no CPU fallback here)."""
        return cls(Context(device))

    def deinit(self) -> None:
        self.ctx.close()

    @property
    def _h(self):
        return self.ctx.handle

    # --- GEMM family
    def _gemm(self, fn, a, b, c, m, n, k, accumulate):
        a, b, c = _f32_in(a), _f32_in(b), _f32_out(c)
        check(fn(self._h, _ptr(a), a.size, _ptr(b), b.size, _ptr(c), c.size, m, n, k, int(bool(accumulate))),
              fn.__name__)

    def matMul(self, a, b, c, m, n, k, accumulate=False):
        """Backend.matMul (src/backend.zig:169-182): C (+)= A[m x k] . B[k x n]."""
        self._gemm(_lib.load().zn_hip_mat_mul, a, b, c, m, n, k, accumulate)

    def matMulBatch(self, a, b, c, batch_size, n, k, accumulate=False):
        """Backend.matMulBatch (src/backend.zig:186-195)."""
        self._gemm(_lib.load().zn_hip_mat_mul_batch, a, b, c, batch_size, n, k, accumulate)

    def matMulTransposeA(self, a, b, c, m, n, k, accumulate=False):
        """Backend.matMulTransposeA (src/backend.zig:298-307): C (+)= A^T . B, A is [k x m]."""
        self._gemm(_lib.load().zn_hip_mat_mul_transpose_a, a, b, c, m, n, k, accumulate)

    def matMulTransposeB(self, a, b, c, m, n, k, accumulate=False):
        """Backend.matMulTransposeB (src/backend.zig:310-325): C (+)= A . B^T, B is [n x k]."""
        self._gemm(_lib.load().zn_hip_mat_mul_transpose_b, a, b, c, m, n, k, accumulate)

    def _bias_gemm(self, fn, a, b, bias, c, batch_size, n, k):
        a, b, bias, c = _f32_in(a), _f32_in(b), _f32_in(bias), _f32_out(c)
        check(fn(self._h, _ptr(a), a.size, _ptr(b), b.size, _ptr(bias), bias.size, _ptr(c), c.size,
                 batch_size, n, k), fn.__name__)

    def matMulBias(self, a, b, bias, c, batch_size, n, k):
        """Backend.matMulBias (src/backend.zig:200-222)."""
        self._bias_gemm(_lib.load().zn_hip_mat_mul_bias, a, b, bias, c, batch_size, n, k)

    def matMulBiasRelu(self, a, b, bias, c, batch_size, n, k):
        """Backend.matMulBiasRelu (src/backend.zig:225-247)."""
        self._bias_gemm(_lib.load().zn_hip_mat_mul_bias_relu, a, b, bias, c, batch_size, n, k)

    def matMulBiasSigmoid(self, a, b, bias, c, batch_size, n, k):
        """Backend.matMulBiasSigmoid (src/backend.zig:250-272)."""
        self._bias_gemm(_lib.load().zn_hip_mat_mul_bias_sigmoid, a, b, bias, c, batch_size, n, k)

    def matMulBiasTanh(self, a, b, bias, c, batch_size, n, k):
        """Backend.matMulBiasTanh (src/backend.zig:275-295)."""
        self._bias_gemm(_lib.load().zn_hip_mat_mul_bias_tanh, a, b, bias, c, batch_size, n, k)

    # --- Dense epilogue / backward helpers
    def addBias(self, output, bias):
        """Backend.addBias (src/backend.zig:658-671)."""
        out, bias = _f32_out(output), _f32_in(bias)
        check(_lib.load().zn_hip_add_bias_host(self._h, _ptr(out), out.size, _ptr(bias), bias.size),
              "zn_hip_add_bias_host")

    def activationForward(self, act, inp, output):
        """Backend.activationForward (src/backend.zig:367-386)."""
        inp, out = _f32_in(inp), _f32_out(output)
        check(_lib.load().zn_hip_activation_forward_host(self._h, act_id(act), _ptr(inp), inp.size, _ptr(out),
                                                         out.size), "zn_hip_activation_forward_host")

    def activationBackward(self, act, inp, grad_output, grad_input):
        """Backend.activationBackward (src/backend.zig:390-399); `inp` is the activated output."""
        y, go, gi = _f32_in(inp), _f32_in(grad_output), _f32_out(grad_input)
        check(_lib.load().zn_hip_activation_backward_host(self._h, act_id(act), _ptr(y), y.size, _ptr(go),
                                                          go.size, _ptr(gi), gi.size),
              "zn_hip_activation_backward_host")

    def accumulateBias(self, grad_bias, grad_after_act):
        """Backend.accumulateBias (src/backend.zig:649-655)."""
        gb, gaa = _f32_out(grad_bias), _f32_in(grad_after_act)
        check(_lib.load().zn_hip_accumulate_bias_host(self._h, _ptr(gb), gb.size, _ptr(gaa), gaa.size),
              "zn_hip_accumulate_bias_host")

    # --- convolution and attention
    def conv2dForward(self, inp, weights, bias, output, in_channels, out_channels, kernel_h, kernel_w, input_h,
                      input_w, output_h, output_w, stride_h, stride_w, padding_h, padding_w):
        """Backend.conv2dForward (src/backend.zig:507-518), NCHW, batch = len(input) / (C*H*W)."""
        x, w, b, out = _f32_in(inp), _f32_in(weights), _f32_in(bias), _f32_out(output)
        check(_lib.load().zn_hip_conv2d_forward_host(
            self._h, _ptr(x), x.size, _ptr(w), w.size, _ptr(b), b.size, _ptr(out), out.size, in_channels,
            out_channels, kernel_h, kernel_w, input_h, input_w, output_h, output_w, stride_h, stride_w, padding_h,
            padding_w), "zn_hip_conv2d_forward_host")

    def conv2dBackward(self, inp, weights, grad_output, grad_input, grad_weights, grad_bias, in_channels,
                       out_channels, kernel_h, kernel_w, input_h, input_w, output_h, output_w, stride_h, stride_w,
                       padding_h, padding_w):
        """Backend.conv2dBackward (src/backend.zig:520, :3049-3095), batch = len(input) / (C*H*W)."""
        x, w, go = _f32_in(inp), _f32_in(weights), _f32_in(grad_output)
        gi, gw, gb = _f32_out(grad_input), _f32_out(grad_weights), _f32_out(grad_bias)
        check(_lib.load().zn_hip_conv2d_backward_host(
            self._h, _ptr(x), x.size, _ptr(w), w.size, _ptr(go), go.size, _ptr(gi), gi.size, _ptr(gw), gw.size,
            _ptr(gb), gb.size, in_channels, out_channels, kernel_h, kernel_w, input_h, input_w, output_h, output_w,
            stride_h, stride_w, padding_h, padding_w), "zn_hip_conv2d_backward_host")

    def attentionForward(self, q, k, v, output, scores_buffer, seq_len, d_k, scaling_factor):
        """Backend.attentionForward (src/backend.zig:631-638), one head [seq_len x d_k]."""
        q, k, v, out = _f32_in(q), _f32_in(k), _f32_in(v), _f32_out(output)
        sc = _f32_out(scores_buffer)
        check(_lib.load().zn_hip_attention_forward_host(
            self._h, _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size, _ptr(out), out.size, _ptr(sc), sc.size,
            seq_len, d_k, float(scaling_factor)), "zn_hip_attention_forward_host")

"""Host-side bookkeeping of DenseDevice's chained backward, with a stand-in
context that records the calls instead of launching kernels (no device).

The chained backward of a layer writes the layer below's derivative
(below.gaa) and marks it ready; the lower layer's own backward then reads it
instead of its grad_out.  A new forward starts a new step, so the mark must
not survive it, and a grad_out handed to a layer whose derivative is already
written is refused rather than silently ignored."""
from __future__ import annotations

import numpy as np
import pytest

from zigneuron_amd import _lib
from zigneuron_amd.layer import DenseDevice


class _Buf:
    def __init__(self, n):
        self.n = n

    def fill(self, value):
        return self


class _Ctx:
    """Records the device calls DenseDevice makes."""

    def __init__(self):
        self.calls = []

    def to_device(self, host):
        return _Buf(np.asarray(host).size)

    def alloc(self, n):
        return _Buf(n)

    def sgemm(self, *args, **kw):
        self.calls.append(("sgemm", args[0]))

    def dense_backward(self, *args):
        self.calls.append(("dense_backward", args[4]))

    def dense_backward_chain(self, *args):
        # args[4] is grad_out (None when the derivative is ready), args[12] `ready`
        self.calls.append(("dense_backward_chain", args[4], args[12]))


def _pair():
    ctx = _Ctx()
    lower = DenseDevice(ctx, 8, 6, "relu", 4, seed=1)
    upper = DenseDevice(ctx, 6, 3, "sigmoid", 4, seed=2)
    return ctx, lower, upper


def test_chained_backward_marks_the_lower_derivative_ready():
    ctx, lower, upper = _pair()
    x, go = _Buf(32), _Buf(12)
    upper.backward(lower.out, go, below=lower)
    assert lower._gaa_ready
    lower.backward(x, None)
    assert ctx.calls[-1] == ("dense_backward_chain", None, True)
    assert not lower._gaa_ready


def test_forward_clears_a_stale_derivative():
    """A backward chained into `lower`, then a new forward: the next
    backward of `lower` must read its grad_out again."""
    ctx, lower, upper = _pair()
    x, go, go_low = _Buf(32), _Buf(12), _Buf(24)
    upper.backward(lower.out, go, below=lower)
    assert lower._gaa_ready
    lower.forward(x)
    assert not lower._gaa_ready
    lower.backward(x, go_low)
    assert ctx.calls[-1] == ("dense_backward", go_low)


def test_grad_out_refused_while_the_derivative_is_ready():
    ctx, lower, upper = _pair()
    x, go = _Buf(32), _Buf(12)
    upper.backward(lower.out, go, below=lower)
    with pytest.raises(_lib.InvalidArgumentError):
        lower.backward(x, _Buf(24))
    with pytest.raises(_lib.InvalidArgumentError):
        lower.backward(x, None, fused=False)

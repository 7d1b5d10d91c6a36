"""GPU parity of the two-layer Dense launches (zn_hip_dense_pair_forward /
_backward) against the oracle, through the C ABI.

Every output of both layers is checked on each case:
  * h and y against the oracle's fused GEMM (Backend.matMulBias*) on the
    GPU's own inputs, within 1e-5*sqrt(K) (plus 4 ulp for sigmoid and tanh);
  * gaa2 = activationBackward(act2, y, grad_y) and gaa1 =
    activationBackward(act1, h, grad_h) bit for bit (the fused kernel
    generates gaa1 wherever it is needed from the grad_h it writes);
  * grad_h = gaa2 . W2^T, grad_x, grad_w1 and grad_w2 within the tolerance,
    the bias gradients within it on top of a non-zero start.
The unfused cases (a head wider than 16, a lower layer of more 16x16 tiles
than CUs, a forced per-layer path) take the per-layer launches and must
agree with the fused ones to the same bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from _parity import tol, uniform
from gpu_common import THREADS, announce, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.close()


# batch, in, hidden, out, act1, act2, forward fused, backward fused
CASES = [
    (256, 784, 128, 10, "relu", "linear", True, True),      # C2
    (256, 784, 128, 10, "tanh", "sigmoid", True, True),
    (100, 77, 50, 7, "tanh", "sigmoid", True, True),          # 4-byte staging, ragged tiles
    (300, 64, 96, 16, "sigmoid", "tanh", True, True),         # two 256-row passes of the column sums
    (1, 5, 3, 1, "relu", "relu", True, True),
    (33, 1000, 40, 12, "linear", "relu", True, True),
    (513, 40, 1024, 3, "relu", "linear", False, True),        # 2112 tiles of 16x16: per-layer forward
    (256, 784, 128, 20, "relu", "linear", False, False),      # a head wider than 16
    (1024, 64, 64, 10, "relu", "linear", True, True),         # 4 passes of the column sums
]


def _run(ctx, batch, d_in, d_h, d_out, act1, act2, seed, grad_x=True, per_layer=False):
    from zigneuron_amd import DenseDevice, pair_backward, pair_forward
    rng = np.random.default_rng(seed)
    x = uniform(rng, (batch, d_in), 0.0, 1.0)
    dy = uniform(rng, (batch, d_out))
    l1 = DenseDevice(ctx, d_in, d_h, act1, batch, bias=uniform(rng, (d_h,), -0.1, 0.1), seed=seed + 1)
    l2 = DenseDevice(ctx, d_h, d_out, act2, batch, bias=uniform(rng, (d_out,), -0.1, 0.1), seed=seed + 2)
    gb1, gb2 = uniform(rng, (d_h,)), uniform(rng, (d_out,))
    l1.grad_bias.upload(gb1)
    l2.grad_bias.upload(gb2)
    dx, ddy = ctx.to_device(x), ctx.to_device(dy)
    if per_layer:
        ctx.set_gemm_wave_split(0)  # a forced path: the per-layer launches
    try:
        pair_forward(l1, l2, dx)
        pair_backward(l1, l2, dx, ddy, grad_input=grad_x)
    finally:
        if per_layer:
            ctx.set_gemm_wave_split(-1)
    ctx.sync()
    out = {"x": x, "dy": dy, "gb1": gb1, "gb2": gb2,
           "W1": l1.weights.download().reshape(d_in, d_h), "b1": l1.bias.download(),
           "W2": l2.weights.download().reshape(d_h, d_out), "b2": l2.bias.download(),
           "H": l1.out.download().reshape(batch, d_h), "Y": l2.out.download().reshape(batch, d_out),
           "gaa2": l2.gaa.download().reshape(batch, d_out), "GH": l2.grad_input.download().reshape(batch, d_h),
           "gaa1": l1.gaa.download().reshape(batch, d_h), "dW1": l1.grad_weights.download().reshape(d_in, d_h),
           "dW2": l2.grad_weights.download().reshape(d_h, d_out), "db1": l1.grad_bias.download(),
           "db2": l2.grad_bias.download()}
    if grad_x:
        out["GX"] = l1.grad_input.download().reshape(batch, d_in)
    return out


def _check_bias(got, start, gaa, what):
    ref = oracle.accumulate_bias(start, gaa)
    den = np.abs(start.astype(np.float64)) + np.abs(gaa.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= tol(gaa.shape[0]) * den), what


def _check(r, batch, d_in, d_h, d_out, act1, act2, fwd_fused, bwd_fused):
    x, dy, W1, W2, b1, b2 = r["x"], r["dy"], r["W1"], r["W2"], r["b1"], r["b2"]
    H, Y = r["H"], r["Y"]
    assert_close(H, oracle.matmul_bias_act(x, W1, b1, batch, d_h, d_in, act1), "nn", x, W1, batch, d_h, d_in,
                 bias=b1, act=act1, what="h")
    Y_ref = oracle.matmul_bias_act(H, W2, b2, batch, d_out, d_h, act2)
    assert_close(Y, Y_ref, "nn", H, W2, batch, d_out, d_h, bias=b2, act=act2, what="y")
    gaa2 = r["gaa2"]
    np.testing.assert_array_equal(gaa2, oracle.activation_backward(act2, Y, dy).reshape(batch, d_out))
    GH_ref = oracle.matmul_nt(gaa2, W2, batch, d_h, d_out)
    assert_close(r["GH"], GH_ref, "nt", gaa2, W2, batch, d_h, d_out, what="grad_h")
    gaa1 = r["gaa1"]
    np.testing.assert_array_equal(gaa1, oracle.activation_backward(act1, H, r["GH"]).reshape(batch, d_h))
    assert_close(r["dW2"], oracle.matmul_tn(H, gaa2, d_h, d_out, batch), "tn", H, gaa2, d_h, d_out, batch,
                 what="grad_w2")
    assert_close(r["dW1"], oracle.matmul_tn(x, gaa1, d_in, d_h, batch, threads=THREADS), "tn", x, gaa1, d_in, d_h,
                 batch, what="grad_w1")
    if "GX" in r:
        assert_close(r["GX"], oracle.matmul_nt(gaa1, W1, batch, d_in, d_h, threads=THREADS), "nt", gaa1, W1, batch,
                     d_in, d_h, what="grad_x")
    _check_bias(r["db2"], r["gb2"], gaa2, "grad_b2")
    _check_bias(r["db1"], r["gb1"], gaa1, "grad_b1")


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:4])) + f"-{c[4]}-{c[5]}")
def test_pair_against_oracle(ctx, case):
    batch, d_in, d_h, d_out, act1, act2, ff, bf = case
    announce(f"pair {case}")
    r = _run(ctx, batch, d_in, d_h, d_out, act1, act2, seed=batch + d_in)
    _check(r, batch, d_in, d_h, d_out, act1, act2, ff, bf)


def test_pair_without_grad_x(ctx):
    """The first layer of a network: grad_x skipped (no NT workgroups)."""
    announce("pair without grad_x")
    r = _run(ctx, 256, 784, 128, 10, "relu", "linear", seed=11, grad_x=False)
    assert "GX" not in r
    _check(r, 256, 784, 128, 10, "relu", "linear", True, True)


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3]], ids=["c2", "ragged", "two-pass"])
def test_pair_matches_per_layer_launches(ctx, case):
    """The per-layer launches (forced, on the same inputs) meet the same bar
    as the fused ones, and both agree within the tolerance on each layer's
    derivative-free outputs."""
    batch, d_in, d_h, d_out, act1, act2, ff, bf = case
    announce(f"pair vs per-layer {case}")
    fused = _run(ctx, batch, d_in, d_h, d_out, act1, act2, seed=5)
    plain = _run(ctx, batch, d_in, d_h, d_out, act1, act2, seed=5, per_layer=True)
    _check(fused, batch, d_in, d_h, d_out, act1, act2, ff, bf)
    _check(plain, batch, d_in, d_h, d_out, act1, act2, False, False)
    x, W1 = fused["x"], fused["W1"]
    assert_close(fused["H"], plain["H"], "nn", x, W1, batch, d_h, d_in, bias=fused["b1"], act=act1,
                 what="h, fused against per-layer")


def test_pair_repeats_bit_identical(ctx):
    """Deterministic: the same inputs give the same bits (counters reset by
    each launch; the bias sums run in a fixed order)."""
    announce("pair determinism")
    a = _run(ctx, 256, 784, 128, 10, "relu", "linear", seed=3)
    b = _run(ctx, 256, 784, 128, 10, "relu", "linear", seed=3)
    for key in a:
        np.testing.assert_array_equal(a[key], b[key], err_msg=key)


def test_pair_argument_errors(ctx):
    from zigneuron_amd import InvalidArgumentError
    announce("pair argument errors")
    buf = ctx.alloc(64)
    with pytest.raises(InvalidArgumentError):  # a Dense layer has at least one output (Dense.init)
        ctx.dense_pair_forward("relu", buf, buf, None, buf, "linear", buf, None, buf, 4, 4, 4, 0)
    with pytest.raises(InvalidArgumentError):
        ctx.dense_pair_forward("relu", None, buf, None, buf, "linear", buf, None, buf, 4, 4, 4, 2)
    with pytest.raises(InvalidArgumentError):  # y is needed for a non-linear head's derivative
        ctx.dense_pair_backward("relu", buf, buf, buf, buf, None, buf, buf, "sigmoid", buf, None, buf, buf, buf,
                                buf, buf, 4, 4, 4, 2)
    buf.close()

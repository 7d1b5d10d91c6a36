"""Pins the CPU oracle (oracle/cpu_gemm.c) before it is trusted as the checker.

Each check is independent of the restatement being tested: the reference's
own known-answer tests, exact integer arithmetic (numpy int64 matmul), the
transpose identities linking NN/TN/NT, a vectorised float32 statement of the
sequential-K definition, fp64 error bounds, and closed forms for epilogues,
im2col and attention.  `test_checks_catch_planted_mistakes` plants plausible
mistakes in oracle outputs (on the CPU) and shows these checks reject them.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import oracle
from _parity import uniform, tol, abs_denominator, componentwise_error

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
U = np.float64(2.0 ** -24)


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build()


@pytest.fixture(scope="module")
def kats():
    return np.load(os.path.join(GOLDEN, "reference_kats.npz"))


def seq_nn(a, b, c0=None):
    """Vectorised float32 statement of the sequential definition: for p
    ascending, C = fl(C + fl(a[:,p] * b[p,:])) (numpy float32 ops are single
    IEEE operations, never fused)."""
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n), np.float32) if c0 is None else c0.copy()
    for p in range(k):
        c = (c + (a[:, p:p + 1] * b[p:p + 1, :]).astype(np.float32)).astype(np.float32)
    return c


def gamma_bound(a, b, k):
    """Deterministic fp32 summation bound gamma_k (|A||B|), gamma_k = k u / (1 - k u)."""
    g = k * U / (1 - k * U)
    return g * abs_denominator(a, b)


# ---------------------------------------------------------------- reference KATs
def test_kat_backend_matmul_correctness(kats):
    m, n, k = kats["correctness_mnk"]
    c = oracle.matmul_batch(kats["correctness_a"], kats["correctness_b"], m, n, k)
    np.testing.assert_array_equal(c.ravel(), kats["correctness_c"])


def test_kat_backend_matmul_large_ones(kats):
    ones = np.ones(64 * 64, np.float32)
    for branch in ("auto", "unblocked", "blocked"):
        c = oracle.matmul(ones, ones, 64, 64, 64, branch=branch)
        np.testing.assert_array_equal(c.ravel(), kats["ones64_c"])
    np.testing.assert_array_equal(oracle.matmul_batch(ones, ones, 64, 64, 64).ravel(), kats["ones64_c"])


def test_kat_backend_matmul_cpu_small(kats):
    m, n, k = kats["cpu_small_mnk"]
    c = oracle.matmul_batch(kats["cpu_small_a"], kats["cpu_small_b"], m, n, k)
    assert c.ravel()[0] == kats["cpu_small_c0"][0]


@pytest.mark.parametrize("tag", ["small64", "medium256", "nonsquare", "accum64"])
def test_kat_integer_matmuls_exact_every_layout(kats, tag):
    m, n, k = (int(x) for x in kats[f"{tag}_mnk"])
    a, b = kats[f"{tag}_a"].reshape(m, k), kats[f"{tag}_b"].reshape(k, n)
    want = kats[f"{tag}_c"].reshape(m, n)
    if tag == "accum64":  # first call overwrites, second accumulates
        c = oracle.matmul(a, b, m, n, k)
        c = oracle.matmul(a, b, m, n, k, accumulate=True, c_init=c)
        np.testing.assert_array_equal(c, 2 * want)
        return
    np.testing.assert_array_equal(oracle.matmul(a, b, m, n, k), want)
    np.testing.assert_array_equal(oracle.matmul(a, b, m, n, k, branch="unblocked"), want)
    np.testing.assert_array_equal(oracle.matmul_batch(a, b, m, n, k), want)
    np.testing.assert_array_equal(oracle.matmul_tn(a.T.copy(), b, m, n, k), want)
    np.testing.assert_array_equal(oracle.matmul_nt(a, b.T.copy(), m, n, k), want)


def test_kat_dense_layer_forward_backward(kats):
    """src/test/unit/layer.zig:16-55,169-241 through the oracle's Dense steps."""
    for act, row in zip(kats["dense_fwd_act"], kats["dense_fwd"]):
        w0, w1, bias, x0, x1, want = row
        y = oracle.matmul_batch(np.float32([x0, x1]), np.float32([w0, w1]), 1, 1, 2)
        y = oracle.add_bias(y, np.float32([bias]))
        y = oracle.activation_forward(str(act), y)
        assert abs(float(y[0, 0]) - float(want)) <= 1e-4
    for act, row in zip(kats["dense_bwd_act"], kats["dense_bwd"]):
        w0, w1, x0, x1, yv, g0, g1 = row
        gaa = oracle.activation_backward(str(act), np.float32([yv]), np.float32([1.0]))
        gx = oracle.matmul_nt(gaa, np.float32([w0, w1]), 1, 2, 1)
        np.testing.assert_allclose(gx.ravel(), [g0, g1], atol=1e-4)


def test_kat_activations(kats):
    x = kats["act_relu_x"]
    np.testing.assert_array_equal(oracle.activation_forward("relu", x), kats["act_relu_y"])
    s = oracle.activation_forward("sigmoid", kats["act_sigmoid_x"])
    assert np.all((s >= 0) & (s <= 1)) and abs(float(s[2]) - 0.5) <= 1e-4
    g = oracle.activation_backward("sigmoid", s, np.ones_like(s))
    np.testing.assert_allclose(g, s * (1 - s), atol=1e-4)


# ------------------------------------------------------------ structural checks
SHAPES = [(1, 1, 1), (3, 5, 7), (31, 33, 32), (32, 32, 32), (37, 45, 29), (64, 96, 70), (70, 33, 129)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_branches_and_layouts_bit_identical(m, n, k):
    rng = np.random.default_rng(m * 10007 + n * 101 + k)
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    ref = seq_nn(a, b)
    for branch in ("auto", "unblocked", "blocked"):
        np.testing.assert_array_equal(oracle.matmul(a, b, m, n, k, branch=branch), ref)
    np.testing.assert_array_equal(oracle.matmul(a, b, m, n, k, branch="blocked", threads=4), ref)
    np.testing.assert_array_equal(oracle.matmul_batch(a, b, m, n, k), ref)
    # C = A B computed as (A^T)^T B and A (B^T)^T: same products, same order.
    np.testing.assert_array_equal(oracle.matmul_tn(a.T.copy(), b, m, n, k), ref)
    np.testing.assert_array_equal(oracle.matmul_nt(a, b.T.copy(), m, n, k), ref)
    np.testing.assert_array_equal(oracle.matmul_tn(a.T.copy(), b, m, n, k, threads=3), ref)
    np.testing.assert_array_equal(oracle.matmul_nt(a, b.T.copy(), m, n, k, threads=3), ref)


@pytest.mark.parametrize("m,n,k", [(5, 6, 7), (40, 33, 35)])
def test_accumulate_semantics(m, n, k):
    """NN accumulates in sequence into C (src/backend.zig:2521); TN/NT form the
    sum from zero and then add it (src/backend.zig:2623-2627, 2640-2644)."""
    rng = np.random.default_rng(7)
    a, b, c0 = uniform(rng, (m, k)), uniform(rng, (k, n)), uniform(rng, (m, n))
    np.testing.assert_array_equal(oracle.matmul(a, b, m, n, k, True, c0), seq_nn(a, b, c0))
    np.testing.assert_array_equal(oracle.matmul_batch(a, b, m, n, k, True, c0), seq_nn(a, b, c0))
    want = (c0 + seq_nn(a, b)).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_tn(a.T.copy(), b, m, n, k, True, c0), want)
    np.testing.assert_array_equal(oracle.matmul_nt(a, b.T.copy(), m, n, k, True, c0), want)


@pytest.mark.parametrize("m,n,k", [(16, 16, 16), (50, 70, 300), (8, 9, 2000)])
def test_fp64_error_bound(m, n, k):
    rng = np.random.default_rng(k)
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    c = oracle.matmul(a, b, m, n, k).astype(np.float64)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.all(np.abs(c - exact) <= gamma_bound(a, b, k))


def test_identity_and_linearity():
    rng = np.random.default_rng(3)
    a = uniform(rng, (40, 40))
    eye = np.eye(40, dtype=np.float32)
    np.testing.assert_array_equal(oracle.matmul(a, eye, 40, 40, 40), a)
    np.testing.assert_array_equal(oracle.matmul(eye, a, 40, 40, 40), a)
    # scaling by a power of two is exact in every step
    b = uniform(rng, (40, 40))
    np.testing.assert_array_equal(oracle.matmul(a * 4, b, 40, 40, 40), 4 * oracle.matmul(a, b, 40, 40, 40))


# ----------------------------------------------------------------- epilogues
def test_epilogue_closed_forms():
    rng = np.random.default_rng(11)
    m, n, k = 23, 17, 41
    a, b, bias = uniform(rng, (m, k)), uniform(rng, (k, n)), uniform(rng, (n,))
    pre = (seq_nn(a, b) + bias[None, :]).astype(np.float32)  # bias after the full K sum
    np.testing.assert_array_equal(oracle.matmul_bias_act(a, b, bias, m, n, k, "linear"), pre)
    np.testing.assert_array_equal(oracle.matmul_bias_act(a, b, bias, m, n, k, "relu"), np.maximum(pre, 0))
    p64 = pre.astype(np.float64)
    sig = oracle.matmul_bias_act(a, b, bias, m, n, k, "sigmoid")
    assert np.all(np.abs(sig - 1 / (1 + np.exp(-p64))) <= 4 * np.spacing(np.abs(sig)))
    th = oracle.matmul_bias_act(a, b, bias, m, n, k, "tanh")
    assert np.all(np.abs(th - np.tanh(p64)) <= 4 * np.spacing(np.abs(th)) + 1e-45)


def test_activation_forward_backward_closed_forms():
    x = np.linspace(-30, 30, 2001).astype(np.float32)
    x64 = x.astype(np.float64)
    s = oracle.activation_forward("sigmoid", x)
    assert np.all(np.abs(s - 1 / (1 + np.exp(-x64))) <= 4 * np.spacing(np.abs(s)))
    t = oracle.activation_forward("tanh", x)
    assert np.all(np.abs(t - np.tanh(x64)) <= 4 * np.spacing(np.abs(t)) + 1e-45)
    np.testing.assert_array_equal(oracle.activation_forward("relu", x), np.maximum(x, 0))
    np.testing.assert_array_equal(oracle.activation_forward("linear", x), x)
    g = np.linspace(-2, 2, x.size).astype(np.float32)
    np.testing.assert_array_equal(oracle.activation_backward("relu", x, g), np.where(x > 0, g, 0).astype(np.float32))
    np.testing.assert_array_equal(oracle.activation_backward("tanh", t, g), (g * (1 - t * t)).astype(np.float32))
    np.testing.assert_array_equal(oracle.activation_backward("sigmoid", s, g), ((g * s) * (1 - s)).astype(np.float32))
    np.testing.assert_array_equal(oracle.activation_backward("linear", s, g), g)


def test_bias_helpers():
    rng = np.random.default_rng(5)
    out, bias = uniform(rng, (7, 9)), uniform(rng, (9,))
    np.testing.assert_array_equal(oracle.add_bias(out, bias), (out + bias[None, :]).astype(np.float32))
    gb0 = uniform(rng, (9,))
    want = gb0.copy()
    for r in range(7):  # rows accumulate in batch order
        want = (want + out[r]).astype(np.float32)
    np.testing.assert_array_equal(oracle.accumulate_bias(gb0, out), want)


# ------------------------------------------------------ im2col, conv, attention
def test_im2col_conv_matches_direct_convolution():
    rng = np.random.default_rng(21)
    B, C, H, W, OC, KH, KW, pad, stride = 2, 3, 6, 5, 4, 3, 3, 1, 1
    x = uniform(rng, (B, C, H, W))
    col = oracle.im2col(x, B, C, H, W, KH, KW, stride=stride, pad=pad)
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    assert col.shape == (B * OH * OW, KH * KW * C)
    w_oihw = uniform(rng, (OC, C, KH, KW))
    w_col = np.ascontiguousarray(w_oihw.transpose(0, 2, 3, 1).reshape(OC, KH * KW * C))  # (kh,kw,ic) order
    bias = uniform(rng, (OC,))
    out = oracle.conv2d_im2col_gemm(col, w_col, bias, B, OC, OH * OW, KH * KW * C)
    xp = np.pad(x.astype(np.float64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    ref = np.zeros((B, OC, OH, OW))
    for oh in range(OH):
        for ow in range(OW):
            patch = xp[:, :, oh * stride:oh * stride + KH, ow * stride:ow * stride + KW]
            ref[:, :, oh, ow] = np.einsum("bchw,ochw->bo", patch, w_oihw.astype(np.float64))
    ref += bias[None, :, None, None]
    assert np.abs(out.reshape(B, OC, OH, OW) - ref).max() <= 1e-5
    # the GEMM contract is C = col . W^T (NT): compare against the NT oracle + bias
    nt = oracle.matmul_nt(col, w_col, B * OH * OW, OC, KH * KW * C) + bias[None, :]
    gemm = out.transpose(0, 2, 1).reshape(B * OH * OW, OC)
    assert np.abs(gemm - nt).max() <= 1e-5


def _ints(rng, shape, lo=-3, hi=4):
    """Small integers as float32: every sum below is exact in fp32."""
    return rng.integers(lo, hi, size=shape).astype(np.float32)


@pytest.mark.parametrize("geo", [(2, 3, 6, 5, 3, 3, 1, 1), (1, 2, 7, 7, 2, 3, 2, 1), (2, 4, 5, 6, 1, 1, 1, 0),
                                 (1, 1, 9, 8, 4, 2, 3, 2)])
def test_col2im_is_the_adjoint_of_im2col(geo):
    """<im2col(x), c> = <x, col2im(c)> exactly (integer data), and
    col2im(im2col(x)) = x times the number of windows covering each pixel."""
    B, C, H, W, KH, KW, stride, pad = geo
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    rng = np.random.default_rng(sum(geo))
    x = _ints(rng, (B, C, H, W))
    c = _ints(rng, (B * OH * OW, KH * KW * C))
    lhs = int((oracle.im2col(x, B, C, H, W, KH, KW, stride, pad).astype(np.int64) * c.astype(np.int64)).sum())
    rhs = int((x.astype(np.int64) * oracle.col2im(c, B, C, H, W, KH, KW, stride, pad).astype(np.int64)).sum())
    assert lhs == rhs
    cover = np.zeros((H, W), np.int64)
    for oh in range(OH):
        for ow in range(OW):
            for kh in range(KH):
                for kw in range(KW):
                    ih, iw = oh * stride - pad + kh, ow * stride - pad + kw
                    if 0 <= ih < H and 0 <= iw < W:
                        cover[ih, iw] += 1
    back = oracle.col2im(oracle.im2col(x, B, C, H, W, KH, KW, stride, pad), B, C, H, W, KH, KW, stride, pad)
    np.testing.assert_array_equal(back, x * cover[None, None].astype(np.float32))


@pytest.mark.parametrize("geo", [(2, 3, 6, 5, 4, 3, 3, 1, 1), (1, 2, 7, 6, 3, 2, 2, 2, 0), (2, 3, 5, 5, 2, 1, 1, 1, 0)])
def test_conv_backward_direct_is_the_adjoint_of_the_forward(geo):
    """Direct branch (NCHW, OIHW): with integer data, <conv(x, w), g> equals
    <x, grad_input> and <w, grad_weights>; grad_bias = the sum of g over b, h, w."""
    B, C, H, W, OC, KH, KW, stride, pad = geo
    OH, OW = (H + 2 * pad - KH) // stride + 1, (W + 2 * pad - KW) // stride + 1
    rng = np.random.default_rng(sum(geo) + 1)
    x, w, g = _ints(rng, (B, C, H, W)), _ints(rng, (OC, C, KH, KW)), _ints(rng, (B, OC, OH, OW))
    zero = np.zeros(OC, np.float32)
    # direct forward: force it with a 1-element batch loop when the switch would pick im2col
    y = np.concatenate([oracle.conv2d_forward(x[b:b + 1], w, zero, C, OC, KH, KW, H, W, stride, pad)
                        for b in range(B)]) if OC * OH * OW < 1024 or KH * KW < 9 else None
    gi, gw, gb = oracle.conv2d_backward(x, w, g, C, OC, KH, KW, H, W, stride, pad, branch="direct")
    ref_y = np.zeros((B, OC, OH, OW), np.int64)
    xp = np.pad(x.astype(np.int64), ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    for oh in range(OH):
        for ow in range(OW):
            patch = xp[:, :, oh * stride:oh * stride + KH, ow * stride:ow * stride + KW]
            ref_y[:, :, oh, ow] = np.einsum("bchw,ochw->bo", patch, w.astype(np.int64))
    if y is not None:
        np.testing.assert_array_equal(y, ref_y.astype(np.float32))
    inner = int((ref_y * g.astype(np.int64)).sum())
    assert inner == int((x.astype(np.int64) * gi.astype(np.int64)).sum())
    assert inner == int((w.astype(np.int64).ravel() * gw.astype(np.int64)).sum())
    np.testing.assert_array_equal(gb, g.sum(axis=(0, 2, 3)))


def _im2col_brute(x, KH, KW, sh, sw, ph, pw):
    """im2col by its definition, col[(b, oh, ow)][(kh, kw, ic)] = x[b, ic, oh*sh - ph + kh, ow*sw - pw + kw]
    (0 outside the image), written independently of the oracle's loops."""
    B, C, H, W = x.shape
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)))
    col = np.empty((B, OH, OW, KH, KW, C), x.dtype)
    for kh in range(KH):
        for kw in range(KW):
            col[:, :, :, kh, kw, :] = xp[:, :, kh:kh + sh * (OH - 1) + 1:sh, kw:kw + sw * (OW - 1) + 1:sw].transpose(0, 2, 3, 1)
    return col.reshape(B * OH * OW, KH * KW * C)


@pytest.mark.parametrize("geo", [(2, 3, 7, 9, 4, 3, 3, (2, 1), (1, 1)), (1, 2, 6, 8, 8, 3, 5, (1, 1), (0, 2)),
                                 (2, 4, 9, 8, 4, 2, 3, (3, 1), (1, 0))])
def test_conv_backward_im2col_contract_unequal_strides(geo):
    """Separate stride_h / stride_w and pad_h / pad_w (the reference takes both
    pairs): im2col equals its definition, and the im2col branch's gradients
    follow its contract exactly on integer data."""
    B, C, H, W, OC, KH, KW, (sh, sw), (ph, pw) = geo
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    rng = np.random.default_rng(sum(geo[:7]) + 5)
    x, w = _ints(rng, (B, C, H, W)), _ints(rng, (OC, KH * KW * C))
    g = _ints(rng, (B, OC, OH, OW))
    col = oracle.im2col(x, B, C, H, W, KH, KW, (sh, sw), (ph, pw))
    np.testing.assert_array_equal(col, _im2col_brute(x, KH, KW, sh, sw, ph, pw))
    gi, gw, gb = oracle.conv2d_backward(x, w, g, C, OC, KH, KW, H, W, (sh, sw), (ph, pw), branch="im2col")
    go2 = g.reshape(B * OH * OW, OC).astype(np.int64)
    np.testing.assert_array_equal(gw, (go2.T @ col.astype(np.int64)).ravel().astype(np.float32))
    grad_col = (go2 @ w.astype(np.int64)).astype(np.float32)
    lhs = int((grad_col.astype(np.int64) * col.astype(np.int64)).sum())  # <grad_col, im2col(x)> = <col2im(grad_col), x>
    assert lhs == int((gi.astype(np.int64) * x.astype(np.int64)).sum())
    np.testing.assert_array_equal(gi, oracle.col2im(grad_col, B, C, H, W, KH, KW, (sh, sw), (ph, pw)))
    np.testing.assert_array_equal(gb, g.sum(axis=(0, 2, 3)))


def test_conv_backward_im2col_contract():
    """The im2col branch reads grad_output as [batch*OH*OW][OC] for both GEMMs
    (NCHW only for grad_bias): grad_weights = go2^T . col, grad_input =
    col2im(go2 . W), exact on integer data; the branch switch follows the
    forward's rule (batch*OC*OH*OW >= 1024 and kH*kW >= 9)."""
    B, C, H, W, OC, KH, KW, stride, pad = 2, 3, 6, 7, 5, 3, 3, 1, 1
    OH, OW = H, W
    rng = np.random.default_rng(77)
    x, w = _ints(rng, (B, C, H, W)), _ints(rng, (OC, KH * KW * C))
    g = _ints(rng, (B, OC, OH, OW))
    gi, gw, gb = oracle.conv2d_backward(x, w, g, C, OC, KH, KW, H, W, stride, pad, branch="im2col")
    col = oracle.im2col(x, B, C, H, W, KH, KW, stride, pad).astype(np.int64)
    go2 = g.reshape(B * OH * OW, OC).astype(np.int64)
    np.testing.assert_array_equal(gw, (go2.T @ col).ravel().astype(np.float32))
    grad_col = (go2 @ w.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(gi, oracle.col2im(grad_col, B, C, H, W, KH, KW, stride, pad))
    np.testing.assert_array_equal(gb, g.sum(axis=(0, 2, 3)))
    # the switch: this size (B*OC*OH*OW = 420 < 1024) runs the direct branch
    auto = oracle.conv2d_backward(x, w, g, C, OC, KH, KW, H, W, stride, pad)
    direct = oracle.conv2d_backward(x, w, g, C, OC, KH, KW, H, W, stride, pad, branch="direct")
    for a, d in zip(auto, direct):
        np.testing.assert_array_equal(a, d)
    big = (4, 3, 8, 8, 5)  # 4*5*8*8 = 1280 >= 1024 with a 3x3 kernel: im2col branch
    xb, gbig = _ints(rng, big[:4]), _ints(rng, (4, 5, 8, 8))
    wb = _ints(rng, (5, 27))
    auto = oracle.conv2d_backward(xb, wb, gbig, 3, 5, 3, 3, 8, 8, 1, 1)
    forced = oracle.conv2d_backward(xb, wb, gbig, 3, 5, 3, 3, 8, 8, 1, 1, branch="im2col")
    for a, f in zip(auto, forced):
        np.testing.assert_array_equal(a, f)


def test_attention_matches_fp64_softmax():
    rng = np.random.default_rng(8)
    S, D = 33, 16
    q, k, v = (rng.standard_normal((S, D)).astype(np.float32) for _ in range(3))
    scale = 1.0 / np.sqrt(D)
    out = oracle.attention(q, k, v, S, D, scale)
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    assert np.abs(out - p @ v.astype(np.float64)).max() <= 1e-5


# --------------------------------------------------------------- golden drift
def test_oracle_matches_committed_cases():
    z = np.load(os.path.join(GOLDEN, "oracle_cases.npz"))
    for name in z["names"]:
        layout, m, n, k, acc, act = z[f"{name}_meta"]
        m, n, k, acc = int(m), int(n), int(k), bool(int(acc))
        a, b, bias, c0 = z[f"{name}_a"], z[f"{name}_b"], z[f"{name}_bias"], z[f"{name}_c0"]
        if act != "none":
            c = oracle.matmul_bias_act(a, b, bias, m, n, k, str(act))
        elif layout == "nn":
            c = oracle.matmul(a, b, m, n, k, acc, c0)
        elif layout == "tn":
            c = oracle.matmul_tn(a, b, m, n, k, acc, c0)
        else:
            c = oracle.matmul_nt(a, b, m, n, k, acc, c0)
        np.testing.assert_array_equal(c, z[f"{name}_c"], err_msg=str(name))


# ------------------------------------------------- the checks are discriminating
def test_checks_catch_planted_mistakes(kats):
    """Plant plausible mistakes in oracle outputs; the pinning checks reject each."""
    rng = np.random.default_rng(99)
    m, n, k = 37, 45, 29
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    good = oracle.matmul(a, b, m, n, k)
    den = abs_denominator(a, b)
    assert componentwise_error(good, seq_nn(a, b), den) == 0.0
    # dropped last K term
    dropped = oracle.matmul(a[:, :-1], b[:-1, :], m, n, k - 1)
    assert componentwise_error(dropped, seq_nn(a, b), den) > tol(k)
    # transposed operand (B^T used as B, square case)
    sq = uniform(rng, (32, 32))
    wrong_t = oracle.matmul(sq, sq.T.copy(), 32, 32, 32)
    assert not np.array_equal(wrong_t, seq_nn(sq, sq))
    # wrong sign on the bias epilogue
    bias = uniform(rng, (n,))
    fused = oracle.matmul_bias_act(a, b, bias, m, n, k, "linear")
    assert componentwise_error(fused - 2 * bias[None, :], seq_nn(a, b) + bias, den + np.abs(bias)) > tol(k)
    # swapped NT index (reading B as [k x n] instead of [n x k]) fails the integer KAT
    mm, nn, kk = (int(x) for x in kats["small64_mnk"])
    ai, bi = kats["small64_a"].reshape(mm, kk), kats["small64_b"].reshape(kk, nn)
    swapped = oracle.matmul_nt(ai, bi, mm, nn, kk)  # B passed without the transpose
    assert not np.array_equal(swapped, kats["small64_c"].reshape(mm, nn))

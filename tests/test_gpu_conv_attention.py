"""GPU parity of the convolution (im2col, implicit GEMM) and attention paths.

im2col is pure data movement and must be bit-exact.  The conv GEMM is held to
the GEMM tolerance 1e-5*sqrt(K), K = C*kH*kW, componentwise against the
oracle with denominator |col|.|W|^T + |bias|.  Attention (the fused
online-softmax kernel for d_k <= 128, the three-kernel path above) is checked
stage by stage (scores, softmax) and end to end with the bound derived from
the stages: a score error e_s <= 1e-5*sqrt(D) (|Q|.|K|^T) * scale perturbs
each softmax row by at most 2*max(e_s) relatively, and the weighted sum over
S keys (with the fused kernel's per-block rescaling, a few ulp) adds
1e-5*sqrt(S) + 1e-6; the oracle carries the same bound, hence the factor 2.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from oracle import oracle
from _parity import abs_denominator, componentwise_error, normal, tol, uniform
from gpu_common import announce, pmap

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def backend(ctx):
    from zigneuron_amd import Backend
    return Backend(ctx)


def pair(v):
    return (v, v) if np.isscalar(v) else tuple(v)


def out_hw(h, w, k_h, k_w, stride, pad):
    (sh, sw), (ph, pw) = pair(stride), pair(pad)
    return (h + 2 * ph - k_h) // sh + 1, (w + 2 * pw - k_w) // sw + 1


CONV_CASES = [  # batch, C, H, W, OC, kH, kW, stride, pad
    (2, 3, 9, 7, 5, 3, 3, 1, 1),
    (1, 4, 8, 8, 6, 3, 3, 2, 1),
    (3, 2, 6, 5, 4, 2, 3, 1, 0),
    (2, 16, 12, 12, 24, 3, 3, 1, 1),
    (1, 1, 5, 5, 1, 1, 1, 1, 0),
    # stride 1 and OC % 4 == 0: grad_input of the im2col branch is one
    # transposed-convolution GEMM (no grad_col, no col2im)
    (2, 6, 10, 9, 8, 3, 3, 1, 1),
    (1, 3, 8, 8, 16, 1, 1, 1, 0),
    (2, 5, 6, 7, 4, 3, 5, 1, 2),
    (3, 7, 17, 19, 12, 3, 3, 1, 1),
    (1, 8, 6, 6, 256, 3, 3, 1, 1),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_im2col_bit_exact(ctx, case):
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    x = uniform(np.random.default_rng(1), (B, C, H, W))
    announce(f"im2col {case}")
    dx = ctx.to_device(x)
    dcol = ctx.alloc(B * OH * OW * KH * KW * C).fill(np.nan)
    ctx.im2col(dx, dcol, B, C, H, W, KH, KW, OH, OW, st, st, pd, pd)
    got = dcol.download().reshape(B * OH * OW, KH * KW * C)
    np.testing.assert_array_equal(got, oracle.im2col(x, B, C, H, W, KH, KW, stride=st, pad=pd))
    dx.close()
    dcol.close()


def conv_check(out, x, w_col, bias, case, what):
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    col = oracle.im2col(x, B, C, H, W, KH, KW, stride=st, pad=pd)
    ref = oracle.conv2d_im2col_gemm(col, w_col, bias, B, OC, OH * OW, KH * KW * C)
    k = KH * KW * C
    for b in range(B):
        cb = col[b * OH * OW:(b + 1) * OH * OW]
        den = abs_denominator(w_col, cb.T.copy()) + np.abs(bias.astype(np.float64))[:, None]
        err = componentwise_error(out[b].reshape(OC, OH * OW), ref[b], den)
        assert err <= tol(k), f"{what} batch {b}: {err:.3e} > {tol(k):.3e}"


@pytest.mark.parametrize("case", CONV_CASES)
def test_conv2d_forward_im2col_device(ctx, case):
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(2)
    x, w, bias = uniform(rng, (B, C, H, W)), uniform(rng, (OC, KH * KW * C)), uniform(rng, (OC,))
    announce(f"conv2d im2col device {case}")
    dx, dw, db = ctx.to_device(x), ctx.to_device(w), ctx.to_device(bias)
    do = ctx.alloc(B * OC * OH * OW).fill(np.nan)
    ctx.conv2d_forward_im2col(dx, dw, db, do, B, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
    conv_check(do.download().reshape(B, OC, OH, OW), x, w, bias, case, "device")
    for buf in (dx, dw, db, do):
        buf.close()


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "32x32"])
@pytest.mark.parametrize("case", [(3, 5, 11, 9, 7, 3, 3, 2, 1), (2, 8, 10, 12, 40, 3, 2, 1, 1),
                                  (2, 7, 13, 11, 20, 5, 5, 2, 2), (1, 64, 9, 9, 33, 1, 1, 1, 0),
                                  (2, 4, 17, 19, 8, 7, 7, 3, 3), (1, 1, 70, 70, 3, 4, 4, 1, 2),
                                  # stride 1 and OW % 4 == 0: the 4-pixel gather, with chunks that
                                  # straddle the left, right or both paddings
                                  (2, 5, 9, 12, 7, 3, 3, 1, 1), (1, 3, 7, 16, 9, 5, 5, 1, 2),
                                  (2, 4, 6, 8, 6, 1, 1, 1, 0), (1, 2, 5, 20, 3, 3, 7, 1, 3),
                                  (2, 3, 4, 4, 5, 3, 3, 1, 1), (1, 6, 3, 2, 4, 1, 3, 1, 1)])
def test_conv_implicit_gemm_every_tile(ctx, case, tile):
    """Both weight orders through every forced tile: im2col order against the
    reference's im2col GEMM, OIHW order against the direct convolution."""
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(9)
    x, w, bias = uniform(rng, (B, C, H, W)), uniform(rng, (OC, C, KH, KW)), uniform(rng, (OC,))
    dx, db = ctx.to_device(x), ctx.to_device(bias)
    do = ctx.alloc(B * OC * OH * OW)
    announce(f"conv implicit tile {tile} {case}")
    ctx.set_gemm_tile(tile)
    try:
        w_col = np.ascontiguousarray(w.transpose(0, 2, 3, 1).reshape(OC, KH * KW * C))
        dw = ctx.to_device(w_col)
        do.fill(np.nan)
        ctx.conv2d_forward_im2col(dx, dw, db, do, B, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
        conv_check(do.download().reshape(B, OC, OH, OW), x, w_col, bias, case, f"{tile} im2col order")
        dw.close()
        dw = ctx.to_device(w)  # OIHW: the same convolution, so the same reference
        do.fill(np.nan)
        ctx.conv2d_forward_direct(dx, dw, db, do, B, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
        conv_check(do.download().reshape(B, OC, OH, OW), x, w_col, bias, case, f"{tile} OIHW order")
        dw.close()
    finally:
        ctx.set_gemm_tile("auto")
    for buf in (dx, db, do):
        buf.close()


@pytest.mark.parametrize("case", CONV_CASES + [(4, 8, 16, 16, 16, 3, 3, 1, 1)])
def test_backend_conv2d_forward_both_branches(backend, case):
    """Backend.conv2dForward keeps the reference's size switch: direct semantics
    (W as [OC][C][kH][kW]) for small problems, im2col semantics otherwise."""
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(3)
    x, w, bias = uniform(rng, (B, C, H, W)), uniform(rng, (OC, C, KH, KW)), uniform(rng, (OC,))
    out = np.empty(B * OC * OH * OW, np.float32)
    announce(f"Backend.conv2dForward {case}")
    backend.conv2dForward(x, w, bias, out, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
    ref = oracle.conv2d_forward(x, w, bias, C, OC, KH, KW, H, W, stride=st, pad=pd)
    im2col_branch = B * OC * OH * OW >= 1024 and KH * KW >= 9
    w_col = w.reshape(OC, -1) if im2col_branch else np.ascontiguousarray(
        w.transpose(0, 2, 3, 1).reshape(OC, KH * KW * C))
    conv_check(out.reshape(B, OC, OH, OW), x, w_col, bias, case, "branch im2col" if im2col_branch else "branch direct")
    # and the oracle's own switch agrees with the semantics used above
    np.testing.assert_allclose(out.reshape(ref.shape), ref, rtol=0, atol=tol(KH * KW * C) * np.abs(ref).max() * 4
                               + 1e-6)


def test_softmax_rows_against_fp64(ctx):
    rng = np.random.default_rng(4)
    for rows, n, scale in ((7, 1, 1.0), (5, 33, 0.5), (64, 1024, 0.125), (3, 3000, 0.3)):
        s = (rng.standard_normal((rows, n)) * 4).astype(np.float32)
        announce(f"softmax {rows}x{n}")
        d = ctx.to_device(s)
        o = ctx.alloc(rows * n)
        ctx.softmax_rows(d, o, rows, n, scale)
        got = o.download().reshape(rows, n)
        z = s.astype(np.float64) * np.float32(scale)
        ref = np.exp(z - z.max(axis=1, keepdims=True))
        ref /= ref.sum(axis=1, keepdims=True)
        assert np.all(np.abs(got - ref) <= 8 * np.spacing(ref.astype(np.float32)) + 1e-6 * ref), (rows, n)
        np.testing.assert_allclose(got.sum(axis=1), 1.0, atol=1e-5)
        ctx.softmax_rows(d, d, rows, n, scale)  # in place
        np.testing.assert_array_equal(d.download().reshape(rows, n), got)
        d.close()
        o.close()


def attention_bound(q, k, v, scale):
    """Componentwise bound on |out - out_exact| for one head (see module docstring)."""
    S, D = q.shape
    q64, k64, v64 = (x.astype(np.float64) for x in (q, k, v))
    s = q64 @ k64.T * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    e_s = tol(D) * (np.abs(q64) @ np.abs(k64).T) * abs(scale)
    rel = 2 * e_s.max(axis=1, keepdims=True) + tol(S) + 1e-6
    return p @ v64, rel * (p @ np.abs(v64))


@pytest.mark.parametrize("batch,seq,d", [(1, 17, 8), (3, 64, 16), (2, 200, 64), (1, 1, 5), (2, 129, 32),
                                         (2, 50, 17), (2, 77, 100), (1, 300, 128), (1, 65, 160), (1, 130, 129)])
def test_attention_forward_device(ctx, batch, seq, d):
    """Fused kernel for every padded head dim (32/64/128, 16-byte and 4-byte
    I/O, ragged query and key blocks); d_k > 128 takes the three-kernel path."""
    rng = np.random.default_rng(seq)
    q, k, v = normal(rng, (batch, seq, d)), normal(rng, (batch, seq, d)), normal(rng, (batch, seq, d))
    scale = 1.0 / np.sqrt(d)
    announce(f"attention {batch}x{seq}x{d}")
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    do = ctx.alloc(batch * seq * d).fill(np.nan)
    ctx.attention_forward(dq, dk, dv, do, batch, seq, d, scale)
    out = do.download().reshape(batch, seq, d)
    for i in range(batch):
        exact, bound = attention_bound(q[i], k[i], v[i], scale)
        ref = oracle.attention(q[i], k[i], v[i], seq, d, scale)
        assert np.all(np.abs(ref - exact) <= bound), "oracle outside its own bound"
        assert np.all(np.abs(out[i] - ref) <= 2 * bound), f"head {i}"
    for buf in (dq, dk, dv, do):
        buf.close()


@pytest.mark.parametrize("scale", [2.0, -0.7, 0.0])
def test_attention_online_softmax_rescaling(ctx, scale):
    """Large, negative and zero score scales: the running maximum moves across
    key blocks (keys sorted so later blocks hold larger scores), and a zero
    scale gives the plain mean of V."""
    rng = np.random.default_rng(3)
    S, D = 515, 64
    q, k, v = normal(rng, (1, S, D)), normal(rng, (1, S, D)), normal(rng, (1, S, D))
    order = np.argsort(k[0] @ q[0].mean(axis=0))
    k = np.ascontiguousarray(k[:, order])
    announce(f"attention rescaling scale={scale}")
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    do = ctx.alloc(S * D).fill(np.nan)
    ctx.attention_forward(dq, dk, dv, do, 1, S, D, scale)
    out = do.download().reshape(S, D)
    exact, bound = attention_bound(q[0], k[0], v[0], scale)
    assert np.all(np.abs(out - exact) <= bound)
    if scale == 0.0:
        np.testing.assert_allclose(out, np.broadcast_to(v[0].astype(np.float64).mean(axis=0), (S, D)), atol=1e-5)
    for buf in (dq, dk, dv, do):
        buf.close()


def test_attention_unaligned_pointers(ctx):
    """Q, K, V and O one float off 16-byte alignment select the 4-byte kernel."""
    rng = np.random.default_rng(4)
    S, D = 150, 64
    q, k, v = normal(rng, (S, D)), normal(rng, (S, D)), normal(rng, (S, D))
    bufs = [ctx.alloc(S * D + 1) for _ in range(4)]
    for buf, x in zip(bufs[:3], (q, k, v)):
        buf.upload(np.concatenate([np.zeros(1, np.float32), x.ravel()]))
    bufs[3].fill(np.nan)
    announce("attention unaligned")
    from zigneuron_amd import _lib
    from zigneuron_amd._lib import check
    check(_lib.load().zn_hip_attention_forward(ctx.handle, *(b.offset(1) for b in bufs), 1, S, D,
                                               ctypes.c_float(0.125)), "attention")
    out = bufs[3].download()[1:].reshape(S, D)
    exact, bound = attention_bound(q, k, v, 0.125)
    assert np.all(np.abs(out - exact) <= bound)
    for buf in bufs:
        buf.close()


def test_backend_attention_forward_host(backend):
    rng = np.random.default_rng(11)
    S, D = 96, 32
    q, k, v = normal(rng, (S, D)), normal(rng, (S, D)), normal(rng, (S, D))
    out = np.empty(S * D, np.float32)
    scores = np.empty(S, np.float32)
    announce("Backend.attentionForward")
    backend.attentionForward(q, k, v, out, scores, S, D, 1.0 / np.sqrt(D))
    exact, bound = attention_bound(q, k, v, 1.0 / np.sqrt(D))
    ref = oracle.attention(q, k, v, S, D, 1.0 / np.sqrt(D))
    assert np.all(np.abs(out.reshape(S, D) - ref) <= 2 * bound)
    from zigneuron_amd import InvalidArgumentError
    with pytest.raises(InvalidArgumentError):
        backend.attentionForward(q, k, v, out, np.empty(S - 1, np.float32), S, D, 1.0)


def test_c5_attention_end_to_end(ctx):
    """[B=8,H=16,S=1024,D=64] through the fused entry point; every one of the
    128 heads against the fp64 bound and against the oracle."""
    rng = np.random.default_rng(5)
    BH, S, D = 128, 1024, 64
    q, k, v = normal(rng, (BH, S, D)), normal(rng, (BH, S, D)), normal(rng, (BH, S, D))
    scale = 1.0 / np.sqrt(D)
    announce("C5 attention end to end")
    dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
    do = ctx.alloc(BH * S * D).fill(np.nan)
    ctx.attention_forward(dq, dk, dv, do, BH, S, D, scale)
    out = do.download().reshape(BH, S, D)
    assert np.all(np.isfinite(out))
    refs = pmap(lambda i: oracle.attention(q[i], k[i], v[i], S, D, scale), range(BH))
    for i in range(BH):
        exact, bound = attention_bound(q[i], k[i], v[i], scale)
        assert np.all(np.abs(out[i] - exact) <= bound), f"head {i}"
        assert np.all(np.abs(out[i] - refs[i]) <= 2 * bound), f"head {i} against the oracle"
    for buf in (dq, dk, dv, do):
        buf.close()


def test_c5_conv_end_to_end(ctx):
    """batch 32, 64->128, 3x3, 56x56, pad 1 through zn_hip_conv2d_forward_im2col;
    all 32 images against the oracle's im2col GEMM."""
    rng = np.random.default_rng(6)
    B, C, H, W, OC = 32, 64, 56, 56, 128
    x, w, bias = uniform(rng, (B, C, H, W)), uniform(rng, (OC, 9 * C)), uniform(rng, (OC,))
    announce("C5 conv end to end")
    dx, dw, db = ctx.to_device(x), ctx.to_device(w), ctx.to_device(bias)
    do = ctx.alloc(B * OC * H * W).fill(np.nan)
    ctx.conv2d_forward_im2col(dx, dw, db, do, B, C, OC, 3, 3, H, W, H, W, 1, 1, 1, 1)
    out = do.download().reshape(B, OC, H, W)
    one = (1, C, H, W, OC, 3, 3, 1, 1)
    pmap(lambda b: conv_check(out[b:b + 1], x[b:b + 1], w, bias, one, f"C5 image {b}"), range(B))
    for buf in (dx, dw, db, do):
        buf.close()


# ------------------------------------------------------------ conv backward
BWD_CASES = [  # batch, C, H, W, OC, kH, kW, stride, pad
    (2, 3, 9, 7, 5, 3, 3, 1, 1),
    (1, 4, 8, 8, 6, 3, 3, 2, 1),
    (3, 2, 6, 5, 4, 2, 3, 1, 0),
    (2, 16, 12, 12, 24, 3, 3, 1, 1),
    (2, 5, 13, 11, 7, 5, 5, 2, 2),
    (1, 1, 5, 5, 1, 1, 1, 1, 0),
    # stride 1 and OC % 4 == 0: grad_input of the im2col branch is one
    # transposed-convolution GEMM (no grad_col, no col2im)
    (2, 6, 10, 9, 8, 3, 3, 1, 1),
    (1, 3, 8, 8, 16, 1, 1, 1, 0),
    (2, 5, 6, 7, 4, 3, 5, 1, 2),
    (3, 7, 17, 19, 12, 3, 3, 1, 1),
    (1, 8, 6, 6, 256, 3, 3, 1, 1),
]


@pytest.mark.parametrize("case", BWD_CASES)
def test_col2im_bit_exact(ctx, case):
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    col = uniform(np.random.default_rng(12), (B * OH * OW, KH * KW * C))
    announce(f"col2im {case}")
    dcol = ctx.to_device(col)
    dout = ctx.alloc(B * C * H * W).fill(np.nan)
    ctx.col2im(dcol, dout, B, C, H, W, KH, KW, OH, OW, st, st, pd, pd)
    np.testing.assert_array_equal(dout.download().reshape(B, C, H, W),
                                  oracle.col2im(col, B, C, H, W, KH, KW, stride=st, pad=pd))
    dcol.close()
    dout.close()


def backward_check(got, x, w, go, case, branch, what):
    """Componentwise against the oracle branch; the denominators are the same
    algorithm run on |x|, |w|, |go| (every output is a sum of products)."""
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    ref = oracle.conv2d_backward(x, w, go, C, OC, KH, KW, H, W, st, pd, branch=branch)
    den = oracle.conv2d_backward(np.abs(x), np.abs(w), np.abs(go), C, OC, KH, KW, H, W, st, pd, branch=branch)
    counts = (OC * KH * KW, B * OH * OW, B * OH * OW)  # terms per grad_input, grad_weights, grad_bias element
    for name, g, r, d, n in zip(("grad_input", "grad_weights", "grad_bias"), got, ref, den, counts):
        d = d.astype(np.float64).ravel()
        err = np.abs(g.astype(np.float64).ravel() - r.astype(np.float64).ravel())
        ok = err <= tol(n) * d + 1e-30
        assert ok.all(), f"{what} {name}: worst {np.max(err / np.maximum(d, 1e-30)):.3e} > {tol(n):.3e}"


def run_backward(ctx, case, branch, seed=13):
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(seed)
    x, w = uniform(rng, (B, C, H, W)), uniform(rng, (OC, KH * KW * C))
    go = uniform(rng, (B, OC, OH, OW))
    dx, dw, dgo = ctx.to_device(x), ctx.to_device(w), ctx.to_device(go)
    dgi = ctx.alloc(B * C * H * W).fill(np.nan)
    dgw = ctx.alloc(OC * KH * KW * C).fill(np.nan)
    dgb = ctx.alloc(OC).fill(np.nan)
    fn = ctx.conv2d_backward_im2col if branch == "im2col" else ctx.conv2d_backward_direct
    (sh, sw), (ph, pw) = pair(st), pair(pd)
    fn(dx, dw, dgo, dgi, dgw, dgb, B, C, OC, KH, KW, H, W, OH, OW, sh, sw, ph, pw)
    got = (dgi.download(), dgw.download(), dgb.download())
    for buf in (dx, dw, dgo, dgi, dgw, dgb):
        buf.close()
    return got, x, w, go


@pytest.mark.parametrize("branch", ["im2col", "direct"])
@pytest.mark.parametrize("case", BWD_CASES)
def test_conv2d_backward_device(ctx, case, branch):
    announce(f"conv2d backward {branch} {case}")
    got, x, w, go = run_backward(ctx, case, branch)
    backward_check(got, x, w, go, case, branch, f"{branch} {case}")


# stride_w 1 and OW % 4 == 0: the weight gradient gathers col from the input
# (no im2col); with stride 1 and OC % 4 == 0 as well, no col buffer at all.
# Chunks straddle the left, right or both paddings; stride_h 2 and 3 keep only
# the weight gradient implicit.
IMPLICIT_W_CASES = [(2, 16, 12, 12, 24, 3, 3, 1, 1), (2, 5, 9, 12, 7, 3, 3, 1, 1), (1, 3, 7, 16, 8, 5, 5, 1, 2),
                    (3, 4, 6, 8, 12, 1, 1, 1, 0), (1, 2, 5, 20, 4, 3, 7, 1, 3), (2, 3, 4, 4, 8, 3, 3, 1, 1),
                    (2, 6, 11, 8, 8, 3, 3, (2, 1), (1, 1)), (1, 5, 13, 12, 6, 3, 3, (3, 1), (0, 1)),
                    (1, 70, 9, 8, 4, 3, 3, 1, 1)]


@pytest.mark.parametrize("tile", ["auto", "256x128", "128x128", "128x64", "64x64", "32x32"])
@pytest.mark.parametrize("case", IMPLICIT_W_CASES)
def test_conv_backward_implicit_weight_grad_every_tile(ctx, case, tile):
    """The weight gradient as an implicit GEMM (col gathered in 4-pixel chunks)
    through every forced tile, with the policy's split-K and 5 forced slices."""
    announce(f"conv backward implicit grad_W tile {tile} {case}")
    ctx.set_gemm_tile(tile)
    try:
        for splits in (0, 5):
            ctx.set_gemm_splits(splits)
            got, x, w, go = run_backward(ctx, case, "im2col", seed=18)
            backward_check(got, x, w, go, case, "im2col", f"{tile} splits {splits} {case}")
    finally:
        ctx.set_gemm_tile("auto")
        ctx.set_gemm_splits(0)


TRANSPOSED_CASES = [(2, 6, 10, 9, 8, 3, 3, 1, 1), (1, 5, 7, 12, 36, 5, 3, 1, 2), (2, 33, 5, 6, 4, 1, 1, 1, 0),
                    (1, 2, 4, 4, 20, 3, 3, 1, 2), (2, 70, 9, 9, 8, 3, 3, 1, 1)]


@pytest.mark.parametrize("tile", ["256x128", "128x128", "128x64", "64x64", "32x32"])
@pytest.mark.parametrize("case", TRANSPOSED_CASES)
def test_conv_backward_transposed_every_tile(ctx, case, tile):
    """The stride-1 input gradient as an implicit transposed convolution
    through every forced tile, with the policy's split-K and with 3 forced
    slices (partial sums reduced in slice order)."""
    announce(f"conv backward transposed tile {tile} {case}")
    ctx.set_gemm_tile(tile)
    try:
        for splits in (0, 3):
            ctx.set_gemm_splits(splits)
            got, x, w, go = run_backward(ctx, case, "im2col", seed=16)
            backward_check(got, x, w, go, case, "im2col", f"{tile} splits {splits} {case}")
    finally:
        ctx.set_gemm_tile("auto")
        ctx.set_gemm_splits(0)


def test_conv_backward_unaligned_grad_output(ctx):
    """grad_output one float off 16-byte alignment: the transposed GEMM needs
    whole 16-byte chunks, so the materialized grad_col + col2im path runs."""
    case = (2, 6, 10, 9, 8, 3, 3, 1, 1)
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(17)
    x, w = uniform(rng, (B, C, H, W)), uniform(rng, (OC, KH * KW * C))
    go = uniform(rng, (B, OC, OH, OW))
    dx, dw = ctx.to_device(x), ctx.to_device(w)
    dgo = ctx.alloc(go.size + 1)
    dgo.upload(np.concatenate([np.zeros(1, np.float32), go.ravel()]))
    dgi = ctx.alloc(B * C * H * W).fill(np.nan)
    dgw = ctx.alloc(OC * KH * KW * C).fill(np.nan)
    dgb = ctx.alloc(OC).fill(np.nan)
    announce("conv backward unaligned grad_output")
    ctx.conv2d_backward_im2col(dx, dw, dgo.offset(1), dgi, dgw, dgb, B, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
    got = (dgi.download(), dgw.download(), dgb.download())
    for buf in (dx, dw, dgo, dgi, dgw, dgb):
        buf.close()
    backward_check(got, x, w, go, case, "im2col", "unaligned grad_output")


@pytest.mark.parametrize("case", [(2, 3, 9, 7, 5, 3, 3, 1, 1), (4, 8, 16, 16, 16, 3, 3, 1, 1),
                                  (2, 4, 10, 10, 6, 2, 2, 1, 0)])
def test_backend_conv2d_backward_host(backend, case):
    """Backend.conv2dBackward on host slices: the reference's size switch
    selects the branch (the last two cases run im2col, then direct on a 2x2)."""
    B, C, H, W, OC, KH, KW, st, pd = case
    OH, OW = out_hw(H, W, KH, KW, st, pd)
    rng = np.random.default_rng(14)
    x, w = uniform(rng, (B, C, H, W)), uniform(rng, (OC, KH * KW * C))
    go = uniform(rng, (B, OC, OH, OW))
    gi = np.full(B * C * H * W, np.nan, np.float32)
    gw = np.full(OC * KH * KW * C, np.nan, np.float32)
    gb = np.full(OC, np.nan, np.float32)
    announce(f"Backend.conv2dBackward {case}")
    backend.conv2dBackward(x.ravel(), w.ravel(), go.ravel(), gi, gw, gb, C, OC, KH, KW, H, W, OH, OW, st, st, pd, pd)
    backward_check((gi, gw, gb), x, w, go, case, "auto", f"host {case}")


@pytest.mark.parametrize("case", [(8, 12, 64, 64, 20, 3, 3, 2, 1), (4, 8, 48, 48, 132, 3, 3, 1, 1)])
def test_conv_backward_weight_grad_long_k(ctx, case):
    """Weight gradients over a long K (batch*OH*OW >= 8192) with few tiles
    and 16-byte grad_output rows, which run as one round of 128x128 tiles x
    K slices on the register-staged loop: grad_weights and grad_bias against
    fp64, grad_input against the col2im form."""
    B, C, H, W, OC, kh, kw, stride, pad = case
    oh, ow = out_hw(H, W, kh, kw, stride, pad)
    rng = np.random.default_rng(list(case))
    x, w, go = uniform(rng, (B, C, H, W)), uniform(rng, (OC, kh * kw * C)), uniform(rng, (B, OC, oh, ow))
    announce(f"conv backward long K {case}")
    dx, dw, dgo = ctx.to_device(x), ctx.to_device(w), ctx.to_device(go)
    dgi, dgw, dgb = ctx.alloc(B * C * H * W), ctx.alloc(OC * kh * kw * C), ctx.alloc(OC)
    ctx.conv2d_backward_im2col(dx, dw, dgo, dgi, dgw, dgb, B, C, OC, kh, kw, H, W, oh, ow, stride, stride, pad, pad)
    gw, gb = dgw.download().reshape(OC, kh * kw * C), dgb.download()
    for buf in (dx, dw, dgo, dgi, dgw, dgb):
        buf.close()
    go2 = go.reshape(B * oh * ow, OC).astype(np.float64)
    col = oracle.im2col(x, B, C, H, W, kh, kw, stride=stride, pad=pad).astype(np.float64)
    gw_ref = go2.T @ col
    assert np.all(np.abs(gw - gw_ref) <= tol(B * oh * ow) * (np.abs(go2).T @ np.abs(col)))
    go64 = go.astype(np.float64)
    assert np.all(np.abs(gb - go64.sum(axis=(0, 2, 3))) <= tol(B * oh * ow) * np.abs(go64).sum(axis=(0, 2, 3)))


def test_c5_conv_backward_properties(ctx):
    """C5 (batch 32, 64->128, 3x3, 56x56, pad 1) through the im2col branch,
    checked in fp64: grad_bias = per-channel sums, grad_weights = go2^T . col,
    grad_input = col2im(go2 . W) for every image (go2 = grad_output as
    [batch*OH*OW][OC], the reference's reading)."""
    B, C, H, W, OC = 32, 64, 56, 56, 128
    rng = np.random.default_rng(15)
    x, w = uniform(rng, (B, C, H, W)), uniform(rng, (OC, 9 * C))
    go = uniform(rng, (B, OC, H, W))
    announce("C5 conv backward")
    dx, dw, dgo = ctx.to_device(x), ctx.to_device(w), ctx.to_device(go)
    dgi, dgw, dgb = ctx.alloc(B * C * H * W), ctx.alloc(OC * 9 * C), ctx.alloc(OC)
    ctx.conv2d_backward_im2col(dx, dw, dgo, dgi, dgw, dgb, B, C, OC, 3, 3, H, W, H, W, 1, 1, 1, 1)
    gi, gw, gb = dgi.download().reshape(B, C, H, W), dgw.download().reshape(OC, 9 * C), dgb.download()
    for buf in (dx, dw, dgo, dgi, dgw, dgb):
        buf.close()
    go64 = go.astype(np.float64)
    gb_ref = go64.sum(axis=(0, 2, 3))
    assert np.all(np.abs(gb - gb_ref) <= tol(B * H * W) * np.abs(go64).sum(axis=(0, 2, 3)))
    go2 = go.reshape(B * H * W, OC).astype(np.float64)
    col = oracle.im2col(x, B, C, H, W, 3, 3, stride=1, pad=1).astype(np.float64)
    gw_ref = go2.T @ col
    gw_den = np.abs(go2).T @ np.abs(col)
    assert np.all(np.abs(gw - gw_ref) <= tol(B * H * W) * gw_den)
    del col
    rows = H * W
    for b in range(B):
        g2 = go2[b * rows:(b + 1) * rows]
        gcol = g2 @ w.astype(np.float64)
        gcol_abs = np.abs(g2) @ np.abs(w.astype(np.float64))
        ref = oracle.col2im(gcol.astype(np.float32), 1, C, H, W, 3, 3, stride=1, pad=1)[0]
        den = oracle.col2im(gcol_abs.astype(np.float32), 1, C, H, W, 3, 3, stride=1, pad=1)[0]
        assert np.all(np.abs(gi[b] - ref) <= tol(9 * OC) * den * 1.01 + 1e-6), f"image {b}"

"""GPU parity at BASELINE.json's configurations (C1-C5).

Every element of every configuration is compared against the oracle, at full
size: 8192^3 (the oracle's blocked NN on all rows, OpenMP over row blocks,
which leaves each element's K order untouched), all 128 QK^T and P.V
problems of the attention batch, and all 100352 rows of the convolution
GEMM.  Row and column checksums (C.1 = A.(B.1), 1^T.C = (1^T.A).B in fp64)
are kept as a size-independent property on top.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from _parity import abs_denominator, normal, tol, uniform
from gpu_common import THREADS, announce, assert_close, assert_close_rows, pmap, ref_gemm, run_gemm

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.close()


def checksum_property(c, a_mk, b_kn, k, what):
    """Row and column sums of C against A.(B.1) and (1^T.A).B in fp64."""
    A, B = a_mk.astype(np.float64), b_kn.astype(np.float64)
    absA, absB = np.abs(A), np.abs(B)
    row = c.astype(np.float64).sum(axis=1)
    row_ref = A @ B.sum(axis=1)
    row_den = absA @ absB.sum(axis=1)
    col = c.astype(np.float64).sum(axis=0)
    col_ref = A.sum(axis=0) @ B
    col_den = absA.sum(axis=0) @ absB
    slack = 1e-12
    assert np.all(np.abs(row - row_ref) <= tol(k) * row_den + slack * row_den + 1e-30), f"{what}: row checksum"
    assert np.all(np.abs(col - col_ref) <= tol(k) * col_den + slack * col_den + 1e-30), f"{what}: column checksum"


def test_c1_nn_512(ctx):
    rng = np.random.default_rng(42)
    m = n = k = 512
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("C1 NN 512^3")
    c = run_gemm(ctx, "nn", a, b, m, n, k)
    assert_close(c, ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k)


def check_bias(got, gaa, fused, start=None):
    start = np.zeros(gaa.shape[1], np.float32) if start is None else start
    ref = oracle.accumulate_bias(start, gaa)
    if not fused:
        np.testing.assert_array_equal(got, ref)
        return
    den = np.abs(start.astype(np.float64)) + np.abs(gaa.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= tol(gaa.shape[0]) * den)


@pytest.mark.parametrize("fused", [False, True, "chain", "pair"])
def test_c2_mlp_training_step(ctx, fused):
    """X[256x784] U[0,1) -> W1 He + b1(0) + ReLU -> W2 + b2(0) linear; dY2 U[-1,1).
    W1 = U[-1,1)*sqrt(2/784) and W2 = U[-1,1)*sqrt(1/128): Dense.init's scales
    for a relu and a linear layer (src/layer.zig:331-333).  BASELINE.json calls
    W2 "Xavier-init", sqrt(2/138), which the reference uses only for sigmoid,
    tanh and softmax layers; the scale does not affect parity.
    Each of the six GEMMs is checked against the oracle on the GPU's own inputs.
    The reference's call sequence gives bit-identical bias gradients; the fused
    backward sums them over row splits (within the GEMM tolerance).  "chain":
    L2's backward also writes L1's activation derivative, and L1's backward
    takes it as ready.  "pair": both layers' forwards in one launch and both
    backwards in another (zn_hip_dense_pair_forward / _backward, the bench's
    step), checked to the same bar."""
    from zigneuron_amd import DenseDevice, pair_backward, pair_forward
    batch, d_in, d_h, d_out = 256, 784, 128, 10
    rng = np.random.default_rng(42)
    x = uniform(rng, (batch, d_in), 0.0, 1.0)
    dy = uniform(rng, (batch, d_out))
    announce(f"C2 MLP step fused={fused}")
    l1 = DenseDevice(ctx, d_in, d_h, "relu", batch, seed=1)
    l2 = DenseDevice(ctx, d_h, d_out, "linear", batch, seed=2)
    dx, ddy = ctx.to_device(x), ctx.to_device(dy)
    if fused == "pair":
        logits = pair_forward(l1, l2, dx)
        h1 = l1.out
    else:
        h1 = l1.forward(dx)
        logits = l2.forward(h1)
    if fused == "pair":
        g_x = pair_backward(l1, l2, dx, ddy)
        g_h1 = l2.grad_input
    elif fused == "chain":
        g_h1 = l2.backward(h1, ddy, below=l1)
        g_x = l1.backward(dx, None)
    else:
        g_h1 = l2.backward(h1, ddy, fused=fused)
        g_x = l1.backward(dx, g_h1, fused=fused)
    ctx.sync()
    W1 = l1.weights.download().reshape(d_in, d_h)
    W2 = l2.weights.download().reshape(d_h, d_out)
    b1, b2 = np.zeros(d_h, np.float32), np.zeros(d_out, np.float32)
    H1 = h1.download().reshape(batch, d_h)
    assert_close(H1, oracle.matmul_bias_act(x, W1, b1, batch, d_h, d_in, "relu"), "nn", x, W1, batch, d_h, d_in,
                 bias=b1, act="relu", what="L1 forward")
    L = logits.download().reshape(batch, d_out)
    L_ref = oracle.matmul_bias_act(H1, W2, b2, batch, d_out, d_h, "linear")
    assert_close(L, L_ref, "nn", H1, W2, batch, d_out, d_h, bias=b2, what="L2 forward")
    # L2 backward: gaa2 = dY (linear), dX2 = gaa2 . W2^T (NT), dW2 = H1^T . gaa2 (TN)
    gaa2 = l2.gaa.download().reshape(batch, d_out)
    np.testing.assert_array_equal(gaa2, dy)
    GH1 = g_h1.download().reshape(batch, d_h)
    GH1_ref = oracle.matmul_nt(gaa2, W2, batch, d_h, d_out)
    assert_close(GH1, GH1_ref, "nt", gaa2, W2, batch, d_h, d_out, what="L2 dX (NT)")
    dW2 = l2.grad_weights.download().reshape(d_h, d_out)
    assert_close(dW2, oracle.matmul_tn(H1, gaa2, d_h, d_out, batch), "tn", H1, gaa2, d_h, d_out, batch,
                 what="L2 dW (TN)")
    check_bias(l2.grad_bias.download(), gaa2, bool(fused))
    # L1 backward: gaa1 = relu'(H1) * GH1, dX1 = gaa1 . W1^T (NT), dW1 = X^T . gaa1 (TN)
    gaa1 = l1.gaa.download().reshape(batch, d_h)
    np.testing.assert_array_equal(gaa1, oracle.activation_backward("relu", H1, GH1).reshape(batch, d_h))
    GX = g_x.download().reshape(batch, d_in)
    assert_close(GX, oracle.matmul_nt(gaa1, W1, batch, d_in, d_h), "nt", gaa1, W1, batch, d_in, d_h,
                 what="L1 dX (NT)")
    dW1 = l1.grad_weights.download().reshape(d_in, d_h)
    assert_close(dW1, oracle.matmul_tn(x, gaa1, d_in, d_h, batch, threads=THREADS), "tn", x, gaa1, d_in, d_h, batch,
                 what="L1 dW (TN)")
    check_bias(l1.grad_bias.download(), gaa1, bool(fused))


@pytest.mark.parametrize("which", ["dW_TN", "dX_NT"])
def test_c3_dense_backward_gemms(ctx, which):
    rng = np.random.default_rng(3)
    s = np.float32(1.0 / 32.0)
    X = (normal(rng, (4096, 1024)) * s).astype(np.float32)
    W = (normal(rng, (1024, 1024)) * s).astype(np.float32)
    dY = (normal(rng, (4096, 1024)) * s).astype(np.float32)
    announce(f"C3 {which}")
    if which == "dW_TN":  # dW[1024x1024] = X^T . dY, K = 4096
        c = run_gemm(ctx, "tn", X, dY, 1024, 1024, 4096)
        assert_close(c, ref_gemm("tn", X, dY, 1024, 1024, 4096), "tn", X, dY, 1024, 1024, 4096)
    else:  # dX[4096x1024] = dY . W^T, K = 1024
        c = run_gemm(ctx, "nt", dY, W, 4096, 1024, 1024)
        assert_close(c, ref_gemm("nt", dY, W, 4096, 1024, 1024), "nt", dY, W, 4096, 1024, 1024)


@pytest.mark.parametrize("m,n,k", [(1000, 1000, 1000), (4097, 1023, 777)])
def test_c4_ragged_full(ctx, m, n, k):
    rng = np.random.default_rng(m + k)
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce(f"C4 NN {m}x{n}x{k}")
    c = run_gemm(ctx, "nn", a, b, m, n, k)
    assert_close(c, ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k)


def test_c4_large_8192(ctx):
    """8192^3 NN: every row against the oracle's blocked NN, plus checksums."""
    rng = np.random.default_rng(8192)
    m = n = k = 8192
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("C4 NN 8192^3")
    c = run_gemm(ctx, "nn", a, b, m, n, k)
    ref = oracle.matmul(a, b, m, n, k, branch="blocked", threads=THREADS)
    assert_close_rows(c, ref, a, b, k, what="8192^3 all rows")
    del ref
    checksum_property(c, a, b, k, "8192^3")


def _softmax_rows_fp64(s):
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    return (p / p.sum(axis=-1, keepdims=True)).astype(np.float32)


def test_c5_attention_batched(ctx):
    """[B=8,H=16,S=1024,D=64]: QK^T (NT, batch 128) then P.V (NN, batch 128);
    all 128 problems of each against the oracle."""
    rng = np.random.default_rng(5)
    BH, S, D = 128, 1024, 64
    q, kk, v = normal(rng, (BH, S, D)), normal(rng, (BH, S, D)), normal(rng, (BH, S, D))
    dq, dk, dv = ctx.to_device(q), ctx.to_device(kk), ctx.to_device(v)
    ds = ctx.alloc(BH * S * S).fill(np.nan)
    announce("C5 QK^T strided batched")
    ctx.sgemm_strided_batched("nt", S, S, D, dq, D, S * D, dk, D, S * D, ds, S, S * S, BH)
    scores = ds.download().reshape(BH, S, S)
    refs = pmap(lambda i: oracle.matmul_nt(q[i], kk[i], S, S, D), range(BH))
    for i in range(BH):
        assert_close(scores[i], refs[i], "nt", q[i], kk[i], S, S, D, what=f"QK^T problem {i}")
    del refs
    for i in range(0, BH, 16):
        checksum_property(scores[i], q[i], kk[i].T, D, f"QK^T checksum {i}")
    del scores
    # P = row softmax of N(0,1) scores (fp64 on the host), then P.V
    p = _softmax_rows_fp64(rng.standard_normal((BH, S, S)))
    dp = ctx.to_device(p)
    do = ctx.alloc(BH * S * D).fill(np.nan)
    announce("C5 PV strided batched")
    ctx.sgemm_strided_batched("nn", S, D, S, dp, S, S * S, dv, D, S * D, do, D, S * D, BH)
    out = do.download().reshape(BH, S, D)
    refs = pmap(lambda i: oracle.matmul(p[i], v[i], S, D, S, branch="blocked"), range(BH))
    for i in range(BH):
        assert_close(out[i], refs[i], "nn", p[i], v[i], S, D, S, what=f"PV problem {i}")
    for i in range(0, BH, 16):
        checksum_property(out[i], p[i], v[i], S, f"PV checksum {i}")
    for buf in (dq, dk, dv, ds, dp, do):
        buf.close()


def test_c5_im2col_conv_gemm(ctx):
    """batch 32, 64->128 channels, 3x3, 56x56, pad 1: C[100352x128] = col[100352x576] . W^T,
    all rows against the oracle."""
    rng = np.random.default_rng(6)
    Bn, C, H, W, OC = 32, 64, 56, 56, 128
    x = uniform(rng, (Bn, C, H, W))
    col = oracle.im2col(x, Bn, C, H, W, 3, 3, stride=1, pad=1)  # K order (kh, kw, ic)
    w = uniform(rng, (OC, 9 * C))  # weights generated directly in the col K order
    M, K = col.shape
    announce("C5 conv NT 100352x128x576")
    c = run_gemm(ctx, "nt", col, w, M, OC, K)
    ref = oracle.matmul_nt(col, w, M, OC, K, threads=THREADS)
    assert_close_rows(c, ref, col, w.T, K, what="conv GEMM all rows", block=8192)
    checksum_property(c, col, w.T, K, "conv")


@pytest.mark.parametrize("path", ["auto", "prologue"])
@pytest.mark.parametrize("act", ["linear", "relu", "sigmoid", "tanh"])
@pytest.mark.parametrize("shape", [(256, 784, 128), (33, 17, 5), (4096, 1024, 1024), (1, 9, 300), (96, 200, 2048),
                                   (2048, 64, 12), (256, 128, 10)])
def test_dense_backward_fused(ctx, act, shape, path):
    """zn_hip_dense_backward against the reference's four steps: the
    activation derivative bit-exact, grad_bias (+= onto a non-zero start)
    within the GEMM tolerance, the NT / TN products componentwise.  "auto"
    runs small layers' GEMMs in one grouped launch of 32x32 tiles whose waves
    split K; "prologue" (wave split off) the grouped launch of unsplit 64x64
    tiles.  Both follow the prologue kernel."""
    ctx.set_gemm_wave_split(-1 if path == "auto" else 0)
    batch, d_in, d_out = shape
    rng = np.random.default_rng(batch + d_in + d_out)
    x, w = uniform(rng, (batch, d_in)), uniform(rng, (d_in, d_out))
    y = oracle.activation_forward(act, uniform(rng, (batch, d_out)) * 3).reshape(batch, d_out)
    go = uniform(rng, (batch, d_out))
    gb0 = uniform(rng, (d_out,))
    announce(f"dense backward {act} {shape}")
    dx, dw, dy, dgo = (ctx.to_device(a) for a in (x, w, y, go))
    dgaa, dgi, dgw = ctx.alloc(batch * d_out), ctx.alloc(batch * d_in), ctx.alloc(d_in * d_out).fill(np.nan)
    dgb = ctx.to_device(gb0)
    ctx.dense_backward(act, dx, dw, dy, dgo, dgaa, dgi, dgw, dgb, batch, d_in, d_out)
    gaa = dgaa.download().reshape(batch, d_out)
    np.testing.assert_array_equal(gaa, oracle.activation_backward(act, y, go).reshape(batch, d_out))
    check_bias(dgb.download(), gaa, True, start=gb0)
    gi = dgi.download().reshape(batch, d_in)
    assert_close(gi, oracle.matmul_nt(gaa, w, batch, d_in, d_out, threads=THREADS), "nt", gaa, w, batch, d_in, d_out,
                 what="grad_input")
    gw = dgw.download().reshape(d_in, d_out)
    assert_close(gw, oracle.matmul_tn(x, gaa, d_in, d_out, batch, threads=THREADS), "tn", x, gaa, d_in, d_out, batch,
                 what="grad_weights")
    # first layer: no grad_input; grad_weights is overwritten (deterministically), not accumulated
    dgaa.fill(np.nan)
    ctx.dense_backward(act, dx, dw, dy, dgo, dgaa, None, dgw, dgb, batch, d_in, d_out)
    np.testing.assert_array_equal(dgw.download().reshape(d_in, d_out), gw)
    np.testing.assert_array_equal(dgaa.download().reshape(batch, d_out), gaa)  # written without grad_input too
    ctx.set_gemm_wave_split(-1)
    for buf in (dx, dw, dy, dgo, dgaa, dgi, dgw, dgb):
        buf.close()


@pytest.mark.parametrize("path", ["auto", "wide", "large"])
@pytest.mark.parametrize("acts", [("relu", "linear"), ("tanh", "sigmoid"), ("sigmoid", "relu"), ("linear", "tanh")])
@pytest.mark.parametrize("shape", [(256, 784, 128, 10), (33, 17, 5, 7), (1, 9, 300, 4), (96, 200, 64, 2048),
                                   (3000, 64, 48, 20)])
def test_dense_backward_chain_bit_identical(ctx, shape, acts, path):
    """Two stacked layers' backward, chained (the upper call writes the lower
    layer's activation derivative, the lower call takes it as ready) against
    the unchained calls: every output bit-identical (both derivatives, both
    grad_inputs, weight and bias gradients).  "auto": 32x32 wave-split tiles
    (the derivative written as the NT tiles finish); "wide": 64x64 tiles (a
    separate activation pass); "large": the ungrouped path (forced tile), as
    is the 3000-row shape on every path.  The unchained results themselves are
    checked against the oracle by test_dense_backward_fused."""
    from zigneuron_amd import DenseDevice
    batch, d_in, d_mid, d_out = shape
    act_lo, act_hi = acts
    rng = np.random.default_rng(batch + d_in + d_mid + d_out)
    x = uniform(rng, (batch, d_in), 0.0, 1.0)
    go = uniform(rng, (batch, d_out))
    gb_lo, gb_hi = uniform(rng, (d_mid,)), uniform(rng, (d_out,))
    announce(f"dense backward chain {shape} {acts} {path}")
    ctx.set_gemm_wave_split(0 if path == "wide" else -1)
    if path == "large":
        ctx.set_gemm_tile("64x64")
    dx, dgo = ctx.to_device(x), ctx.to_device(go)
    lo = DenseDevice(ctx, d_in, d_mid, act_lo, batch, seed=3)
    hi = DenseDevice(ctx, d_mid, d_out, act_hi, batch, seed=4)
    lo.forward(dx)
    hi.forward(lo.out)
    results = {}
    for mode in ("plain", "chain"):
        lo.grad_bias.upload(gb_lo)
        hi.grad_bias.upload(gb_hi)
        for b in (lo.gaa, hi.gaa, lo.grad_input, hi.grad_input, lo.grad_weights, hi.grad_weights):
            b.fill(np.nan)
        if mode == "plain":
            g = hi.backward(lo.out, dgo)
            lo.backward(dx, g)
        else:
            hi.backward(lo.out, dgo, below=lo)
            lo.backward(dx, None)
        results[mode] = [b.download() for b in (hi.gaa, lo.gaa, hi.grad_input, lo.grad_input, hi.grad_weights,
                                                lo.grad_weights, hi.grad_bias, lo.grad_bias)]
    names = ("hi.gaa", "lo.gaa", "hi.grad_input", "lo.grad_input", "hi.grad_weights", "lo.grad_weights",
             "hi.grad_bias", "lo.grad_bias")
    for name, a, b in zip(names, results["plain"], results["chain"]):
        assert not np.isnan(a).any(), name
        np.testing.assert_array_equal(b, a, err_msg=name)
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_wave_split(-1)
    for b in (dx, dgo):
        b.close()


@pytest.mark.parametrize("pair", [False, True])
def test_graph_replay_of_mlp_step_matches_eager(ctx, pair):
    """The C2 training step (bias-gradient reset by a fill kernel, two fused
    forwards, two chained backwards; or the pair launches, whose forward
    hands rows over through counters that each launch leaves at zero)
    captured once and replayed three times, with unrelated eager GEMMs and
    synchronisations between the replays: every replay reproduces the eager
    step bit for bit."""
    from zigneuron_amd import DenseDevice, InvalidArgumentError, pair_backward, pair_forward
    batch = 256
    rng = np.random.default_rng(7)
    x = ctx.to_device(uniform(rng, (batch, 784), 0.0, 1.0))
    dy = ctx.to_device(uniform(rng, (batch, 10)))
    l1 = DenseDevice(ctx, 784, 128, "relu", batch, seed=1)
    l2 = DenseDevice(ctx, 128, 10, "linear", batch, seed=2)

    def step():
        l1.grad_bias.fill(0.0)
        l2.grad_bias.fill(0.0)
        if pair:
            pair_forward(l1, l2, x)
            pair_backward(l1, l2, x, dy)
            return
        h = l1.forward(x)
        l2.forward(h)
        l2.backward(h, dy, below=l1)
        l1.backward(x, None)

    def outputs():
        return [b.download() for b in (l1.out, l2.out, l2.grad_input, l1.grad_input, l1.grad_weights,
                                       l2.grad_weights, l1.grad_bias, l2.grad_bias)]

    announce(f"graph replay MLP step pair={pair}")
    step()
    ctx.sync()
    eager = outputs()
    with pytest.raises(InvalidArgumentError):
        ctx.capture(ctx.sync)  # waiting for the device is refused under capture
    graph = ctx.capture(step)
    other_a, other_b = ctx.to_device(uniform(rng, (300, 200))), ctx.to_device(uniform(rng, (200, 100)))
    other_c = ctx.alloc(300 * 100)
    for _ in range(3):
        for b in (l1.out, l2.out, l2.grad_input, l1.grad_input, l1.grad_weights, l2.grad_weights):
            b.fill(np.nan)
        graph.launch()
        ctx.sync()
        for got, ref in zip(outputs(), eager):
            np.testing.assert_array_equal(got, ref)
        ctx.sgemm("nn", 300, 100, 200, other_a, 200, other_b, 100, other_c, 100)
        ctx.sync()
    graph.close()
    step()  # the context keeps working eagerly after the graph is gone
    ctx.sync()
    for got, ref in zip(outputs(), eager):
        np.testing.assert_array_equal(got, ref)
    for b in (x, dy, other_a, other_b, other_c):
        b.close()


def test_graph_replay_of_large_tiles_matches_eager(ctx):
    """The register-staged tiles under graph capture: a 256x256-tile GEMM
    (4096 x 4096 x 512), whole rounds of 128x128 tiles (4096 x 2048 x 256)
    and one round of 128x128 tiles in 4 K slices with the split-K reduce
    (C3's 1024 x 1024 x 4096 TN), captured once and replayed three times
    with outputs poisoned and unrelated eager GEMMs in between: every replay
    reproduces the eager results bit for bit."""
    rng = np.random.default_rng(17)
    probs = [("nn", 4096, 4096, 512), ("nn", 4096, 2048, 256), ("tn", 1024, 1024, 4096)]
    bufs = []
    for lay, m, n, k in probs:
        a_shape = (k, m) if lay == "tn" else (m, k)
        a, b = ctx.to_device(uniform(rng, a_shape)), ctx.to_device(uniform(rng, (k, n)))
        bufs.append((lay, m, n, k, a, b, ctx.alloc(m * n), m if lay == "tn" else k))

    def run():
        for lay, m, n, k, a, b, c, lda in bufs:
            ctx.sgemm(lay, m, n, k, a, lda, b, n, c, n)

    announce("graph replay of large tiles")
    run()
    ctx.sync()
    eager = [c.download() for *_, c, _ in bufs]
    graph = ctx.capture(run)
    other_a, other_b = ctx.to_device(uniform(rng, (300, 200))), ctx.to_device(uniform(rng, (200, 100)))
    other_c = ctx.alloc(300 * 100)
    for _ in range(3):
        for *_, c, _ in bufs:
            c.fill(np.nan)
        graph.launch()
        ctx.sync()
        for (*_, c, _), ref in zip(bufs, eager):
            np.testing.assert_array_equal(c.download(), ref)
        ctx.sgemm("nn", 300, 100, 200, other_a, 200, other_b, 100, other_c, 100)
        ctx.sync()
    graph.close()
    for lay, m, n, k, a, b, c, lda in bufs:
        for x in (a, b, c):
            x.close()
    for x in (other_a, other_b, other_c):
        x.close()


def test_znn_model_loads_into_hbm_and_matches_oracle(ctx, tmp_path):
    """A C2-shaped MLP (784 -> 128 relu -> 10 linear) written as a .znn file,
    loaded straight into HBM, run forward on the GPU against the oracle's
    matMulBias path on the same weights, and written back byte for byte."""
    from zigneuron_amd import serialization as znn
    from zigneuron_amd.layer import init_weights
    rng = np.random.default_rng(11)
    specs = [znn.DenseSpec(784, 128, "relu", init_weights(784, 128, "relu", 3), uniform(rng, (128,))),
             znn.DenseSpec(128, 10, "linear", init_weights(128, 10, "linear", 4), uniform(rng, (10,)))]
    path = tmp_path / "mlp.znn"
    znn.save_model(specs, str(path))
    batch = 256
    announce("znn load + forward")
    layers = znn.load_model(str(path), ctx, batch=batch)
    x = uniform(rng, (batch, 784), 0.0, 1.0)
    h = ctx.to_device(x)
    inp = x
    for spec, layer in zip(specs, layers):
        out = layer.forward(h)
        got = out.download().reshape(batch, spec.output_size)
        ref = oracle.matmul_bias_act(inp, spec.weights, spec.bias, batch, spec.output_size, spec.input_size, spec.act)
        assert_close(got, ref, "nn", inp, spec.weights, batch, spec.output_size, spec.input_size, bias=spec.bias,
                     act=spec.act, what=f"znn layer {spec.input_size}->{spec.output_size}")
        h, inp = out, got
    back = tmp_path / "back.znn"
    znn.save_model(layers, str(back))
    assert back.read_bytes() == path.read_bytes()


def test_graph_and_buffer_outlive_their_context():
    """Closing a context releases its graphs: a graph or buffer closed later is
    a no-op, and launching such a graph raises instead of touching freed state."""
    from zigneuron_amd import Context, InvalidArgumentError
    c = Context(0)
    a, b, out = c.to_device(np.ones((64, 64), np.float32)), c.to_device(np.ones((64, 64), np.float32)), c.alloc(4096)
    c.sgemm("nn", 64, 64, 64, a, 64, b, 64, out, 64)
    c.sync()
    g = c.capture(lambda: c.sgemm("nn", 64, 64, 64, a, 64, b, 64, out, 64))
    g.launch()
    c.sync()
    np.testing.assert_array_equal(out.download(), np.full(4096, 64.0, np.float32))
    c.close()
    with pytest.raises(InvalidArgumentError):
        g.launch()
    g.close()
    for buf in (a, b, out):
        buf.close()

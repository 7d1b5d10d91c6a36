"""Seeded random sweeps through the C ABI, beside the hand-picked cases.

Each test draws its cases from a fixed seed (the seed and the case are
announced before every GPU call), so a failure is reproducible by its id:
  * GEMMs: every layout, random sizes (1..700), padded leading dimensions,
    operands one float off 16-byte alignment, accumulate, fused bias and
    activation, forced tiles and split-K slices, strided batches;
  * convolutions: random geometry with separate strides and pads, forward in
    both weight orders and backward in both branches, against the oracle;
  * attention: random sequence lengths, head dims and scales.
The bar is the one of the other parity tests: componentwise <= 1e-5*sqrt(K)
against fp64 (or the oracle for the convolution backward)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle
from _parity import abs_denominator, as_kn, as_mk, componentwise_error, normal, tol, uniform
from gpu_common import announce, assert_close, stored_shapes

pytestmark = pytest.mark.gpu

TILES = ["auto", "256x128", "128x128", "128x64", "64x64", "32x32", "128x128k32", "64x64k16", "256x256"]
ACTS = ["linear", "relu", "sigmoid", "tanh"]


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    assert c.arch.startswith("gfx950"), c.arch
    yield c
    c.close()


def _fp64_act(x, act):
    if act == "relu":
        return np.maximum(x, 0.0)
    if act == "sigmoid":
        return 1.0 / (1.0 + np.exp(-x))
    if act == "tanh":
        return np.tanh(x)
    return x


def _size(rng):
    """Log-uniform in [1, 700], with a bias towards tile edges (31..33, 63..65, 127..129)."""
    if rng.random() < 0.25:
        return int(rng.choice([31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 257]))
    return int(np.exp(rng.uniform(0.0, np.log(700.0))))


@pytest.mark.parametrize("seed", range(8))
def test_random_gemms(ctx, seed):
    rng = np.random.default_rng(1000 + seed)
    for case in range(16):
        layout = str(rng.choice(["nn", "nt", "tn"]))
        m, n, k = _size(rng), _size(rng), _size(rng)
        a_shape, b_shape = stored_shapes(layout, m, n, k)
        pad_a, pad_b, pad_c = (int(rng.choice([0, 0, 1, 3, 4])) for _ in range(3))
        off_a, off_b, off_c = (int(rng.choice([0, 0, 1])) for _ in range(3))
        fused = layout == "nn" and rng.random() < 0.35
        accumulate = (not fused) and rng.random() < 0.3
        act = str(rng.choice(ACTS)) if fused else "linear"
        tile = str(rng.choice(TILES))
        splits = int(rng.choice([0, 0, 0, 2, 3]))
        lda, ldb, ldc = a_shape[1] + pad_a, b_shape[1] + pad_b, n + pad_c
        a_full, b_full = uniform(rng, (a_shape[0], lda)), uniform(rng, (b_shape[0], ldb))
        c_full = uniform(rng, (m, ldc))
        bias = uniform(rng, (n,)) if fused else None
        announce(f"random gemm seed {seed} case {case}: {layout} {m}x{n}x{k} ld+({pad_a},{pad_b},{pad_c}) "
                 f"off({off_a},{off_b},{off_c}) acc={accumulate} bias={fused} act={act} tile={tile} splits={splits}")
        bufs = [ctx.to_device(np.concatenate([np.zeros(o, np.float32), x.ravel()]).astype(np.float32))
                for o, x in ((off_a, a_full), (off_b, b_full), (off_c, c_full))]
        dbias = ctx.to_device(bias) if fused else None
        ctx.set_gemm_tile(tile)
        ctx.set_gemm_splits(splits)
        try:
            ctx.sgemm(layout, m, n, k, bufs[0].offset(off_a), lda, bufs[1].offset(off_b), ldb,
                      bufs[2].offset(off_c), ldc, accumulate, dbias, act)
        finally:
            ctx.set_gemm_tile("auto")
            ctx.set_gemm_splits(0)
        got = bufs[2].download()[off_c:].reshape(m, ldc)
        a = np.ascontiguousarray(a_full[:, :a_shape[1]])
        b = np.ascontiguousarray(b_full[:, :b_shape[1]])
        a_mk, b_kn = as_mk(a, layout, m, k).astype(np.float64), as_kn(b, layout, k, n).astype(np.float64)
        ref = a_mk @ b_kn
        c0 = c_full[:, :n]
        if accumulate:
            ref = ref + c0
        if fused:
            ref = _fp64_act(ref + bias.astype(np.float64)[None, :], act)
        assert_close(got[:, :n], ref, layout, a, b, m, n, k, c0=c0.copy() if accumulate else None,
                     accumulate=accumulate, bias=bias, act=act, what=f"seed {seed} case {case}")
        assert np.array_equal(got[:, n:], c_full[:, n:]), "wrote into the padding of C rows"
        for buf in bufs + ([dbias] if dbias is not None else []):
            buf.close()


@pytest.mark.parametrize("seed", range(3))
def test_random_strided_batched(ctx, seed):
    rng = np.random.default_rng(2000 + seed)
    for case in range(6):
        layout = str(rng.choice(["nn", "nt", "tn"]))
        m, n, k = (int(rng.integers(1, 200)) for _ in range(3))
        batch = int(rng.integers(1, 9))
        a_shape, b_shape = stored_shapes(layout, m, n, k)
        gap_a, gap_b, gap_c = (int(rng.choice([0, 1, 5])) for _ in range(3))
        sa, sb, sc = a_shape[0] * a_shape[1] + gap_a, b_shape[0] * b_shape[1] + gap_b, m * n + gap_c
        a = uniform(rng, (batch, sa))
        b = uniform(rng, (batch, sb))
        announce(f"random strided batched seed {seed} case {case}: {layout} {m}x{n}x{k} x{batch} gaps "
                 f"({gap_a},{gap_b},{gap_c})")
        da, db = ctx.to_device(a), ctx.to_device(b)
        dc = ctx.alloc(batch * sc).fill(-3.0)
        ctx.sgemm_strided_batched(layout, m, n, k, da, a_shape[1], sa, db, b_shape[1], sb, dc, n, sc, batch)
        got = dc.download().reshape(batch, sc)
        for i in range(batch):
            ai = a[i, :a_shape[0] * a_shape[1]].reshape(a_shape)
            bi = b[i, :b_shape[0] * b_shape[1]].reshape(b_shape)
            ref = as_mk(ai, layout, m, k).astype(np.float64) @ as_kn(bi, layout, k, n).astype(np.float64)
            assert_close(got[i, :m * n].reshape(m, n), ref, layout, ai, bi, m, n, k, what=f"problem {i}")
            assert np.all(got[i, m * n:] == -3.0), "wrote between problems"
        for buf in (da, db, dc):
            buf.close()


def _conv_case(rng):
    while True:
        B, C, OC = int(rng.integers(1, 4)), int(rng.integers(1, 10)), int(rng.integers(1, 14))
        KH, KW = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        H, W = int(rng.integers(1, 15)), int(rng.integers(1, 17))
        sh, sw = int(rng.choice([1, 1, 2, 3])), int(rng.choice([1, 1, 2, 3]))
        ph, pw = int(rng.integers(0, KH)), int(rng.integers(0, KW))
        OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
        if OH >= 1 and OW >= 1:
            return B, C, H, W, OC, KH, KW, (sh, sw), (ph, pw), OH, OW


@pytest.mark.parametrize("seed", range(4))
def test_random_convolutions(ctx, seed):
    """Forward in both weight orders (implicit GEMM) and backward in both
    branches, on random geometry with separate strides and pads."""
    rng = np.random.default_rng(3000 + seed)
    for case in range(8):
        B, C, H, W, OC, KH, KW, (sh, sw), (ph, pw), OH, OW = _conv_case(rng)
        x, w, bias = uniform(rng, (B, C, H, W)), uniform(rng, (OC, C, KH, KW)), uniform(rng, (OC,))
        go = uniform(rng, (B, OC, OH, OW))
        announce(f"random conv seed {seed} case {case}: B{B} C{C} {H}x{W} OC{OC} k{KH}x{KW} s({sh},{sw}) "
                 f"p({ph},{pw})")
        w_col = np.ascontiguousarray(w.transpose(0, 2, 3, 1).reshape(OC, KH * KW * C))
        col = oracle.im2col(x, B, C, H, W, KH, KW, (sh, sw), (ph, pw)).astype(np.float64)
        ref = (col @ w_col.T.astype(np.float64)).reshape(B, OH * OW, OC).transpose(0, 2, 1) + bias[None, :, None]
        den = (np.abs(col) @ np.abs(w_col.T.astype(np.float64))).reshape(B, OH * OW, OC).transpose(0, 2, 1) \
            + np.abs(bias.astype(np.float64))[None, :, None]
        dx, db = ctx.to_device(x), ctx.to_device(bias)
        do = ctx.alloc(B * OC * OH * OW)
        for order, wt in (("im2col", w_col), ("direct", w)):
            dw = ctx.to_device(wt)
            do.fill(np.nan)
            fn = ctx.conv2d_forward_im2col if order == "im2col" else ctx.conv2d_forward_direct
            fn(dx, dw, db, do, B, C, OC, KH, KW, H, W, OH, OW, sh, sw, ph, pw)
            got = do.download().reshape(B, OC, OH * OW)
            err = np.abs(got - ref) / np.maximum(den, 1e-30)
            assert err.max() <= tol(KH * KW * C), f"forward {order}: {err.max():.3e}"
            dw.close()
        for branch, wt in (("im2col", w_col), ("direct", w)):
            dw, dgo = ctx.to_device(wt), ctx.to_device(go)
            dgi, dgw, dgb = ctx.alloc(B * C * H * W).fill(np.nan), ctx.alloc(w.size).fill(np.nan), ctx.alloc(OC)
            fn = ctx.conv2d_backward_im2col if branch == "im2col" else ctx.conv2d_backward_direct
            fn(dx, dw, dgo, dgi, dgw, dgb, B, C, OC, KH, KW, H, W, OH, OW, sh, sw, ph, pw)
            got = (dgi.download(), dgw.download(), dgb.download())
            refs = oracle.conv2d_backward(x, wt, go, C, OC, KH, KW, H, W, (sh, sw), (ph, pw), branch=branch)
            dens = oracle.conv2d_backward(np.abs(x), np.abs(wt), np.abs(go), C, OC, KH, KW, H, W, (sh, sw), (ph, pw),
                                          branch=branch)
            for name, g, r, d, terms in zip(("grad_input", "grad_weights", "grad_bias"), got, refs, dens,
                                            (OC * KH * KW, B * OH * OW, B * OH * OW)):
                e = np.abs(g.astype(np.float64).ravel() - r.astype(np.float64).ravel())
                assert np.all(e <= tol(terms) * d.astype(np.float64).ravel() + 1e-30), f"backward {branch} {name}"
            for buf in (dw, dgo, dgi, dgw, dgb):
                buf.close()
        for buf in (dx, db, do):
            buf.close()


@pytest.mark.parametrize("seed", range(2))
def test_random_attention(ctx, seed):
    rng = np.random.default_rng(4000 + seed)
    for case in range(6):
        batch, seq, d = int(rng.integers(1, 4)), int(rng.integers(1, 320)), int(rng.integers(1, 160))
        scale = float(rng.choice([1.0 / np.sqrt(d), 0.5, -0.3, 1.7]))
        q, k, v = normal(rng, (batch, seq, d)), normal(rng, (batch, seq, d)), normal(rng, (batch, seq, d))
        announce(f"random attention seed {seed} case {case}: {batch}x{seq}x{d} scale {scale:.3f}")
        dq, dk, dv = ctx.to_device(q), ctx.to_device(k), ctx.to_device(v)
        do = ctx.alloc(batch * seq * d).fill(np.nan)
        ctx.attention_forward(dq, dk, dv, do, batch, seq, d, scale)
        out = do.download().reshape(batch, seq, d)
        for i in range(batch):
            q64, k64, v64 = (t[i].astype(np.float64) for t in (q, k, v))
            s = q64 @ k64.T * scale
            p = np.exp(s - s.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            e_s = tol(d) * (np.abs(q64) @ np.abs(k64).T) * abs(scale)
            rel = 2 * e_s.max(axis=1, keepdims=True) + tol(seq) + 1e-6
            bound = rel * (p @ np.abs(v64))
            assert np.all(np.abs(out[i] - p @ v64) <= 2 * bound), f"head {i}"
        for buf in (dq, dk, dv, do):
            buf.close()

"""GPU parity of the 128x128 register-staged GEMM on rows that are not whole
float4s (zn_sgemm_<layout>_r_u): operands loaded as they lie, 16 bytes at a
4-byte aligned offset, instead of packed copies or 4-byte loads.

Checks, per layout (Backend.matMul, matMulTransposeB, matMulTransposeA:
src/backend.zig:169-182, 298-325):
- against the oracle for K = 1, 2, 3 mod 4 and M, N off multiples of 4,
  split and unsplit, with accumulation and the fused epilogues;
- bit-identical to the 16-byte kernel on zero-padded aligned copies of the
  same operands (same tile, same K order: the padding adds exact zeros);
- a K-contiguous load that runs past K reads the next row's first values:
  with +Inf planted there (and NaN in the row padding past K when the
  leading dimension is longer than K), the other rows stay finite and
  within tolerance, so those values never reach C;
- strided batches with unaligned strides.
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import uniform
from gpu_common import announce, assert_close, ref_gemm, run_gemm, stored_shapes

pytestmark = pytest.mark.gpu

TILE = "128x128k32"


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.set_gemm_tile("auto")
    c.set_gemm_splits(0)
    c.close()


def forced(ctx, splits=0):
    ctx.set_gemm_tile(TILE)
    ctx.set_gemm_splits(splits)


SHAPES = [(130, 131, 97), (257, 129, 250), (200, 300, 771), (96, 130, 1), (131, 65, 6), (1, 129, 515)]


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("m,n,k", SHAPES)
@pytest.mark.parametrize("splits", [1, 3])
def test_unaligned_rows_against_oracle(ctx, layout, m, n, k, splits):
    rng = np.random.default_rng(m * 7 + n * 3 + k + splits)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    c0 = uniform(rng, (m, n))
    forced(ctx, splits)
    try:
        announce(f"unaligned r tile {layout} {m}x{n}x{k} splits {splits}")
        out = run_gemm(ctx, layout, a, b, m, n, k)
        assert_close(out, ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k, what="unaligned")
        out = run_gemm(ctx, layout, a, b, m, n, k, c0=c0.copy(), accumulate=True)
        assert_close(out, ref_gemm(layout, a, b, m, n, k, c0=c0, accumulate=True), layout, a, b, m, n, k,
                     c0=c0, accumulate=True, what="unaligned accumulate")
    finally:
        forced(ctx, 0)
        ctx.set_gemm_tile("auto")


@pytest.mark.parametrize("act", ["linear", "relu", "sigmoid", "tanh"])
def test_unaligned_rows_fused_epilogues(ctx, act):
    m, n, k = 257, 130, 99
    rng = np.random.default_rng(11)
    a, b, bias = uniform(rng, (m, k)), uniform(rng, (k, n)), uniform(rng, (n,))
    forced(ctx)
    try:
        announce(f"unaligned r tile bias+{act}")
        out = run_gemm(ctx, "nn", a, b, m, n, k, bias=bias, act=act)
        assert_close(out, ref_gemm("nn", a, b, m, n, k, bias=bias, act=act), "nn", a, b, m, n, k, bias=bias, act=act,
                     what=f"unaligned bias {act}")
    finally:
        ctx.set_gemm_tile("auto")


def pad_rows(x):
    """x with its rows zero-padded to whole float4s."""
    rows, cols = x.shape
    out = np.zeros((rows, (cols + 3) & ~3), np.float32)
    out[:, :cols] = x
    return out


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("m,n,k,splits", [(257, 131, 517, 1), (260, 255, 203, 2), (129, 385, 1003, 4)])
def test_unaligned_matches_padded_copies_bitwise(ctx, layout, m, n, k, splits):
    rng = np.random.default_rng(k)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    ap, bp = pad_rows(a), pad_rows(b)
    forced(ctx, splits)
    try:
        announce(f"unaligned vs padded {layout} {m}x{n}x{k} splits {splits}")
        out_u = run_gemm(ctx, layout, a, b, m, n, k)
        da, db, dc = ctx.to_device(ap), ctx.to_device(bp), ctx.alloc(m * n).fill(np.nan)
        ctx.sgemm(layout, m, n, k, da, ap.shape[1], db, bp.shape[1], dc, n)
        out_v = dc.download(m * n).reshape(m, n)
        for buf in (da, db, dc):
            buf.close()
    finally:
        forced(ctx, 0)
        ctx.set_gemm_tile("auto")
    np.testing.assert_array_equal(out_u.view(np.uint32), out_v.view(np.uint32))


@pytest.mark.parametrize("layout", ["nn", "nt"])
@pytest.mark.parametrize("extra", [0, 3])
def test_values_past_k_never_reach_c(ctx, layout, extra):
    """Rows of A (and of B for NT) stored with leading dimension K + extra,
    K = 3 mod 4: +Inf at column 0 of every odd row (the value a load running
    past K in the row above reads) and NaN in the padding columns.  The even
    rows (columns) of C must be finite and match the oracle."""
    m, n, k = 200, 136, 131
    rng = np.random.default_rng(extra + (7 if layout == "nt" else 0))
    a = uniform(rng, (m, k))
    b = uniform(rng, (n, k) if layout == "nt" else (k, n))
    a[1::2, 0] = np.inf
    if layout == "nt":
        b[1::2, 0] = np.inf
    lda = k + extra
    ldb = k + extra if layout == "nt" else n
    a_st = np.full((m, lda), np.nan, np.float32)
    a_st[:, :k] = a
    b_st = np.full((n, ldb), np.nan, np.float32) if layout == "nt" else b.copy()
    if layout == "nt":
        b_st[:, :k] = b
    forced(ctx)
    try:
        announce(f"values past K {layout} lda {lda}")
        da, db, dc = ctx.to_device(a_st), ctx.to_device(b_st), ctx.alloc(m * n).fill(np.nan)
        ctx.sgemm(layout, m, n, k, da, lda, db, ldb, dc, n)
        out = dc.download(m * n).reshape(m, n)
        for buf in (da, db, dc):
            buf.close()
    finally:
        ctx.set_gemm_tile("auto")
    rows = np.arange(0, m, 2)
    cols = np.arange(0, n, 2) if layout == "nt" else np.arange(n)
    a_even = np.ascontiguousarray(a[rows])
    b_even = np.ascontiguousarray(b[cols]) if layout == "nt" else b
    sub = out[np.ix_(rows, cols)]
    ref = ref_gemm(layout, a_even, b_even, len(rows), len(cols), k)
    assert_close(sub, ref, layout, a_even, b_even, len(rows), len(cols), k, what=f"past K {layout}")


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_unaligned_strided_batches(ctx, layout):
    m, n, k, batch = 129, 130, 67, 3
    rng = np.random.default_rng(5)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    sa, sb, sc = a_shape[0] * a_shape[1] + 1, b_shape[0] * b_shape[1] + 3, m * n + 1
    a = uniform(rng, (batch * sa,))
    b = uniform(rng, (batch * sb,))
    forced(ctx)
    try:
        announce(f"unaligned strided batch {layout}")
        da, db, dc = ctx.to_device(a), ctx.to_device(b), ctx.alloc(batch * sc).fill(np.nan)
        ctx.sgemm_strided_batched(layout, m, n, k, da, a_shape[1], sa, db, b_shape[1], sb, dc, n, sc, batch)
        out = dc.download(batch * sc)
        for buf in (da, db, dc):
            buf.close()
    finally:
        ctx.set_gemm_tile("auto")
    for z in range(batch):
        az = a[z * sa:z * sa + a_shape[0] * a_shape[1]].reshape(a_shape)
        bz = b[z * sb:z * sb + b_shape[0] * b_shape[1]].reshape(b_shape)
        cz = out[z * sc:z * sc + m * n].reshape(m, n)
        assert_close(cz, ref_gemm(layout, az, bz, m, n, k), layout, az, bz, m, n, k, what=f"batch {z}")


@pytest.mark.parametrize("layout,mode", [(lay, mode) for lay in ("nn", "nt", "tn") for mode in ("plain", "accumulate")]
                         + [("nn", "bias_relu")])  # the fused bias epilogue is Backend.matMulBias*, NN only
def test_row_tail_folded_into_unaligned_launch(ctx, layout, mode):
    """C4's 4097 x 1023 x 777: the automatic choice runs rows 0..4095 on the
    unaligned 128x128 tiles and the last row as dot products inside the same
    launch.  The first 4096 rows are bit-identical to one launch of the same
    kernel over all rows (forcing the tile turns the row split off); the last
    row and sampled rows match the oracle."""
    m, n, k = 4097, 1023, 777
    rng = np.random.default_rng(10 * "nn nt tn".split().index(layout) + "plain accumulate bias_relu".split().index(mode))
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    c0 = uniform(rng, (m, n)) if mode == "accumulate" else None
    bias = uniform(rng, (n,)) if mode == "bias_relu" else None
    act = "relu" if mode == "bias_relu" else "linear"
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    dbias = ctx.to_device(bias) if bias is not None else None
    outs = []
    for tile in ("auto", TILE):
        announce(f"folded row tail {layout} {mode} tile {tile}")
        ctx.set_gemm_tile(tile)
        dc = ctx.to_device(c0) if c0 is not None else ctx.alloc(m * n).fill(np.nan)
        ctx.sgemm(layout, m, n, k, da, lda, db, ldb, dc, n, c0 is not None, dbias, act)
        outs.append(dc.download().reshape(m, n))
        dc.close()
    ctx.set_gemm_tile("auto")
    for buf in (da, db, dbias):
        if buf is not None:
            buf.close()
    split, whole = outs
    assert np.isfinite(split).all()
    np.testing.assert_array_equal(split[:m - 1].view(np.uint32), whole[:m - 1].view(np.uint32))
    rows = np.unique(np.r_[np.linspace(0, m - 1, 8).astype(int), m - 1])
    a_rows = np.ascontiguousarray(a[:, rows] if layout == "tn" else a[rows])
    c0_rows = np.ascontiguousarray(c0[rows]) if c0 is not None else None
    ref = ref_gemm(layout, a_rows, b, len(rows), n, k, c0=c0_rows, accumulate=c0 is not None, bias=bias, act=act)
    assert_close(split[rows], ref, layout, a_rows, b, len(rows), n, k, c0=c0_rows, accumulate=c0 is not None,
                 bias=bias, act=act, what=f"folded tail {mode}")

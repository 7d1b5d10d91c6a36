"""GPU: the persistent GEMM kernels (zn_sgemmp_*) against the plain ones.

A persistent workgroup walks several (problem, tile) items and keeps its LDS
pipeline running across tile boundaries; each output element still sums K in
the same order, so results must be bit-identical to the plain kernels for
every layout, tile, epilogue, accumulation and batch.  The plain kernels are
checked against the oracle elsewhere; one case here is also checked against
the oracle directly.  The deferred-store kernels (zn_sgemmpd_*) are held to
the same bar.
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import uniform
from gpu_common import announce, assert_close, ref_gemm, stored_shapes

pytestmark = pytest.mark.gpu

TILES = {"256x128": 0, "128x128": 1, "128x64": 2, "64x64": 3}


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.set_gemm_tile("auto")
    c.set_gemm_persistent(-1)
    c.close()


def _both(ctx, layout, m, n, k, batch, tile, acc=False, bias=False, act="linear", seed=0):
    rng = np.random.default_rng(seed)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    c0 = uniform(rng, (batch, m, n))
    bv = uniform(rng, (n,)) if bias else None
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    dbias = ctx.to_device(bv) if bias else None
    outs = []
    ctx.set_gemm_tile(TILES[tile])
    for mode in (0, 1):
        ctx.set_gemm_persistent(mode)
        dc = ctx.to_device(c0)
        if batch == 1:
            ctx.sgemm(layout, m, n, k, da, lda, db, ldb, dc, n, acc, dbias, act)
        else:
            ctx.sgemm_strided_batched(layout, m, n, k, da, lda, a_shape[0] * a_shape[1], db, ldb,
                                      b_shape[0] * b_shape[1], dc, n, m * n, batch)
        outs.append(dc.download().reshape(batch, m, n))
        dc.close()
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_persistent(-1)
    for x in (da, db, dbias):
        if x is not None:
            x.close()
    return outs, a, b, c0, bv


CASES = [
    # layout, m, n, k, batch, tile
    ("nt", 1024, 1024, 64, 16, "128x128"),   # the C5 QK^T shape, 16 heads
    ("nn", 1024, 64, 1024, 8, "64x64"),
    ("tn", 780, 516, 96, 3, "128x64"),        # ragged edges in every tile row and column
    ("nn", 1000, 1000, 40, 1, "256x128"),
    ("nt", 4097, 300, 128, 1, "64x64"),
    ("tn", 2048, 2048, 256, 1, "256x128"),
    ("nn", 96, 80, 8, 40, "64x64"),           # K shorter than one slice
]


@pytest.mark.parametrize("layout,m,n,k,batch,tile", CASES)
def test_persistent_bit_identical(ctx, layout, m, n, k, batch, tile):
    announce(f"persistent {layout} {m}x{n}x{k} batch {batch} tile {tile}")
    (plain, pers), *_ = _both(ctx, layout, m, n, k, batch, tile, seed=m + n + k)
    assert np.isfinite(plain).all()
    np.testing.assert_array_equal(pers.view(np.uint32), plain.view(np.uint32))


DEFER_CASES = [
    # layout, m, n, k, batch: plain problems, 128x128 tiles all inside C, K >= 4 slices of 16
    ("nt", 1024, 1024, 64, 16),    # the C5 QK^T shape, 16 heads (stores spread over all 4 slices)
    ("nt", 256, 384, 1024, 3),     # long K: stores in the first 4 of 64 slices
    ("nn", 512, 768, 96, 3),
    ("tn", 384, 256, 80, 5),
    ("nn", 128, 128, 49, 7),       # K one past 3 slices; one tile per problem
    ("nt", 2048, 1024, 64, 1),
    ("nn", 384, 640, 64, 3),       # 45 work items: uneven chunks over the 8 XCDs
]


@pytest.mark.parametrize("layout,m,n,k,batch", DEFER_CASES)
def test_persistent_deferred_stores_bit_identical(ctx, layout, m, n, k, batch):
    """zn_sgemmpd_*: each finished tile is stored during the first four slices
    of the workgroup's next tile, each XCD's workgroups walking a contiguous
    run of work items (8 or more workgroups).  Against the plain persistent kernel (mode 1)
    and the plain kernels (mode 0): the same bits, the default policy (mode -1)
    included, and a second run gives them again."""
    rng = np.random.default_rng(m + 3 * n + k)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    outs = []
    announce(f"deferred stores {layout} {m}x{n}x{k} batch {batch}")
    ctx.set_gemm_tile("128x128")
    for mode in (0, 1, 2, 2, -1):
        ctx.set_gemm_persistent(mode)
        dc = ctx.alloc(batch * m * n).fill(np.nan)
        ctx.sgemm_strided_batched(layout, m, n, k, da, lda, a_shape[0] * a_shape[1], db, ldb,
                                  b_shape[0] * b_shape[1], dc, n, m * n, batch)
        outs.append(dc.download().reshape(batch, m, n))
        dc.close()
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_persistent(-1)
    da.close()
    db.close()
    assert np.isfinite(outs[0]).all()
    for got in outs[1:]:
        np.testing.assert_array_equal(got.view(np.uint32), outs[0].view(np.uint32))
    ref = ref_gemm(layout, a[-1], b[-1], m, n, k)
    assert_close(outs[2][-1], ref, layout, a[-1], b[-1], m, n, k, what="deferred stores")


@pytest.mark.parametrize("act", ["linear", "relu", "sigmoid", "tanh"])
def test_persistent_epilogues_and_accumulate(ctx, act):
    for tile in ("128x128", "64x64"):
        announce(f"persistent epilogue {act} tile {tile}")
        (plain, pers), *_ = _both(ctx, "nn", 700, 900, 72, 1, tile, acc=True, bias=True, act=act, seed=7)
        np.testing.assert_array_equal(pers.view(np.uint32), plain.view(np.uint32))


def test_persistent_against_oracle(ctx):
    m, n, k = 1500, 700, 100
    announce(f"persistent vs oracle nt {m}x{n}x{k}")
    (plain, pers), a, b, c0, _ = _both(ctx, "nt", m, n, k, 1, "128x128", acc=True, seed=3)
    ref = ref_gemm("nt", a[0], b[0], m, n, k, c0=c0[0], accumulate=True)
    assert_close(pers[0], ref, "nt", a[0], b[0], m, n, k, c0=c0[0], accumulate=True, what="persistent")


@pytest.mark.parametrize("layout,m,n,k", [("nn", 4097, 1023, 777), ("tn", 2049, 2048, 512), ("nt", 4100, 1000, 256)])
def test_row_tail_split(ctx, layout, m, n, k):
    """A last row of 64x64 tiles that would put one more workgroup on the
    busiest CU runs as a second, small GEMM: the rows above it are
    bit-identical to the unsplit launch (forcing the tile turns the row split
    off), and sampled rows, the tail included, match the oracle."""
    rng = np.random.default_rng(m + n)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    outs = []
    for tile in ("auto", "64x64"):
        announce(f"row tail {layout} {m}x{n}x{k} tile {tile}")
        ctx.set_gemm_tile(tile)
        dc = ctx.alloc(m * n).fill(np.nan)
        ctx.sgemm(layout, m, n, k, da, lda, db, ldb, dc, n)
        outs.append(dc.download().reshape(m, n))
        dc.close()
    ctx.set_gemm_tile("auto")
    da.close()
    db.close()
    split, whole = outs
    main = (m - 1) // 64 * 64
    assert np.isfinite(split).all()
    np.testing.assert_array_equal(split[:main].view(np.uint32), whole[:main].view(np.uint32))
    rows = np.unique(np.r_[np.linspace(0, m - 1, 16).astype(int), np.arange(main, m)])
    a_rows = np.ascontiguousarray(a[:, rows] if layout == "tn" else a[rows])
    ref = ref_gemm(layout, a_rows, b, len(rows), n, k)
    assert_close(split[rows], ref, layout, a_rows, b, len(rows), n, k, what="row tail")

"""GPU: the intra-workgroup split-K kernels (zn_sgemmk<4|8>_*).

The waves of a workgroup each multiply one 32x32 tile over their own slice of
K and sum the partial tiles in wave order, then apply C_old, the bias and the
activation.  That is the arithmetic of the 32x32 tile split into as many K
slices by separate workgroups and finished by the ordered reduce, so the two
paths must agree bit for bit whenever every wave has a non-empty slice; the
automatic policy is checked against the oracle.  Problems of at most half
the CUs of tiles split K over workgroups too; the last workgroup of a tile
adds the partial tiles in slice order, again the split-K arithmetic.
Problems of at most one 16x16 tile per CU run on 16x16 tiles whose four
waves split K (unless K >= 1536 and the tiles fill under half the CUs).
"""
from __future__ import annotations

import numpy as np
import pytest

from _parity import uniform
from gpu_common import announce, assert_close, ref_gemm, stored_shapes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    yield c
    c.set_gemm_tile("auto")
    c.set_gemm_splits(0)
    c.set_gemm_wave_split(-1)
    c.close()


def _run(ctx, layout, m, n, k, batch, a, b, c0, bias, act, acc, lda, ldb):
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    da, db = ctx.to_device(a), ctx.to_device(b)
    dbias = ctx.to_device(bias) if bias is not None else None
    dc = ctx.to_device(c0)
    if batch == 1:
        ctx.sgemm(layout, m, n, k, da, lda, db, ldb, dc, n, acc, dbias, act)
    else:
        ctx.sgemm_strided_batched(layout, m, n, k, da, lda, a_shape[0] * a_shape[1], db, ldb,
                                  b_shape[0] * b_shape[1], dc, n, m * n, batch)
    out = dc.download().reshape(batch, m, n)
    for x in (da, db, dc, dbias):
        if x is not None:
            x.close()
    return out


CASES = [
    # layout, m, n, k, batch, waves, bias, act, acc
    ("nn", 512, 512, 512, 1, 8, False, "linear", False),
    ("nn", 256, 128, 784, 1, 4, True, "relu", False),   # the C2 first layer
    ("nn", 256, 10, 128, 1, 4, True, "linear", False),  # the C2 second layer (unaligned rows)
    ("tn", 784, 128, 256, 1, 4, False, "linear", False),
    ("nt", 256, 784, 128, 1, 4, False, "linear", True),
    ("nt", 100, 70, 1000, 1, 8, True, "sigmoid", True),  # ragged everywhere
    ("tn", 64, 96, 300, 3, 4, False, "tanh", False),
    ("nn", 33, 65, 200, 5, 4, False, "linear", False),
]


@pytest.mark.parametrize("layout,m,n,k,batch,waves,bias,act,acc", CASES)
def test_wave_split_matches_split_k(ctx, layout, m, n, k, batch, waves, bias, act, acc):
    rng = np.random.default_rng(m * 7 + n + k)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    c0 = uniform(rng, (batch, m, n))
    bv = uniform(rng, (n,)) if bias else None
    if batch > 1:
        bv, act, acc = None, "linear", False  # the strided-batched entry point has no epilogue
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    chunk = -(-(-(-k // waves)) // 32) * 32
    assert (waves - 1) * chunk < k, "every wave has a slice"
    announce(f"wave split {waves} {layout} {m}x{n}x{k} batch {batch} act {act} acc {acc}")
    ctx.set_gemm_wave_split(waves)
    got = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    ctx.set_gemm_wave_split(0)
    ctx.set_gemm_tile("32x32")
    ctx.set_gemm_splits(waves)
    want = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_splits(0)
    ctx.set_gemm_wave_split(-1)
    assert np.isfinite(got).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    if batch == 1:
        ref = ref_gemm(layout, a[0], b[0], m, n, k, c0=c0[0] if acc else None, accumulate=acc, bias=bv, act=act) \
            if (bv is None or layout == "nn") and not (bv is not None and acc) else None
        if ref is not None:
            assert_close(got[0], ref, layout, a[0], b[0], m, n, k, c0=c0[0] if acc else None, accumulate=acc,
                         bias=bv, act=act, what="wave split")


WG_CASES = [
    # layout, m, n, k, batch, bias, act, acc: at most half the CUs of 32x32 tiles, K >= 1536
    ("nn", 256, 96, 1600, 1, True, "relu", False),      # 7 workgroups per tile, 25 slices of 64
    ("nt", 100, 70, 2000, 1, True, "sigmoid", True),    # ragged everywhere
    ("nn", 64, 64, 4096, 1, True, "linear", True),      # 32 slices of 128 (two stages per wave)
    ("nn", 128, 200, 3000, 1, False, "tanh", False),    # 96-wide slices
    ("nt", 32, 32, 1537, 1, False, "linear", False),    # 4-byte staging; the last slice is one column of K
    ("tn", 64, 96, 2048, 3, False, "linear", False),
    ("nn", 33, 65, 1800, 5, False, "linear", False),    # the last workgroup has one slice
]


@pytest.mark.parametrize("layout,m,n,k,batch,bias,act,acc", WG_CASES)
def test_workgroup_split_matches_split_k(ctx, layout, m, n, k, batch, bias, act, acc):
    """Small problems whose K the policy also splits over workgroups: slice q
    (chunk floats of K) goes to wave q % 4 of workgroup q / 4, and the last
    workgroup of each tile adds the slices in order.  That is the 32x32 tile
    split into the same slices by split-K launches and the ordered reduce,
    so the two agree bit for bit; run twice in a row (the tile counters are
    set back to zero by each launch), and checked against the oracle."""
    cus = ctx.compute_units
    tiles = -(-m // 32) * -(-n // 32) * batch
    assert tiles * 2 <= cus
    assert 2 * (-(-m // 16) * -(-n // 16) * batch) < cus, "too few 16x16 tiles for the 16x16 kernels"
    assert k >= 1536
    s0 = min(cus // tiles, -(-k // 128), 8)
    chunk = -(-(-(-k // (4 * s0))) // 32) * 32
    slices = -(-k // chunk)
    assert slices > 4, "more than one workgroup per tile"
    assert -(-(-(-k // slices)) // 32) * 32 == chunk, "split-K with this many slices cuts K the same way"
    rng = np.random.default_rng(m * 3 + n + k)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    c0 = uniform(rng, (batch, m, n))
    bv = uniform(rng, (n,)) if bias else None
    if batch > 1:
        bv, act, acc = None, "linear", False
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    announce(f"workgroup split {layout} {m}x{n}x{k} batch {batch}: {slices} slices of {chunk}")
    got = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    again = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    ctx.set_gemm_wave_split(0)
    ctx.set_gemm_tile("32x32")
    ctx.set_gemm_splits(slices)
    want = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_splits(0)
    ctx.set_gemm_wave_split(-1)
    assert np.isfinite(got).all()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
    # an activation without bias is checked as the oracle's fused form with a zero bias
    rb = bv if bv is not None or act == "linear" else np.zeros(n, np.float32)
    for i in range(batch):
        if rb is not None and (layout != "nn" or acc):
            continue  # the oracle's fused form: NN, bias, no accumulate
        ref = ref_gemm(layout, a[i], b[i], m, n, k, c0=c0[i] if acc else None, accumulate=acc, bias=rb, act=act)
        assert_close(got[i], ref, layout, a[i], b[i], m, n, k, c0=c0[i] if acc else None, accumulate=acc, bias=rb,
                     act=act, what=f"workgroup split problem {i}")


Q_CASES = [
    # layout, m, n, k, batch, bias, act, acc
    ("nn", 256, 128, 784, 1, True, "relu", False),     # the C2 first layer (the policy's choice)
    ("nn", 256, 10, 128, 1, True, "linear", False),    # the C2 second layer (4-byte B rows)
    ("nt", 256, 784, 128, 1, False, "linear", True),
    ("tn", 784, 128, 256, 1, False, "linear", False),
    ("nn", 100, 70, 1000, 1, True, "sigmoid", False),  # ragged
    ("tn", 64, 96, 300, 3, False, "linear", False),
    ("nn", 33, 65, 200, 5, False, "linear", False),
    ("nn", 17, 9, 3000, 1, False, "tanh", False),      # eight waves, 11-12 slices each through one stage (4-byte B)
    ("nt", 31, 47, 4099, 1, False, "linear", True),    # 4-byte staging, 16-17 slices per wave
    ("nn", 64, 64, 2048, 1, False, "linear", False),   # 8 slices per wave through one stage
    ("nt", 48, 40, 224, 2, False, "linear", False),    # four waves (K < 256), every slice in flight
]


@pytest.mark.parametrize("layout,m,n,k,batch,bias,act,acc", Q_CASES)
def test_quarter_tiles_against_oracle(ctx, layout, m, n, k, batch, bias, act, acc):
    """16x16 tiles whose waves split K, forced on every case (K < 256: four
    waves with every slice in flight, zn_sgemmq4_*; else eight waves with
    one LDS stage each, zn_sgemmq8_*): against the oracle, the same bits on
    a second run, and the same
    bits as the automatic choice where the policy picks them (64 <= K <=
    4096 and at most one 32x32 tile per CU; at most one 16x16 tile per CU
    and K < 1536 or tiles for at least half the CUs, or two to three 16x16
    tiles per CU on the two-stage kernels)."""
    rng = np.random.default_rng(m * 5 + n + k)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    c0 = uniform(rng, (batch, m, n))
    bv = uniform(rng, (n,)) if bias else None
    if batch > 1:
        bv, act, acc = None, "linear", False
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    announce(f"16x16 wave split {layout} {m}x{n}x{k} batch {batch} act {act} acc {acc}")
    ctx.set_gemm_wave_split(16)
    got = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    again = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
    ctx.set_gemm_wave_split(-1)
    assert np.isfinite(got).all()
    np.testing.assert_array_equal(again.view(np.uint32), got.view(np.uint32))
    cus = ctx.compute_units
    tiles16 = -(-m // 16) * -(-n // 16) * batch
    tiles32 = -(-m // 32) * -(-n // 32) * batch
    picked = (tiles16 <= cus and (k < 1536 or 2 * tiles16 >= cus)) or cus < tiles16 <= 3 * cus
    if picked and tiles32 <= cus and 64 <= k <= 4096:
        auto = _run(ctx, layout, m, n, k, batch, a, b, c0, bv, act, acc, lda, ldb)
        np.testing.assert_array_equal(auto.view(np.uint32), got.view(np.uint32))
    rb = bv if bv is not None or act == "linear" else np.zeros(n, np.float32)
    for i in range(batch):
        ref = ref_gemm(layout, a[i], b[i], m, n, k, c0=c0[i] if acc else None, accumulate=acc, bias=rb, act=act)
        assert_close(got[i], ref, layout, a[i], b[i], m, n, k, c0=c0[i] if acc else None, accumulate=acc, bias=rb,
                     act=act, what=f"16x16 wave split problem {i}")


def test_policy_small_problems_against_oracle(ctx):
    """The automatic choice for problems of at most one 32x32 tile per CU."""
    rng = np.random.default_rng(5)
    for layout, m, n, k in (("nn", 512, 512, 512), ("nt", 256, 784, 128), ("tn", 784, 128, 256),
                            ("nn", 256, 128, 784), ("nn", 300, 200, 3000)):
        a_shape, b_shape = stored_shapes(layout, m, n, k)
        a, b = uniform(rng, a_shape), uniform(rng, b_shape)
        announce(f"wave split policy {layout} {m}x{n}x{k}")
        got = _run(ctx, layout, m, n, k, 1, a[None], b[None], np.full((1, m, n), np.nan, np.float32), None, "linear",
                   False, m if layout == "tn" else k, k if layout == "nt" else n)[0]
        assert_close(got, ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k, what="wave split policy")


def test_tuning_hooks_reject_bad_values(ctx):
    from zigneuron_amd import InvalidArgumentError
    for bad in (1, 2, 5, 32, -2):
        with pytest.raises(InvalidArgumentError):
            ctx.set_gemm_wave_split(bad)
    for bad in (3, -2):
        with pytest.raises(InvalidArgumentError):
            ctx.set_gemm_persistent(bad)
    from zigneuron_amd import _lib
    for bad in (max(_lib.TILES.values()) + 1, -2):
        with pytest.raises(InvalidArgumentError):
            ctx.set_gemm_tile(bad)
    for name in _lib.TILES:
        ctx.set_gemm_tile(name)
    ctx.set_gemm_tile("auto")
    ctx.set_gemm_wave_split(-1)
    ctx.set_gemm_persistent(-1)

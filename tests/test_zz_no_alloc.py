"""zn_hip_sgemm_noalloc against zn_hip_sgemm, through the C ABI.

The no-allocation GEMM keeps split-K partial sums (and the partial tiles of
the workgroup-split tiles) in the library's fixed 64 MiB per-device scratch
and never packs operands.  Two calls in a row, the
second on a smaller problem, must match zn_hip_sgemm bit for bit wherever
both split K alike, and the oracle within 1e-5*sqrt(K) everywhere; a policy
split too large for the scratch runs unsplit, and a forced one is refused.
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
    c.close()


def run_both(ctx, layout, m, n, k, a, b, lda=None, ldb=None, bias=None, act="linear", c0=None):
    """The same GEMM through zn_hip_sgemm and zn_hip_sgemm_noalloc; returns both C."""
    from zigneuron_amd import _lib
    from zigneuron_amd._lib import check
    from zigneuron_amd.backend import act_id, layout_id
    lda = lda or (m if layout == "tn" else k)
    ldb = ldb or (k if layout == "nt" else n)
    da, db = ctx.to_device(a), ctx.to_device(b)
    dbias = ctx.to_device(bias) if bias is not None else None
    acc = c0 is not None
    outs = []
    for fn in (_lib.load().zn_hip_sgemm, _lib.load().zn_hip_sgemm_noalloc):
        dc = ctx.to_device(c0) if acc else ctx.alloc(m * n).fill(np.nan)
        check(fn(ctx.handle, layout_id(layout), m, n, k, da.ptr, lda, db.ptr, ldb, dc.ptr, n, int(acc),
                 dbias.ptr if dbias is not None else None, act_id(act)), fn.__name__)
        outs.append(dc.download().reshape(m, n))
        dc.close()
    for buf in (da, db, dbias):
        if buf is not None:
            buf.close()
    return outs


def test_noalloc_matches_sgemm_two_calls(ctx):
    """A split-K problem (C3 dW, four slices of K in the scratch), then a
    smaller one with a fused epilogue and accumulation."""
    rng = np.random.default_rng(77)
    m, n, k = 1024, 1024, 4096
    a_shape, b_shape = stored_shapes("tn", m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    announce("noalloc call 1: TN 1024x1024x4096")
    ref_c, got = run_both(ctx, "tn", m, n, k, a, b)
    np.testing.assert_array_equal(got, ref_c)
    assert_close(got, ref_gemm("tn", a, b, m, n, k), "tn", a, b, m, n, k, what="noalloc TN")

    m, n, k = 300, 200, 2000
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    bias, c0 = uniform(rng, (n,)), uniform(rng, (m, n))
    announce("noalloc call 2: NN 300x200x2000 + bias + relu")
    ref_c, got = run_both(ctx, "nn", m, n, k, a, b, bias=bias, act="relu")
    np.testing.assert_array_equal(got, ref_c)
    assert_close(got, ref_gemm("nn", a, b, m, n, k, bias=bias, act="relu"), "nn", a, b, m, n, k, bias=bias,
                 act="relu", what="noalloc bias relu")
    announce("noalloc call 3: NT 300x200x2000 accumulate")
    b_nt = uniform(rng, (n, k))
    ref_c, got = run_both(ctx, "nt", m, n, k, a, b_nt, c0=c0)
    np.testing.assert_array_equal(got, ref_c)
    assert_close(got, ref_gemm("nt", a, b_nt, m, n, k, c0=c0, accumulate=True), "nt", a, b_nt, m, n, k, c0=c0,
                 accumulate=True, what="noalloc accumulate")


def test_noalloc_workgroup_split_tiles(ctx):
    """Few tiles with deep K take the 32x32 tiles whose K is split over
    workgroups too; their partial tiles go to the scratch here and to the
    context's workspace in zn_hip_sgemm, with the same slices and the same
    order.  Two calls in a row (the tile counters are back at zero after
    each), then a smaller problem on the 16x16 tiles."""
    rng = np.random.default_rng(78)
    for m, n, k, bias in ((64, 64, 4096, False), (100, 70, 2000, True), (32, 96, 1600, False)):
        a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
        bv = uniform(rng, (n,)) if bias else None
        announce(f"noalloc workgroup split NN {m}x{n}x{k} bias {bias}")
        for _ in range(2):
            ref_c, got = run_both(ctx, "nn", m, n, k, a, b, bias=bv, act="tanh" if bias else "linear")
            np.testing.assert_array_equal(got.view(np.uint32), ref_c.view(np.uint32))
        assert_close(got, ref_gemm("nn", a, b, m, n, k, bias=bv, act="tanh" if bias else "linear"), "nn", a, b, m,
                     n, k, bias=bv, act="tanh" if bias else "linear", what="noalloc workgroup split")
    m, n, k = 256, 128, 784
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("noalloc 16x16 tiles NN 256x128x784")
    ref_c, got = run_both(ctx, "nn", m, n, k, a, b)
    np.testing.assert_array_equal(got.view(np.uint32), ref_c.view(np.uint32))
    assert_close(got, ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k, what="noalloc 16x16")


def test_noalloc_unaligned_rows_are_not_packed(ctx):
    """Rows that are not whole float4s: zn_hip_sgemm may pack them into
    padded rows (a pooled allocation); the no-allocation GEMM never does and
    stages them with 4-byte loads (or 16-byte loads of the rows as they lie,
    on the 128x128 register-staged tile).  The zeros past K are the same, so
    the result is too."""
    rng = np.random.default_rng(78)
    m, n, k = 1025, 1023, 777
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("noalloc unaligned NN 1025x1023x777")
    ref_c, got = run_both(ctx, "nn", m, n, k, a, b)
    np.testing.assert_array_equal(got, ref_c)
    assert_close(got, ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k, what="noalloc unaligned")


def test_noalloc_split_beyond_scratch(ctx):
    """4097^2 x 4096 NN: the policy splits K three ways (201 MiB of partial
    sums, more than the scratch), so the no-allocation GEMM runs unsplit:
    within the tolerance of the oracle.  A forced split that needs more than
    the scratch is refused; one that fits matches zn_hip_sgemm bit for bit."""
    from zigneuron_amd import InvalidArgumentError
    rng = np.random.default_rng(79)
    m = n = 4097
    k = 4096
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("noalloc NN 4097x4097x4096 (policy split beyond the scratch)")
    _, got = run_both(ctx, "nn", m, n, k, a, b)
    assert_close(got, ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k, what="noalloc unsplit")
    m2, n2, k2 = 1024, 1024, 4096
    a2, b2 = uniform(rng, (m2, k2)), uniform(rng, (k2, n2))
    try:
        ctx.set_gemm_splits(32)  # 32 x 4 MiB of partial sums > 64 MiB
        announce("noalloc forced 32 splits: refused")
        with pytest.raises(InvalidArgumentError):
            run_both(ctx, "nn", m2, n2, k2, a2, b2)
        ctx.set_gemm_splits(8)  # 32 MiB: fits
        announce("noalloc forced 8 splits")
        ref_c, got = run_both(ctx, "nn", m2, n2, k2, a2, b2)
        np.testing.assert_array_equal(got, ref_c)
    finally:
        ctx.set_gemm_splits(0)
    assert_close(got, ref_gemm("nn", a2, b2, m2, n2, k2), "nn", a2, b2, m2, n2, k2, what="noalloc forced split")


def test_noalloc_two_contexts_on_one_device():
    """Two host threads, each with its own context (its own stream) on
    device 0, issue split-K no-allocation GEMMs at the same time.  Both use
    the device's one scratch array; each call waits for the previous call of
    the other context before its kernels run, so every result matches
    zn_hip_sgemm of the same context bit for bit."""
    import threading

    from zigneuron_amd import Context, _lib
    from zigneuron_amd._lib import check
    from zigneuron_amd.backend import layout_id
    lib = _lib.load()
    m, n, k = 1024, 1024, 4096  # TN: four slices of K, 16 MiB of partial sums in the scratch
    rounds = 6
    rng = np.random.default_rng(80)
    a_shape, b_shape = stored_shapes("tn", m, n, k)
    jobs = []
    for i in range(2):
        c = Context(0)
        a, b = uniform(rng, a_shape), uniform(rng, b_shape)
        da, db = c.to_device(a), c.to_device(b)
        ref = c.alloc(m * n).fill(np.nan)
        check(lib.zn_hip_sgemm(c.handle, layout_id("tn"), m, n, k, da.ptr, m, db.ptr, n, ref.ptr, n, 0, None, 0),
              "zn_hip_sgemm")
        outs = [c.alloc(m * n).fill(np.nan) for _ in range(rounds)]
        c.sync()
        jobs.append(dict(ctx=c, a=a, b=b, da=da, db=db, ref=ref, outs=outs, rc=[]))
    start = threading.Barrier(2)

    def issue(job):
        start.wait()
        c = job["ctx"]
        for out in job["outs"]:
            job["rc"].append(lib.zn_hip_sgemm_noalloc(c.handle, layout_id("tn"), m, n, k, job["da"].ptr, m,
                                                      job["db"].ptr, n, out.ptr, n, 0, None, 0))

    announce(f"noalloc from two contexts in two threads: TN {m}x{n}x{k}, {rounds} calls each")
    threads = [threading.Thread(target=issue, args=(job,)) for job in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    try:
        for i, job in enumerate(jobs):
            assert job["rc"] == [0] * rounds, job["rc"]
            want = job["ref"].download().reshape(m, n)
            for r, out in enumerate(job["outs"]):
                got = out.download().reshape(m, n)
                np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32),
                                              err_msg=f"context {i}, call {r}")
            assert_close(want, ref_gemm("tn", job["a"], job["b"], m, n, k), "tn", job["a"], job["b"], m, n, k,
                         what=f"context {i}")
    finally:
        for job in jobs:
            for buf in [job["da"], job["db"], job["ref"]] + job["outs"]:
                buf.close()
            job["ctx"].close()

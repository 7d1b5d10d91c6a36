"""GPU parity: the HIP path against the oracle and the committed fixtures.

Bar: bit-exact where the reference's own known answers are exact (integer
inputs), otherwise max componentwise relative error <= 1e-5 * sqrt(K) in
fp64 (tests/_parity.py).  Every call goes through the C ABI.
"""
from __future__ import annotations

import os
import zlib

import numpy as np
import pytest

from oracle import oracle
from _parity import as_kn, as_mk, normal, tol, uniform
from gpu_common import announce, assert_close, ref_gemm, run_gemm, stored_shapes

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def ctx():
    from zigneuron_amd import Context
    c = Context(0)
    assert c.arch.startswith("gfx950"), c.arch
    yield c
    c.close()


@pytest.fixture(scope="module")
def backend(ctx):
    from zigneuron_amd import Backend
    return Backend(ctx)


@pytest.fixture(scope="module")
def kats():
    return np.load(os.path.join(GOLDEN, "reference_kats.npz"))


# ------------------------------------------------- reference known answers
def test_kat_matmul_correctness(backend, kats):
    announce("kat correctness 2x2x3")
    m, n, k = (int(x) for x in kats["correctness_mnk"])
    c = np.zeros(m * n, np.float32)
    backend.matMul(kats["correctness_a"], kats["correctness_b"], c, m, n, k, False)
    np.testing.assert_array_equal(c, kats["correctness_c"])


def test_kat_matmul_large_ones(backend, kats):
    announce("kat ones 64^3")
    ones = np.ones(64 * 64, np.float32)
    c = np.zeros(64 * 64, np.float32)
    backend.matMul(ones, ones, c, 64, 64, 64, False)
    np.testing.assert_array_equal(c, kats["ones64_c"])


def test_kat_matmul_cpu_small(backend, kats):
    announce("kat cpu small")
    m, n, k = (int(x) for x in kats["cpu_small_mnk"])
    c = np.zeros(m * n, np.float32)
    backend.matMul(kats["cpu_small_a"], kats["cpu_small_b"], c, m, n, k, False)
    assert abs(float(c[0]) - float(kats["cpu_small_c0"][0])) < 1e-4  # the reference test's tolerance


@pytest.mark.parametrize("tag", ["small64", "medium256", "nonsquare", "accum64"])
def test_kat_integer_matmuls_bit_exact(backend, kats, tag):
    """Integer inputs keep every product and partial sum exact: all layouts must match exactly."""
    m, n, k = (int(x) for x in kats[f"{tag}_mnk"])
    a, b = kats[f"{tag}_a"].reshape(m, k), kats[f"{tag}_b"].reshape(k, n)
    want = kats[f"{tag}_c"]
    announce(f"kat integer {tag}")
    c = np.zeros(m * n, np.float32)
    backend.matMul(a, b, c, m, n, k, False)
    if tag == "accum64":
        backend.matMul(a, b, c, m, n, k, True)
        np.testing.assert_array_equal(c, 2 * want)
        return
    np.testing.assert_array_equal(c, want)
    c[:] = np.nan
    backend.matMulTransposeA(a.T.copy(), b, c, m, n, k, False)
    np.testing.assert_array_equal(c, want)
    c[:] = np.nan
    backend.matMulTransposeB(a, b.T.copy(), c, m, n, k, False)
    np.testing.assert_array_equal(c, want)


@pytest.mark.parametrize("layout", ["nn", "nt"])
def test_host_slice_chunked_pipeline(ctx, backend, layout):
    """Host-slice NN/NT calls with A of 16 MiB or more run as row chunks whose
    uploads, GEMMs and downloads overlap on three streams.  Every chunk is an
    unsplit GEMM like the whole problem, so the result is bit-identical to the
    device-pointer call; ragged rows, accumulate and the fused epilogue are
    checked against the oracle."""
    rng = np.random.default_rng(91)
    m, n, k = 4096, 1000, 1024  # two chunks of 2048 rows
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    announce(f"host-slice chunked {layout} {m}x{n}x{k}")
    c = np.full(m * n, np.nan, np.float32)
    fn = backend.matMul if layout == "nn" else backend.matMulTransposeB
    fn(a, b, c, m, n, k, False)
    np.testing.assert_array_equal(c.reshape(m, n), run_gemm(ctx, layout, a, b, m, n, k))
    # ragged rows (three balanced chunks), accumulating
    m = 4100
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    c0 = uniform(rng, (m, n))
    c = c0.ravel().copy()
    announce(f"host-slice chunked {layout} {m}x{n}x{k} accumulate")
    fn(a, b, c, m, n, k, True)
    ref = ref_gemm(layout, a, b, m, n, k, c0=c0, accumulate=True)
    assert_close(c.reshape(m, n), ref, layout, a, b, m, n, k, c0=c0, accumulate=True, what="chunked host")
    if layout == "nn":
        bias = uniform(rng, (n,))
        announce(f"host-slice chunked nn {m}x{n}x{k} bias relu")
        c = np.full(m * n, np.nan, np.float32)
        backend.matMulBiasRelu(a, b, bias, c, m, n, k)
        ref = ref_gemm("nn", a, b, m, n, k, bias=bias, act="relu")
        assert_close(c.reshape(m, n), ref, "nn", a, b, m, n, k, bias=bias, act="relu", what="chunked host")


def test_kat_dense_layer(backend, kats):
    """src/test/unit/layer.zig:16-55,169-241 through the Dense mirror."""
    from zigneuron_amd import Dense
    announce("kat dense layer")
    for act, row in zip(kats["dense_fwd_act"], kats["dense_fwd"]):
        w0, w1, bias, x0, x1, want = (float(v) for v in row)
        lyr = Dense(backend, 2, 1, str(act))
        lyr.weights[:] = [w0, w1]
        lyr.bias[:] = [bias]
        out = np.zeros(1, np.float32)
        lyr.forward(np.float32([x0, x1]), out)
        assert abs(float(out[0]) - want) <= 1e-4, (act, row)
    for act, row in zip(kats["dense_bwd_act"], kats["dense_bwd"]):
        w0, w1, x0, x1, yv, g0, g1 = (float(v) for v in row)
        lyr = Dense(backend, 2, 1, str(act))
        lyr.weights[:] = [w0, w1]
        gi = np.zeros(2, np.float32)
        lyr.backward(np.float32([x0, x1]), np.float32([1.0]), gi, np.float32([yv]))
        np.testing.assert_allclose(gi, [g0, g1], atol=1e-4)


def test_kat_activations(backend, kats):
    announce("kat activations")
    x = kats["act_relu_x"]
    y = np.empty_like(x)
    backend.activationForward("relu", x, y)
    np.testing.assert_array_equal(y, kats["act_relu_y"])
    xs = kats["act_sigmoid_x"]
    s = np.empty_like(xs)
    backend.activationForward("sigmoid", xs, s)
    assert np.all((s >= 0) & (s <= 1)) and abs(float(s[2]) - 0.5) <= 1e-4
    g = np.empty_like(s)
    backend.activationBackward("sigmoid", s, np.ones_like(s), g)
    np.testing.assert_allclose(g, s * (1 - s), atol=1e-4)


# ---------------------------------------------------- committed fixtures
def test_committed_oracle_cases(ctx):
    z = np.load(os.path.join(GOLDEN, "oracle_cases.npz"))
    for name in z["names"]:
        layout, m, n, k, acc, act = (str(v) for v in z[f"{name}_meta"])
        m, n, k, acc = int(m), int(n), int(k), bool(int(acc))
        a, b, bias, c0, want = (z[f"{name}_{s}"] for s in ("a", "b", "bias", "c0", "c"))
        announce(f"fixture {name}")
        if act != "none":
            c = run_gemm(ctx, layout, a, b, m, n, k, bias=bias, act=act)
            assert_close(c, want, layout, a, b, m, n, k, bias=bias, act=act, what=str(name))
        else:
            c = run_gemm(ctx, layout, a, b, m, n, k, c0=c0 if acc else None, accumulate=acc)
            assert_close(c, want, layout, a, b, m, n, k, c0=c0, accumulate=acc, what=str(name))


# ------------------------------------------------------- seeded shapes
SHAPES = [(1, 1, 1), (1, 9, 13), (5, 7, 3), (31, 33, 17), (37, 45, 29), (64, 64, 64), (96, 80, 72),
          (127, 129, 130), (200, 300, 100), (257, 255, 33), (300, 520, 260), (129, 1030, 16)]


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_layouts_against_oracle(ctx, layout, m, n, k):
    rng = np.random.default_rng(zlib.crc32(f"{layout}-{m}-{n}-{k}".encode()))
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    announce(f"{layout} {m}x{n}x{k}")
    c = run_gemm(ctx, layout, a, b, m, n, k)
    assert_close(c, ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k)


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("m,n,k", [(33, 47, 29), (130, 260, 70)])
def test_accumulate_against_oracle(ctx, layout, m, n, k):
    rng = np.random.default_rng(17)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b, c0 = uniform(rng, a_shape), uniform(rng, b_shape), uniform(rng, (m, n))
    announce(f"accumulate {layout} {m}x{n}x{k}")
    c = run_gemm(ctx, layout, a, b, m, n, k, c0=c0, accumulate=True)
    ref = ref_gemm(layout, a, b, m, n, k, c0=c0, accumulate=True)
    assert_close(c, ref, layout, a, b, m, n, k, c0=c0, accumulate=True)


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("batch_size,n,k", [(1, 10, 128), (1, 300, 7), (37, 130, 70), (256, 10, 784),
                                            (513, 65, 33)])
def test_backend_mat_mul_batch(backend, batch_size, n, k, accumulate):
    """Backend.matMulBatch (src/backend.zig:186-195): rows of A against a shared
    B, against the CPU arm cpuMatMulBatch (:2609-2613) row by row.  Host slices
    in and out, with and without accumulate, one row and ragged row counts.
    C is exactly batch_size*n long: the CPU arm's per-row memset clears its
    slice to the end (:2521), which past batch_size*n is a side effect of that
    defect, not part of the operator's result."""
    rng = np.random.default_rng(batch_size * 1000 + n + k)
    a, b = uniform(rng, (batch_size, k)), uniform(rng, (k, n))
    c0 = uniform(rng, (batch_size * n,))
    announce(f"Backend.matMulBatch {batch_size}x{n}x{k} acc={accumulate}")
    c = c0.copy()
    backend.matMulBatch(a.ravel(), b.ravel(), c, batch_size, n, k, accumulate)
    ref = oracle.matmul_batch(a, b, batch_size, n, k, accumulate, c0)
    assert_close(c.reshape(batch_size, n), ref, "nn", a, b, batch_size, n, k,
                 c0=c0 if accumulate else None, accumulate=accumulate, what="matMulBatch")


def test_k_zero_and_empty(ctx):
    announce("k=0 and empty shapes")
    rng = np.random.default_rng(2)
    bias = uniform(rng, (5,))
    c = run_gemm(ctx, "nn", np.zeros(0, np.float32), np.zeros(0, np.float32), 3, 5, 0, bias=bias, act="relu")
    np.testing.assert_array_equal(c, np.broadcast_to(np.maximum(bias, 0), (3, 5)))
    c0 = uniform(rng, (3, 5))
    c = run_gemm(ctx, "nt", np.zeros(0, np.float32), np.zeros(0, np.float32), 3, 5, 0, c0=c0, accumulate=True)
    np.testing.assert_array_equal(c, c0)
    ctx.sgemm("nn", 0, 5, 7, None, 7, None, 5, None, 5)  # m == 0: no-op, no launch


# ---------------------------------------------------------- epilogues
@pytest.mark.parametrize("act", ["linear", "relu", "sigmoid", "tanh"])
@pytest.mark.parametrize("m,n,k", [(256, 128, 784), (256, 10, 128), (45, 33, 70), (300, 257, 129)])
def test_fused_epilogues(ctx, act, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a, b, bias = uniform(rng, (m, k)), uniform(rng, (k, n)), uniform(rng, (n,))
    announce(f"epilogue {act} {m}x{n}x{k}")
    c = run_gemm(ctx, "nn", a, b, m, n, k, bias=bias, act=act)
    ref = ref_gemm("nn", a, b, m, n, k, bias=bias, act=act)
    assert_close(c, ref, "nn", a, b, m, n, k, bias=bias, act=act)


@pytest.mark.parametrize("name", ["matMulBias", "matMulBiasRelu", "matMulBiasSigmoid", "matMulBiasTanh"])
def test_backend_bias_methods(backend, name):
    act = {"matMulBias": "linear", "matMulBiasRelu": "relu", "matMulBiasSigmoid": "sigmoid",
           "matMulBiasTanh": "tanh"}[name]
    rng = np.random.default_rng(4)
    m, n, k = 64, 50, 90
    a, b, bias = uniform(rng, (m, k)), uniform(rng, (k, n)), uniform(rng, (n,))
    c = np.zeros(m * n, np.float32)
    announce(f"Backend.{name}")
    getattr(backend, name)(a, b, bias, c, m, n, k)
    ref = oracle.matmul_bias_act(a, b, bias, m, n, k, act)
    assert_close(c.reshape(m, n), ref, "nn", a, b, m, n, k, bias=bias, act=act)


def test_backend_elementwise_helpers(backend):
    rng = np.random.default_rng(12)
    out, bias = uniform(rng, (13, 37)), uniform(rng, (37,))
    announce("addBias / activation / accumulateBias")
    o = out.ravel().copy()
    backend.addBias(o, bias)
    np.testing.assert_array_equal(o, oracle.add_bias(out, bias).ravel())
    x = np.linspace(-12, 12, 3001).astype(np.float32)
    for act in ("linear", "relu", "sigmoid", "tanh"):
        y = np.empty_like(x)
        backend.activationForward(act, x, y)
        ref = oracle.activation_forward(act, x)
        assert np.all(np.abs(y - ref) <= 2 * np.spacing(np.abs(ref)) + 1e-45), act
        g = uniform(rng, x.shape)
        gi = np.empty_like(x)
        backend.activationBackward(act, ref, g, gi)
        np.testing.assert_array_equal(gi, oracle.activation_backward(act, ref, g))
    gb0 = uniform(rng, (37,))
    gb = gb0.copy()
    backend.accumulateBias(gb, out.ravel())
    np.testing.assert_array_equal(gb, oracle.accumulate_bias(gb0, out))  # same row order: bit-exact


@pytest.mark.parametrize("act", ["linear", "relu", "sigmoid", "tanh"])
def test_dense_forward_reference_sequence_in_place(backend, act):
    """Dense.forward as the reference runs it where the fused dispatch is not
    taken (src/layer.zig:384-407): host-slice matMul into the output, addBias
    on the output in place, then activationForward with the output as its own
    input (`output, output_buf, output, output_buf`).  Each call is checked
    against the oracle on the GPU's own intermediate: the GEMM within the
    tolerance, addBias bit for bit, the in-place activation bit for bit for
    linear and relu and within 2 ulp for sigmoid and tanh; the whole sequence
    also agrees with the fused Backend.matMulBias* within the tolerance."""
    rng = np.random.default_rng(31)
    batch, d_in, d_out = 256, 784, 128  # C2's first layer
    x, w, bias = uniform(rng, (batch, d_in), 0.0, 1.0), uniform(rng, (d_in, d_out)), uniform(rng, (d_out,))
    announce(f"Dense.forward reference sequence, in place, {act}")
    out = np.empty(batch * d_out, np.float32)
    backend.matMul(x, w, out, batch, d_out, d_in, False)
    mm = out.reshape(batch, d_out).copy()
    assert_close(mm, ref_gemm("nn", x, w, batch, d_out, d_in), "nn", x, w, batch, d_out, d_in, what="matMul")
    backend.addBias(out, bias)
    np.testing.assert_array_equal(out, oracle.add_bias(mm, bias).ravel())
    biased = out.copy()
    backend.activationForward(act, out, out)
    ref = oracle.activation_forward(act, biased)
    if act in ("linear", "relu"):
        np.testing.assert_array_equal(out, ref)
    else:
        assert np.all(np.abs(out - ref) <= 2 * np.spacing(np.abs(ref)) + 1e-45), act
    fused = np.empty_like(out)
    getattr(backend, {"linear": "matMulBias", "relu": "matMulBiasRelu", "sigmoid": "matMulBiasSigmoid",
                      "tanh": "matMulBiasTanh"}[act])(x, w, bias, fused, batch, d_out, d_in)
    assert_close(out.reshape(batch, d_out), fused.reshape(batch, d_out), "nn", x, w, batch, d_out, d_in, bias=bias,
                 act=act, what="unfused sequence against matMulBias*")


def test_host_slice_staging_paths(ctx, backend):
    """Host-slice calls take three routes by size: small ones stage their
    inputs through one pinned block (one DMA) and, for small results, let the
    kernel write straight into it; streaming elementwise ops run on the pinned
    block itself; large ones copy through the pinned ring.  Every route must
    give the device-pointer path's (or the oracle's) bits."""
    rng = np.random.default_rng(44)
    cases = [(100, 200, 300), (1024, 512, 64), (1500, 1400, 700)]  # zero-copy C, C by DMA, large
    for m, n, k in cases:
        a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
        bias, c0 = uniform(rng, (n,)), uniform(rng, (m, n))
        announce(f"host-slice staging {m}x{n}x{k}")
        c = np.empty(m * n, np.float32)
        backend.matMulBiasRelu(a, b, bias, c, m, n, k)
        np.testing.assert_array_equal(c.reshape(m, n), run_gemm(ctx, "nn", a, b, m, n, k, bias=bias, act="relu"))
        c = c0.ravel().copy()
        backend.matMulTransposeB(a, np.ascontiguousarray(b.T), c, m, n, k, True)
        np.testing.assert_array_equal(c.reshape(m, n), run_gemm(ctx, "nt", a, np.ascontiguousarray(b.T), m, n, k,
                                                                c0=c0, accumulate=True))
    for rows, cols in ((30, 1000), (300, 1000), (1200, 1000)):  # zero-copy, copies, pinned ring
        announce(f"host-slice elementwise {rows}x{cols}")
        out, bias = uniform(rng, (rows, cols)), uniform(rng, (cols,))
        o = out.ravel().copy()
        backend.addBias(o, bias)
        np.testing.assert_array_equal(o, oracle.add_bias(out, bias).ravel())
        y = oracle.activation_forward("sigmoid", out.ravel())
        got = np.empty_like(y)
        backend.activationForward("sigmoid", out.ravel(), got)
        assert np.all(np.abs(got - y) <= 2 * np.spacing(np.abs(y)) + 1e-45)
        g, gi = uniform(rng, (rows * cols,)), np.empty(rows * cols, np.float32)
        backend.activationBackward("tanh", y, g, gi)
        np.testing.assert_array_equal(gi, oracle.activation_backward("tanh", y, g))
        gb0 = uniform(rng, (cols,))
        gb = gb0.copy()
        backend.accumulateBias(gb, out.ravel())
        np.testing.assert_array_equal(gb, oracle.accumulate_bias(gb0, out))


# ------------------------------------------------------ strided batched
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_strided_batched_against_oracle(ctx, layout):
    rng = np.random.default_rng(31)
    batch, m, n, k = 6, 70, 40, 33
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.alloc(batch * m * n).fill(np.nan)
    announce(f"strided batched {layout}")
    ctx.sgemm_strided_batched(layout, m, n, k, da, lda, m * k, db, ldb, k * n, dc, n, m * n, batch)
    c = dc.download().reshape(batch, m, n)
    for i in range(batch):
        assert_close(c[i], ref_gemm(layout, a[i], b[i], m, n, k), layout, a[i], b[i], m, n, k, what=f"batch {i}")
    # stride 0 shares B across the batch (CudaBackend.matMulBatch's shared B)
    ctx.sgemm_strided_batched(layout, m, n, k, da, lda, m * k, db, ldb, 0, dc, n, m * n, batch)
    c = dc.download().reshape(batch, m, n)
    for i in range(batch):
        assert_close(c[i], ref_gemm(layout, a[i], b[0], m, n, k), layout, a[i], b[0], m, n, k, what=f"shared B {i}")
    for buf in (da, db, dc):
        buf.close()


@pytest.mark.parametrize("layout", ["nn", "tn"])
def test_strided_batched_multi_round_128x128(ctx, layout):
    """A batch whose 128x128 tiles fill three whole rounds (64 problems of
    512 x 384 x 320) goes to the register-staged 128x128 loop: every problem
    bit-identical to the forced two-stage 128x128 kernel and within the
    oracle's tolerance."""
    rng = np.random.default_rng(37)
    batch, m, n, k = 64, 512, 384, 320
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a = uniform(rng, (batch,) + a_shape)
    b = uniform(rng, (batch,) + b_shape)
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.alloc(batch * m * n).fill(np.nan)
    announce(f"strided batched multi-round {layout}")
    ctx.sgemm_strided_batched(layout, m, n, k, da, lda, m * k, db, ldb, k * n, dc, n, m * n, batch)
    auto = dc.download().reshape(batch, m, n)
    ctx.set_gemm_tile("128x128")
    try:
        ctx.sgemm_strided_batched(layout, m, n, k, da, lda, m * k, db, ldb, k * n, dc, n, m * n, batch)
    finally:
        ctx.set_gemm_tile("auto")
    two_stage = dc.download().reshape(batch, m, n)
    assert np.array_equal(auto.view(np.uint32), two_stage.view(np.uint32))
    for i in (0, 17, batch - 1):
        assert_close(auto[i], ref_gemm(layout, a[i], b[i], m, n, k), layout, a[i], b[i], m, n, k, what=f"batch {i}")
    for buf in (da, db, dc):
        buf.close()


# ------------------------------------------- unaligned pointers / leading dims
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_padded_and_unaligned_operands(ctx, layout):
    """Leading dims larger than the row and 4-byte-offset base pointers take the scalar-load path."""
    rng = np.random.default_rng(5)
    m, n, k = 150, 90, 70
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    lda, ldb, ldc = a_shape[1] + 3, b_shape[1] + 5, n + 7
    a_full = uniform(rng, (a_shape[0], lda))
    b_full = uniform(rng, (b_shape[0], ldb))
    da, db = ctx.to_device(np.concatenate([[0.0], a_full.ravel()])), ctx.to_device(b_full)
    dc = ctx.alloc(1 + m * ldc).fill(-7.0)
    announce(f"padded/unaligned {layout}")
    ctx.sgemm(layout, m, n, k, da.offset(1), lda, db, ldb, dc.offset(1), ldc)
    c_full = dc.download()[1:].reshape(m, ldc)
    a = np.ascontiguousarray(a_full[:, :a_shape[1]])
    b = np.ascontiguousarray(b_full[:, :b_shape[1]])
    assert_close(c_full[:, :n], ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k)
    assert np.all(c_full[:, n:] == -7.0), "wrote outside the n columns of a padded C row"
    for buf in (da, db, dc):
        buf.close()


@pytest.mark.parametrize("layout,m,n,k", [("nn", 4097, 1023, 777), ("nt", 1501, 1003, 999), ("tn", 999, 1502, 1001),
                                           ("nn", 40000, 1000, 18), ("nt", 30000, 997, 21)])
def test_large_unaligned_operands_are_packed(ctx, layout, m, n, k):
    """Large problems whose rows are not 16-byte aligned whole float4s are
    staged with 16-byte loads: from zero-padded aligned copies, or on the
    128x128 register-staged tile from the rows as they lie.  Bit-identical to
    the problem with every dimension padded to a multiple of 4 with zeros
    (16-byte staging, no copy), except for a row tail that the 128x128 tile
    computes as dot products in the same launch (another summation order:
    the last 127 rows are compared against fp64 instead), and within
    tolerance of fp64.  The base pointer of A is also one float off
    alignment.  The last two pack rows of only 5 and 6 float4s."""
    rng = np.random.default_rng(6)
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    announce(f"packed operands {layout} {m}x{n}x{k}")
    da = ctx.to_device(np.concatenate([[0.0], a.ravel()]).astype(np.float32))
    db = ctx.to_device(b)
    dc = ctx.alloc(m * n).fill(np.nan)
    ctx.sgemm(layout, m, n, k, da.offset(1), a_shape[1], db, b_shape[1], dc, n)
    c = dc.download().reshape(m, n)
    mp, np_, kp = (-(-d // 4) * 4 for d in (m, n, k))
    pa_shape, pb_shape = stored_shapes(layout, mp, np_, kp)
    pa = np.zeros(pa_shape, np.float32)
    pa[:a_shape[0], :a_shape[1]] = a
    pb = np.zeros(pb_shape, np.float32)
    pb[:b_shape[0], :b_shape[1]] = b
    dpa, dpb = ctx.to_device(pa), ctx.to_device(pb)
    dc2 = ctx.alloc(mp * np_).fill(np.nan)
    ctx.sgemm(layout, mp, np_, kp, dpa, pa_shape[1], dpb, pb_shape[1], dc2, np_)
    bitwise = m - 127  # rows that no folded row tail can hold
    np.testing.assert_array_equal(c[:bitwise], dc2.download().reshape(mp, np_)[:bitwise, :n])
    rows = np.unique(np.r_[np.random.default_rng(7).choice(m, 48, replace=False), np.arange(bitwise, m)])
    a_mk, b_kn = as_mk(a, layout, m, k), as_kn(b, layout, k, n)
    ref = a_mk[rows].astype(np.float64) @ b_kn.astype(np.float64)
    den = np.abs(a_mk[rows]).astype(np.float64) @ np.abs(b_kn).astype(np.float64)
    assert np.all(np.abs(c[rows] - ref) <= tol(k) * den), "packed GEMM outside 1e-5*sqrt(K) of fp64"
    for buf in (da, db, dc, dpa, dpb, dc2):
        buf.close()


# ----------------------------------------------------------- determinism
def test_deterministic_bitwise(ctx):
    rng = np.random.default_rng(9)
    m, n, k = 300, 260, 500
    a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
    announce("determinism")
    c1 = run_gemm(ctx, "nn", a, b, m, n, k)
    c2 = run_gemm(ctx, "nn", a, b, m, n, k)
    np.testing.assert_array_equal(c1, c2)


# ------------------------------------------------------- argument errors
def test_invalid_arguments_are_errors(ctx, backend):
    from zigneuron_amd import InvalidArgumentError
    announce("argument errors")
    d = ctx.alloc(64)
    with pytest.raises(InvalidArgumentError):
        ctx.sgemm(7, 4, 4, 4, d, 4, d, 4, d, 4)  # bad layout
    with pytest.raises(InvalidArgumentError):
        ctx.sgemm("nn", 4, 4, 4, d, 3, d, 4, d, 4)  # lda < k
    with pytest.raises(InvalidArgumentError):
        ctx.sgemm("nn", 4, 4, 4, d, 4, d, 4, d, 4, act=9)
    with pytest.raises(InvalidArgumentError):
        backend.matMul(np.zeros(3, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 2, 2, 2)
    with pytest.raises(InvalidArgumentError):
        backend.activationBackward("relu", np.zeros(3, np.float32), np.zeros(4, np.float32),
                                   np.zeros(3, np.float32))
    d.close()


# ------------------------------------------------ every kernel variant
TILES = ["256x128", "128x128", "128x64", "64x64", "32x32", "128x128k32", "64x64k16", "256x256"]


@pytest.mark.parametrize("aligned", [True, False], ids=["vec16", "vec4"])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
@pytest.mark.parametrize("tile", TILES)
def test_every_tile_variant(ctx, tile, layout, aligned):
    """Force each macro tile on ragged shapes, for both staging widths: plain
    GEMM, then accumulate + bias + tanh through the same kernel."""
    m, n, k = (300, 260, 136) if aligned else (301, 259, 133)
    rng = np.random.default_rng(zlib.crc32(f"{tile}-{layout}-{aligned}".encode()))
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    c0, bias = uniform(rng, (m, n)), uniform(rng, (n,))
    announce(f"tile {tile} {layout} {'vec16' if aligned else 'vec4'}")
    ctx.set_gemm_tile(tile)
    try:
        c = run_gemm(ctx, layout, a, b, m, n, k)
        assert_close(c, ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k, what=tile)
        c = run_gemm(ctx, layout, a, b, m, n, k, c0=c0, accumulate=True, bias=bias, act="tanh")
    finally:
        ctx.set_gemm_tile("auto")
    pre = (ref_gemm(layout, a, b, m, n, k, c0=c0, accumulate=True) + bias[None, :]).astype(np.float32)
    ref = np.tanh(pre.astype(np.float64)).astype(np.float32)
    assert_close(c, ref, layout, a, b, m, n, k, c0=c0, accumulate=True, bias=bias, act="tanh", what=tile + " epi")


@pytest.mark.parametrize("layout", ["nn", "nt", "tn"])
def test_pinned_tiles_bit_identical(ctx, layout):
    """The three-stage loops (pinned: 64x64, 128x128k32, 64x64k16; wide:
    256x256) keep the two-stage loop's K order per element: unsplit results
    are bit-identical to the 128x128 two-stage kernel's, on interior tiles
    (short store path) and edge tiles alike; split into K slices they match
    the oracle."""
    m, n, k = 520, 392, 1040
    rng = np.random.default_rng(zlib.crc32(f"pinned-{layout}".encode()))
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    out = {}
    try:
        ctx.set_gemm_splits(1)
        for tile in ("128x128", "64x64", "128x128k32", "64x64k16", "256x256"):
            announce(f"pinned {layout} {tile} unsplit")
            ctx.set_gemm_tile(tile)
            out[tile] = run_gemm(ctx, layout, a, b, m, n, k)
        for tile in ("64x64", "128x128k32", "64x64k16", "256x256"):
            assert np.array_equal(out[tile].view(np.uint32), out["128x128"].view(np.uint32)), tile
        ref = ref_gemm(layout, a, b, m, n, k)
        assert_close(out["128x128"], ref, layout, a, b, m, n, k, what="128x128")
        ctx.set_gemm_splits(3)
        for tile in ("64x64", "128x128k32", "64x64k16", "256x256"):
            announce(f"pinned {layout} {tile} split 3")
            ctx.set_gemm_tile(tile)
            c = run_gemm(ctx, layout, a, b, m, n, k)
            assert_close(c, ref, layout, a, b, m, n, k, what=tile + " split")
    finally:
        ctx.set_gemm_tile("auto")
        ctx.set_gemm_splits(0)

@pytest.mark.parametrize("layout,m,n,k", [("nn", 4096, 2048, 192), ("nt", 3840, 2048, 160), ("tn", 2048, 4096, 144)])
def test_multi_round_128x128_policy(ctx, layout, m, n, k):
    """Whole rounds of 128x128 tiles with 16-byte rows (two rounds, and 1.9
    for NT) go to the register-staged 128x128 loop by the policy: the result
    is bit-identical to the forced two-stage 128x128 kernel's and matches the
    oracle."""
    rng = np.random.default_rng(zlib.crc32(f"rounds-{layout}-{m}".encode()))
    a_shape, b_shape = stored_shapes(layout, m, n, k)
    a, b = uniform(rng, a_shape), uniform(rng, b_shape)
    announce(f"multi-round 128x128 {layout} {m}x{n}x{k}")
    auto = run_gemm(ctx, layout, a, b, m, n, k)
    ctx.set_gemm_tile("128x128")
    try:
        two_stage = run_gemm(ctx, layout, a, b, m, n, k)
    finally:
        ctx.set_gemm_tile("auto")
    assert np.array_equal(auto.view(np.uint32), two_stage.view(np.uint32))
    assert_close(auto, ref_gemm(layout, a, b, m, n, k), layout, a, b, m, n, k, what="multi-round")


@pytest.mark.parametrize("tile", TILES)
def test_every_tile_strided_batched(ctx, tile):
    rng = np.random.default_rng(77)
    batch, m, n, k = 3, 130, 70, 40
    a, b = uniform(rng, (batch, m, k)), uniform(rng, (batch, n, k))
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.alloc(batch * m * n).fill(np.nan)
    announce(f"tile {tile} batched nt")
    ctx.set_gemm_tile(tile)
    try:
        ctx.sgemm_strided_batched("nt", m, n, k, da, k, m * k, db, k, n * k, dc, n, m * n, batch)
        c = dc.download().reshape(batch, m, n)
    finally:
        ctx.set_gemm_tile("auto")
    for i in range(batch):
        assert_close(c[i], ref_gemm("nt", a[i], b[i], m, n, k), "nt", a[i], b[i], m, n, k, what=f"{tile} {i}")
    for buf in (da, db, dc):
        buf.close()

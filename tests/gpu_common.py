"""Helpers shared by the GPU parity tests: run a GEMM through the C ABI on
device buffers, compute the oracle's answer, and apply the tolerance."""
from __future__ import annotations

import os

import numpy as np

from oracle import oracle
from _parity import abs_denominator, as_kn, as_mk, componentwise_error, normwise_error, tol

THREADS = max(1, min(16, oracle.cpu_count()))


def stored_shapes(layout, m, n, k):
    a_shape = (k, m) if layout == "tn" else (m, k)
    b_shape = (n, k) if layout == "nt" else (k, n)
    return a_shape, b_shape


def run_gemm(ctx, layout, a, b, m, n, k, c0=None, accumulate=False, bias=None, act="linear"):
    """One GEMM on device buffers with the reference's implicit leading dims."""
    lda = m if layout == "tn" else k
    ldb = k if layout == "nt" else n
    da, db = ctx.to_device(a), ctx.to_device(b)
    dc = ctx.to_device(c0) if c0 is not None else ctx.alloc(m * n).fill(np.nan if not accumulate else 0.0)
    dbias = ctx.to_device(bias) if bias is not None else None
    ctx.sgemm(layout, m, n, k, da, max(lda, 1), db, max(ldb, 1), dc, n, accumulate, dbias, act)
    out = dc.download(m * n).reshape(m, n)
    for buf in (da, db, dc, dbias):
        if buf is not None:
            buf.close()
    return out


def ref_gemm(layout, a, b, m, n, k, c0=None, accumulate=False, bias=None, act="linear"):
    """The oracle's answer for one problem (bias/act via the fused CPU fallback semantics)."""
    if bias is not None:
        assert layout == "nn" and not accumulate
        return oracle.matmul_bias_act(a, b, bias, m, n, k, act)
    if layout == "nn":
        if m >= 32 and n >= 32 and k >= 32:
            return oracle.matmul(a, b, m, n, k, accumulate, c0, branch="blocked", threads=THREADS)
        return oracle.matmul(a, b, m, n, k, accumulate, c0)
    if layout == "tn":
        return oracle.matmul_tn(a, b, m, n, k, accumulate, c0, threads=THREADS)
    return oracle.matmul_nt(a, b, m, n, k, accumulate, c0, threads=THREADS)


def assert_close(c, ref, layout, a, b, m, n, k, c0=None, accumulate=False, bias=None, act="linear", what=""):
    den = abs_denominator(as_mk(a, layout, m, k), as_kn(b, layout, k, n), bias,
                          c0.reshape(m, n) if (accumulate and c0 is not None) else None)
    slack = 4 if act in ("sigmoid", "tanh") else 0
    err = componentwise_error(c, ref, den, ulp_slack=slack)
    bound = tol(k)
    assert np.all(np.isfinite(c)), f"{what}: non-finite output"
    assert err <= bound, (f"{what} {layout} m={m} n={n} k={k} acc={accumulate} act={act}: componentwise "
                          f"err {err:.3e} > tol {bound:.3e} (normwise {normwise_error(c, ref):.3e})")
    return err


def assert_close_rows(c, ref, a_mk, b_kn, k, what="", block=1024):
    """assert_close for a large problem, with the fp64 denominators taken in
    row blocks so host memory stays at a few blocks' worth."""
    bound = tol(k)
    abs_b = np.abs(b_kn.astype(np.float64))
    worst = 0.0
    for r0 in range(0, c.shape[0], block):
        r1 = min(c.shape[0], r0 + block)
        cb = c[r0:r1]
        assert np.all(np.isfinite(cb)), f"{what}: non-finite output in rows {r0}:{r1}"
        den = np.abs(a_mk[r0:r1].astype(np.float64)) @ abs_b
        err = componentwise_error(cb, ref[r0:r1], den)
        assert err <= bound, f"{what} rows {r0}:{r1}: componentwise err {err:.3e} > tol {bound:.3e}"
        worst = max(worst, err)
    return worst


def pmap(fn, items, threads=THREADS):
    """fn over items on a thread pool (the oracle's ctypes calls release the
    GIL, so single-threaded oracle functions run side by side)."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        return list(ex.map(fn, items))


def announce(msg: str) -> None:
    """Name the case before each GPU step (flushed), so a failure names it."""
    print(f"[gpu] {msg}", flush=True)
    os.sys.stdout.flush()

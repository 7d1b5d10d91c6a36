"""Error paths that need a device: a code object that loads but lacks a
kernel (ZN_ERR_SYMBOL, the role of src/cuda.zig:262-290), and failures while
the host-slice staging is set up, forced from the host
(ZN_HIP_TEST_SETUP_FAULT, honoured only with ZN_HIP_ENABLE_TEST_HOOKS=1),
after which the context must still work.

Every kernel that runs here is an ordinary, valid launch; the faults are
simulated in host code before any device work uses the staging memory.
"""
from __future__ import annotations

import os
import shutil

import numpy as np
import pytest

from _parity import uniform
from gpu_common import announce, assert_close, ref_gemm, run_gemm

pytestmark = pytest.mark.gpu

OBJECTS = ("zn_gemm_gfx950.hsaco", "zn_conv_gfx950.hsaco", "zn_elementwise_gfx950.hsaco",
           "zn_attention_gfx950.hsaco", "zn_mlp_gfx950.hsaco")


def copy_objects(dst):
    from zigneuron_amd import _lib
    for name in OBJECTS:
        shutil.copyfile(os.path.join(_lib.LIB_DIR, name), os.path.join(dst, name))


def test_missing_kernel_symbol(tmp_path):
    """A valid gfx950 code object without the elementwise kernels in the
    elementwise slot loads, then fails symbol resolution."""
    from zigneuron_amd import Context, SymbolError
    copy_objects(tmp_path)
    shutil.copyfile(tmp_path / "zn_attention_gfx950.hsaco", tmp_path / "zn_elementwise_gfx950.hsaco")
    announce("code object without its kernels")
    with pytest.raises(SymbolError):
        Context(0, str(tmp_path))


def test_copied_code_objects_work(tmp_path):
    from zigneuron_amd import Context
    copy_objects(tmp_path)
    announce("code objects from another directory")
    c = Context(0, str(tmp_path))
    try:
        a = np.ones((64, 64), np.float32)
        np.testing.assert_array_equal(run_gemm(c, "nn", a, a, 64, 64, 64), np.full((64, 64), 64, np.float32))
    finally:
        c.close()


# Set-up steps: 1-5 the pinned staging pair (buffers, events, copier), 11-21
# the chunked pipeline (download ring, chunk events, streams).
STAGING_STEPS = [1, 2, 3, 4, 5]
PIPELINE_STEPS = [11, 12, 14, 15, 18, 19, 20, 21]


@pytest.mark.parametrize("step", STAGING_STEPS + PIPELINE_STEPS)
def test_setup_failure_leaves_a_working_context(monkeypatch, step):
    """A host-slice call whose staging set-up fails at `step` returns
    ZN_ERR_OOM; the next call sets up again from nothing and is correct.
    Small calls use only the staging pair; A of 16 MiB or more also the
    pipeline."""
    from zigneuron_amd import Backend, Context, OutOfMemoryError
    c = Context(0)  # fresh: no staging made yet
    be = Backend(c)
    try:
        rng = np.random.default_rng(step)
        if step < 10:
            m, n, k = 64, 48, 80
        else:
            m, n, k = 2048, 64, 2048  # A is 16 MiB: the chunked pipeline
        a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
        out = np.full(m * n, np.nan, np.float32)
        announce(f"staging set-up fault at step {step}")
        monkeypatch.setenv("ZN_HIP_ENABLE_TEST_HOOKS", "1")
        monkeypatch.setenv("ZN_HIP_TEST_SETUP_FAULT", str(step))
        with pytest.raises(OutOfMemoryError):
            be.matMul(a, b, out, m, n, k)
        monkeypatch.delenv("ZN_HIP_TEST_SETUP_FAULT")
        monkeypatch.delenv("ZN_HIP_ENABLE_TEST_HOOKS")
        be.matMul(a, b, out, m, n, k)
        assert_close(out.reshape(m, n), ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k, what="after the fault")
        again = np.full(m * n, np.nan, np.float32)
        be.matMul(a, b, again, m, n, k)  # and once more on the set-up it made
        np.testing.assert_array_equal(again, out)
    finally:
        c.close()


def test_setup_fault_hook_needs_the_opt_in(monkeypatch):
    """ZN_HIP_TEST_SETUP_FAULT alone changes nothing: without
    ZN_HIP_ENABLE_TEST_HOOKS=1 a host-slice call sets up and computes."""
    from zigneuron_amd import Backend, Context
    c = Context(0)
    be = Backend(c)
    try:
        rng = np.random.default_rng(7)
        m, n, k = 64, 48, 80
        a, b = uniform(rng, (m, k)), uniform(rng, (k, n))
        out = np.full(m * n, np.nan, np.float32)
        announce("set-up fault variable without the opt-in")
        monkeypatch.delenv("ZN_HIP_ENABLE_TEST_HOOKS", raising=False)
        monkeypatch.setenv("ZN_HIP_TEST_SETUP_FAULT", "1")
        be.matMul(a, b, out, m, n, k)
        assert_close(out.reshape(m, n), ref_gemm("nn", a, b, m, n, k), "nn", a, b, m, n, k, what="hook off")
    finally:
        c.close()


def test_hold_stream_waits_on_the_device_and_checks_its_argument():
    """zn_hip_hold_stream (the timing aid that keeps the stream busy while
    the host queues launches): the events around a 300 us hold read at least
    300 us and well under a millisecond; a negative or over-long hold is
    refused before anything is launched."""
    from zigneuron_amd import Context, InvalidArgumentError
    c = Context(0)
    try:
        announce("hold_stream 300 us")
        e0, e1 = c.event(), c.event()
        c.hold_stream(1.0)
        c.sync()
        e0.record()
        c.hold_stream(300.0)
        e1.record()
        ms = e0.elapsed_ms(e1)
        assert 0.3 <= ms < 1.0, ms
        e0.close()
        e1.close()
        for bad in (-1.0, 100001.0, float("nan")):
            with pytest.raises(InvalidArgumentError):
                c.hold_stream(bad)
        c.sync()
    finally:
        c.close()

"""The host library's no-device paths under AddressSanitizer and UBSan (CPU).

zigneuron_amd/lib/asan/libzn_hip.so is the same runtime built with ASan and
UBSan on its host code.  A child Python process loads it with the clang ASan
runtime preloaded and drives what runs without a GPU: the argument checks of
every entry point on null contexts, the status strings, and zn_hip_create's
code-object checks on good, damaged and randomly corrupted copies of this
build's code objects (the bundle-table and ELF-header parser reads untrusted
files).  Any out-of-bounds read, leak of control or undefined behaviour aborts
the child; the test then shows the sanitizer's report.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ASAN_LIB = os.path.join(ROOT, "zigneuron_amd", "lib", "asan", "libzn_hip.so")
RUNTIMES = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))

CHILD = textwrap.dedent(r'''
    import ctypes, os, random, shutil, struct, sys, tempfile
    sys.path.insert(0, ROOT)
    from zigneuron_amd import _lib
    L = ctypes.CDLL(ASAN_LIB)
    for name, (res, args) in _lib.SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    # status strings, including out-of-range codes
    for s in range(-12, 3):
        assert L.zn_hip_status_string(s)
    assert L.zn_hip_abi_version() == 1
    # every entry point that takes a context first: a null context is an argument error
    # (zn_hip_destroy and zn_hip_event_destroy accept null; zn_hip_stream returns null)
    for name, (res, args) in _lib.SIGNATURES.items():
        if not args or args[0] is not _lib.P or name in ("zn_hip_destroy", "zn_hip_stream", "zn_hip_graph_destroy",
                                                         "zn_hip_event_destroy", "zn_hip_last_hip_error"):
            continue
        zeros = []
        for a in args:
            zeros.append(0.0 if a is _lib.F else (None if a in (_lib.P,) or a.__name__.startswith("LP_") else 0))
        rc = getattr(L, name)(*zeros)
        assert rc == _lib.ZN_ERR_INVALID_ARG, (name, rc)
    assert L.zn_hip_destroy(None) == 0 and L.zn_hip_event_destroy(None) == 0
    h = ctypes.c_void_p()
    names = ("zn_gemm_gfx950.hsaco", "zn_conv_gfx950.hsaco", "zn_elementwise_gfx950.hsaco", "zn_attention_gfx950.hsaco",
             "zn_mlp_gfx950.hsaco")
    d = tempfile.mkdtemp()
    for n in names:
        shutil.copyfile(os.path.join(ROOT, "zigneuron_amd", "lib", n), os.path.join(d, n))
    good = L.zn_hip_create(0, d.encode(), ctypes.byref(h))
    assert good in (_lib.ZN_ERR_NO_DEVICE, _lib.ZN_OK), good
    if good == _lib.ZN_OK:
        L.zn_hip_destroy(h)
    assert L.zn_hip_create(0, b"/nonexistent/dir", ctypes.byref(h)) == _lib.ZN_ERR_CODE_OBJECT
    path = os.path.join(d, "zn_elementwise_gfx950.hsaco")  # the smallest of the five
    blob = open(path, "rb").read()
    rng = random.Random(7)
    outcomes = set()
    for trial in range(300):
        b = bytearray(blob)
        kind = trial % 4
        if kind == 0:  # truncate anywhere
            del b[rng.randrange(len(b)):]
        elif kind == 1:  # corrupt the bundle table (first 4 KiB)
            for _ in range(rng.randrange(1, 8)):
                b[rng.randrange(min(len(b), 4096))] = rng.randrange(256)
        elif kind == 2:  # corrupt the ELF header and program/section header fields
            off = blob.index(b"\x7fELF")
            for _ in range(rng.randrange(1, 6)):
                b[off + rng.randrange(64)] = rng.randrange(256)
        else:  # huge entry counts / offsets / sizes in the bundle table
            pos = 24 + 8 * rng.randrange(8)
            if pos + 8 <= len(b):
                struct.pack_into("<Q", b, pos, rng.choice([0, 1, 2**31, 2**63, 2**64 - 1, rng.randrange(2**64)]))
        open(path, "wb").write(bytes(b))
        rc = L.zn_hip_create(0, d.encode(), ctypes.byref(h))
        if rc == _lib.ZN_OK:
            L.zn_hip_destroy(h)
        outcomes.add(rc)
    assert outcomes <= {_lib.ZN_ERR_CODE_OBJECT, _lib.ZN_ERR_NO_DEVICE, _lib.ZN_ERR_SYMBOL, _lib.ZN_OK}, outcomes
    assert _lib.ZN_ERR_CODE_OBJECT in outcomes
    shutil.rmtree(d)
    print("SANITIZED_OK", sorted(outcomes))
''')


@pytest.mark.skipif(not RUNTIMES, reason="clang ASan runtime not found")
@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="the no-device paths need a host without a GPU")
def test_host_library_under_asan_and_ubsan(tmp_path):
    assert os.path.exists(ASAN_LIB), f"{ASAN_LIB} is missing; run __graft_entry__.build()"
    script = tmp_path / "child.py"
    script.write_text(f"ROOT = {ROOT!r}\nASAN_LIB = {ASAN_LIB!r}\n" + CHILD)
    env = dict(os.environ)
    env["LD_PRELOAD"] = ":".join(p for p in (RUNTIMES[-1], os.environ.get("LD_PRELOAD", "")) if p)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, str(script)], env=env, capture_output=True, text=True, timeout=300)
    report = (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0 and "SANITIZED_OK" in r.stdout, report
    assert "AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, report

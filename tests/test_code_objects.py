"""Code-object errors of zn_hip_create, on the CPU.

zn_hip_create checks the five gfx950 code objects on the host before it
touches a device (the role of the module checks in CudaBackend.init,
src/cuda.zig:262-290, and of checkCuda's error mapping,
src/cuda_driver.zig:1119-1160).  A missing directory, a missing, truncated or
foreign file, or a bundle without a gfx950 ELF entry is ZN_ERR_CODE_OBJECT
with or without a GPU; a good directory gets past the check (here: to
ZN_ERR_NO_DEVICE).  The files are this build's own code objects, copied and
altered in a temporary directory.
"""
from __future__ import annotations

import os
import shutil
import struct

import pytest

OBJECTS = ("zn_gemm_gfx950.hsaco", "zn_conv_gfx950.hsaco", "zn_elementwise_gfx950.hsaco",
           "zn_attention_gfx950.hsaco", "zn_mlp_gfx950.hsaco")
BUNDLE = b"__CLANG_OFFLOAD_BUNDLE__"
NO_GPU = not os.path.exists("/dev/kfd")


def lib_dir():
    from zigneuron_amd import _lib
    return _lib.LIB_DIR


def good_copy(dst):
    for name in OBJECTS:
        shutil.copyfile(os.path.join(lib_dir(), name), os.path.join(dst, name))
    return str(dst)


def gfx_entry(blob):
    """(offset, size, triple offset) of the amdgcn entry of an offload bundle."""
    assert blob.startswith(BUNDLE)
    n, = struct.unpack_from("<Q", blob, len(BUNDLE))
    at = len(BUNDLE) + 8
    for _ in range(n):
        off, size, tlen = struct.unpack_from("<QQQ", blob, at)
        at += 24
        triple = blob[at:at + tlen]
        if b"amdgcn" in triple:
            return off, size, at
        at += tlen
    raise AssertionError("no amdgcn entry")


def create(code_dir):
    """Status of zn_hip_create on device 0 with `code_dir`; destroys a context it made."""
    import ctypes
    from zigneuron_amd import _lib
    L = _lib.load()
    h = ctypes.c_void_p()
    rc = L.zn_hip_create(0, code_dir.encode() if code_dir else None, ctypes.byref(h))
    if rc == _lib.ZN_OK:
        L.zn_hip_destroy(h)
    return rc


def alter(path, fn):
    blob = bytearray(open(path, "rb").read())
    fn(blob)
    open(path, "wb").write(bytes(blob))


def test_missing_directory_and_files(tmp_path):
    from zigneuron_amd import _lib
    assert create(str(tmp_path / "nowhere")) == _lib.ZN_ERR_CODE_OBJECT
    assert create(str(tmp_path)) == _lib.ZN_ERR_CODE_OBJECT  # empty directory
    for missing in OBJECTS:
        d = tmp_path / missing.split("_")[1]
        d.mkdir()
        good_copy(d)
        os.remove(d / missing)
        assert create(str(d)) == _lib.ZN_ERR_CODE_OBJECT, missing


@pytest.mark.parametrize("damage", ["truncated_elf", "truncated_table", "garbage", "empty", "other_arch_triple",
                                    "other_arch_elf", "not_amdgpu_elf", "entry_past_end"])
def test_damaged_code_object(tmp_path, damage):
    from zigneuron_amd import _lib
    d = good_copy(tmp_path)
    path = os.path.join(d, "zn_gemm_gfx950.hsaco")
    blob = open(path, "rb").read()
    off, size, tri = gfx_entry(blob)

    def truncated_elf(b):   # the file ends inside the gfx950 ELF
        del b[off + size // 2:]

    def truncated_table(b):  # ELF header intact, section header table cut off
        shoff, = struct.unpack_from("<Q", b, off + 40)
        del b[off + shoff + 8:]

    def garbage(b):
        b[:] = os.urandom(4096)

    def empty(b):
        del b[:]

    def other_arch_triple(b):
        i = b.index(b"gfx950", tri)
        b[i:i + 6] = b"gfx942"

    def other_arch_elf(b):  # EF_AMDGPU_MACH of gfx942 in the ELF header
        flags, = struct.unpack_from("<I", b, off + 48)
        struct.pack_into("<I", b, off + 48, (flags & ~0xFF) | 0x4C)

    def not_amdgpu_elf(b):  # e_machine x86-64
        struct.pack_into("<H", b, off + 18, 62)

    def entry_past_end(b):  # the bundle table claims more bytes than the file holds
        n, = struct.unpack_from("<Q", b, len(BUNDLE))
        at = len(BUNDLE) + 8
        for _ in range(n):
            o, s, t = struct.unpack_from("<QQQ", b, at)
            if o == off:
                struct.pack_into("<Q", b, at + 8, len(b))
            at += 24 + t

    alter(path, locals()[damage])
    assert create(d) == _lib.ZN_ERR_CODE_OBJECT


def test_environment_directory(tmp_path, monkeypatch):
    """With no directory argument, $ZN_HIP_CODE_OBJECT_DIR names it."""
    from zigneuron_amd import _lib
    monkeypatch.setenv("ZN_HIP_CODE_OBJECT_DIR", str(tmp_path))
    assert create(None) == _lib.ZN_ERR_CODE_OBJECT


@pytest.mark.skipif(not NO_GPU, reason="a GPU is present")
def test_good_copy_gets_past_the_check(tmp_path):
    from zigneuron_amd import _lib
    assert create(good_copy(tmp_path)) == _lib.ZN_ERR_NO_DEVICE
    assert create(None) == _lib.ZN_ERR_NO_DEVICE

"""CPU-side tests of the C ABI (no GPU needed): the library loads, exports every
symbol include/zn_hip.h declares, the ctypes table matches the header, the
code objects hold every kernel the runtime resolves, and argument/device
errors come back as status codes."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zn_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zn_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from zigneuron_amd import _lib
    return _lib.load()


def test_header_declares_the_boundary():
    fns = header_functions()
    assert len(fns) >= 35
    for must in ("zn_hip_create", "zn_hip_sgemm", "zn_hip_sgemm_strided_batched", "zn_hip_mat_mul",
                 "zn_hip_mat_mul_transpose_a", "zn_hip_mat_mul_transpose_b", "zn_hip_mat_mul_bias_relu"):
        assert must in fns


def test_library_exports_every_declared_symbol(lib):
    from zigneuron_amd import _lib
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = set(re.findall(r"\sT\s(zn_hip_\w+)", out.stdout))
    missing = [f for f in header_functions() if f not in exported]
    assert not missing, missing
    for f in header_functions():
        assert hasattr(lib, f)


def test_ctypes_table_matches_header():
    from zigneuron_amd import _lib
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_code_objects_hold_every_kernel():
    from zigneuron_amd import _lib
    gemm = open(os.path.join(_lib.LIB_DIR, "zn_gemm_gfx950.hsaco"), "rb").read()
    conv = open(os.path.join(_lib.LIB_DIR, "zn_conv_gfx950.hsaco"), "rb").read()
    elt = open(os.path.join(_lib.LIB_DIR, "zn_elementwise_gfx950.hsaco"), "rb").read()
    attn = open(os.path.join(_lib.LIB_DIR, "zn_attention_gfx950.hsaco"), "rb").read()
    mlp = open(os.path.join(_lib.LIB_DIR, "zn_mlp_gfx950.hsaco"), "rb").read()
    for blob in (gemm, conv, elt, attn, mlp):  # an offload bundle (hipcc --genco) or a bare ELF code object
        assert blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__") or blob[:4] == b"\x7fELF"
    for lay in ("nn", "nt", "tn"):
        for t in ("x", "l", "n", "m", "s", "r", "h"):
            for v in ("", "_v"):
                assert f"zn_sgemm_{lay}_{t}{v}".encode() in gemm
        assert f"zn_sgemm_{lay}_w_v".encode() in gemm  # 16-byte staging only
        for t in ("x", "l", "n", "m"):
            assert f"zn_sgemmp_{lay}_{t}_v".encode() in gemm
        assert f"zn_sgemmpd_{lay}_l_v".encode() in gemm
        assert f"zn_sgemmpd4_{lay}_l_v".encode() in gemm
        for waves in ("4", "8", "4s"):
            for v in ("", "_v"):
                assert f"zn_sgemmk{waves}_{lay}{v}".encode() in gemm
        for v in ("", "_v"):
            for q in ("q4", "q4m"):
                assert f"zn_sgemm{q}_{lay}{v}".encode() in gemm
    for t in ("x", "l", "n", "m", "s"):
        for v in ("", "_v"):
            for g in ("", "_g"):
                assert f"zn_conv_nn_{t}{v}{g}".encode() in conv
            for fam in ("zn_convt_nt", "zn_convw_tn", "zn_convf_nt", "zn_convwn_tn"):
                assert f"{fam}_{t}{v}".encode() in conv
    assert b"zn_convwn_tn_r_v" in conv  # the NHWC weight gradient on the register-staged 128x128 loop
    for lay in ("nn", "nt", "tn"):
        for fam in ("zn_sgemmq4", "zn_sgemmq4m", "zn_sgemmq8"):
            for v in ("", "_v"):
                assert f"{fam}_{lay}{v}".encode() in gemm
        for v in ("_v", "_u"):
            assert f"zn_sgemm_{lay}_r{v}".encode() in gemm
    for k in ("zn_splitk_reduce", "zn_dense_bwd_m", "zn_dense_bwd_m_v", "zn_dense_bwd_k", "zn_dense_bwd_k_v"):
        assert k.encode() in gemm
    for k in ("zn_fill_f32", "zn_copy_f32", "zn_add_bias", "zn_activation_forward", "zn_activation_backward",
              "zn_accumulate_bias", "zn_im2col", "zn_softmax_rows", "zn_col2im", "zn_row_sum", "zn_dense_grad_prologue",
              "zn_hold_stream"):
        assert k.encode() in elt
    for d in (32, 64, 128):
        for v in ("", "_v"):
            assert f"zn_attention_d{d}{v}".encode() in attn
    for k in ("zn_dense_pair_fwd", "zn_dense_pair_fwd_v"):
        assert k.encode() in mlp
    for a1 in range(4):
        for a2 in range(2):
            for v in ("", "_v"):
                assert f"zn_dense_pair_bwd_{a1}{a2}{v}".encode() in mlp
    assert b"gfx950" in gemm and b"gfx950" in conv and b"gfx950" in attn and b"gfx950" in mlp


def test_abi_version_and_status_strings(lib):
    from zigneuron_amd import _lib
    assert lib.zn_hip_abi_version() == 1
    names = {lib.zn_hip_status_string(s).decode().split(":")[0] for s in range(-8, 1)}
    assert len(names) == 9
    assert lib.zn_hip_status_string(-99).decode() == "ZN_ERR_UNKNOWN"


def test_null_and_bad_arguments_without_device(lib):
    """Argument checks that run before any device call."""
    from zigneuron_amd import _lib
    assert lib.zn_hip_set_gemm_tile(None, 0) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_set_gemm_splits(None, 0) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_set_gemm_persistent(None, -1) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_set_gemm_wave_split(None, 4) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_create(0, None, None) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_destroy(None) == _lib.ZN_OK
    assert lib.zn_hip_sgemm(None, 0, 1, 1, 1, None, 1, None, 1, None, 1, 0, None, 0) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_mat_mul(None, None, 0, None, 0, None, 0, 1, 1, 1, 0) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_sync(None) == _lib.ZN_ERR_INVALID_ARG
    assert lib.zn_hip_event_destroy(None) == _lib.ZN_OK
    assert lib.zn_hip_stream(None) is None


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_is_a_clean_error():
    import zigneuron_amd as zn
    assert zn.available() is False
    with pytest.raises(zn.NoDeviceError):
        zn.Context(0)
    with pytest.raises(zn.NoDeviceError):
        zn.Backend.init()


def test_backend_rejects_non_gemm_activation():
    from zigneuron_amd import InvalidArgumentError
    from zigneuron_amd.backend import act_id
    assert act_id("relu") == 1 and act_id("tanh") == 3
    with pytest.raises(InvalidArgumentError):
        act_id("softmax")


def test_dense_init_scales_match_reference():
    """src/layer.zig:330-334: He for relu, Xavier for sigmoid/tanh, sqrt(1/in) for linear."""
    from zigneuron_amd.layer import init_scale, init_weights
    assert init_scale("relu", 784, 128) == pytest.approx((2 / 784) ** 0.5)
    assert init_scale("sigmoid", 128, 10) == pytest.approx((2 / 138) ** 0.5)
    assert init_scale("linear", 128, 10) == pytest.approx((1 / 128) ** 0.5)
    w = init_weights(784, 128, "relu", seed=1)
    assert w.dtype == np.float32 and w.shape == (784, 128)
    assert np.abs(w).max() <= (2 / 784) ** 0.5


@pytest.mark.parametrize("obj", ["zn_gemm_gfx950.s", "zn_conv_gfx950.s", "zn_attention_gfx950.s", "zn_mlp_gfx950.s"])
def test_lds_dma_m0_use_is_confined(obj):
    """The LDS-DMA staging sets M0 right before each buffer_load ... lds; no other
    instruction in the code objects that use it may read or write M0."""
    from zigneuron_amd import _lib
    path = os.path.join(_lib.LIB_DIR, obj)
    lines = [ln.split(";")[0].strip() for ln in open(path)]
    insts = [ln for ln in lines if ln and not ln.startswith((".", "#")) and not ln.endswith(":")]
    m0_writes = 0
    for i, ins in enumerate(insts):
        if re.search(r"\bm0\b", ins):
            assert re.match(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$", ins), ins
            nxt = insts[i + 1]
            assert re.match(r"buffer_load_dword(x4)? ", nxt) and nxt.endswith(" lds"), (ins, nxt)
            m0_writes += 1
        if " lds" in ins and ins.startswith("buffer_load"):
            assert re.match(r"s_mov_b32 m0, (s\d+|vcc_lo|vcc_hi)$", insts[i - 1]), ins
    assert m0_writes > 0

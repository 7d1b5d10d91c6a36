"""The Zig side of the boundary, checked against the C header on the CPU.

No Zig toolchain exists in this image, so zig/hip.zig and
zig/backend_hip.patch are not compiled here.  These tests tie them to
include/zn_hip.h instead, so that neither can drift from the library:
  - every function the header declares has one `pub extern fn` in hip.zig with
    the same name, parameter names and order, and the Zig spelling of each C
    type (and nothing else is declared extern);
  - the enums and the status mapping agree with the header's constants;
  - every HipBackend method calls declared externs with the right number of
    arguments, and every call the patch makes names a HipBackend method with
    the right number of arguments;
  - the patch only inserts lines, and (where the reference tree is present)
    applies to its src/backend.zig and build.zig.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "zn_hip.h")
HIP_ZIG = os.path.join(ROOT, "zig", "hip.zig")
PATCH = os.path.join(ROOT, "zig", "backend_hip.patch")
REFERENCE = "/root/reference"

# C type (as written in the header) -> Zig type in the extern declarations
C_TO_ZIG = {
    "int": "c_int", "int64_t": "i64", "size_t": "usize", "float": "f32",
    "zn_ctx *": "?*Ctx", "const zn_ctx *": "?*const Ctx", "zn_ctx **": "*?*Ctx",
    "const char *": "?[*:0]const u8", "void *": "?*anyopaque", "const void *": "?*const anyopaque",
    "void **": "*?*anyopaque", "zn_device_info *": "*DeviceInfo",
    "zn_graph **": "*?*Graph", "zn_graph *": "?*Graph", "zn_event **": "*?*Event", "zn_event *": "?*Event",
    "const float *": "?[*]const f32", "float *": "?[*]f32",
}
RET_TO_ZIG = {"int": "c_int", "const char *": "[*:0]const u8", "void *": "?*anyopaque"}
OUT_PARAMS = {("zn_hip_event_elapsed_ms", "ms"): "*f32"}  # a single float written back


def norm_ctype(t):
    t = " ".join(t.replace("*", " * ").split())
    return re.sub(r"\* \*", "**", t).replace(" *", " *")


def header_protos():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"((?:const\s+)?\w+\s*\**)\s*(zn_hip_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.S):
        params = []
        args = " ".join(args.split())
        if args != "void":
            for a in args.split(","):
                m = re.match(r"(.*?)(\w+)$", a.strip())
                params.append((m.group(2), norm_ctype(m.group(1))))
        out[name] = (norm_ctype(ret), params)
    return out


def zig_externs():
    text = open(HIP_ZIG).read()
    out = {}
    for name, params, ret in re.findall(r"pub extern fn (\w+)\((.*?)\) ([^;]+);", text):
        ps = []
        if params.strip():
            for p in params.split(", "):
                pn, pt = p.split(": ", 1)
                ps.append((pn, pt.strip()))
        assert name not in out, f"{name} declared twice"
        out[name] = (ret.strip(), ps)
    return out


def split_args(s):
    """Top-level comma split of an argument list."""
    depth, cur, out = 0, "", []
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append(cur.strip())
            cur = ""
        else:
            cur += ch
    if cur.strip():
        out.append(cur.strip())
    return out


def calls(text, prefix):
    """(name, argument count) of every call `prefix<name>(...)` in text."""
    out = []
    for m in re.finditer(re.escape(prefix) + r"(\w+)\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        out.append((m.group(1), len(split_args(text[m.end():i - 1]))))
    return out


def backend_methods():
    text = open(HIP_ZIG).read()
    body = text[text.index("pub const HipBackend = struct {"):]
    out = {}
    for name, params in re.findall(r"pub fn (\w+)\((.*?)\) ", body):
        ps = split_args(params)
        out[name] = len(ps) - (1 if ps and ps[0].startswith("self") else 0)
    return out, body


def test_every_header_function_is_declared_with_its_c_types():
    hdr, zig = header_protos(), zig_externs()
    assert len(hdr) >= 60
    assert sorted(hdr) == sorted(zig), (sorted(set(hdr) ^ set(zig)))
    for name, (cret, cparams) in hdr.items():
        zret, zparams = zig[name]
        assert zret == RET_TO_ZIG[cret], (name, cret, zret)
        assert [p for p, _ in zparams] == [p for p, _ in cparams], (name, zparams, cparams)
        for (pn, ct), (_, zt) in zip(cparams, zparams):
            want = OUT_PARAMS.get((name, pn), C_TO_ZIG[ct])
            assert zt == want, f"{name}({pn}): C {ct!r} -> Zig {zt!r}, expected {want!r}"


def test_constants_agree_with_the_header():
    hdr = open(HEADER).read()
    zig = open(HIP_ZIG).read()
    codes = dict(re.findall(r"#define (ZN_(?:OK|ERR_\w+))\s+\(?(-?\d+)\)?", hdr))
    mapping = dict(re.findall(r"(-?\d+) => error\.(\w+)", zig))
    names = {"ZN_ERR_NO_DEVICE": "NoDevice", "ZN_ERR_CODE_OBJECT": "CodeObject", "ZN_ERR_SYMBOL": "Symbol",
             "ZN_ERR_INVALID_ARG": "InvalidArgument", "ZN_ERR_OOM": "OutOfMemory", "ZN_ERR_LAUNCH": "Launch",
             "ZN_ERR_HIP": "Hip", "ZN_ERR_OVERFLOW": "Overflow"}
    assert codes["ZN_OK"] == "0"
    for c, z in names.items():
        assert mapping[codes[c]] == z, c
    assert len(mapping) == len(names)
    for kind, zig_enum in (("LAYOUT", "Layout"), ("ACT", "Act")):
        hvals = {k.lower(): v for k, v in re.findall(rf"ZN_{kind}_(\w+) = (\d+)", hdr)}
        zdecl = re.search(rf"pub const {zig_enum} = enum\(c_int\) \{{([^}}]*)\}};", zig).group(1)
        zvals = dict(re.findall(r"(\w+) = (\d+)", zdecl))
        assert hvals == zvals, (kind, hvals, zvals)
    assert re.search(r"pub const ABI_VERSION: c_int = (\d+);", zig).group(1) == \
        re.search(r"#define ZN_HIP_ABI_VERSION (\d+)", hdr).group(1)


def test_backend_methods_call_declared_externs():
    zig = zig_externs()
    _, body = backend_methods()
    assert calls(body, "zn_hip_"), "HipBackend calls no extern"
    for name, nargs in calls(body, "zn_"):
        full = "zn_" + name
        assert full in zig, full
        assert nargs == len(zig[full][1]), (full, nargs, len(zig[full][1]))
    # every Backend drop-in of the header (host slices) has a HipBackend method
    methods, _ = backend_methods()
    for must in ("matMul", "matMulBatch", "matMulTransposeA", "matMulTransposeB", "matMulBias", "matMulBiasRelu",
                 "matMulBiasSigmoid", "matMulBiasTanh", "addBias", "accumulateBias", "activationForward",
                 "activationBackward", "conv2dForward", "conv2dBackward", "attentionForward", "sgemm",
                 "sgemmNoAlloc", "sgemmStridedBatched", "denseBackward", "graphBegin", "graphEnd", "graphLaunch"):
        assert must in methods, must


def patch_text():
    return open(PATCH).read()


def test_patch_only_inserts_and_calls_existing_methods():
    text = patch_text()
    hunks = [ln for ln in text.splitlines() if ln.startswith(("+", "-")) and not ln.startswith(("+++", "---"))]
    assert hunks and all(ln.startswith("+") for ln in hunks), "the patch must only insert lines"
    methods, _ = backend_methods()
    added = "\n".join(ln[1:] for ln in hunks)
    used = calls(added, "hip_be.")
    assert {n for n, _ in used} >= {"matMul", "matMulBatch", "matMulTransposeA", "matMulTransposeB", "matMulBias",
                                    "matMulBiasRelu", "matMulBiasSigmoid", "matMulBiasTanh", "addBias",
                                    "accumulateBias", "activationForward", "activationBackward", "conv2dForward",
                                    "conv2dBackward", "attentionForward", "deinit"}
    for name, nargs in used:
        assert name in methods, name
        assert nargs == methods[name], (name, nargs, methods[name])
    assert "hip.HipBackend.init(0)" in added and "hip.actId(act)" in added
    assert re.search(r'b\.option\(bool, "hip"', added)


# Backend's fused Dense-forward methods and their parameter count after self (src/backend.zig:200-295:
# a, a_buf, b, b_buf, bias, bias_buf, c, c_buf, batch_size, n, k)
FUSED_FORWARD = {"linear": "matMulBias", "relu": "matMulBiasRelu", "sigmoid": "matMulBiasSigmoid",
                 "tanh": "matMulBiasTanh"}


def layer_hunk():
    text = patch_text()
    part = text[text.index("--- a/src/layer.zig"):]
    nxt = part.find("\n--- a/", 1)
    return "\n".join(ln[1:] for ln in (part if nxt < 0 else part[:nxt]).splitlines()
                     if ln.startswith("+") and not ln.startswith("+++"))


def test_layer_hunk_routes_dense_forward_to_the_fused_methods():
    """Dense.forward on the HIP backend dispatches each GEMM activation to its
    fused Backend.matMulBias* method with the layer's tensors in the
    method's argument order (the insert sits after Dense.forward's output-size
    check, src/layer.zig:380-382)."""
    added = layer_hunk()
    assert 'const hip_options = @import("hip_options");' in added
    assert "if (hip_options.enable_hip)" in added and "self.backend.hip_backend != null" in added
    used = dict(calls(added, "self.backend."))
    for act, method in FUSED_FORWARD.items():
        assert re.search(rf"\.{act} => return self\.backend\.{method}\(", added), act
        assert used[method] == 11, (method, used[method])
    for method in FUSED_FORWARD.values():
        args = split_args(re.search(rf"self\.backend\.{method}\((.*?)\),?\n", added).group(1))
        assert args == ["input", "input_buf", "w", "w_buf", "b", "b_buf", "output", "output_buf", "batch_size",
                        "self.output_size", "self.input_size"], (method, args)
    # every other activation (softmax, gelu, ...) keeps the reference's three calls
    assert "else => {}," in added


@pytest.mark.skipif(not os.path.isdir(os.path.join(REFERENCE, "src")), reason="reference tree not present")
@pytest.mark.skipif(shutil.which("git") is None, reason="git not available")
def test_patch_applies_to_the_reference(tmp_path):
    os.makedirs(tmp_path / "src")
    shutil.copyfile(os.path.join(REFERENCE, "src", "backend.zig"), tmp_path / "src" / "backend.zig")
    shutil.copyfile(os.path.join(REFERENCE, "build.zig"), tmp_path / "build.zig")
    shutil.copyfile(os.path.join(REFERENCE, "src", "layer.zig"), tmp_path / "src" / "layer.zig")
    subprocess.run(["git", "init", "-q", str(tmp_path)], check=True)
    r = subprocess.run(["git", "apply", "--unidiff-zero", PATCH], cwd=tmp_path, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    patched = (tmp_path / "src" / "backend.zig").read_text()
    # each dispatch line sits right after its method's signature
    for name in ("matMul", "matMulBatch", "matMulTransposeA", "matMulTransposeB", "conv2dForward", "addBias"):
        m = re.search(r"pub fn " + name + r"\(self: Backend,[^\n]*\n([^\n]*)", patched)
        assert m and "hip_be." + name + "(" in m.group(1), name
    # the fused methods the layer hunk calls take 11 arguments after self in the reference
    for method in FUSED_FORWARD.values():
        sig = re.search(r"pub fn " + method + r"\(self: Backend, (.*?)\) !void", patched).group(1)
        assert len(split_args(sig)) == 11, (method, sig)
    layer = (tmp_path / "src" / "layer.zig").read_text()
    fwd = layer[layer.index("pub fn forward(self: *Dense"):]
    fwd = fwd[:fwd.index("pub fn backward(")]
    check = fwd.index("return error.InvalidOutputSize;")
    assert check < fwd.index("if (hip_options.enable_hip)") < fwd.index("try self.backend.matMul(")

"""ctypes front-end of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Restates ZigNeuron's CPU GEMM family (src/backend.zig:2520-2647 and the
epilogue/bias/activation helpers); see oracle/cpu_gemm.c for the per-function
citations and the bit-exactness argument.  Inputs are numpy float32 arrays in
the reference's row-major layouts; every function returns a new array.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ACT = {"linear": 0, "relu": 1, "sigmoid": 2, "tanh": 3}

_lib = None


def build() -> None:
    """Compile oracle/liboracle.so with its Makefile (always rebuilds)."""
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P, S, I, F = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
        sig = {
            "zno_matmul": [P, P, P, S, S, S, I],
            "zno_matmul_unblocked": [P, P, P, S, S, S, I],
            "zno_matmul_blocked": [P, P, P, S, S, S, I],
            "zno_matmul_blocked_omp": [P, P, P, S, S, S, I, I],
            "zno_matmul_batch": [P, P, P, S, S, S, I],
            "zno_matmul_tn": [P, P, P, S, S, S, I],
            "zno_matmul_nt": [P, P, P, S, S, S, I],
            "zno_matmul_tn_omp": [P, P, P, S, S, S, I, I],
            "zno_matmul_nt_omp": [P, P, P, S, S, S, I, I],
            "zno_matmul_bias_act": [P, P, P, P, S, S, S, I],
            "zno_add_bias": [P, S, P, S],
            "zno_activation_forward": [I, P, P, S],
            "zno_activation_backward": [I, P, P, P, S],
            "zno_accumulate_bias": [P, S, P, S],
            "zno_im2col": [P, P] + [S] * 12,
            "zno_conv2d_im2col_gemm": [P, P, P, P, S, S, S, S],
            "zno_attention": [P, P, P, P, P, S, S, F],
            "zno_conv2d_forward": [P, S, P, P, P] + [S] * 12,
            "zno_col2im": [P, P] + [S] * 12,
            "zno_conv2d_backward_direct": [P, P, P, P, P, P] + [S] * 13,
            "zno_conv2d_backward_im2col": [P, P, P, P, P, P] + [S] * 13,
            "zno_conv2d_backward": [P, S, P, P, P, P, P] + [S] * 12,
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        _lib = L
    return _lib


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _p(x: np.ndarray) -> int:
    return x.ctypes.data


def _c_init(c_init, shape):
    return np.zeros(shape, np.float32) if c_init is None else _f32(c_init).reshape(shape).copy()


def matmul(a, b, m, n, k, accumulate=False, c_init=None, branch="auto", threads=1):
    """cpuMatMul: C[m x n] (+)= A[m x k] . B[k x n]."""
    a, b = _f32(a), _f32(b)
    assert a.size == m * k and b.size == k * n
    c = _c_init(c_init if accumulate else None, (m, n))
    L = lib()
    if branch == "auto":
        L.zno_matmul(_p(a), _p(b), _p(c), m, n, k, int(accumulate))
    elif branch == "unblocked":
        L.zno_matmul_unblocked(_p(a), _p(b), _p(c), m, n, k, int(accumulate))
    elif branch == "blocked":
        if threads > 1:
            L.zno_matmul_blocked_omp(_p(a), _p(b), _p(c), m, n, k, int(accumulate), threads)
        else:
            L.zno_matmul_blocked(_p(a), _p(b), _p(c), m, n, k, int(accumulate))
    else:
        raise ValueError(branch)
    return c


def matmul_batch(a, b, batch, n, k, accumulate=False, c_init=None):
    """cpuMatMulBatch (the path Backend.matMul takes for m > 1)."""
    a, b = _f32(a), _f32(b)
    c = _c_init(c_init if accumulate else None, (batch, n))
    lib().zno_matmul_batch(_p(a), _p(b), _p(c), batch, n, k, int(accumulate))
    return c


def matmul_tn(a, b, m, n, k, accumulate=False, c_init=None, threads=1):
    """cpuMatMulTransposeA: C[m x n] (+)= A^T B with A stored [k x m]."""
    a, b = _f32(a), _f32(b)
    assert a.size == k * m and b.size == k * n
    c = _c_init(c_init if accumulate else None, (m, n))
    if threads > 1:
        lib().zno_matmul_tn_omp(_p(a), _p(b), _p(c), m, n, k, int(accumulate), threads)
    else:
        lib().zno_matmul_tn(_p(a), _p(b), _p(c), m, n, k, int(accumulate))
    return c


def matmul_nt(a, b, m, n, k, accumulate=False, c_init=None, threads=1):
    """cpuMatMulTransposeB: C[m x n] (+)= A B^T with B stored [n x k]."""
    a, b = _f32(a), _f32(b)
    assert a.size == m * k and b.size == n * k
    c = _c_init(c_init if accumulate else None, (m, n))
    if threads > 1:
        lib().zno_matmul_nt_omp(_p(a), _p(b), _p(c), m, n, k, int(accumulate), threads)
    else:
        lib().zno_matmul_nt(_p(a), _p(b), _p(c), m, n, k, int(accumulate))
    return c


def matmul_bias_act(a, b, bias, batch, n, k, act="linear"):
    """matMulBias{,Relu,Sigmoid,Tanh} CPU fallbacks."""
    a, b, bias = _f32(a), _f32(b), _f32(bias)
    c = np.zeros((batch, n), np.float32)
    lib().zno_matmul_bias_act(_p(a), _p(b), _p(bias), _p(c), batch, n, k, ACT[act])
    return c


def add_bias(out, bias):
    out, bias = _f32(out).copy(), _f32(bias)
    lib().zno_add_bias(_p(out), out.size, _p(bias), bias.size)
    return out


def activation_forward(act, x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().zno_activation_forward(ACT[act], _p(x), _p(y), x.size)
    return y


def activation_backward(act, y, grad_out):
    y, g = _f32(y), _f32(grad_out)
    gi = np.empty_like(y)
    lib().zno_activation_backward(ACT[act], _p(y), _p(g), _p(gi), y.size)
    return gi


def accumulate_bias(grad_bias, gaa):
    gb, gaa = _f32(grad_bias).copy(), _f32(gaa)
    lib().zno_accumulate_bias(_p(gb), gb.size, _p(gaa), gaa.size)
    return gb


def _geometry(in_h, in_w, k_h, k_w, stride, pad):
    """stride and pad as one int or an (h, w) pair -> (out_h, out_w, sh, sw, ph, pw)."""
    sh, sw = (stride, stride) if np.isscalar(stride) else tuple(stride)
    ph, pw = (pad, pad) if np.isscalar(pad) else tuple(pad)
    return (in_h + 2 * ph - k_h) // sh + 1, (in_w + 2 * pw - k_w) // sw + 1, sh, sw, ph, pw


def im2col(x, batch, channels, in_h, in_w, k_h, k_w, stride=1, pad=0):
    x = _f32(x)
    out_h, out_w, sh, sw, ph, pw = _geometry(in_h, in_w, k_h, k_w, stride, pad)
    col = np.empty((batch * out_h * out_w, k_h * k_w * channels), np.float32)
    lib().zno_im2col(_p(x), _p(col), batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, sh, sw, ph, pw)
    return col


def conv2d_im2col_gemm(col, weights, bias, batch, out_channels, col_height, col_width):
    col, w, bias = _f32(col), _f32(weights), _f32(bias)
    out = np.empty((batch, out_channels, col_height), np.float32)
    lib().zno_conv2d_im2col_gemm(_p(col), _p(w), _p(bias), _p(out), batch, out_channels,
                                 col_height, col_width)
    return out


def conv2d_forward(x, weights, bias, channels, out_channels, k_h, k_w, in_h, in_w, stride=1, pad=0):
    """cpuConv2dForward with its naive / im2col switch; returns [batch, OC, OH, OW]."""
    x, w, bias = _f32(x), _f32(weights), _f32(bias)
    out_h, out_w, sh, sw, ph, pw = _geometry(in_h, in_w, k_h, k_w, stride, pad)
    batch = x.size // (channels * in_h * in_w)
    out = np.empty((batch, out_channels, out_h, out_w), np.float32)
    lib().zno_conv2d_forward(_p(x), x.size, _p(w), _p(bias), _p(out), channels, out_channels, k_h, k_w, in_h, in_w,
                             out_h, out_w, sh, sw, ph, pw)
    return out


def col2im(col, batch, channels, in_h, in_w, k_h, k_w, stride=1, pad=0):
    """Backend.col2im: col [batch*OH*OW, kH*kW*C] -> NCHW [batch, C, H, W]."""
    col = _f32(col)
    out_h, out_w, sh, sw, ph, pw = _geometry(in_h, in_w, k_h, k_w, stride, pad)
    out = np.empty((batch, channels, in_h, in_w), np.float32)
    lib().zno_col2im(_p(col), _p(out), batch, channels, in_h, in_w, k_h, k_w, out_h, out_w, sh, sw, ph, pw)
    return out


def conv2d_backward(x, weights, grad_output, channels, out_channels, k_h, k_w, in_h, in_w, stride=1, pad=0,
                    branch="auto"):
    """cpuConv2dBackward (branch "auto": the reference's size switch; "direct" or
    "im2col" force one branch).  stride and pad: an int or an (h, w) pair.
    Returns (grad_input, grad_weights, grad_bias)."""
    x, w, go = _f32(x), _f32(weights), _f32(grad_output)
    out_h, out_w, sh, sw, ph, pw = _geometry(in_h, in_w, k_h, k_w, stride, pad)
    batch = x.size // (channels * in_h * in_w)
    gi = np.empty((batch, channels, in_h, in_w), np.float32)
    gw = np.empty(out_channels * channels * k_h * k_w, np.float32)
    gb = np.empty(out_channels, np.float32)
    geo = (channels, out_channels, k_h, k_w, in_h, in_w, out_h, out_w, sh, sw, ph, pw)
    if branch == "auto":
        lib().zno_conv2d_backward(_p(x), x.size, _p(w), _p(go), _p(gi), _p(gw), _p(gb), *geo)
    else:
        fn = {"direct": lib().zno_conv2d_backward_direct, "im2col": lib().zno_conv2d_backward_im2col}[branch]
        fn(_p(x), _p(w), _p(go), _p(gi), _p(gw), _p(gb), batch, *geo)
    return gi, gw, gb


def attention(q, k, v, seq_len, d_k, scale):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty((seq_len, d_k), np.float32)
    scores = np.empty(seq_len, np.float32)
    lib().zno_attention(_p(q), _p(k), _p(v), _p(out), _p(scores), seq_len, d_k, float(scale))
    return out


def cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1

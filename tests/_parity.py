"""Shared parity helpers for the tests (seeded inputs, the tolerance metric).

Tolerance: max relative error <= 1e-5 * sqrt(K) in
fp32, measured componentwise in fp64 as

    max_ij |C_gpu - C_ref|_ij / (|A| . |B|)_ij

(entries whose denominator is zero must match exactly).  The normwise value
max|dC| / max|C_ref| is reported alongside.  For fused epilogues the
denominator also carries |bias_j| and, with accumulate, |C0_ij|; sigmoid, tanh
and relu are 1-Lipschitz so the same bound holds on their outputs, plus a
4-ulp allowance for the device exp/tanh.
"""
from __future__ import annotations

import numpy as np


def tol(k: int) -> float:
    return 1e-5 * float(np.sqrt(max(int(k), 1)))


def uniform(rng, shape, lo=-1.0, hi=1.0):
    return (rng.random(shape, dtype=np.float32) * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)


def normal(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def abs_denominator(a_mk, b_kn, bias=None, c0=None):
    """(|A|.|B|)_ij in fp64, plus |bias_j| and |C0_ij| when present."""
    d = np.abs(a_mk.astype(np.float64)) @ np.abs(b_kn.astype(np.float64))
    if bias is not None:
        d = d + np.abs(bias.astype(np.float64))[None, :]
    if c0 is not None:
        d = d + np.abs(c0.astype(np.float64))
    return d


def componentwise_error(c, c_ref, denom, ulp_slack=0):
    """max |c - c_ref| / denom (fp64); entries with denom == 0 must match."""
    c64, r64 = c.astype(np.float64), c_ref.astype(np.float64)
    diff = np.abs(c64 - r64)
    if ulp_slack:
        diff = np.maximum(diff - ulp_slack * np.spacing(np.abs(c_ref).astype(np.float32)).astype(np.float64), 0.0)
    zero = denom == 0
    if np.any(zero) and np.any(diff[zero] != 0):
        return float("inf")
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(zero, 0.0, diff / np.where(zero, 1.0, denom))
    return float(r.max()) if r.size else 0.0


def normwise_error(c, c_ref):
    r64 = c_ref.astype(np.float64)
    scale = np.abs(r64).max() if r64.size else 0.0
    if scale == 0:
        return float(np.abs(c.astype(np.float64)).max()) if c.size else 0.0
    return float(np.abs(c.astype(np.float64) - r64).max() / scale)


def as_mk(a, layout, m, k):
    """A as an [m x k] view for the layout's storage (TN stores A as [k x m])."""
    return a.reshape(k, m).T if layout == "tn" else a.reshape(m, k)


def as_kn(b, layout, k, n):
    """B as a [k x n] view for the layout's storage (NT stores B as [n x k])."""
    return b.reshape(n, k).T if layout == "nt" else b.reshape(k, n)

"""Residual add + RMSNorm restated (test oracle only): the C function
oracle_add_rmsnorm in oracle/c/norm.c follows fastllm_py/graph_decode.py:300-322
(per-thread fma accumulation in the reference's order, halving-tree sum,
fp32 throughout).

Pins (tests/test_oracle_norm.py): a closed form (constant rows of 2.0 with
eps = 0 give inv = 1/2 exactly, so h == w), invariance of h under scaling
x + delta by powers of two (eps = 0), the float64 formula of the reference's
own test (tests/test_fused_ops.py:10-14) within float32 rounding, and xnew ==
x + delta exactly.
"""
from __future__ import annotations

import ctypes

import numpy as np

from .router import _clib


def add_rmsnorm(x, delta, w, eps: float):
    """x, delta (rows, dim), w (dim,) of any float dtype -> (xnew fp32, h fp16)."""
    x = np.asarray(x).astype(np.float32)
    d = np.asarray(delta).astype(np.float32)
    w = np.ascontiguousarray(np.asarray(w).astype(np.float32))
    dim = x.shape[-1]
    x2 = np.ascontiguousarray(x.reshape(-1, dim))
    d2 = np.ascontiguousarray(d.reshape(-1, dim))
    rows = x2.shape[0]
    xnew = np.empty_like(x2)
    y = np.empty_like(x2)
    lib = _clib()
    f = lib.oracle_add_rmsnorm
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_int, ctypes.c_float]
    f(x2.ctypes.data, d2.ctypes.data, w.ctypes.data, xnew.ctypes.data, y.ctypes.data, rows, dim,
      float(eps))
    return xnew.reshape(x.shape), y.astype(np.float16).reshape(x.shape)

"""Elementwise ops adjacent to the quantized matmuls, on the native library.

``add_rmsnorm`` is the reference's fused residual-add + RMSNorm
(fastllm_py/graph_decode.py:291-326 kernel, 715-731 ``_add_rmsnorm``) that
feeds every decode projection; ``swiglu`` between gate/up and down is fused
into the gate/up GEMV instead (``marlin.gemm_swiglu``).
"""
from __future__ import annotations

from .. import _native as nat


def add_rmsnorm(x, delta, weight, eps: float, out=None, stream=None):
    """(x + delta, rmsnorm(x + delta) * weight) for rows of the last axis.

    x, delta, weight: fp32 or fp16 (each independently), on the device.
    Returns (xnew fp32, h fp16) shaped like x, as the reference's
    ``_add_rmsnorm`` does.  ``out`` may be a (xnew, h) pair of preallocated
    contiguous tensors (graph capture)."""
    t = nat.torch()
    ok = (t.float32, t.float16)
    xd, dd, wd = (nat.to_device(v) for v in (x, delta, weight))
    for name, v in (("x", xd), ("delta", dd), ("weight", wd)):
        if v.dtype not in ok:
            raise TypeError(f"add_rmsnorm: {name} must be fp32 or fp16, got {v.dtype}")
    dim = xd.shape[-1]
    if dd.shape != xd.shape or wd.numel() != dim:
        raise ValueError(f"add_rmsnorm: shapes x {tuple(xd.shape)}, delta {tuple(dd.shape)}, "
                         f"weight {tuple(wd.shape)}")
    xd, dd, wd = xd.contiguous(), dd.contiguous(), wd.contiguous()
    rows = xd.numel() // dim
    if out is not None:
        xnew, h = out
    else:
        xnew = t.empty(xd.shape, dtype=t.float32, device=xd.device)
        h = t.empty(xd.shape, dtype=t.float16, device=xd.device)
    hs = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_add_rmsnorm(
        nat.ptr(xd), int(xd.dtype == t.float32), nat.ptr(dd), int(dd.dtype == t.float32),
        nat.ptr(wd), int(wd.dtype == t.float32), nat.ptr(xnew), nat.ptr(h), rows, dim,
        float(eps), hs)
    nat.check_rc(rc, "fastllm_add_rmsnorm")
    return xnew, h

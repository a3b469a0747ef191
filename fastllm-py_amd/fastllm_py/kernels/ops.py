"""Elementwise ops adjacent to the quantized matmuls, on the native library.

``add_rmsnorm`` is the reference's fused residual-add + RMSNorm
(fastllm_py/graph_decode.py:291-326 kernel, 715-731 ``_add_rmsnorm``) that
feeds every decode projection; ``swiglu`` between gate/up and down
(fastllm_py/kernels/ops.py:144-163) normally runs as the epilogue of the
gate/up GEMV (``marlin.gemm_swiglu``) and here on its own for the shapes that
kernel does not take.
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
        nat.check_out(xnew, xd.numel(), (t.float32,), xd.device, "out[0] (xnew)")
        nat.check_out(h, xd.numel(), (t.float16,), xd.device, "out[1] (h)")
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


def swiglu(gate, up, out=None, stream=None):
    """silu(gate) * up in fp32, stored fp16 (reference ops.py:157-163 with fp16
    inputs).  gate and up: fp16 device tensors of one shape (..., cols),
    rows may be strided views (e.g. the two halves of a gate/up output).
    ``out``: optional contiguous fp16 tensor of the same shape."""
    t = nat.torch()
    g, u = nat.to_device(gate), nat.to_device(up)
    if g.dtype != t.float16 or u.dtype != t.float16:
        raise TypeError("swiglu: gate and up must be fp16")
    if g.shape != u.shape:
        raise ValueError(f"swiglu: gate {tuple(g.shape)} and up {tuple(u.shape)} differ")
    cols = g.shape[-1]
    g2, u2 = g.reshape(-1, cols), u.reshape(-1, cols)
    for v in (g2, u2):
        if v.stride(-1) != 1:
            raise ValueError("swiglu: rows must be contiguous")
    rows = g2.shape[0]
    if out is None:
        out = t.empty(g.shape, dtype=t.float16, device=g.device)
    else:
        nat.check_out(out, g.numel(), (t.float16,), g.device)
    hs = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_swiglu(nat.ptr(g2), nat.ptr(u2), nat.ptr(out), rows, cols,
                                  g2.stride(0), u2.stride(0), cols, hs)
    nat.check_rc(rc, "fastllm_swiglu")
    return out

"""GEMV on quantize_int4_group's INT4 format, on the GPU.

The reference stores this format with ``fastllm_py/quantizer.py:97-117``
(``QuantizedTensor`` kind ``"int4_group"``) and reads it only on the host:
``dequantize_int4_group`` (``quantizer.py:120-129``) followed by a numpy
matmul.  This module is that read, done by the HIP kernel
``fastllm_int4_group_gemv`` without materialising the fp32 weights:

  data   : (out, in/2) uint8, two nibbles per byte, even column low
  scales : (out, in/group) float32
  zeros  : (out, in/group) float32, the group minimum
  W[o, i] = q[o, i] * scales[o, i // group] + zeros[o, i // group]
"""
from __future__ import annotations

from .. import _native as nat


def gemv(x, qt, out=None, out_dtype=None):
    """y = x @ dequant(qt)^T.

    x: (in,) or (M, in), fp16 or fp32 (other dtypes are cast to fp32).
    qt: a QuantizedTensor of kind "int4_group" (numpy or device arrays).
    out: optional preallocated (M, out) fp32 or fp16 device tensor.
    out_dtype: fp32 (default) or fp16 when ``out`` is not given.
    Returns a device tensor of shape (out,) for 1-D x, else (M, out)."""
    t = nat.torch()
    if getattr(qt, "kind", None) != "int4_group":
        raise ValueError("gemv needs a QuantizedTensor of kind 'int4_group'")
    out_f, in_f = qt.shape
    xd = nat.to_device(x)
    if xd.dtype not in (t.float32, t.float16):
        xd = xd.to(t.float32)
    if xd.shape[-1] != in_f:
        raise ValueError(f"x has {xd.shape[-1]} features, the weight expects {in_f}")
    x2 = xd.reshape(-1, in_f)
    M = x2.shape[0]
    data = nat.to_device(qt.data, t.uint8)
    scales = nat.to_device(qt.scales, t.float32)
    zeros = nat.to_device(qt.zeros, t.float32)
    if tuple(data.shape) != (out_f, in_f // 2) or scales.numel() != out_f * (in_f // qt.block_size):
        raise ValueError("QuantizedTensor arrays do not match its shape and block size")
    if out is None:
        y = t.empty((M, out_f), dtype=out_dtype or t.float32, device=xd.device)
    else:
        nat.check_out(out, M * out_f, (t.float32, t.float16), xd.device, "out")
        y = out
    rc = nat.lib().fastllm_int4_group_gemv(
        nat.ptr(x2), 1 if x2.dtype == t.float32 else 0, nat.ptr(data), nat.ptr(scales),
        nat.ptr(zeros), nat.ptr(y), 1 if y.dtype == t.float32 else 0, M, out_f, in_f,
        qt.block_size, nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_int4_group_gemv")
    return y.reshape(-1) if (xd.dim() == 1 and out is None) else y

"""Weight quantization: FP8-E4M3 128x128 block and INT4 group quantization.

Same API as the reference's ``fastllm_py/quantizer.py`` (lines 13-129); the
arithmetic runs in gfx950 HIP kernels (csrc/packers.hip) that reproduce the
reference's numpy formulas bit for bit.  numpy input gives numpy output
(computed on the GPU and copied back); torch input gives device tensors.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native as nat

FP8_E4M3_MAX = 448.0


@dataclass
class QuantizedTensor:
    """A packed weight.  Fields keep the reference's names and order (its
    loaders construct and read them positionally): ``kind`` names the format,
    "fp8_e4m3_block" or "int4_group"; ``data`` holds the packed codes as
    uint8 (numpy or a device tensor); ``scales`` the float32 scale per block
    or group; ``shape`` the unpacked (out_features, in_features);
    ``block_size`` the block edge or group length; ``zeros`` the int4 group
    minimum (None for fp8)."""

    kind: str
    data: object
    scales: object
    shape: tuple[int, int]
    block_size: int
    zeros: object = None


def _f32_device(x):
    t = nat.torch()
    if isinstance(x, np.ndarray):
        return nat.to_device(np.ascontiguousarray(x, dtype=np.float32))
    return nat.to_device(x, t.float32)


def _fp8_e4m3_encode(x, xp=np):
    """float array -> uint8 e4m3fn bytes, the reference encoder
    (quantizer.py:26-51, including its subnormal clip-to-7)."""
    t = nat.torch()
    numpy_in = nat.host_out(x, xp)
    xd = _f32_device(np.asarray(x) if numpy_in else x)
    out = t.empty(xd.shape, dtype=t.uint8, device=xd.device)
    rc = nat.lib().fastllm_fp8_e4m3_encode(nat.ptr(xd), nat.ptr(out), xd.numel(),
                                           nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_fp8_e4m3_encode")
    return nat.as_output(out, numpy_in)


def _fp8_e4m3_decode(b, xp=np):
    """uint8 e4m3fn -> float32, exact (quantizer.py:54-62)."""
    t = nat.torch()
    numpy_in = nat.host_out(b, xp)
    bd = nat.to_device(np.asarray(b).astype(np.uint8) if numpy_in else b, t.uint8)
    out = t.empty(bd.shape, dtype=t.float32, device=bd.device)
    rc = nat.lib().fastllm_fp8_e4m3_decode(nat.ptr(bd), nat.ptr(out), bd.numel(),
                                           nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_fp8_e4m3_decode")
    return nat.as_output(out, numpy_in)


def quantize_fp8_block(w, block_size: int = 128, xp=np) -> QuantizedTensor:
    """Per (bs x bs) 2-D block scaling (quantizer.py:65-85).

    w: (out_features, in_features). scales: (ceil(out/bs), ceil(in/bs)) fp32;
    data cropped to (out, in) uint8."""
    t = nat.torch()
    numpy_in = nat.host_out(w, xp)
    wd = _f32_device(w)
    out_f, in_f = wd.shape
    bs = int(block_size)
    q = t.empty((out_f, in_f), dtype=t.uint8, device=wd.device)
    scales = t.empty(((out_f + bs - 1) // bs, (in_f + bs - 1) // bs), dtype=t.float32,
                     device=wd.device)
    rc = nat.lib().fastllm_quantize_fp8_block(nat.ptr(wd), nat.ptr(q), nat.ptr(scales), out_f,
                                              in_f, bs, nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_fp8_block")
    return QuantizedTensor("fp8_e4m3_block", nat.as_output(q, numpy_in),
                           nat.as_output(scales, numpy_in), (out_f, in_f), bs)


def dequantize_fp8_block(qt: QuantizedTensor, xp=np):
    """decode(q) * block scale (quantizer.py:88-94)."""
    t = nat.torch()
    numpy_in = nat.host_out(qt.data, xp)
    out_f, in_f = qt.shape
    q = nat.to_device(qt.data, t.uint8)
    s = _f32_device(qt.scales)
    out = t.empty((out_f, in_f), dtype=t.float32, device=q.device)
    rc = nat.lib().fastllm_dequantize_fp8_block(nat.ptr(q), nat.ptr(s), nat.ptr(out), out_f, in_f,
                                                qt.block_size, nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_dequantize_fp8_block")
    return nat.as_output(out, numpy_in)


def quantize_int4_group(w, group_size: int = 128, xp=np) -> QuantizedTensor:
    """Asymmetric INT4 with per-group min/max scaling along in_features
    (quantizer.py:97-117).  data (out, in/2) uint8, even column in the low
    nibble; scales and zeros (= group minimum) (out, in/group) float32."""
    t = nat.torch()
    numpy_in = nat.host_out(w, xp)
    wd = _f32_device(w)
    out_f, in_f = wd.shape
    assert in_f % group_size == 0 and in_f % 2 == 0
    packed = t.empty((out_f, in_f // 2), dtype=t.uint8, device=wd.device)
    scales = t.empty((out_f, in_f // group_size), dtype=t.float32, device=wd.device)
    zeros = t.empty_like(scales)
    rc = nat.lib().fastllm_quantize_int4_group(nat.ptr(wd), nat.ptr(packed), nat.ptr(scales),
                                               nat.ptr(zeros), out_f, in_f, group_size,
                                               nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_int4_group")
    return QuantizedTensor("int4_group", nat.as_output(packed, numpy_in),
                           nat.as_output(scales, numpy_in), (out_f, in_f), group_size,
                           zeros=nat.as_output(zeros, numpy_in))


def dequantize_int4_group(qt: QuantizedTensor, xp=np):
    """q * scale + zero (quantizer.py:120-129)."""
    t = nat.torch()
    numpy_in = nat.host_out(qt.data, xp)
    out_f, in_f = qt.shape
    p = nat.to_device(qt.data, t.uint8)
    s = _f32_device(qt.scales)
    z = _f32_device(qt.zeros)
    out = t.empty((out_f, in_f), dtype=t.float32, device=p.device)
    rc = nat.lib().fastllm_dequantize_int4_group(nat.ptr(p), nat.ptr(s), nat.ptr(z), nat.ptr(out),
                                                 out_f, in_f, qt.block_size,
                                                 nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_dequantize_int4_group")
    return nat.as_output(out, numpy_in)


def quantize_mxfp4(w, xp=np) -> QuantizedTensor:
    """OCP MXFP4 (Microscaling v1.0): blocks of 32 consecutive in_features
    share a power-of-two scale 2^(floor(log2 amax) - 2), stored as an E8M0
    byte; elements are E2M1 (magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6) rounded to
    nearest, ties to the even code, saturating at 6.  data (out, in/2) uint8,
    even column in the low nibble; scales (out, in/32) uint8 E8M0; block_size
    32.  No reference counterpart: the format of the planned MXFP4 experts
    (docs/next-optimizations.md:160-184)."""
    t = nat.torch()
    numpy_in = nat.host_out(w, xp)
    wd = _f32_device(w).contiguous()
    out_f, in_f = wd.shape
    if in_f % 32:
        raise ValueError(f"quantize_mxfp4: in_features {in_f} is not a multiple of 32")
    codes = t.empty((out_f, in_f // 2), dtype=t.uint8, device=wd.device)
    e8 = t.empty((out_f, in_f // 32), dtype=t.uint8, device=wd.device)
    rc = nat.lib().fastllm_quantize_mxfp4(nat.ptr(wd), nat.ptr(codes), nat.ptr(e8), out_f, in_f,
                                          nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_mxfp4")
    return QuantizedTensor("mxfp4", nat.as_output(codes, numpy_in), nat.as_output(e8, numpy_in),
                           (out_f, in_f), 32)


def dequantize_mxfp4(qt: QuantizedTensor, xp=np):
    """E2M1(code) * 2^(e8 - 127) as float32 (out, in)."""
    t = nat.torch()
    numpy_in = nat.host_out(qt.data, xp)
    out_f, in_f = qt.shape
    c = nat.to_device(qt.data, t.uint8).contiguous()
    e = nat.to_device(qt.scales, t.uint8).contiguous()
    out = t.empty((out_f, in_f), dtype=t.float32, device=c.device)
    rc = nat.lib().fastllm_dequantize_mxfp4(nat.ptr(c), nat.ptr(e), nat.ptr(out), out_f, in_f,
                                            nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_dequantize_mxfp4")
    return nat.as_output(out, numpy_in)

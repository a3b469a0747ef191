"""Marlin-format INT4 packers and the per-expert INT4 FFN.

Hot-path parts of the reference's ``fastllm_py/moe.py`` (lines 30-81): the
engine's Marlin packer ``quantize_marlin_matrix``, ``build_marlin_expert_payload``
and ``_expert_ffn_marlin``.  Quantization, GPTQ packing, repacking and the
scale/zero permutation all run on the GPU (csrc/packers.hip,
csrc/int4_marlin.hip); the results are bit-identical to the reference's numpy
packer followed by this library's repack.
"""
from __future__ import annotations

import numpy as np

from . import _native as nat
from .kernels import marlin


def _quantize_marlin_device(w, group_size: int = 128):
    """Device RTN with integer zero point (moe.py:40-46).

    Returns (q u8 [N, K], scale f32 [N, G], zero i32 [N, G]) device tensors."""
    t = nat.torch()
    wd = nat.to_device(w, t.float32)
    size_n, size_k = wd.shape
    G = size_k // group_size
    q = t.empty((size_n, size_k), dtype=t.uint8, device=wd.device)
    scale = t.empty((size_n, G), dtype=t.float32, device=wd.device)
    zero = t.empty((size_n, G), dtype=t.int32, device=wd.device)
    rc = nat.lib().fastllm_quantize_int4_marlin(nat.ptr(wd), nat.ptr(q), nat.ptr(scale),
                                                nat.ptr(zero), size_n, size_k, group_size,
                                                nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_int4_marlin")
    return q, scale, zero


def quantize_marlin_matrix_device(w, group_size: int = 128) -> dict:
    """(out, in) float matrix -> {"qweight": u32 tile layout, "scales": fp16
    [G, N] permuted, "zeros": u32 [G, N/8] permuted}, all device tensors."""
    t = nat.torch()
    wd = nat.to_device(w)
    size_n, size_k = wd.shape
    q, scale, zero = _quantize_marlin_device(wd, group_size)
    std = marlin.pack_gptq_qweight(q.view(t.uint8).to(t.int32).view(t.uint32))
    repacked = marlin.marlin_repack(std, size_k, size_n)
    scales, zeros = marlin.build_marlin_scales_zeros(scale, zero, group_size)
    return {"qweight": repacked, "scales": scales, "zeros": zeros}


def quantize_marlin_matrix(w, group_size: int = 128) -> dict:
    """Quantize one (out, in) float matrix to upload-ready Marlin INT4
    (moe.py:30-50): {"qweight": u32, "scales": fp16, "zeros": u32} numpy arrays."""
    pay = quantize_marlin_matrix_device(nat.to_device(np.asarray(w)), group_size)
    return {k: v.cpu().numpy() for k, v in pay.items()}


def build_marlin_expert_payload(w_fp16: dict, group_size: int = 128) -> dict:
    """One expert's {gate, up, down} -> flat "<proj>.qweight/..." dict
    (moe.py:53-59)."""
    payload = {}
    for proj, w in w_fp16.items():
        for k, v in quantize_marlin_matrix(w, group_size).items():
            payload[f"{proj}.{k}"] = v
    return payload


def _expert_ffn_marlin(x_fp16, w, stream=None):
    """One expert's FFN on its Marlin payload for the rows routed to it
    (moe.py:62-81): gate and up GEMMs, swiglu, down GEMM.  ``w`` is the flat
    payload of ``build_marlin_expert_payload`` on the device ("gate.qweight",
    "gate.scales", ..., "down.zeros"); x (n, hidden) fp16.  Every step runs
    in this library on ``stream`` (None: the current stream), with no
    per-call validation, as the reference's hot loop expects.  Returns
    (n, hidden) fp16."""
    from .kernels import ops

    if stream is None:  # one stream for all four launches
        stream = nat.current_stream_handle()
    hidden = x_fp16.shape[1]
    inter = w["gate.scales"].shape[1]
    g = marlin.gemm_fast(x_fp16, w["gate.qweight"], w["gate.scales"], w["gate.zeros"], inter,
                         hidden, stream=stream)
    u = marlin.gemm_fast(x_fp16, w["up.qweight"], w["up.scales"], w["up.zeros"], inter, hidden,
                         stream=stream)
    act = ops.swiglu(g, u, stream=stream)
    return marlin.gemm_fast(act, w["down.qweight"], w["down.scales"], w["down.zeros"], hidden,
                            inter, stream=stream)

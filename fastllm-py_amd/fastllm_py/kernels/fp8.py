"""FP8-E4M3 block-scaled GEMV (small-batch decode path) on gfx950.

Drop-in for the reference's ``fastllm_py/kernels/fp8.py`` (lines 1-142) with
PyTorch-ROCm tensors as buffers.  Two weight formats:

* the reference .so's interleaved inline-scale layout (``quantize`` /
  ``fp8_gemv``): each weight row is ``[128 e4m3 codes][fp32 scale]`` repeated
  ``m/128`` times, ``perRow = m + 4*m/128`` bytes;
* the separate-scale 128x128 block format of ``quantizer.quantize_fp8_block``
  (``fp8_gemv_block``), with fp16 or bf16 activations and in-features that
  need only be a multiple of 64.

GEMV semantics: ``C[n, k] = A[n, m] @ dequant(W).T`` with ``k`` output rows.
"""
from __future__ import annotations

import numpy as np

from .. import _native as nat


def _load():
    return nat.load()


def available() -> bool:
    try:
        _load()
        return True
    except Exception:
        return False


def packed_row_bytes(m: int) -> int:
    """Bytes per weight row in the inline layout = m + (m/128)*4 (fp8.py:68-70)."""
    return _load().fastllm_fp8_block128_packed_row_bytes(int(m))


def quantize(weight_fp16, is_bf16: bool = False):
    """[k(out), m(in)] fp16/bf16 device weight -> uint8 [k, perRow] inline layout
    (fp8.py:73-95).  m % 128 == 0.  Scale per (row, 128-block) = amax/448;
    codes are round-to-nearest-even, saturating e4m3 of x * (1/scale)."""
    t = nat.torch()
    lib = _load()
    w = nat.to_device(weight_fp16)
    k, m = w.shape
    if m % 128 != 0:
        raise ValueError(f"quantize: the inline format packs 128-wide blocks; m={m} is not a "
                         f"multiple of 128")
    want = t.bfloat16 if is_bf16 else t.float16
    if w.dtype != want:
        w = w.to(want)
    per_row = packed_row_bytes(m)
    out = t.empty((k, per_row), dtype=t.uint8, device=w.device)
    rc = lib.fastllm_fp8_block128_quantize(nat.ptr(w), nat.ptr(out), k, m, 1 if is_bf16 else 0)
    if rc != 0:
        raise RuntimeError(f"quantize: the library refused the call (rc={rc}: 1 = arguments, "
                           f"2/3 = device or launch)")
    return out


def fp8_gemv(x_fp16, weight_fp8_block128, scales=None, out=None, k=None):
    """Inline-layout FP8 GEMV/GEMM (fp8.py:98-142): fp16 [n, m] activations,
    uint8 weight [k, perRow] (or flat with k given).  Returns fp16 [n, k]."""
    t = nat.torch()
    lib = _load()
    if scales is not None:
        raise ValueError("fp8_gemv: the inline format carries its own block scales, so "
                         "`scales` must stay None")
    x = nat.to_device(x_fp16, t.float16)
    n, m = x.shape
    per_row = packed_row_bytes(m)
    w = nat.to_device(weight_fp8_block128)
    if w.dim() == 2:
        k = w.shape[0]
        if w.shape[1] != per_row:
            raise ValueError(f"fp8_gemv: weight rows hold {w.shape[1]} bytes; m={m} needs "
                             f"{per_row}")
    else:
        if k is None:
            raise ValueError("fp8_gemv: a flat weight needs its row count k")
        if w.numel() != k * per_row:
            raise ValueError(f"fp8_gemv: flat weight has {w.numel()} bytes, k={k} rows need "
                             f"{k * per_row}")
    if out is None:
        out = t.empty((n, k), dtype=t.float16, device=x.device)
    rc = lib.fastllm_fp8_block128_gemv_fp16(nat.ptr(x), nat.ptr(w), nat.ptr(out), None, n, m, k,
                                            per_row)
    if rc != 0:
        raise RuntimeError(f"fp8_gemv: the library refused the call (rc={rc}: 1 = arguments, "
                           f"2/3 = device or launch)")
    return out


# one zeroed split-K workspace per device for the prefill GEMM, grown as
# shapes need it (its tile counters are left at zero by every call).  A
# smaller workspace it replaces is kept alive to the end of the process: a
# launch on a caller's stream, or a captured graph, may still read it, and
# freeing it would let the caching allocator hand its block to a new tensor.
_gemm_ws: dict = {}
_gemm_ws_retired: list = []


def _gemm_workspace(M: int, N: int, K: int):
    t = nat.torch()
    need = int(_load().fastllm_fp8_b128x128_gemm_ws_bytes(M, N, K))
    if need == 0:
        return None, 0
    dev = t.cuda.current_device()
    ws = _gemm_ws.get(dev)
    if ws is None or ws.numel() < need:
        if ws is not None:
            _gemm_ws_retired.append(ws)
        # round up so a run of growing shapes retires few buffers
        size = 1 << max(20, (need - 1).bit_length())
        ws = t.zeros(size, dtype=t.uint8, device="cuda")
        _gemm_ws[dev] = ws
    return ws, ws.numel()


def fp8_gemv_block(x, q, scales, out=None, bias=None, stream=None, workspace=None):
    """128x128-block FP8 GEMV: x [M, K] fp16/bf16, q uint8 [N, K], scales fp32
    [ceil(N/128), ceil(K/128)] (quantizer.quantize_fp8_block's format).
    Returns [M, N] in x's dtype.  K % 64 == 0, K >= 128.  Above 64 rows with
    fewer than 256 output tiles the GEMM splits K; its partials go to
    ``workspace`` (a zeroed uint8 device tensor of at least
    fastllm_fp8_b128x128_gemm_ws_bytes bytes) or to a per-device workspace
    shared by calls without one (such calls must not overlap)."""
    t = nat.torch()
    lib = _load()
    x = nat.to_device(x)
    if x.dtype not in (t.float16, t.bfloat16):
        x = x.to(t.bfloat16)
    M, K = x.shape
    qd = nat.to_device(q, t.uint8)
    N = qd.shape[0]
    sd = nat.to_device(scales, t.float32)
    if out is None:
        out = t.empty((M, N), dtype=x.dtype, device=x.device)
    b = nat.to_device(bias, x.dtype) if bias is not None else None
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    if workspace is not None:
        ws, wsb = workspace, workspace.numel() * workspace.element_size()
    else:
        ws, wsb = _gemm_workspace(M, N, K)
    rc = lib.fastllm_fp8_b128x128_gemm_ws(nat.ptr(x), nat.ptr(qd), nat.ptr(sd),
                                          nat.ptr(b) if b is not None else None, nat.ptr(out),
                                          M, N, K, 1 if x.dtype == t.bfloat16 else 0,
                                          nat.ptr(ws) if ws is not None else None, wsb, h)
    if rc != 0:
        raise RuntimeError(f"fastllm_fp8_b128x128_gemm_ws failed (rc={rc})")
    return out

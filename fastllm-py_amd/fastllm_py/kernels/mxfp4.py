"""Dense MXFP4 GEMV (decode) and GEMM (prefill) on gfx950.

The reference plans MXFP4 weights for both its expert kernels and a dense
decode GEMV / prefill GEMM (docs/next-optimizations.md:160-184) without a
format or kernel of its own; this module is the dense pair.  Weights
use the same OCP MXFP4 quantization (``fastllm_quantize_mxfp4``: E2M1 codes,
one E8M0 scale per 32 inputs) and the same MFMA tile layout as this
library's MXFP4 experts (``moe_int4.stack_lowp``), one matrix instead of a
stack.

GEMV semantics: ``C[M, N] = A[M, K] @ dequant(W).T``, fp16 in and out.
"""
from __future__ import annotations

from .. import _native as nat
from . import moe_int4


def quantize(W) -> dict:
    """(N, K) float weight (device tensor or numpy; N and K multiples of
    128) -> {"qtile", "e8w", "shape"}: the MXFP4 tiles of one expert
    (``stack_lowp`` with E = 1), quantized on the GPU."""
    t = nat.torch()
    w = nat.to_device(W, t.float32)
    if w.dim() != 2:
        raise ValueError(f"mxfp4.quantize: weight must be 2-D (N, K), got {tuple(w.shape)}")
    st = moe_int4.stack_lowp("mxfp4", "w", w.unsqueeze(0))
    return {"qtile": st["w.qtile"][0], "e8w": st["w.sz"][0], "shape": st["w.shape"]}


def gemv(A, wq: dict, out=None, stream=None):
    """C = A @ dequant(W).T for A (M, K) fp16 on the GPU and ``wq`` from
    :func:`quantize`: up to 64 rows the decode GEMV (fast for M <= 16; it
    reads the weights once per 16 rows), above the MFMA prefill GEMM.
    Returns C (M, N) fp16; ``out`` may be given."""
    t = nat.torch()
    N, K = wq["shape"]
    a = nat.to_device(A, t.float16)
    if a.dim() != 2 or a.shape[1] != K:
        raise ValueError(f"mxfp4.gemv: A must be (M, {K}), got {tuple(a.shape)}")
    a = a.contiguous()
    M = a.shape[0]
    if out is None:
        out = t.empty((M, N), dtype=t.float16, device=a.device)
    elif out.dtype != t.float16 or tuple(out.shape) != (M, N) or not out.is_contiguous():
        raise ValueError(f"mxfp4.gemv: out must be contiguous fp16 ({M}, {N})")
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_mxfp4_gemv(nat.ptr(a), nat.ptr(wq["qtile"]), nat.ptr(wq["e8w"]),
                                      nat.ptr(out), M, N, K, h)
    nat.check_rc(rc, "fastllm_mxfp4_gemv")
    return out

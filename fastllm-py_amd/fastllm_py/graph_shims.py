"""Stand-ins for the two RawKernel factories of the reference's graph decoder.

``GraphDecoder`` (fastllm_py/graph_decode.py) compiles two CuPy RawKernels on
the quantized path and launches them with CuPy's call convention
``kernel(grid, block, args, shared_mem=...)``:

* ``_dense_gemv_kernel(cp, ctype)`` (graph_decode.py:170-216), the row-major
  INT4 GEMV of the attention projections, launched by ``_dgemv``
  (graph_decode.py:748-765) with ``args = (x, qweight, scales, zeros, y,
  in_f, out_f, gs, rpb)``;
* ``_route_topk_kernel(cp)`` (graph_decode.py:242-285), the one-token
  router of ``_moe_branch`` (graph_decode.py:682-686) with ``args = (logits,
  rw, aidx, E, K, norm, scale)``.

``dense_gemv_kernel`` and ``route_topk_kernel`` return objects with that call
convention that launch this library's kernels instead, on the caller's
current CuPy stream (so they capture into the caller's graph), reading the
CuPy arrays through their device pointers.  Grid, block and shared-memory
arguments are the reference kernels' own launch shape and are ignored.
``fastllm_py.swap.install`` puts them in place of the factories.

Behaviour relative to the reference kernels: the GEMV is the same function
(fp32 accumulation, fp16 or fp32 in and out); the router is numpy-exact
(the reference kernel uses ``__expf`` and keeps every expert tied at the
k-th value), writing the same ``rw`` (E,) weights and ``aidx`` (K,) list in
descending weight order.
"""
from __future__ import annotations

from . import _native as nat


def _stream_of(cp, stream):
    if stream is not None:
        return nat.stream_handle(stream)
    return int(cp.cuda.get_current_stream().ptr) if cp is not None else nat.current_stream_handle()


class _DenseGemv:
    def __init__(self, cp, ctype: str):
        if ctype not in ("__half", "float"):
            raise TypeError(f"dense GEMV: activation type {ctype!r} is not fp16 or fp32")
        self.cp, self.f32 = cp, 1 if ctype == "float" else 0

    def __call__(self, grid, block, args, shared_mem=0, stream=None):
        x, qweight, scales, zeros, y, in_f, out_f, gs, _rpb = args
        rc = nat.lib().fastllm_int4_rowmajor_gemv(
            nat.ptr(x), self.f32, nat.ptr(qweight), nat.ptr(scales), nat.ptr(zeros), nat.ptr(y),
            self.f32, 1, int(out_f), int(in_f), int(gs), _stream_of(self.cp, stream))
        nat.check_rc(rc, "fastllm_int4_rowmajor_gemv")


class _RouteTopk:
    def __init__(self, cp):
        self.cp = cp
        self._w = {}  # top_k -> persistent fp32 (top_k,) weight buffer (allocated outside capture)

    def prepare(self, top_k: int):
        """Allocate the per-top_k scratch now (before any graph capture)."""
        if top_k not in self._w:
            t = nat.torch()
            self._w[top_k] = t.empty((top_k,), dtype=t.float32, device="cuda")
        return self._w[top_k]

    def __call__(self, grid, block, args, shared_mem=0, stream=None):
        logits, rw, aidx, E, K, norm, scale = args
        w = self.prepare(int(K))
        rc = nat.lib().fastllm_route_topk(
            nat.ptr(logits), 1, int(E), int(K), 0, int(norm), float(scale), None, 0, 0,
            nat.ptr(aidx), nat.ptr(w), nat.ptr(rw), None, None, None, None, None, None, None,
            _stream_of(self.cp, stream))
        nat.check_rc(rc, "fastllm_route_topk")


_DENSE: dict = {}
_ROUTE: dict = {}


def dense_gemv_kernel(cp, ctype: str):
    """``_dense_gemv_kernel(cp, ctype)``: a launcher of the row-major INT4 GEMV."""
    if ctype not in _DENSE:
        _DENSE[ctype] = _DenseGemv(cp, ctype)
    return _DENSE[ctype]


def route_topk_kernel(cp):
    """``_route_topk_kernel(cp)``: a launcher of the numpy-exact router."""
    if "k" not in _ROUTE:
        _ROUTE["k"] = _RouteTopk(cp)
    return _ROUTE["k"]

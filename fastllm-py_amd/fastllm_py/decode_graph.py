"""One decoder layer's quantized-matmul chain, captured once in a HIP graph.

The reference turns kernel time into tok/s by capturing a segment of decoder
layers in a CUDA graph with persistent buffers and per-call-site workspaces
(``GraphDecoder._segment_step``, fastllm_py/graph_decode.py:782-874, replayed
by 896-922).  ``DecodeLayerGraph`` is that capture for this library's path,
for one dense layer (INT4 Marlin weights):

    xnew1, h1 = add_rmsnorm(x, pending, ln1)      # previous layer's residual
    qkv       = h1 @ Wqkv^T                        # Marlin GEMV
    ctx       = qkv[:, :q_dim]                     # stand-in for attention
    o         = ctx @ Wo^T
    xnew2, h2 = add_rmsnorm(xnew1, o, ln2)
    hh        = swiglu(h2 @ Wgu^T)                 # gate/up GEMV + SwiGLU, one launch
    pending'  = hh @ Wdown^T

Attention, RoPE and the KV cache are not part of this library (the reference's
attention kernels are outside the quantized-matmul path), so the context is
the q slice of the projection: the shapes and the data dependence between the
launches stay those of a decode step.  A MoE layer replaces the last two lines
with ``kernels.moe_int4.moe_branch``, which is capturable the same way.

Every tensor the graph touches is allocated once here; ``x`` and ``pending``
are the inputs (write them, then ``replay()``), ``x_out`` and ``pending_out``
the outputs.  No launch in the chain records a memset.

At M = 1 (``fuse_norm``, the default there) each add_rmsnorm runs in the
prologue of the projection that consumes it (``marlin.gemm_add_rmsnorm``):
four launches per layer instead of six, and the normalised rows never leave
the chip.
"""
from __future__ import annotations

from . import _native as nat
from .kernels import marlin, ops


class DecodeLayerGraph:
    def __init__(self, weights: dict, M: int, hidden: int, q_dim: int, inter: int,
                 eps: float = 1e-6, fuse_norm: bool | None = None):
        """weights: ``ln1``, ``ln2`` (hidden,) fp16/fp32 norm weights and Marlin
        payloads (``quantize_marlin_matrix_device`` dicts) ``qkv`` (N_qkv x
        hidden), ``o`` (hidden x q_dim), ``gate_up`` (2 inter x hidden: gate
        rows then up rows) and ``down`` (hidden x inter)."""
        t = nat.torch()
        self.t, self.w, self.M, self.eps = t, weights, M, eps
        self.fuse_norm = (M == 1) if fuse_norm is None else bool(fuse_norm)
        if self.fuse_norm and M != 1:
            raise ValueError("DecodeLayerGraph: the fused add_rmsnorm prologue takes one row")
        self.hidden, self.q_dim, self.inter = hidden, q_dim, inter
        self.n_qkv = weights["qkv"]["scales"].shape[1]
        dev = weights["qkv"]["qweight"].device
        f32, f16 = t.float32, t.float16
        e = lambda n, dt: t.zeros((M, n), dtype=dt, device=dev)  # noqa: E731
        self.x, self.pending = e(hidden, f32), e(hidden, f16)
        self.xnew1, self.h1 = e(hidden, f32), e(hidden, f16)
        self.qkv, self.ctx, self.o = e(self.n_qkv, f16), e(q_dim, f16), e(hidden, f16)
        self.x_out, self.h2 = e(hidden, f32), e(hidden, f16)
        self.hh, self.pending_out = e(inter, f16), e(hidden, f16)
        self.ws = {k: marlin.make_workspace(self.w[k]["scales"].shape[1]) for k in ("qkv", "o", "down")}
        self.graph = None
        self.stream = None

    def _lin(self, name, a, out, stream):
        p = self.w[name]
        return marlin.gemm_fast(a, p["qweight"], p["scales"], p["zeros"], p["scales"].shape[1],
                                a.shape[1], stream=stream, workspace=self.ws[name], out=out)

    def step(self, stream=None):
        """Issue the chain once on ``stream`` (eager; also what is captured)."""
        w = self.w
        gu = w["gate_up"]
        if self.fuse_norm:
            p = w["qkv"]
            marlin.gemm_add_rmsnorm(self.x, self.pending, w["ln1"], self.eps, p["qweight"],
                                    p["scales"], p["zeros"], self.n_qkv, self.hidden,
                                    out=self.qkv, xnew=self.xnew1, stream=stream)
        else:
            ops.add_rmsnorm(self.x, self.pending, w["ln1"], self.eps, out=(self.xnew1, self.h1),
                            stream=stream)
            self._lin("qkv", self.h1, self.qkv, stream)
        self.ctx.copy_(self.qkv[:, :self.q_dim])
        self._lin("o", self.ctx, self.o, stream)
        if self.fuse_norm:
            marlin.gemm_add_rmsnorm(self.xnew1, self.o, w["ln2"], self.eps, gu["qweight"],
                                    gu["scales"], gu["zeros"], 2 * self.inter, self.hidden,
                                    swiglu=True, out=self.hh, xnew=self.x_out, stream=stream)
        else:
            ops.add_rmsnorm(self.xnew1, self.o, w["ln2"], self.eps, out=(self.x_out, self.h2),
                            stream=stream)
            marlin.gemm_swiglu(self.h2, gu["qweight"], gu["scales"], gu["zeros"], 2 * self.inter,
                               self.hidden, out=self.hh, stream=stream)
        self._lin("down", self.hh, self.pending_out, stream)

    def capture(self, warmup: int = 2):
        """Warm up on a side stream, then capture ``step`` into a graph."""
        t = self.t
        self.stream = t.cuda.Stream()
        self.stream.wait_stream(t.cuda.current_stream())
        with t.cuda.stream(self.stream):
            for _ in range(warmup):
                self.step(stream=self.stream)
        t.cuda.current_stream().wait_stream(self.stream)
        self.graph = t.cuda.CUDAGraph()
        with t.cuda.graph(self.graph, stream=self.stream):
            self.step(stream=self.stream)
        return self

    def replay(self):
        self.graph.replay()

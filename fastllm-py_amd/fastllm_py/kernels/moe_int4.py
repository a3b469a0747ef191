"""Row-major INT4 group-quant GEMV, gate matvec and the fused selective MoE FFN.

Drop-in for the reference's ``fastllm_py/kernels/moe_int4.py`` (lines 1-506)
and the hot-path kernels of ``fastllm_py/graph_decode.py`` (``_dgemv``
:748-765, ``_route_topk_kernel`` :242-285, ``_moe_branch`` :669-700), with
PyTorch-ROCm tensors as buffers and gfx950 HIP kernels (csrc/moe_int4.hip,
csrc/packers.hip) doing the work.

Format for a weight W of shape (out, in), group size gs along ``in``:
  qweight : (out, in//2) uint8   -- two int4 nibbles/byte, even col in low nibble
  scales  : (out, in//gs) fp16
  zeros   : (out, in//gs) fp16   -- dequant(W[o,i]) = (q - zero) * scale

Differences from the reference kernels, all in the direction of the numpy
reference: the fused MoE combines experts in a fixed order (no atomics), so a
call is deterministic; activations feed the matrix cores as fp16.
"""
from __future__ import annotations

import numpy as np

from .. import _native as nat


# ----------------------------------------------------------------- packers
def _rowmajor_device(W, group_size):
    """(..., out, in) float -> (qweight, scales, zeros) device tensors."""
    t = nat.torch()
    w = nat.to_device(W, t.float32)
    lead = tuple(w.shape[:-2])
    out_f, in_f = w.shape[-2:]
    assert in_f % group_size == 0 and in_f % 2 == 0
    batch = int(np.prod(lead)) if lead else 1
    qw = t.empty(lead + (out_f, in_f // 2), dtype=t.uint8, device=w.device)
    sc = t.empty(lead + (out_f, in_f // group_size), dtype=t.float16, device=w.device)
    ze = t.empty_like(sc)
    rc = nat.lib().fastllm_quantize_int4_rowmajor(nat.ptr(w), nat.ptr(qw), nat.ptr(sc),
                                                  nat.ptr(ze), batch, out_f, in_f, group_size,
                                                  nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_quantize_int4_rowmajor")
    return qw, sc, ze


def quantize_int4_rowmajor(w, group_size: int = 128, xp=np) -> dict:
    """RTN group INT4, row-major (moe_int4.py:24-40).  numpy in -> numpy arrays
    out (computed on the GPU); torch in -> device tensors."""
    numpy_in = isinstance(w, np.ndarray) or xp is np and not nat.is_tensor(w)
    qw, sc, ze = _rowmajor_device(np.asarray(w) if numpy_in else w, group_size)
    out_f, in_f = qw.shape[0], qw.shape[1] * 2
    return {"qweight": nat.as_output(qw, numpy_in), "scales": nat.as_output(sc, numpy_in),
            "zeros": nat.as_output(ze, numpy_in), "shape": (out_f, in_f), "group": group_size}


def dequantize_int4_rowmajor(payload, xp=np):
    """(q - zero) * scale -> fp32 (moe_int4.py:43-54)."""
    t = nat.torch()
    numpy_in = isinstance(payload["qweight"], np.ndarray)
    qw = nat.to_device(payload["qweight"], t.uint8)
    sc = nat.to_device(payload["scales"], t.float16)
    ze = nat.to_device(payload["zeros"], t.float16)
    out_f, in_f = payload["shape"]
    batch = qw.numel() // (out_f * (in_f // 2))
    out = t.empty(tuple(qw.shape[:-2]) + (out_f, in_f), dtype=t.float32, device=qw.device)
    rc = nat.lib().fastllm_dequantize_int4_rowmajor(nat.ptr(qw), nat.ptr(sc), nat.ptr(ze),
                                                    nat.ptr(out), batch, out_f, in_f,
                                                    payload["group"], nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_dequantize_int4_rowmajor")
    return nat.as_output(out, numpy_in)


def _quantize_int4_rowmajor_batched(W, group_size: int, xp=np):
    """(E, out, in) -> (qweight (E,out,in/2), scales, zeros, (out,in))
    (moe_int4.py:97-113), one GPU launch for all E."""
    qw, sc, ze = _rowmajor_device(W, group_size)
    return qw, sc, ze, (qw.shape[-2], qw.shape[-1] * 2)


def build_stacked_experts(expert_ws, group_size: int = 128, xp=np) -> dict:
    """Stack E experts' {gate, up, down} into (E, out, in/2) INT4 device tensors
    indexable by expert id (moe_int4.py:116-133)."""
    t = nat.torch()
    out = {"group": group_size}
    for proj in ("gate", "up", "down"):
        ws = [w[proj] for w in expert_ws]
        if nat.is_tensor(ws[0]):
            stack = t.stack([nat.to_device(w) for w in ws])
        else:
            stack = np.stack([np.asarray(w) for w in ws])
        qw, sc, ze, shp = _quantize_int4_rowmajor_batched(stack, group_size)
        out[f"{proj}.qweight"] = qw
        out[f"{proj}.scales"] = sc
        out[f"{proj}.zeros"] = ze
        out[f"{proj}.shape"] = shp
    return out


# ------------------------------------------------------------------ GEMVs
def _rm_gemv(x, payload, out, y_dtype):
    t = nat.torch()
    out_f, in_f = payload["shape"]
    x = nat.to_device(x)
    if x.dtype not in (t.float32, t.float16):
        x = x.to(t.float32)
    x2 = x.reshape(-1, in_f)
    M = x2.shape[0]
    y = out if out is not None else t.empty((M, out_f), dtype=y_dtype, device=x.device)
    rc = nat.lib().fastllm_int4_rowmajor_gemv(
        nat.ptr(x2), 1 if x2.dtype == t.float32 else 0, nat.ptr(payload["qweight"]),
        nat.ptr(payload["scales"]), nat.ptr(payload["zeros"]), nat.ptr(y),
        1 if y.dtype == t.float32 else 0, M, out_f, in_f, payload["group"],
        nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_int4_rowmajor_gemv")
    return y


def gemv_int4(x, payload, out=None):
    """y = x @ dequant(W).T for decode rows (moe_int4.py:490-506).  x (in,) or
    (M, in) fp32 -> fp32 (out,) / (M, out)."""
    t = nat.torch()
    y = _rm_gemv(x, payload, out, t.float32)
    return y.reshape(-1) if (nat.to_device(x).dim() == 1 and out is None) else y


def dgemv(x, payload, out=None):
    """graph_decode._dgemv (graph_decode.py:748-765): x (1, in) or (in,) fp16 or
    fp32 -> same dtype (1, out), written into ``out`` when given."""
    t = nat.torch()
    xd = nat.to_device(x)
    y = _rm_gemv(xd, payload, out, xd.dtype if xd.dtype in (t.float16, t.float32) else t.float32)
    return y.reshape(1, -1)


def gate_matvec(x, gate_w, E, hidden, out=None, threads=128):
    """logits (E,) = x (hidden,) @ gate_w (E, hidden).T in fp32 (moe_int4.py:162-169).
    x may also be (T, hidden) -> (T, E)."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32)
    x2 = xd.reshape(-1, hidden)
    T = x2.shape[0]
    gw = nat.to_device(gate_w, t.float16)
    y = out if out is not None else t.empty((T, E) if xd.dim() > 1 else (E,), dtype=t.float32,
                                            device=xd.device)
    rc = nat.lib().fastllm_gate_matvec(nat.ptr(x2), nat.ptr(gw), None, nat.ptr(y), None, T, E,
                                       hidden, nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_gate_matvec")
    return y


# -------------------------------------------------------------- fused MoE
def _stacked_ptrs(st):
    return [nat.ptr(st[f"{p}.{k}"]) for p in ("gate", "up", "down")
            for k in ("qweight", "scales", "zeros")]


def moe_forward(x, stacked, E, hidden, inter, *, rw=None, active=None, n_active=None,
                host_active=None, slot_coef=None, shared=None, shared_inter=0,
                shared_coef=None, out=None, inter_buf=None, max_active=None, stream=None):
    """Fused selective INT4 MoE FFN for T <= 16 tokens (x (T, hidden) fp32):

    y[t] = sum_{slots s} coef(s, t) * down_e(silu(gate_e x_t) * up_e x_t)
           + shared_coef[t] * shared(x_t)

    Routing comes either as dense weights ``rw`` (T, E) with the active expert
    list ``active`` (device int32) and its length ``n_active`` (device (1,)
    int32) or ``host_active`` (int), or as per-slot weights ``slot_coef``
    (S, T) for the experts listed in ``active``.  Experts are combined in slot
    order inside the matrix cores: no atomics, deterministic."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32)
    x2 = xd.reshape(-1, hidden).contiguous()
    T = x2.shape[0]
    if T > 16:
        raise ValueError("moe_forward handles up to 16 tokens per call")
    act = nat.to_device(active, t.int32)
    S = int(act.numel()) if max_active is None else int(max_active)
    gs = stacked["group"]
    pad = max(inter, shared_inter or 0)
    nslots = S + (1 if shared is not None else 0)
    need = nslots * T * pad
    if inter_buf is not None and inter_buf.numel() * inter_buf.element_size() >= need * 2 \
            and inter_buf.is_contiguous():
        ib = inter_buf
    else:
        ib = t.empty((nslots, T, pad), dtype=t.float16, device=xd.device)
    y = out if out is not None else t.empty((T, hidden), dtype=t.float32, device=xd.device)
    sp = _stacked_ptrs(shared) if shared is not None else [None] * 9
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_moe_int4_fused(
        nat.ptr(x2), T, hidden, gs, E, inter, *_stacked_ptrs(stacked),
        int(shared_inter or 0) if shared is not None else 0, *sp,
        nat.ptr(shared_coef) if shared_coef is not None else None,
        nat.ptr(n_active) if n_active is not None else None,
        int(host_active if host_active is not None else S), nat.ptr(act), S,
        nat.ptr(rw) if rw is not None else None,
        nat.ptr(slot_coef) if slot_coef is not None else None,
        nat.ptr(ib), pad, nat.ptr(y), h)
    nat.check_rc(rc, "fastllm_moe_int4_fused")
    return y


def fused_moe_weighted(x, stacked, rw, E, hidden, inter, out=None, inter_buf=None,
                       threads=256, rpb=8, aidx=None):
    """(E,)-routing-weight-driven selective MoE FFN (moe_int4.py:263-294):
    y (hidden,) = sum_{e: rw[e] > 0} rw[e] * FFN_e(x).  ``aidx`` (K,) lists the
    active experts; without it every expert is visited and zero weights skip
    nothing but contribute 0."""
    t = nat.torch()
    rwd = nat.to_device(rw, t.float32).reshape(1, -1)
    if aidx is None:
        act = t.arange(E, dtype=t.int32, device=rwd.device)
    else:
        act = nat.to_device(aidx, t.int32).reshape(-1)
    y = out.reshape(1, hidden) if out is not None else None
    r = moe_forward(x, stacked, E, hidden, inter, rw=rwd, active=act, out=y,
                    inter_buf=inter_buf)
    return r.reshape(hidden)


def fused_moe_ffn2(x, stacked, eidx, rw, hidden, inter, out=None, inter_buf=None, threads=128):
    """Index-driven selective MoE FFN (moe_int4.py:372-396):
    y = sum_k rw[k] * FFN_{eidx[k]}(x)."""
    t = nat.torch()
    act = nat.to_device(eidx, t.int32).reshape(-1)
    coef = nat.to_device(rw, t.float32).reshape(-1, 1).contiguous()
    E = stacked["gate.qweight"].shape[0]
    y = out.reshape(1, hidden) if out is not None else None
    r = moe_forward(x, stacked, E, hidden, inter, slot_coef=coef, active=act, out=y,
                    inter_buf=inter_buf)
    return r.reshape(hidden)


def fused_moe_ffn(x, stacked, eidx, rw, hidden, inter, out=None):
    """One-launch-per-expert variant in the reference (moe_int4.py:466-487);
    same math, same kernels here."""
    return fused_moe_ffn2(x, stacked, eidx, rw, hidden, inter, out=out)


# ------------------------------------------------------- graph decode branch
def route_topk_gpu(logits, top_k, *, norm=False, scale=1.0, rw=None, aidx=None):
    """graph_decode._route_topk_kernel (graph_decode.py:242-285) for one token:
    writes the (E,) weight vector and the (K,) active expert list.  Selection
    and weights are numpy-exact (the reference kernel's __expf is not)."""
    from ..expert_router import route_topk_device

    r = route_topk_device(logits, top_k, norm_topk_prob=norm, routed_scaling=scale)
    if rw is not None:
        rw.copy_(r["rw"].reshape(rw.shape))
    if aidx is not None:
        aidx.copy_(r["topk_ids"].reshape(aidx.shape))
    return r


def moe_branch(x, gate_w, stacked, top_k, *, E, hidden, inter, norm=False, scale=1.0,
               shared=None, shared_inter=0, shared_gate_w=None, bufs=None, stream=None):
    """One fused MoE layer for T <= 16 tokens, all on the device with no host
    sync (graph_decode._moe_branch, graph_decode.py:669-700):
    gate matvec (+ shared gate) -> router -> fused routed + shared FFN.
    Returns (T, hidden) fp32.  ``bufs`` may carry persistent buffers for
    graph capture (keys of route_topk_device plus logits, slogit, inter_buf,
    out)."""
    from ..expert_router import route_topk_device

    t = nat.torch()
    xd = nat.to_device(x, t.float32).reshape(-1, hidden).contiguous()
    T = xd.shape[0]
    b = bufs if bufs is not None else {}
    logits = b.get("logits")
    if logits is None:
        logits = t.empty((T, E), dtype=t.float32, device=xd.device)
    sl = None
    if shared_gate_w is not None:
        sl = b.get("slogit")
        if sl is None:
            sl = t.empty((T,), dtype=t.float32, device=xd.device)
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    gw = nat.to_device(gate_w, t.float16)
    sgw = nat.to_device(shared_gate_w, t.float16) if shared_gate_w is not None else None
    rc = nat.lib().fastllm_gate_matvec(nat.ptr(xd), nat.ptr(gw),
                                       nat.ptr(sgw) if sgw is not None else None,
                                       nat.ptr(logits), nat.ptr(sl) if sl is not None else None,
                                       T, E, hidden, h)
    nat.check_rc(rc, "fastllm_gate_matvec")
    r = route_topk_device(logits, top_k, norm_topk_prob=norm, routed_scaling=scale,
                          shared_logit=sl, out=b, stream=stream)
    max_active = min(E, T * top_k)
    return moe_forward(xd, stacked, E, hidden, inter, rw=r["rw"], active=r["active"],
                       n_active=r["n_active"], max_active=max_active, shared=shared,
                       shared_inter=shared_inter,
                       shared_coef=r.get("shared_coef") if shared_gate_w is not None else None,
                       out=b.get("out"), inter_buf=b.get("inter_buf"), stream=stream)

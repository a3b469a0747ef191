"""Top-k expert routing on the GPU.

Same API and arithmetic as the reference's ``route_topk``
(fastllm_py/expert_router.py:15-71): softmax (Qwen/Mixtral) or sigmoid + bias
(DeepSeek V3) scoring, DeepSeek group-limited selection, optional
renormalisation and routed scaling; returns one ``ExpertTask`` per activated
expert, experts ascending, tokens ascending within an expert.  Scores run in
the HIP router (csrc/moe_int4.hip), which evaluates numpy's float32 exp and
pairwise sums exactly, so probabilities and weights are bit-identical to the
reference's numpy.  Where experts tie, the selection and its order are those
of np.argpartition as numpy 2.x runs it on an AVX512_SKX host (x86-simd-sort's
bitonic key/index network, simulated in the router for tied rows).

``route_topk_device`` returns the device tensors the fused MoE kernels and
graph-captured decode consume.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native as nat


@dataclass
class ExpertTask:
    """One expert's share of a batch: ``token_idx`` (int32, ascending) are
    the batch rows routed to expert ``expert_id`` and ``weights`` (float32)
    their combine weights, in the same order.  Field names and order are the
    reference's, which its MoE layer reads."""

    expert_id: int
    token_idx: np.ndarray
    weights: np.ndarray


def route_topk_device(scores, top_k: int, *, norm_topk_prob: bool = False,
                      scoring: str = "softmax", routed_scaling: float = 1.0,
                      e_score_bias=None, n_group: int = 0, topk_group: int = 0,
                      shared_logit=None, out: dict | None = None, stream=None) -> dict:
    """scores (T, E) logits (any float dtype; cast to fp32 exactly like the
    reference's ``astype(float32)``) -> dict of device tensors:
    topk_ids (T, k) int32, topk_w (T, k) f32 (descending selection order),
    rw (T, E) f32 dense weights, n_active (1,) int32, active (E,) int32,
    offsets (E+1,) int32, tok (T*k,) int32, tokw (T*k,) f32 and, when
    shared_logit (T,) is given, shared_coef (T,) = sigmoid(shared_logit).
    ``out`` may hold preallocated tensors of those names (graph capture)."""
    t = nat.torch()
    s = nat.to_device(scores)
    if s.dim() == 1:
        s = s[None]
    if s.dtype != t.float32:
        s = s.to(t.float32)
    s = s.contiguous()
    T, E = s.shape
    dev = s.device
    o = out if out is not None else {}

    def buf(name, shape, dtype):
        if name not in o:
            o[name] = t.empty(shape, dtype=dtype, device=dev)
        return o[name]

    ids = buf("topk_ids", (T, top_k), t.int32)
    w = buf("topk_w", (T, top_k), t.float32)
    rw = buf("rw", (T, E), t.float32)
    na = buf("n_active", (1,), t.int32)
    act = buf("active", (E,), t.int32)
    offs = buf("offsets", (E + 1,), t.int32)
    tok = buf("tok", (T * top_k,), t.int32)
    tokw = buf("tokw", (T * top_k,), t.float32)
    bias = None
    if scoring == "sigmoid" and e_score_bias is not None:
        bias = nat.to_device(e_score_bias, t.float32)
    sl = sc = None
    if shared_logit is not None:
        sl = nat.to_device(shared_logit, t.float32).reshape(-1)
        sc = buf("shared_coef", (T,), t.float32)
    h = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_route_topk(
        nat.ptr(s), T, E, int(top_k), 1 if scoring == "sigmoid" else 0,
        1 if norm_topk_prob else 0, float(routed_scaling),
        nat.ptr(bias) if bias is not None else None, int(n_group or 0), int(topk_group or 0),
        nat.ptr(ids), nat.ptr(w), nat.ptr(rw), nat.ptr(sl) if sl is not None else None,
        nat.ptr(sc) if sc is not None else None, nat.ptr(na), nat.ptr(act), nat.ptr(offs),
        nat.ptr(tok), nat.ptr(tokw), h)
    nat.check_rc(rc, "fastllm_route_topk")
    return o


def route_topk(scores: np.ndarray, top_k: int, *, norm_topk_prob: bool = False,
               scoring: str = "softmax", routed_scaling: float = 1.0,
               e_score_bias: np.ndarray | None = None,
               n_group: int = 0, topk_group: int = 0) -> list[ExpertTask]:
    """scores: (T, num_experts) raw gate logits -> one ExpertTask per activated
    expert (expert_router.py:22-71)."""
    r = route_topk_device(scores, top_k, norm_topk_prob=norm_topk_prob, scoring=scoring,
                          routed_scaling=routed_scaling, e_score_bias=e_score_bias,
                          n_group=n_group, topk_group=topk_group)
    na = int(r["n_active"].cpu()[0])
    act = r["active"][:na].cpu().numpy()
    offs = r["offsets"][:na + 1].cpu().numpy()
    tok = r["tok"].cpu().numpy()
    tokw = r["tokw"].cpu().numpy()
    return [ExpertTask(int(act[i]), tok[offs[i]:offs[i + 1]].astype(np.int32).copy(),
                       tokw[offs[i]:offs[i + 1]].astype(np.float32).copy()) for i in range(na)]

"""numpy restatement of the reference's expert router (test oracle only).

route_topk follows fastllm_py/expert_router.py:22-71 operation by operation.
numpy's float32 exp is taken from the C restatement in oracle/c/npexp.c
(pinned bit-for-bit against the installed np.exp in tests/test_oracle_router.py)
so the oracle gives the same probabilities on any host, whichever SIMD path
that host's numpy dispatches.

Selection: the reference calls np.argpartition, whose choice among values
tied at the k-th position (and whose output order) is left to numpy's
selection algorithm.  ``route_topk`` here takes it from
``oracle/argpartition.py``, the restatement of that algorithm as numpy 2.2.6
runs it on an AVX512_SKX host (x86-simd-sort's key/index network), pinned
against the installed np.argpartition in tests/test_oracle_argpartition.py,
so the oracle selects the same experts as the reference on any host.
``route_topk_canonical`` breaks ties by lowest expert index instead (a
reference point for the tests: the two agree on every token without a tie,
which ``boundary_ties`` reports).

Pins: the reference's known answers (tests/test_router.py:36-64), brute
force (sort-based selection) on tie-free inputs, and np.argpartition itself
on tie-heavy rows.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

from .argpartition import argpartition_rows

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None


def _clib():
    global _lib
    if _lib is None:
        from . import build_oracle

        path = build_oracle.OUT
        if not os.path.exists(path):
            build_oracle.build()
        lib = ctypes.CDLL(path)
        lib.np_expf_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long]
        lib.np_sum_rows_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long,
                                        ctypes.c_long]
        _lib = lib
    return _lib


def np_exp_f32(x) -> np.ndarray:
    """numpy's float32 SIMD exp (restated in C)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    _clib().np_expf_array(x.ctypes.data, y.ctypes.data, x.size)
    return y


def np_rowsum_f32(a) -> np.ndarray:
    """numpy's pairwise row sum of a 2-D float32 array (restated in C)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape[0], dtype=np.float32)
    _clib().np_sum_rows_f32(a.ctypes.data, out.ctypes.data, a.shape[0], a.shape[1])
    return out


@dataclass
class ExpertTask:
    expert_id: int
    token_idx: np.ndarray
    weights: np.ndarray


def _scores(scores, scoring, e_score_bias):
    s = np.asarray(scores, dtype=np.float32)
    if scoring == "sigmoid":
        probs = (np.float32(1.0) / (np.float32(1.0) + np_exp_f32(-s))).astype(np.float32)
        bias = np.float32(0.0) if e_score_bias is None else np.asarray(e_score_bias, np.float32)
        select = (probs + bias).astype(np.float32)
    else:
        m = s.max(-1, keepdims=True)
        e = np_exp_f32(s - m)
        probs = (e / np_rowsum_f32(e)[:, None]).astype(np.float32)
        select = probs
    return probs, select


def _group_mask(select, n_group, topk_group, canonical):
    T, E = select.shape
    gsz = E // n_group
    gs = select.reshape(T, n_group, gsz)
    ntop = min(2, gsz)
    group_score = np.sort(gs, axis=-1)[:, :, -ntop:].sum(-1)
    if canonical:
        order = np.lexsort((np.broadcast_to(np.arange(n_group), group_score.shape), -group_score), axis=-1)
        keep = order[:, :topk_group]
    else:
        keep = argpartition_rows(-group_score, topk_group - 1)[:, :topk_group]
    masked = np.ones((T, n_group), dtype=bool)
    np.put_along_axis(masked, keep, False, axis=-1)
    return np.where(np.repeat(masked, gsz, axis=1), np.float32(-np.inf), select)


def _finish(probs, topk_idx, top_k, norm_topk_prob, routed_scaling):
    T = probs.shape[0]
    topk_w = np.take_along_axis(probs, topk_idx, axis=-1)
    if norm_topk_prob:
        topk_w = topk_w / (np_rowsum_f32(topk_w)[:, None] + np.float32(1e-20))
    topk_w = (topk_w * np.float32(routed_scaling)).astype(np.float32)
    tasks = []
    flat_e = topk_idx.ravel()
    flat_t = np.repeat(np.arange(T, dtype=np.int32), top_k)
    flat_w = topk_w.ravel().astype(np.float32)
    order = np.argsort(flat_e, kind="stable")
    fe, ft, fw = flat_e[order], flat_t[order], flat_w[order]
    E = probs.shape[1]
    bounds = np.searchsorted(fe, np.arange(E + 1))
    for eid in np.unique(fe):
        lo, hi = bounds[eid], bounds[eid + 1]
        tasks.append(ExpertTask(int(eid), ft[lo:hi].copy(), fw[lo:hi].copy()))
    return tasks, topk_idx, topk_w


def route_topk(scores, top_k, *, norm_topk_prob=False, scoring="softmax", routed_scaling=1.0,
               e_score_bias=None, n_group=0, topk_group=0, return_arrays=False):
    """fastllm_py/expert_router.py:22-71, with np.argpartition's selection
    (fastllm_py/expert_router.py:50,55) restated for rows of <= 256 experts."""
    probs, select = _scores(scores, scoring, e_score_bias)
    if n_group and n_group > 1 and 0 < topk_group < n_group:
        select = _group_mask(select, n_group, topk_group, canonical=False)
    topk_idx = argpartition_rows(-select, top_k - 1)[:, :top_k]
    out = _finish(probs, topk_idx, top_k, norm_topk_prob, routed_scaling)
    return out if return_arrays else out[0]


def route_topk_canonical(scores, top_k, *, norm_topk_prob=False, scoring="softmax",
                         routed_scaling=1.0, e_score_bias=None, n_group=0, topk_group=0,
                         return_arrays=False):
    """Same arithmetic; ties broken by lowest index, experts of a token listed by
    descending selection value (the GPU router's order)."""
    probs, select = _scores(scores, scoring, e_score_bias)
    if n_group and n_group > 1 and 0 < topk_group < n_group:
        select = _group_mask(select, n_group, topk_group, canonical=True)
    T, E = select.shape
    order = np.lexsort((np.broadcast_to(np.arange(E), select.shape), -select), axis=-1)
    topk_idx = order[:, :top_k]
    out = _finish(probs, topk_idx, top_k, norm_topk_prob, routed_scaling)
    return out if return_arrays else out[0]


def boundary_ties(scores, top_k, *, scoring="softmax", e_score_bias=None, n_group=0,
                  topk_group=0) -> np.ndarray:
    """Tokens whose k-th and (k+1)-th selection values are equal (where the
    reference's argpartition may pick either expert)."""
    probs, select = _scores(scores, scoring, e_score_bias)
    if n_group and n_group > 1 and 0 < topk_group < n_group:
        select = _group_mask(select, n_group, topk_group, canonical=True)
    s = -np.sort(-select, axis=-1)
    if top_k >= select.shape[1]:
        return np.zeros(select.shape[0], dtype=bool)
    return s[:, top_k - 1] == s[:, top_k]


def tasks_to_dict(tasks):
    return {t.expert_id: (t.token_idx.tolist(), t.weights.view(np.uint32).tolist()) for t in tasks}

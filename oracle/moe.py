"""fp32 reference of the selective MoE FFN (test oracle only).

Follows the reference's per-expert numpy FFN (tests/test_moe_int4.py:42-52,
fastllm_py/moe.py:22-26,161-175): for each routed (token, expert, weight),
g = x Wg^T, u = x Wu^T, y += w * ((g / (1 + exp(-g))) * u) Wd^T, with the
weights dequantized from the very packed payload the kernels read; plus the
shared expert scaled by sigmoid(x sg^T) (fastllm_py/moe.py:227-232).
"""
import numpy as np

from . import quant as Q


def dequant_stacked(stacked_np, gs):
    """{proj.qweight/scales/zeros} numpy (E, out, in/2) -> {proj: (E, out, in) fp32}."""
    return {p: Q.dequantize_int4_rowmajor(stacked_np[f"{p}.qweight"], stacked_np[f"{p}.scales"],
                                          stacked_np[f"{p}.zeros"], gs)
            for p in ("gate", "up", "down")}


def expert_ffn(x, wg, wu, wd):
    x = np.asarray(x, np.float32)
    g = x @ wg.T
    u = x @ wu.T
    return ((g / (1.0 + np.exp(-g))) * u) @ wd.T


def moe_ref(x, deq, topk_idx, topk_w, shared_deq=None, shared_coef=None):
    """x (T, hidden); deq from dequant_stacked; topk_idx/topk_w (T, k)."""
    x = np.asarray(x, np.float32)
    T = x.shape[0]
    y = np.zeros((T, deq["down"].shape[1]), np.float32)
    for t in range(T):
        for e, w in zip(np.asarray(topk_idx[t]).tolist(), np.asarray(topk_w[t]).tolist()):
            y[t] += np.float32(w) * expert_ffn(x[t:t + 1], deq["gate"][e], deq["up"][e],
                                               deq["down"][e])[0]
    if shared_deq is not None:
        s = expert_ffn(x, shared_deq["gate"][0], shared_deq["up"][0], shared_deq["down"][0])
        c = np.ones(T, np.float32) if shared_coef is None else np.asarray(shared_coef, np.float32)
        y += c[:, None] * s
    return y


def moe_ref_grouped(x, deq, topk_idx, topk_w, shared_deq=None, shared_coef=None):
    """moe_ref evaluated expert by expert (each expert's tokens in one batch),
    the way MoELayer._run_gpu_experts groups its tasks (fastllm_py/moe.py:
    135-159); same arithmetic as moe_ref up to fp32 summation order."""
    x = np.asarray(x, np.float32)
    idx = np.asarray(topk_idx)
    w = np.asarray(topk_w, np.float32)
    T = x.shape[0]
    y = np.zeros((T, deq["down"].shape[1]), np.float32)
    for e in np.unique(idx):
        tt, kk = np.nonzero(idx == e)
        f = expert_ffn(x[tt], deq["gate"][e], deq["up"][e], deq["down"][e])
        np.add.at(y, tt, w[tt, kk][:, None] * f)
    if shared_deq is not None:
        s = expert_ffn(x, shared_deq["gate"][0], shared_deq["up"][0], shared_deq["down"][0])
        c = np.ones(T, np.float32) if shared_coef is None else np.asarray(shared_coef, np.float32)
        y += c[:, None] * s
    return y

"""Pins of the MoE oracle (oracle/moe.py) on the CPU.

The oracle restates the reference's per-expert numpy FFN
(fastllm_py/moe.py:22-26,161-175; tests/test_moe_int4.py:42-52).  It is
checked here against a brute-force scalar evaluation on tiny shapes, and
against what the mathematics fixes: linearity in the routing weights, a
repeated expert summing its weights, zero weights vanishing, and the
expert-grouped evaluation equal to the per-token one.
"""
import math

import numpy as np

from oracle import moe as OM


def _rand_experts(rng, E, hidden, inter):
    return {"gate": rng.standard_normal((E, inter, hidden)).astype(np.float32) * 0.3,
            "up": rng.standard_normal((E, inter, hidden)).astype(np.float32) * 0.3,
            "down": rng.standard_normal((E, hidden, inter)).astype(np.float32) * 0.3}


def _ffn_scalar(x, wg, wu, wd):
    """silu(x wg^T) * (x wu^T) then wd, one scalar at a time."""
    inter, hidden = wg.shape
    h = []
    for i in range(inter):
        g = sum(float(x[k]) * float(wg[i, k]) for k in range(hidden))
        u = sum(float(x[k]) * float(wu[i, k]) for k in range(hidden))
        h.append(g / (1.0 + math.exp(-g)) * u)
    return np.array([sum(h[i] * float(wd[o, i]) for i in range(inter))
                     for o in range(wd.shape[0])])


def test_expert_ffn_brute_force():
    rng = np.random.default_rng(1)
    d = _rand_experts(rng, 1, 6, 5)
    x = rng.standard_normal((3, 6)).astype(np.float32)
    got = OM.expert_ffn(x, d["gate"][0], d["up"][0], d["down"][0])
    for t in range(3):
        np.testing.assert_allclose(got[t], _ffn_scalar(x[t], d["gate"][0], d["up"][0], d["down"][0]),
                                   rtol=1e-5, atol=1e-6)


def test_moe_ref_brute_force_and_shared():
    rng = np.random.default_rng(2)
    E, hidden, inter, T = 4, 5, 3, 2
    d = _rand_experts(rng, E, hidden, inter)
    sh = _rand_experts(rng, 1, hidden, 7)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    idx = np.array([[2, 0], [3, 2]])
    w = np.array([[0.7, 0.3], [0.25, 0.5]], np.float32)
    coef = np.array([0.2, 0.9], np.float32)
    got = OM.moe_ref(x, d, idx, w, sh, coef)
    for t in range(T):
        want = sum(w[t, j] * _ffn_scalar(x[t], d["gate"][e], d["up"][e], d["down"][e])
                   for j, e in enumerate(idx[t]))
        want = want + coef[t] * _ffn_scalar(x[t], sh["gate"][0], sh["up"][0], sh["down"][0])
        np.testing.assert_allclose(got[t], want, rtol=1e-5, atol=1e-6)


def test_moe_ref_weight_identities():
    rng = np.random.default_rng(3)
    E, hidden, inter, T = 5, 8, 6, 4
    d = _rand_experts(rng, E, hidden, inter)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    idx = rng.integers(0, E, size=(T, 3))
    w = rng.random((T, 3)).astype(np.float32)
    y = OM.moe_ref(x, d, idx, w)
    # linear in the routing weights
    np.testing.assert_allclose(OM.moe_ref(x, d, idx, 2 * w), 2 * y, rtol=1e-5, atol=1e-6)
    # zero weights contribute nothing
    assert not OM.moe_ref(x, d, idx, np.zeros_like(w)).any()
    # one expert listed twice == listed once with the summed weight
    idx2 = np.array([[1, 1]] * T)
    w2 = np.array([[0.25, 0.5]] * T, np.float32)
    np.testing.assert_allclose(OM.moe_ref(x, d, idx2, w2),
                               OM.moe_ref(x, d, idx2[:, :1], np.full((T, 1), 0.75, np.float32)),
                               rtol=1e-5, atol=1e-6)


def test_grouped_equals_per_token():
    rng = np.random.default_rng(4)
    E, hidden, inter, T, K = 16, 32, 24, 40, 4
    d = _rand_experts(rng, E, hidden, inter)
    sh = _rand_experts(rng, 1, hidden, 20)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(T)])
    w = rng.random((T, K)).astype(np.float32)
    coef = rng.random(T).astype(np.float32)
    np.testing.assert_allclose(OM.moe_ref_grouped(x, d, idx, w, sh, coef),
                               OM.moe_ref(x, d, idx, w, sh, coef), rtol=2e-5, atol=1e-5)

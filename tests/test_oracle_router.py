"""Pins of the router oracle (oracle/router.py) — CPU only."""
import numpy as np
import pytest

from oracle import router as R


def test_np_exp_restatement_matches_numpy():
    rng = np.random.default_rng(0)
    for lo, hi in [(-87.0, 0.0), (-2.0, 2.0), (-30.0, 0.0), (0.0, 88.0)]:
        x = rng.uniform(lo, hi, 500_000).astype(np.float32)
        np.testing.assert_array_equal(R.np_exp_f32(x).view(np.uint32), np.exp(x).view(np.uint32))
    # strided bit sweep of the routing range [-30, 0]
    b = np.arange(0x80000000, 0xC1F00000, 251, dtype=np.uint64).astype(np.uint32)
    x = b.view(np.float32)
    np.testing.assert_array_equal(R.np_exp_f32(x).view(np.uint32), np.exp(x).view(np.uint32))
    sp = np.array([0.0, -0.0, 88.7, 88.73, -103.9, -104.0, np.inf, -np.inf], np.float32)
    np.testing.assert_array_equal(R.np_exp_f32(sp), np.exp(sp))


@pytest.mark.parametrize("E", [1, 4, 7, 8, 9, 60, 64, 127, 128, 129, 200, 256])
def test_pairwise_rowsum_matches_numpy(E):
    rng = np.random.default_rng(E)
    a = rng.random((500, E)).astype(np.float32)
    np.testing.assert_array_equal(R.np_rowsum_f32(a), a.sum(-1))


def test_softmax_probs_match_numpy_formula():
    # the reference's exact expression, with the installed numpy
    rng = np.random.default_rng(1)
    s = rng.standard_normal((256, 60)).astype(np.float16).astype(np.float32)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    p_ref = e / e.sum(-1, keepdims=True)
    p, _ = R._scores(s, "softmax", None)
    np.testing.assert_array_equal(p.view(np.uint32), p_ref.view(np.uint32))


def _selected(scores, top_k, fn=R.route_topk, **kw):
    sel = {}
    for t in fn(scores, top_k, **kw):
        for tok in t.token_idx.tolist():
            sel.setdefault(int(tok), set()).add(t.expert_id)
    return sel


def test_group_routing_known_answer():
    # reference tests/test_router.py:36-43
    logits = np.array([[5, 4, -9, -9, 6, 3, -9, -9]], dtype=np.float32)
    bias = np.zeros(8, dtype=np.float32)
    for fn in (R.route_topk, R.route_topk_canonical):
        sel = _selected(logits, 2, fn, scoring="sigmoid", e_score_bias=bias, n_group=4,
                        topk_group=2)
        assert sel[0] == {0, 4}


def _ref_group(logits, top_k, n_group, topk_group, bias):
    # brute force of reference tests/test_router.py:17-33
    T, E = logits.shape
    gsz = E // n_group
    probs = 1.0 / (1.0 + np.exp(-logits))
    select = probs + bias
    gs = select.reshape(T, n_group, gsz)
    group_score = np.sort(gs, -1)[:, :, -2:].sum(-1)
    out = {}
    for t in range(T):
        keep = set(np.argsort(-group_score[t])[:topk_group].tolist())
        masked = select[t].copy()
        for g in range(n_group):
            if g not in keep:
                masked[g * gsz:(g + 1) * gsz] = -np.inf
        out[t] = set(np.argsort(-masked)[:top_k].tolist())
    return out


def test_group_routing_matches_brute_force():
    # reference tests/test_router.py:46-55
    rng = np.random.default_rng(0)
    E, n_group, topk_group, top_k, T = 16, 4, 2, 4, 6
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    ref = _ref_group(logits, top_k, n_group, topk_group, bias)
    for fn in (R.route_topk, R.route_topk_canonical):
        got = _selected(logits, top_k, fn, scoring="sigmoid", e_score_bias=bias, n_group=n_group,
                        topk_group=topk_group)
        for t in range(T):
            assert got[t] == ref[t]


def test_no_groups_is_unchanged():
    # reference tests/test_router.py:58-64
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((4, 8)).astype(np.float32)
    assert _selected(logits, 2, scoring="softmax") == _selected(logits, 2, scoring="softmax",
                                                                  n_group=0, topk_group=0)


@pytest.mark.parametrize("T,E,k,norm", [(16, 60, 4, False), (64, 128, 8, True), (300, 60, 4, True)])
def test_selection_vs_sort_brute_force(T, E, k, norm):
    rng = np.random.default_rng(T + E)
    s = rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)
    ties = R.boundary_ties(s, k)
    _, idx_a, w_a = R.route_topk(s, k, norm_topk_prob=norm, return_arrays=True)
    _, idx_c, w_c = R.route_topk_canonical(s, k, norm_topk_prob=norm, return_arrays=True)
    probs, _ = R._scores(s, "softmax", None)
    for t in range(T):
        brute = set(np.argsort(-probs[t], kind="stable")[:k].tolist())
        if not ties[t]:
            assert set(idx_a[t].tolist()) == brute == set(idx_c[t].tolist())
        # canonical order: descending probability
        assert np.all(np.diff(probs[t][idx_c[t]]) <= 0)
    if not norm:
        # unnormalised weights are the probabilities themselves: bit-equal as sets
        for t in np.nonzero(~ties)[0]:
            a = dict(zip(idx_a[t].tolist(), w_a[t].view(np.uint32).tolist()))
            c = dict(zip(idx_c[t].tolist(), w_c[t].view(np.uint32).tolist()))
            assert a == c


def test_norm_weights_agree_within_one_ulp_across_orders():
    rng = np.random.default_rng(7)
    s = rng.standard_normal((512, 128)).astype(np.float16).astype(np.float32)
    ties = R.boundary_ties(s, 8)
    _, idx_a, w_a = R.route_topk(s, 8, norm_topk_prob=True, return_arrays=True)
    _, idx_c, w_c = R.route_topk_canonical(s, 8, norm_topk_prob=True, return_arrays=True)
    for t in np.nonzero(~ties)[0]:
        a = dict(zip(idx_a[t].tolist(), w_a[t].tolist()))
        for e, wc in zip(idx_c[t].tolist(), w_c[t].tolist()):
            assert abs(np.float32(a[e]).view(np.int32) - np.float32(wc).view(np.int32)) <= 1

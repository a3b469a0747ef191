"""oracle/argpartition.py against the installed np.argpartition.

The restatement models numpy 2.2.6's float32 argpartition on an AVX512_SKX
host (x86-simd-sort's key/index network for rows of <= 256 elements).  It is
pinned here by comparing the whole output permutation -- the selected set
and its order, ties included -- with np.argpartition on router rows with
forced ties: softmax probabilities of fp16 logits drawn from a few distinct
values (so most rows hold tied probabilities), E in {60, 128, 256},
kth = k - 1 for k in {2, 4, 8}; 1.02 million rows in all.  Plus every row
length 1..256 on small tie-heavy batches, and all-equal rows (where the
network must leave the index order unchanged).
"""
import numpy as np
import pytest

from oracle import argpartition as AP
from oracle import router as R

def _avx512_skx() -> bool:
    try:
        from numpy._core._multiarray_umath import __cpu_features__
    except ImportError:
        return False
    return bool(__cpu_features__.get("AVX512_SKX"))


pytestmark = pytest.mark.skipif(
    not _avx512_skx() or int(np.__version__.split(".")[0]) < 2,
    reason="np.argpartition here is not the numpy >= 2 AVX512_SKX path the restatement models")


def _router_keys(rng, rows, E, levels):
    vals = rng.standard_normal(levels).astype(np.float16)
    logits = vals[rng.integers(0, levels, size=(rows, E))].astype(np.float32)
    probs, _ = R._scores(logits, "softmax", None)
    return -probs


@pytest.mark.parametrize("E,rows", [(60, 400_000), (128, 400_000), (256, 220_000)])
def test_router_rows_with_ties(E, rows):
    rng = np.random.default_rng(E)
    n_tied = 0
    for start in range(0, rows, 20_000):
        keys = _router_keys(rng, 20_000, E, levels=int(rng.integers(3, 12)))
        mine = AP.network_argsort(keys)
        for k in (2, 4, 8):
            ref = np.argpartition(keys, k - 1, axis=-1)
            bad = np.nonzero((mine != ref).any(axis=1))[0]
            assert bad.size == 0, (E, k, start + bad[:5])
        s = np.sort(keys, axis=-1)
        n_tied += int((s[:, 3] == s[:, 4]).sum())
    assert n_tied > rows // 10  # the rows really hold ties at the boundary


def test_every_length_and_all_equal():
    rng = np.random.default_rng(1)
    for N in range(1, 257):
        keys = rng.integers(0, 3, size=(200, N)).astype(np.float32)
        mine = AP.network_argsort(keys)
        for kth in {0, N // 2, N - 1}:
            np.testing.assert_array_equal(mine, np.argpartition(keys, kth, axis=-1), err_msg=str(N))
        eq = np.zeros((1, N), np.float32)
        np.testing.assert_array_equal(AP.network_argsort(eq)[0], np.arange(N))


def test_infinities_and_group_scores():
    """+inf keys (experts of dropped groups) and short rows (group scores)."""
    rng = np.random.default_rng(2)
    keys = rng.integers(0, 4, size=(5000, 64)).astype(np.float32)
    keys[rng.random(keys.shape) < 0.4] = np.inf
    np.testing.assert_array_equal(AP.network_argsort(keys), np.argpartition(keys, 7, axis=-1))
    g = rng.integers(0, 3, size=(5000, 8)).astype(np.float32)
    np.testing.assert_array_equal(AP.network_argsort(g), np.argpartition(g, 3, axis=-1))

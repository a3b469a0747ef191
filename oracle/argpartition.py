"""Restatement of numpy's float32 ``np.argpartition`` for rows of at most 256
elements, as numpy 2.2.6 runs it on an x86-64 host with AVX512_SKX (test
oracle only).

Why it is needed: the reference selects experts with
``np.argpartition(-p, k - 1)[:, :k]`` (fastllm_py/expert_router.py:50,55).
Which of several experts tied at the k-th value that picks is not defined by
numpy's documentation; it is whatever the selection algorithm leaves.

Third-party algorithm: numpy >= 2.0 sends a single-kth float32 argpartition
to the vendored x86-simd-sort library (``argquickselect_dispatch`` ->
``avx512_argselect``) when the CPU has AVX512_SKX.  Arrays of at most 256
elements are not partitioned at all there: they are fully sorted by a
bitonic key/index network (``argsort_n``) on 8-lane registers (8 float keys,
8 int64 indices), and the first k positions are the selection.  The network
(x86-simd-sort's published design):

  1. pad the row to maxN = max(8, the next power of two >= N) with +inf keys
     and index 0; split it into maxN/8 registers of 8 lanes;
  2. sort each register with the 6-step bitonic network
     (partner lane l^1, mask 0xAA), (l -> 4*(l//4)+3-l%4, 0xCC), (l^1, 0xAA),
     (l -> 7-l, 0xF0), (l^2, 0xCC), (l^1, 0xAA);
  3. merge registers in groups of 2, 4, ... maxN/8: within a group of n,
     register i is compare-exchanged lane-wise with register n-1-i read in
     reversed lane order (written back reversed), then half-cleaners across
     registers (i with i + m/2 inside blocks of m = n/2, n/4, ... 2), then
     each register's in-lane bitonic merge (l^4, 0xF0), (l^2, 0xCC),
     (l^1, 0xAA).
A "mask" step keeps max(own, partner) in the lanes whose mask bit is set and
the min in the others; the index follows the key, and a lane whose result
equals its own key keeps its own index.  So equal keys never swap: ties are
resolved only by the network's wiring, which is what this restatement pins
(tests/test_oracle_argpartition.py checks the full output permutation
against the installed ``np.argpartition`` on tie-heavy rows).

Not restated: rows longer than 256 (a vectorised quickselect partition;
the router here takes E <= 256), rows holding NaN (numpy then takes another
path), and other CPUs (an AVX2-only or non-x86 host runs a different
algorithm and can break ties differently).
"""
from __future__ import annotations

import numpy as np

_L = np.arange(8)
SORT8 = [(_L ^ 1, 0xAA), (4 * (_L // 4) + 3 - _L % 4, 0xCC), (_L ^ 1, 0xAA),
         (7 - _L, 0xF0), (_L ^ 2, 0xCC), (_L ^ 1, 0xAA)]
MERGE8 = [(_L ^ 4, 0xF0), (_L ^ 2, 0xCC), (_L ^ 1, 0xAA)]
_STAGES: dict = {}


def _lane_stage(maxN, perm, mask):
    x = np.arange(maxN)
    partner = 8 * (x // 8) + perm[x % 8]
    take_max = ((mask >> (x % 8)) & 1).astype(bool)
    return partner, take_max


def stages(maxN: int) -> list:
    """The network's steps for maxN positions as (partner position, keep-max)
    arrays: position x holds lane x % 8 of register x // 8."""
    if maxN in _STAGES:
        return _STAGES[maxN]
    st = [_lane_stage(maxN, perm, mask) for perm, mask in SORT8]
    nv = maxN // 8
    x = np.arange(maxN)
    R, lane = x // 8, x % 8
    n = 2
    while n <= nv:
        # register R against register g + n - 1 - (R - g), lanes reversed
        g = R - R % n
        a = R - g
        st.append((8 * (g + n - 1 - a) + (7 - lane), a >= n // 2))
        m = n // 2
        while m >= 2:  # half-cleaners across registers, distance m/2
            d = m // 2
            hi = (R % m) >= d
            st.append((8 * np.where(hi, R - d, R + d) + lane, hi))
            m //= 2
        st += [_lane_stage(maxN, perm, mask) for perm, mask in MERGE8]
        n *= 2
    _STAGES[maxN] = st
    return st


def network_argsort(keys: np.ndarray) -> np.ndarray:
    """keys (rows, N) float32, N <= 256, no NaN -> (rows, N) int64: the index
    order the network leaves (ascending keys; ties by wiring)."""
    keys = np.asarray(keys, dtype=np.float32)
    rows, N = keys.shape
    assert 1 <= N <= 256
    maxN = 8
    while maxN < N:
        maxN *= 2
    # positions on the first axis: each step gathers whole rows of `rows` values
    k = np.full((maxN, rows), np.inf, dtype=np.float32)
    k[:N] = keys.T
    i = np.zeros((maxN, rows), dtype=np.int32)
    i[:N] = np.arange(N, dtype=np.int32)[:, None]
    for partner, take_max in stages(maxN):
        pk = k[partner]
        r = np.where(take_max[:, None], np.maximum(k, pk), np.minimum(k, pk))
        i = np.where(r == k, i, i[partner])  # a lane keeps its index when it keeps its key
        k = r
    return i[:N].T.astype(np.int64)


def argpartition_rows(keys: np.ndarray, kth: int) -> np.ndarray:
    """``np.argpartition(keys, kth, axis=-1)`` for float32 rows of N <= 256
    elements on the host described above (the whole order, which for these
    sizes is the network's full sort)."""
    keys = np.asarray(keys, dtype=np.float32)
    assert 0 <= kth < keys.shape[-1]
    return network_argsort(keys.reshape(-1, keys.shape[-1])).reshape(keys.shape)

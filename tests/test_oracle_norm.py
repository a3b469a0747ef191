"""Pins of the add_rmsnorm oracle (oracle/norm.py, oracle/c/norm.c)."""
import numpy as np
import pytest

from oracle import norm as ON


def test_closed_form_constant_rows():
    # v = 2 everywhere, eps = 0: sum of squares 4 * dim exactly, inv = 1/2, h = w
    dim = 4096
    x = np.full((3, dim), 1.5, np.float32)
    d = np.full((3, dim), 0.5, np.float32)
    w = np.random.default_rng(0).standard_normal(dim).astype(np.float16)
    xnew, h = ON.add_rmsnorm(x, d, w, 0.0)
    assert (xnew == 2.0).all()
    np.testing.assert_array_equal(h, np.broadcast_to(w, h.shape))


@pytest.mark.parametrize("k", [-3, 5])
def test_power_of_two_scale_invariance(k):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 1000)).astype(np.float32)
    d = rng.standard_normal((4, 1000)).astype(np.float32)
    w = rng.standard_normal(1000).astype(np.float32)
    _, h0 = ON.add_rmsnorm(x, d, w, 0.0)
    _, h1 = ON.add_rmsnorm(x * np.float32(2.0 ** k), d * np.float32(2.0 ** k), w, 0.0)
    np.testing.assert_array_equal(h0, h1)


@pytest.mark.parametrize("rows,dim", [(5, 1024), (1, 2048), (3, 200), (2, 4096)])
def test_matches_float64_formula(rows, dim):
    # the reference's own test formula (tests/test_fused_ops.py:10-14), in float64
    rng = np.random.default_rng(rows * 7 + dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float16)
    w = rng.standard_normal(dim).astype(np.float16)
    eps = 1e-6
    xnew, h = ON.add_rmsnorm(x, d, w, eps)
    v = x.astype(np.float64) + d.astype(np.float64)
    np.testing.assert_array_equal(xnew, (x + d.astype(np.float32)))
    ref = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps) * w.astype(np.float64)
    np.testing.assert_allclose(h.astype(np.float64), ref, rtol=1e-3, atol=2e-3)
    # a wrong mean (dim - 1) or a dropped weight would fail this
    assert np.abs(h.astype(np.float64) - ref).max() < 4e-3

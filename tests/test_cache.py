"""Versioned on-disk caches (fastllm_py/cache.py): round trips, the format
tag, atomic writes.  CPU only (numpy payloads, device=None)."""
import numpy as np
import pytest

from fastllm_py import cache


def test_marlin_payload_round_trip(tmp_path):
    rng = np.random.default_rng(0)
    p = {"qweight": rng.integers(0, 2 ** 32, size=(64, 32), dtype=np.uint64).astype(np.uint32),
         "scales": rng.standard_normal((2, 32)).astype(np.float16),
         "zeros": rng.integers(0, 2 ** 32, size=(2, 4), dtype=np.uint64).astype(np.uint32)}
    f = tmp_path / "m" / "w.npz"
    cache.save_marlin_payload(f, p)
    assert f.exists() and not (tmp_path / "m" / "w.npz.tmp.npz").exists()
    back = cache.load_marlin_payload(f, device=None)
    assert set(back) == set(p)
    for k in p:
        np.testing.assert_array_equal(back[k], p[k])
        assert back[k].dtype == p[k].dtype


def test_expert_payloads_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    pays = {e: {"qweight": rng.integers(0, 255, size=(8, 8)).astype(np.uint32),
                "scales": rng.standard_normal((1, 8)).astype(np.float16)} for e in (0, 3, 11)}
    f = tmp_path / "marlin.L0.npz"
    cache.save_expert_payloads(f, pays)
    back = cache.load_expert_payloads(f, device=None)
    assert sorted(back) == [0, 3, 11]
    for e in pays:
        for k in pays[e]:
            np.testing.assert_array_equal(back[e][k], pays[e][k])


def test_stacked_round_trip_and_scalars(tmp_path):
    rng = np.random.default_rng(2)
    st = {"group": 128, "layout": "tile16x128",
          "gate.qtile": rng.integers(0, 255, size=(2, 4, 2, 1024)).astype(np.uint8),
          "gate.sz": rng.integers(0, 2 ** 31, size=(2, 4, 2, 16)).astype(np.int32),
          "gate.shape": (64, 256)}
    f = tmp_path / "experts.L3.npz"
    cache.save_stacked(f, st)
    back = cache.load_stacked(f, device=None)
    assert back["group"] == 128 and isinstance(back["group"], int)
    assert back["layout"] == "tile16x128"
    assert back["gate.shape"] == (64, 256)
    np.testing.assert_array_equal(back["gate.qtile"], st["gate.qtile"])
    np.testing.assert_array_equal(back["gate.sz"], st["gate.sz"])


def test_foreign_or_untagged_cache_is_refused(tmp_path):
    f = tmp_path / "ref.npz"
    np.savez(f, qweight=np.zeros(4, np.uint32))  # a reference-style cache: no tag
    with pytest.raises(ValueError):
        cache.load_marlin_payload(f, device=None)
    cache.save_stacked(tmp_path / "s.npz", {"group": 128})
    with pytest.raises(ValueError):  # right file, wrong kind
        cache.load_marlin_payload(tmp_path / "s.npz", device=None)

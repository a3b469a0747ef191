"""Caches written from device payloads load back into working kernels."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_marlin_cache_on_device(torch_gpu, tmp_path):
    from fastllm_py import cache
    from fastllm_py.kernels import marlin
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    rng = np.random.default_rng(5)
    W = torch.from_numpy((rng.standard_normal((512, 1024)) * 0.02).astype(np.float32)).cuda()
    pay = quantize_marlin_matrix_device(W, 128)
    cache.save_marlin_payload(tmp_path / "w.npz", pay)
    back = cache.load_marlin_payload(tmp_path / "w.npz")
    a = torch.from_numpy(rng.standard_normal((4, 1024)).astype(np.float16)).cuda()
    y0 = marlin.marlin_gemm_int4(a, pay["qweight"], pay["scales"], pay["zeros"])
    y1 = marlin.marlin_gemm_int4(a, back["qweight"], back["scales"], back["zeros"])
    assert torch.equal(y0, y1)


def test_stacked_cache_on_device(torch_gpu, tmp_path):
    from fastllm_py import cache
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(6)
    E, hidden, inter = 8, 256, 384
    ews = [{"gate": (rng.standard_normal((inter, hidden)) * 0.05).astype(np.float16),
            "up": (rng.standard_normal((inter, hidden)) * 0.05).astype(np.float16),
            "down": (rng.standard_normal((hidden, inter)) * 0.05).astype(np.float16)} for _ in range(E)]
    st = moe_int4.build_stacked_experts(ews, 128)
    cache.save_stacked(tmp_path / "experts.L0.npz", st)
    st2 = cache.load_stacked(tmp_path / "experts.L0.npz")
    x = torch.from_numpy(rng.standard_normal((2, hidden)).astype(np.float32)).cuda()
    r = route_topk_device(rng.standard_normal((2, E)).astype(np.float32), 2)
    kw = dict(max_slots=4, max_entries=4)
    y0 = moe_int4.moe_forward(x, st, E, hidden, inter, r, **kw).cpu().numpy()
    y1 = moe_int4.moe_forward(x, st2, E, hidden, inter, r, **kw).cpu().numpy()
    np.testing.assert_allclose(y1, y0, rtol=1e-6, atol=1e-7)

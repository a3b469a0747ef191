"""The Python drop-in layer on the GPU: _expert_ffn_marlin against the
oracle at config-5 expert shapes, and the CuPy interop of the swap adapters
and the graph-decoder shims (through a stand-in array type exposing
__cuda_array_interface__, as CuPy's arrays do)."""
import sys
import types

import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu


def _marlin_hat(W, gs=128):
    q, s, z = Q.quantize_int4_marlin(W, gs)
    s16, zp = Q.marlin_scales_zeros(s, z)
    return Q.marlin_dequant(q, s16, zp, gs)


@pytest.mark.parametrize("M", [1, 32, 100])
def test_expert_ffn_marlin_config5(torch_gpu, M):
    """Qwen3-30B-A3B expert (hidden 2048, inter 768): gate, up, swiglu, down on
    one Marlin payload (moe.py:62-81) vs the fp32 chain on the same packed
    weights."""
    from fastllm_py.moe import _expert_ffn_marlin, build_marlin_expert_payload

    torch = torch_gpu
    hidden, inter = 2048, 768
    rng = np.random.default_rng(5500 + M)
    w = {"gate": (rng.standard_normal((inter, hidden)) * 0.02).astype(np.float16),
         "up": (rng.standard_normal((inter, hidden)) * 0.02).astype(np.float16),
         "down": (rng.standard_normal((hidden, inter)) * 0.02).astype(np.float16)}
    pay = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda()
           for k, v in build_marlin_expert_payload(w).items()}
    x = rng.standard_normal((M, hidden)).astype(np.float16)
    y = _expert_ffn_marlin(torch.from_numpy(x).cuda(), pay)
    assert y.shape == (M, hidden) and y.dtype == torch.float16
    hat = {k: _marlin_hat(v.astype(np.float32)) for k, v in w.items()}
    xf = x.astype(np.float32)
    g, u = xf @ hat["gate"].T, xf @ hat["up"].T
    ref = ((g / (1.0 + np.exp(-g))) * u) @ hat["down"].T
    assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < 1e-2


class _FakeArray:
    """Stand-in for a CuPy array: only __cuda_array_interface__ and shape."""

    __module__ = "cupy_standin"

    def __init__(self, t):
        self._t = t
        self.__cuda_array_interface__ = t.__cuda_array_interface__
        self.shape = tuple(t.shape)


@pytest.fixture
def fake_cupy(torch_gpu):
    torch = torch_gpu
    mod = types.ModuleType("cupy")
    mod.asarray = lambda t: _FakeArray(t.contiguous())
    stream = types.SimpleNamespace(ptr=int(torch.cuda.current_stream().cuda_stream))
    mod.cuda = types.SimpleNamespace(get_current_stream=lambda: stream)
    saved = sys.modules.get("cupy")
    sys.modules["cupy"] = mod
    yield mod
    if saved is None:
        del sys.modules["cupy"]
    else:
        sys.modules["cupy"] = saved


def test_adapter_round_trips_device_arrays(torch_gpu, fake_cupy):
    from fastllm_py import swap
    from fastllm_py.kernels import marlin, moe_int4
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    N, K = 512, 1024
    W = torch.randn((N, K), generator=torch.Generator().manual_seed(1)).mul_(0.02).cuda()
    pay = quantize_marlin_matrix_device(W, 128)
    x = torch.randn((2, K), device="cuda").half()
    direct = marlin.gemm_fast(x, pay["qweight"], pay["scales"], pay["zeros"], N, K)
    fa = {k: _FakeArray(v) for k, v in pay.items()}
    out = swap.adapt(marlin.gemm_fast)(_FakeArray(x), fa["qweight"], fa["scales"], fa["zeros"], N, K)
    assert isinstance(out, _FakeArray)
    torch.cuda.synchronize()
    assert torch.equal(out._t, direct)
    # xp=cupy with a host weight (graph_decode.py:563): device results come back
    w = (np.random.default_rng(2).standard_normal((64, 256)) * 0.02).astype(np.float32)
    p = swap.adapt(moe_int4.quantize_int4_rowmajor)(w, 128, xp=fake_cupy)
    assert isinstance(p["qweight"], _FakeArray) and p["shape"] == (64, 256)
    ref = moe_int4.quantize_int4_rowmajor(w, 128)
    np.testing.assert_array_equal(p["qweight"]._t.cpu().numpy(), ref["qweight"])


class _FakeStream:
    """Stand-in for a cupy.cuda.Stream: CuPy streams expose their handle as
    ``.ptr`` (not ``.cuda_stream``) and live in module cupy.cuda.stream."""

    __module__ = "cupy.cuda.stream"

    def __init__(self, ptr):
        self.ptr = int(ptr)


def test_adapter_passes_cupy_streams(torch_gpu, fake_cupy):
    """The reference's hot callers pass stream=<cupy Stream> (graph_decode.py:778,
    batched.py:161, moe.py:152): the adapted gemm_fast and _expert_ffn_marlin
    launch on that stream and equal the direct calls bit for bit."""
    from fastllm_py import swap
    from fastllm_py.kernels import marlin
    from fastllm_py.moe import _expert_ffn_marlin, build_marlin_expert_payload

    torch = torch_gpu
    side = torch.cuda.Stream()
    fs = _FakeStream(side.cuda_stream)
    N, K = 768, 2048
    rng = np.random.default_rng(11)
    w = {"gate": (rng.standard_normal((N, K)) * 0.02).astype(np.float16),
         "up": (rng.standard_normal((N, K)) * 0.02).astype(np.float16),
         "down": (rng.standard_normal((K, N)) * 0.02).astype(np.float16)}
    pay = {k: torch.from_numpy(np.ascontiguousarray(v)).cuda()
           for k, v in build_marlin_expert_payload(w).items()}
    for M in (1, 3):
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16)).cuda()
        ws = marlin.make_workspace(N)
        direct = marlin.gemm_fast(x, pay["gate.qweight"], pay["gate.scales"], pay["gate.zeros"],
                                  N, K, stream=torch.cuda.current_stream(), workspace=ws)
        ffn = _expert_ffn_marlin(x, pay)
        torch.cuda.synchronize()
        fa = {k: _FakeArray(v) for k, v in pay.items()}
        ws2 = _FakeArray(marlin.make_workspace(N))
        out = swap.adapt(marlin.gemm_fast)(_FakeArray(x), fa["gate.qweight"], fa["gate.scales"],
                                           fa["gate.zeros"], N, K, stream=fs, workspace=ws2)
        out2 = swap.adapt(_expert_ffn_marlin)(_FakeArray(x), fa, stream=fs)
        # torch tensors in, only the stream from CuPy: results still leave as CuPy arrays
        out3 = swap.adapt(marlin.gemm_fast)(x, pay["gate.qweight"], pay["gate.scales"],
                                            pay["gate.zeros"], N, K, stream=fs,
                                            workspace=marlin.make_workspace(N))
        side.synchronize()
        assert isinstance(out, _FakeArray) and isinstance(out2, _FakeArray)
        assert isinstance(out3, _FakeArray)
        assert torch.equal(out._t, direct) and torch.equal(out3._t, direct)
        assert torch.equal(out2._t, ffn)


def test_graph_shims_match_library_paths(torch_gpu, fake_cupy):
    from fastllm_py import graph_shims
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    torch = torch_gpu
    rng = np.random.default_rng(3)
    W = (rng.standard_normal((768, 1024)) * 0.02).astype(np.float16)
    pay = moe_int4.quantize_int4_rowmajor(torch.from_numpy(W).cuda(), 128)
    x = torch.from_numpy(rng.standard_normal((1, 1024)).astype(np.float16)).cuda()
    y = torch.empty(768, dtype=torch.float16, device="cuda")
    k = graph_shims.dense_gemv_kernel(fake_cupy, "__half")
    k((48,), (512,), (_FakeArray(x.reshape(-1)), _FakeArray(pay["qweight"]),
                      _FakeArray(pay["scales"]), _FakeArray(pay["zeros"]), _FakeArray(y),
                      np.int32(1024), np.int32(768), np.int32(128), np.int32(16)),
      shared_mem=2048)
    ref = moe_int4.dgemv(x, pay)
    torch.cuda.synchronize()
    assert torch.equal(y, ref.reshape(-1))
    E, K = 60, 4
    logits = torch.from_numpy(rng.standard_normal(E).astype(np.float16).astype(np.float32)).cuda()
    rw = torch.empty(E, device="cuda")
    aidx = torch.empty(K, dtype=torch.int32, device="cuda")
    r = graph_shims.route_topk_kernel(fake_cupy)
    r((1,), (128,), (_FakeArray(logits), _FakeArray(rw), _FakeArray(aidx), np.int32(E),
                     np.int32(K), np.int32(0), np.float32(1.0)), shared_mem=(E + 128) * 4)
    ref = route_topk_device(logits.reshape(1, E), K)
    torch.cuda.synchronize()
    assert torch.equal(aidx, ref["topk_ids"].reshape(-1))
    assert torch.equal(rw, ref["rw"].reshape(-1))

"""Dense MXFP4 GEMV / prefill GEMM (fastllm_mxfp4_gemv) on the GPU vs the oracle.

The weights go through the GPU quantizer and tile repack (both pinned
bit-exact against oracle/mx.py in test_gpu_moe_lowp.py); the reference is the
fp64 product of the fp16 activations with oracle/mx.py's dequantization of
the same weights.  The kernels feed the MFMAs fp16(code x scale), exact at
these weights' scales (>= 2^-14), and accumulate in fp32, so their only
deviations are the fp32 summation order and the final fp16 rounding (2^-11
relative): max-abs-rel 2e-3.
"""
import numpy as np
import pytest

from oracle import mx
from oracle import quant as Q

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _case(torch, rng, N, K, M, scale=0.05):
    from fastllm_py.kernels import mxfp4

    W = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    wq = mxfp4.quantize(torch.from_numpy(W).cuda())
    p, e8 = mx.quantize_mxfp4(W)
    Wd = mx.dequantize_mxfp4(p, e8).astype(np.float64)
    A = (rng.standard_normal((M, K)) * 0.5).astype(np.float16)
    ref = A.astype(np.float64) @ Wd.T
    return wq, A, ref


@pytest.mark.parametrize("N,K,M", [
    (256, 512, 1),        # one block per wave
    (384, 2048, 3),       # two blocks per wave
    (2048, 4096, 8),      # Qwen3-8B o-like K, 8 rows
    (16384, 1024, 16),    # wide output: two tiles per workgroup
    (512, 8192, 5),       # four blocks per wave
    (256, 12288, 2),      # two phases of three blocks (Qwen3-8B down K)
    (256, 4224, 4),       # 33 blocks: the last wave's blocks partly past K
    (640, 1152, 20),      # two 16-row groups, the second ragged
    (128, 256, 33),
    # above 64 rows: the MFMA GEMM (64 x 256 workgroup tiles)
    (512, 1024, 65),      # one row past a tile
    (384, 2048, 130),     # a 256-column strip only partly inside N
    (2048, 4096, 512),    # prefill-sized
    (256, 12288, 100),
])
def test_mxfp4_gemv_matches_oracle(torch_gpu, N, K, M):
    from fastllm_py.kernels import mxfp4

    torch = torch_gpu
    rng = np.random.default_rng(100 + N + K + M)
    wq, A, ref = _case(torch, rng, N, K, M)
    a = torch.from_numpy(A).cuda()
    y = mxfp4.gemv(a, wq)
    y2 = mxfp4.gemv(a, wq)
    torch.cuda.synchronize()
    yc = y.cpu().numpy()
    assert np.isfinite(yc).all()
    assert Q.max_abs_rel(yc, ref) < TOL
    np.testing.assert_array_equal(yc.view(np.uint16), y2.cpu().numpy().view(np.uint16))  # fixed order


def test_mxfp4_gemv_rows_independent(torch_gpu):
    """Row m of C depends only on row m of A: the 16-row groups and the row
    clamping inside a group leak nothing between rows (bit-identical to
    one-row calls)."""
    from fastllm_py.kernels import mxfp4

    torch = torch_gpu
    rng = np.random.default_rng(7)
    wq, A, _ = _case(torch, rng, 512, 2048, 19)
    a = torch.from_numpy(A).cuda()
    y = mxfp4.gemv(a, wq)
    for m in (0, 5, 15, 16, 18):
        ym = mxfp4.gemv(a[m:m + 1].contiguous(), wq)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y[m].cpu().numpy().view(np.uint16), ym[0].cpu().numpy().view(np.uint16))


def test_mxfp4_gemv_argument_checks(torch_gpu):
    from fastllm_py import _native as nat

    torch = torch_gpu
    lib = nat.lib()
    a = torch.zeros((1, 256), dtype=torch.float16, device="cuda")
    q = torch.zeros((16, 2, 1024), dtype=torch.uint8, device="cuda")
    e = torch.zeros((16, 2, 16), dtype=torch.int32, device="cuda")
    c = torch.zeros((1, 256), dtype=torch.float16, device="cuda")
    args = [nat.ptr(a), nat.ptr(q), nat.ptr(e), nat.ptr(c)]
    assert lib.fastllm_mxfp4_gemv(*args, 1, 256, 256, None) == 0
    torch.cuda.synchronize()
    assert lib.fastllm_mxfp4_gemv(*args, 1, 250, 256, None) == 1      # N % 16
    assert lib.fastllm_mxfp4_gemv(*args, 1, 256, 200, None) == 1      # K % 128
    assert lib.fastllm_mxfp4_gemv(*args, 1, 256, 12416, None) == 1    # K > 12288
    assert lib.fastllm_mxfp4_gemv(*args, 0, 256, 256, None) == 1      # M
    assert lib.fastllm_mxfp4_gemv(None, *args[1:], 1, 256, 256, None) == 1


def test_mxfp4_graph_replays(torch_gpu):
    """Capturable (the roadmap's requirement for these kernels): the decode
    GEMV and the prefill GEMM captured in one HIP graph replay bit-identical
    to eager calls, three replays with fresh inputs and eager work between."""
    from fastllm_py.kernels import mxfp4

    torch = torch_gpu
    rng = np.random.default_rng(21)
    wq, _, _ = _case(torch, rng, 1024, 2048, 1)
    a1 = torch.zeros((4, 2048), dtype=torch.float16, device="cuda")
    a2 = torch.zeros((200, 2048), dtype=torch.float16, device="cuda")
    y1 = torch.empty((4, 1024), dtype=torch.float16, device="cuda")
    y2 = torch.empty((200, 1024), dtype=torch.float16, device="cuda")
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):  # warm the allocator and the library off-capture
        mxfp4.gemv(a1, wq, out=y1, stream=st)
        mxfp4.gemv(a2, wq, out=y2, stream=st)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        mxfp4.gemv(a1, wq, out=y1, stream=torch.cuda.current_stream())
        mxfp4.gemv(a2, wq, out=y2, stream=torch.cuda.current_stream())
    for r in range(3):
        a1.copy_(torch.from_numpy((rng.standard_normal((4, 2048)) * 0.5).astype(np.float16)))
        a2.copy_(torch.from_numpy((rng.standard_normal((200, 2048)) * 0.5).astype(np.float16)))
        g.replay()
        torch.cuda.synchronize()
        e1, e2 = mxfp4.gemv(a1, wq), mxfp4.gemv(a2, wq)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(y1.cpu().numpy().view(np.uint16), e1.cpu().numpy().view(np.uint16), err_msg=f"replay {r}")
        np.testing.assert_array_equal(y2.cpu().numpy().view(np.uint16), e2.cpu().numpy().view(np.uint16), err_msg=f"replay {r}")

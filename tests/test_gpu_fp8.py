"""FP8-E4M3 GEMV paths on the GPU vs the numpy oracle.

Mirrors tests/test_native_kernels.py:39-73 of the reference (inline layout,
n in {1, 16}, MoE-like shapes) plus the 128x128-block format at the
BASELINE config-3 shapes with bf16 activations.  Packing is bit-exact; GEMV
outputs are within max-abs-rel 1e-2 of the fp32 dequantize-then-matmul of the
same packed bytes.
"""
import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _bf16_to_f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("is_bf16", [False, True])
def test_inline_quantize_bit_exact(torch_gpu, is_bf16):
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(31 + is_bf16)
    W = rng.standard_normal((96, 640)).astype(np.float32) * 0.1
    W[5, :128] = 0.0  # all-zero block -> scale 1
    W[7, 128:256] *= 1e-4  # tiny block: subnormal codes
    wt = torch.from_numpy(W).cuda().to(torch.bfloat16 if is_bf16 else torch.float16)
    got = fp8.quantize(wt, is_bf16=is_bf16).cpu().numpy()
    want = Q.quantize_fp8_inline(wt.float().cpu().numpy())
    assert got.shape == (96, fp8.packed_row_bytes(640)) == want.shape
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n", [1, 3, 8, 16, 20])
@pytest.mark.parametrize("m,k", [(1024, 512), (2048, 1408), (1408, 2048), (2048, 136), (512, 8192)])
def test_fp8_gemv_inline(torch_gpu, n, m, k):
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(1234 + n + m + k)
    W = rng.standard_normal((k, m)).astype(np.float32) * 0.1
    x = rng.standard_normal((n, m)).astype(np.float32) * 0.5
    wq = fp8.quantize(torch.from_numpy(W).cuda().half())
    out = fp8.fp8_gemv(torch.from_numpy(x).cuda().half(), wq)
    assert out.shape == (n, k) and out.dtype == torch.float16
    w_hat = Q.dequantize_fp8_inline(wq.cpu().numpy(), m)
    ref = Q.matmul_ref(x.astype(np.float16).astype(np.float32), w_hat)
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL
    # the reference's own acceptance: rel-Frobenius vs the unquantized product < 0.05
    full = x.astype(np.float16).astype(np.float32) @ W.astype(np.float16).astype(np.float32).T
    o = out.float().cpu().numpy()
    assert np.linalg.norm(o - full) / np.linalg.norm(full) < 0.05


def test_fp8_gemv_inline_bias_and_stream_entry(torch_gpu):
    from fastllm_py import _native as nat
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(5)
    m, k, n = 1024, 640, 4
    W = torch.from_numpy(rng.standard_normal((k, m)).astype(np.float32) * 0.1).cuda().half()
    x = torch.from_numpy(rng.standard_normal((n, m)).astype(np.float32)).cuda().half()
    b = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).cuda().half()
    wq = fp8.quantize(W)
    c0 = torch.empty((n, k), dtype=torch.float16, device="cuda")
    c1 = torch.empty_like(c0)
    lib = nat.lib()
    assert lib.fastllm_fp8_block128_gemv_fp16(x.data_ptr(), wq.data_ptr(), c0.data_ptr(),
                                              b.data_ptr(), n, m, k, fp8.packed_row_bytes(m)) == 0
    s = torch.cuda.Stream()
    assert lib.fastllm_fp8_block128_gemv_stream(x.data_ptr(), wq.data_ptr(), c1.data_ptr(),
                                                b.data_ptr(), n, m, k, fp8.packed_row_bytes(m), 0,
                                                s.cuda_stream) == 0
    s.synchronize()
    assert torch.equal(c0, c1)
    nob = fp8.fp8_gemv(x, wq)
    np.testing.assert_allclose(c0.float().cpu().numpy(),
                               nob.float().cpu().numpy() + b.float().cpu().numpy()[None], rtol=2e-3,
                               atol=2e-3)


def test_fp8_gemv_rejects_bad_args(torch_gpu):
    from fastllm_py import _native as nat

    torch = torch_gpu
    a = torch.zeros((1, 200), dtype=torch.float16, device="cuda")
    lib = nat.lib()
    # m % 128 != 0 -> 1, no launch
    assert lib.fastllm_fp8_block128_gemv_fp16(a.data_ptr(), a.data_ptr(), a.data_ptr(), None, 1,
                                              200, 8, 208) == 1
    assert lib.fastllm_fp8_block128_quantize(a.data_ptr(), a.data_ptr(), 1, 200, 0) == 1


@pytest.mark.parametrize("act", ["bf16", "fp16"])
def test_fp8_decode_exhaustive_through_gemv(torch_gpu, act):
    """Every finite e4m3 code through the 128x128-block GEMV with unit scales
    and a one-hot activation: C[0, n] = decode(code n) exactly."""
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    codes = np.arange(256, dtype=np.uint8)
    codes[[0x7F, 0xFF]] = 0  # NaN in e4m3fn; the reference encoders never emit them
    N, K = 256, 128
    q = np.zeros((N, K), dtype=np.uint8)
    q[:, 0] = codes
    scales = np.ones((2, 1), dtype=np.float32)
    dt = torch.bfloat16 if act == "bf16" else torch.float16
    x = torch.zeros((1, K), dtype=dt, device="cuda")
    x[0, 0] = 1.0
    out = fp8.fp8_gemv_block(x, torch.from_numpy(q).cuda(), torch.from_numpy(scales).cuda())
    np.testing.assert_array_equal(out.float().cpu().numpy()[0], Q.e4m3_decode(codes))


CFG3 = [(2048, 2048), (10944, 2048), (2048, 10944)]


@pytest.mark.parametrize("M", [1, 8])
@pytest.mark.parametrize("N,K", CFG3)
def test_fp8_block_gemv_config3(torch_gpu, M, N, K):
    from fastllm_py import quantizer
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(3000 + M + N + K)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda().to(torch.bfloat16)
    qt = quantizer.quantize_fp8_block(torch.from_numpy(W).cuda(), 128)
    q_ref, s_ref = Q.quantize_fp8_block(W, 128)
    np.testing.assert_array_equal(qt.data.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(qt.scales.cpu().numpy(), s_ref)
    out = fp8.fp8_gemv_block(x, qt.data, qt.scales)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    ref = Q.matmul_ref(_bf16_to_f32(x), Q.dequantize_fp8_block(q_ref, s_ref, 128))
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL


# N not a multiple of 16, K ending in a 64-wide block; all but the first take
# the halved 8-row kernel (M <= 8 and K >= 512; at M <= 4 only from K = 8192)
@pytest.mark.parametrize("N,K,M", [(200, 320, 5), (200, 704, 6), (2000, 1088, 8), (200, 8256, 3),
                                   (2000, 8192, 1)])
def test_fp8_block_gemv_fp16_bias_ragged(torch_gpu, N, K, M):
    from fastllm_py import quantizer
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(77 + N + K + M)
    W = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda().half()
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda().half()
    qt = quantizer.quantize_fp8_block(torch.from_numpy(W).cuda(), 128)
    out = fp8.fp8_gemv_block(x, qt.data, qt.scales, bias=b)
    q_ref, s_ref = Q.quantize_fp8_block(W, 128)
    ref = Q.matmul_ref(x.float().cpu().numpy(), Q.dequantize_fp8_block(q_ref, s_ref, 128))
    ref = ref + b.float().cpu().numpy()[None]
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL


# prefill-shaped (M > 64): the MFMA GEMM, ragged M and N, K ending in a 64-wide block,
# both activation types, bias
@pytest.mark.parametrize("M,N,K,bf16", [(128, 2048, 2048, True), (200, 1000, 1024, False),
                                        (65, 4096, 512, True), (512, 10944, 2048, True),
                                        (128, 2048, 10944, True), (96, 256, 320, False),
                                        (512, 2048, 2048, True)])
def test_fp8_block_gemm_prefill(torch_gpu, M, N, K, bf16):
    from fastllm_py import quantizer
    from fastllm_py.kernels import fp8

    torch = torch_gpu
    rng = np.random.default_rng(8100 + M + N + K)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    dt = torch.bfloat16 if bf16 else torch.float16
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda().to(dt)
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda().to(dt)
    qt = quantizer.quantize_fp8_block(torch.from_numpy(W).cuda(), 128)
    out = fp8.fp8_gemv_block(x, qt.data, qt.scales, bias=b)
    assert out.shape == (M, N) and out.dtype == dt
    q_ref, s_ref = Q.quantize_fp8_block(W, 128)
    ref = Q.matmul_ref(x.float().cpu().numpy(), Q.dequantize_fp8_block(q_ref, s_ref, 128))
    ref = ref + b.float().cpu().numpy()[None]
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL


def test_fp8_block_gemm_split_k(torch_gpu):
    """Split-K of the prefill GEMM (grids under 256 tiles): within the
    oracle's tolerance, bit-identical on a repeat (partials summed in split
    order), equal in tolerance to the unsplit entry, and one workspace shared
    by calls of different shapes (tile counters left at zero)."""
    from fastllm_py import _native, quantizer

    torch = torch_gpu
    lib = _native.lib()
    rng = np.random.default_rng(8300)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    outs = []
    for M, N, K in ((512, 2048, 4096), (128, 2048, 10944), (200, 1000, 4096), (256, 2048, 8192)):
        need = lib.fastllm_fp8_b128x128_gemm_ws_bytes(M, N, K)
        assert 0 < need <= ws.numel(), (M, N, K, need)
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).cuda().to(torch.bfloat16)
        b = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).cuda().to(torch.bfloat16)
        qt = quantizer.quantize_fp8_block(torch.from_numpy(W).cuda(), 128)
        q_ref, s_ref = Q.quantize_fp8_block(W, 128)
        ref = Q.matmul_ref(x.float().cpu().numpy(), Q.dequantize_fp8_block(q_ref, s_ref, 128))
        ref = ref + b.float().cpu().numpy()[None]
        args = (x.data_ptr(), qt.data.data_ptr(), qt.scales.data_ptr(), b.data_ptr())
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        assert lib.fastllm_fp8_b128x128_gemm_ws(*args, y.data_ptr(), M, N, K, 1, ws.data_ptr(),
                                                ws.numel(), None) == 0
        y0 = torch.empty_like(y)
        assert lib.fastllm_fp8_b128x128_gemv(*args, y0.data_ptr(), M, N, K, 1, None) == 0
        torch.cuda.synchronize()
        assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < TOL
        assert Q.max_abs_rel(y.float().cpu().numpy(), y0.float().cpu().numpy()) < 1e-2
        outs.append((args, M, N, K, y, (x, b, qt)))  # the tensors stay alive for the repeats
    for args, M, N, K, y, _keep in outs:  # repeats after the other shapes on the same workspace
        y2 = torch.empty_like(y)
        assert lib.fastllm_fp8_b128x128_gemm_ws(*args, y2.data_ptr(), M, N, K, 1, ws.data_ptr(),
                                                ws.numel(), None) == 0
        torch.cuda.synchronize()
        assert torch.equal(y, y2), (M, N, K)
    assert int(ws[:1024].count_nonzero()) == 0  # counters back at zero

"""INT4 Marlin-ABI path on the GPU vs the numpy oracle.

Packers are bit-exact; the GEMM is within max-abs-rel 1e-2 of the fp32
dequantize-then-matmul of the very same packed weights (the bar the path is
held to; its fp16 output rounding alone is ~5e-4).
Mirrors tests/test_native_kernels.py:79-154 of the reference.
"""
import ctypes

import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _prep(torch, W, gs):
    """W fp32 (N, K) -> GPU Marlin payload through the product packers, plus the
    oracle's W_hat of the same payload."""
    from fastllm_py.kernels import marlin
    from fastllm_py.moe import quantize_marlin_matrix_device

    N, K = W.shape
    pay = quantize_marlin_matrix_device(torch.from_numpy(W).cuda(), gs)
    q, s, z = Q.quantize_int4_marlin(W, gs)
    s16, zp = Q.marlin_scales_zeros(s, z)
    w_hat = Q.marlin_dequant(q, s16, zp, gs)
    return pay, w_hat, (q, s16, zp)


@pytest.mark.parametrize("K,N", [(128, 64), (1024, 512), (2048, 1408 // 64 * 64), (4096, 256)])
def test_repack_roundtrip_bit_exact(torch_gpu, K, N):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(K + N)
    std = rng.integers(0, 2 ** 32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    tile = marlin.marlin_repack(torch.from_numpy(std).cuda(), K, N)
    assert tile.numel() == std.size
    back = marlin.marlin_unrepack(tile, K, N)
    np.testing.assert_array_equal(back.cpu().numpy(), std)
    # a bijection, not the identity
    assert not np.array_equal(tile.cpu().numpy().reshape(-1), std.reshape(-1))


def test_packers_bit_exact(torch_gpu):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(12)
    W = (rng.standard_normal((192, 512)) * 0.02).astype(np.float32)
    W[3, :128] = 0.5  # constant group
    for gs in (128, 32):
        q, s, z = Q.quantize_int4_marlin(W, gs)
        # numpy-in / numpy-out like the reference host helpers
        np.testing.assert_array_equal(marlin.pack_gptq_qweight(q), Q.pack_gptq(q))
        s16, zp = marlin.build_marlin_scales_zeros(s, z, gs)
        rs16, rzp = Q.marlin_scales_zeros(s, z)
        np.testing.assert_array_equal(s16.view(np.uint16), rs16.view(np.uint16))
        np.testing.assert_array_equal(zp, rzp)
        # device quantizer of moe.quantize_marlin_matrix
        from fastllm_py.moe import _quantize_marlin_device

        qd, sd, zd = _quantize_marlin_device(torch.from_numpy(W).cuda(), gs)
        np.testing.assert_array_equal(qd.cpu().numpy(), q)
        np.testing.assert_array_equal(sd.cpu().numpy().view(np.uint32), s.view(np.uint32))
        np.testing.assert_array_equal(zd.cpu().numpy(), z)


SHAPES = [(1024, 512), (2048, 1408 // 64 * 64), (1408 // 64 * 64, 2048), (4096, 4096), (12288, 4096),
          (192, 64)]


# (K, N, group) with K a multiple of the group (192 x 64 runs at group 32 only)
SHAPE_CASES = [(K, N, gs) for K, N in SHAPES for gs in (128, 32) if K % gs == 0]


@pytest.mark.parametrize("K,N,gs", SHAPE_CASES)
@pytest.mark.parametrize("M", [1, 4, 8, 16])
def test_gemm_parity(torch_gpu, M, K, N, gs):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(1000 * M + K + N + gs)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, gs)
    ws = marlin.make_workspace(N)
    out = marlin.marlin_gemm_int4(torch.from_numpy(a).cuda(), pay["qweight"], pay["scales"],
                                  pay["zeros"], ws)
    assert out.shape == (M, N) and out.dtype == torch.float16
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    err = Q.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err < TOL, err


# Config 2: the four Qwen3-8B decode linears (N x K) at their exact shapes,
# each at every batch of the config (each (shape, M) has its own launch
# configuration).  Seeds 2000 + i per shape i, W drawn before x.
QWEN3_8B = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (24576, 4096),
            "down": (4096, 12288)}
_qwen_cache = {}


def _qwen_payload(torch, name):
    if name not in _qwen_cache:
        N, K = QWEN3_8B[name]
        rng = np.random.default_rng(2000 + list(QWEN3_8B).index(name))
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float16).astype(np.float32)
        pay, w_hat, _ = _prep(torch, W, 128)
        _qwen_cache.clear()  # one shape's fp32 W_hat at a time (gate_up's is 400 MB)
        _qwen_cache[name] = (pay, w_hat, rng)
    return _qwen_cache[name]


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("name", list(QWEN3_8B))  # closest decorator = outer loop
def test_gemm_parity_qwen3_8b(torch_gpu, name, M):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    pay, w_hat, rng = _qwen_payload(torch, name)
    N, K = QWEN3_8B[name]
    a = rng.standard_normal((M, K)).astype(np.float16)
    out = marlin.marlin_gemm_int4(torch.from_numpy(a).cuda(), pay["qweight"], pay["scales"],
                                  pay["zeros"], marlin.make_workspace(N))
    assert out.shape == (M, N)
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    err = Q.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err < TOL, (name, M, err)


def test_gemv_scales_off_16_byte_alignment(torch_gpu):
    """The ABI takes a scale array at any 2-byte alignment
    (marlin.py:250-299 passes whatever the caller's tensor holds): a scale
    pointer 2 bytes past a 16-byte boundary, at the two- and four-tile
    launches (N = 16384), gives the aligned call's results bit for bit."""
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    N, K = 16384, 1024  # two tiles up to M = 8, four above
    rng = np.random.default_rng(77)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    pay, w_hat, _ = _prep(torch, W, 128)
    s = pay["scales"]
    buf = torch.empty(s.numel() + 8, dtype=s.dtype, device=s.device)
    su = buf[1:1 + s.numel()].view(s.shape)
    su.copy_(s)
    assert su.data_ptr() % 16 != 0
    for M in (1, 4, 8, 16):
        a = rng.standard_normal((M, K)).astype(np.float16)
        ad = torch.from_numpy(a).cuda()
        ref_dev = marlin.marlin_gemm_int4(ad, pay["qweight"], s, pay["zeros"], marlin.make_workspace(N))
        out = marlin.marlin_gemm_int4(ad, pay["qweight"], su, pay["zeros"], marlin.make_workspace(N))
        ref = Q.matmul_ref(a.astype(np.float32), w_hat)
        err = Q.max_abs_rel(out.float().cpu().numpy(), ref)
        assert err < TOL, (M, err)
        assert torch.equal(out, ref_dev), M  # the same kernels, fixed reduction order


@pytest.mark.parametrize("M", [17, 33, 64, 100, 130])
def test_gemm_parity_larger_m(torch_gpu, M):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    K, N, gs = 2048, 512, 128
    rng = np.random.default_rng(77 + M)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, gs)
    out = marlin.marlin_gemm_int4(torch.from_numpy(a).cuda(), pay["qweight"], pay["scales"],
                                  pay["zeros"])
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL


# prefill shapes on the MFMA GEMM (M > 64): config 5's dense 8192x2048 at
# M=512, ragged M and N (N % 128 == 64), group 32
@pytest.mark.parametrize("M,K,N,gs", [(512, 2048, 8192, 128), (65, 1024, 576, 128),
                                      (200, 2048, 1408, 128), (129, 512, 192, 32),
                                      (300, 768, 2048, 128), (256, 1024, 1024, 32)])
def test_gemm_mfma_parity(torch_gpu, M, K, N, gs):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(5000 + M + K + N + gs)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, gs)
    out = marlin.marlin_gemm_int4(torch.from_numpy(a).cuda(), pay["qweight"], pay["scales"],
                                  pay["zeros"])
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    err = Q.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err < TOL, err


@pytest.mark.parametrize("M", [1, 16, 256])
def test_stream_entry_bit_identical(torch_gpu, M):
    # reference tests/test_native_kernels.py:132-154
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    K, N, gs = 2048, 1408 // 64 * 64, 128
    rng = np.random.default_rng(7)
    W = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    a = torch.from_numpy((rng.standard_normal((M, K)) * 0.5).astype(np.float16)).cuda()
    pay, _, _ = _prep(torch, W, gs)
    default = marlin.gemm_fast(a, pay["qweight"], pay["scales"], pay["zeros"], N, K)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        streamed = marlin.gemm_fast(a, pay["qweight"], pay["scales"], pay["zeros"], N, K, stream=s)
    s.synchronize()
    assert torch.equal(default, streamed)


def test_rejects_bad_shapes(torch_gpu):
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    a = torch.zeros((1, 96), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        marlin.marlin_gemm_int4(a, torch.zeros(96 * 64 // 8, dtype=torch.uint32, device="cuda"),
                                torch.zeros((1, 64), dtype=torch.float16, device="cuda"),
                                torch.zeros((1, 8), dtype=torch.uint32, device="cuda"))
    lib = __import__("fastllm_py._native", fromlist=["x"]).lib()
    # group 64 is not a Marlin group size: the entry returns false, no launch
    assert not lib.FastllmCudaMarlinHalfInt4Gemm(a.data_ptr(), a.data_ptr(), a.data_ptr(),
                                                 a.data_ptr(), a.data_ptr(), 1, 64, 128, 64, None)


@pytest.mark.parametrize("M", [5, 9, 16])
@pytest.mark.parametrize("gs", [128, 32])
def test_gemv_four_tiles(torch_gpu, M, gs):
    """Wide N above M = 8 takes four n-tiles per workgroup with the
    activations in registers; explicit launch configs of that variant too."""
    from fastllm_py import _native
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    K, N = 2048, 16384
    rng = np.random.default_rng(300 + M + gs)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, gs)
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    ad = torch.from_numpy(a).cuda()
    out = marlin.marlin_gemm_int4(ad, pay["qweight"], pay["scales"], pay["zeros"])
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL
    lib = _native.lib()
    for tiles, waves, nb in ((4, 16, 1), (4, 8, 2), (4, 4, 4)):
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        assert lib.fastllm_int4_gemm_config(ad.data_ptr(), pay["qweight"].data_ptr(),
                                            pay["scales"].data_ptr(), pay["zeros"].data_ptr(),
                                            y.data_ptr(), M, N, K, gs, tiles, waves, nb, None)
        torch.cuda.synchronize()
        assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < TOL, (tiles, waves, nb)


@pytest.mark.parametrize("M,N,K", [(5, 16448, 1152), (13, 16448, 4096), (16, 24576, 384), (8, 16384, 8192)])
def test_gemv_column_split(torch_gpu, M, N, K):
    """Wide outputs (N / 16 >= 1024) at 5..16 rows, group 128: the
    column-split GEMV (one n-tile per wave over all of K). 1028 tiles leave
    the last workgroup with two live waves; 9 and 3 blocks end half way
    through a two-block chunk; M = 8 at K = 8192 stages 8 rows (64 KB)."""
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(400 + M + K)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, 128)
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    ad = torch.from_numpy(a).cuda()
    out = marlin.marlin_gemm_int4(ad, pay["qweight"], pay["scales"], pay["zeros"])
    out2 = marlin.marlin_gemm_int4(ad, pay["qweight"], pay["scales"], pay["zeros"])
    torch.cuda.synchronize()
    assert Q.max_abs_rel(out.float().cpu().numpy(), ref) < TOL
    # no atomics or splits: a repeat is bit-identical
    assert torch.equal(out, out2)


@pytest.mark.parametrize("gs", [128, 32])
def test_gemv_split_k(torch_gpu, gs):
    """Split-K decode GEMV through fastllm_int4_gemm_ws: every forced
    {tiles, waves, blocks per wave, splits} within the oracle's tolerance,
    bit-identical on a repeat (the last split of each strip sums the partials
    in split order), and one workspace shared by calls of different M and
    split (the strip counters sit at one offset and are left at zero)."""
    from fastllm_py import _native

    torch = torch_gpu
    lib = _native.lib()
    K, N = 4096, 2048
    rng = np.random.default_rng(410 + gs)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    pay, w_hat, _ = _prep(torch, W, gs)
    ws_bytes = 1024 * N + 65536  # 16 splits x 16 rows x N fp32 + the counters
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    cfgs = [(4, 16, 1, 2), (4, 8, 1, 4), (2, 4, 2, 4), (1, 4, 1, 8), (4, 4, 1, 8), (1, 2, 1, 16)]

    def run(ad, M, cfg):
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        c = None if cfg is None else (ctypes.c_int * 4)(*cfg)
        rc = lib.fastllm_int4_gemm_ws(ad.data_ptr(), pay["qweight"].data_ptr(),
                                      pay["scales"].data_ptr(), pay["zeros"].data_ptr(),
                                      y.data_ptr(), M, N, K, gs, ws.data_ptr(), ws_bytes, c, None)
        assert rc == 0, (M, cfg, rc)
        return y

    first = {}
    for M in (1, 3, 5, 8, 16):
        a = rng.standard_normal((M, K)).astype(np.float16)
        ad = torch.from_numpy(a).cuda()
        ref = Q.matmul_ref(a.astype(np.float32), w_hat)
        for cfg in cfgs + [None]:
            y = run(ad, M, cfg)
            torch.cuda.synchronize()
            assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < TOL, (M, cfg)
            first[(M, cfg)] = (ad, y)
    # repeats after calls of other shapes on the same workspace: bit-identical
    for (M, cfg), (ad, y) in first.items():
        assert torch.equal(run(ad, M, cfg), y), (M, cfg)
    torch.cuda.synchronize()
    assert int(ws[:65536].count_nonzero()) == 0  # counters back at zero
    # a forced split with too small a workspace is refused, no launch
    y = torch.empty((8, N), dtype=torch.float16, device="cuda")
    ad = first[(8, None)][0]
    assert lib.fastllm_int4_gemm_ws(ad.data_ptr(), pay["qweight"].data_ptr(), pay["scales"].data_ptr(),
                                    pay["zeros"].data_ptr(), y.data_ptr(), 8, N, K, gs,
                                    ws.data_ptr(), 1024, (ctypes.c_int * 4)(4, 8, 1, 4), None) == 2


def test_gemv_split_k_workspace_across_widths(torch_gpu):
    """One workspace shared by split-K calls of different output widths,
    interleaved: a narrow call's partials must not land on a wide call's
    strip counters (they sit in a fixed region whatever N), so every call
    stays within the oracle's tolerance and bit-identical to its first run."""
    from fastllm_py import _native

    torch = torch_gpu
    lib = _native.lib()
    K, M = 2048, 16
    rng = np.random.default_rng(433)
    ws_bytes = 65536 + 2 * M * 4096 * 4
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device="cuda")
    cases = []
    for N in (4096, 256, 1024):
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        pay, w_hat, _ = _prep(torch, W, 128)
        a = rng.standard_normal((M, K)).astype(np.float16)
        cases.append((N, pay, torch.from_numpy(a).cuda(), Q.matmul_ref(a.astype(np.float32), w_hat)))

    def run(N, pay, ad):
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        rc = lib.fastllm_int4_gemm_ws(ad.data_ptr(), pay["qweight"].data_ptr(), pay["scales"].data_ptr(),
                                      pay["zeros"].data_ptr(), y.data_ptr(), M, N, K, 128, ws.data_ptr(),
                                      ws_bytes, (ctypes.c_int * 4)(1, 16, 1, 2), None)
        assert rc == 0, N
        return y

    first = {}
    for _ in range(3):
        for N, pay, ad, ref in cases:
            y = run(N, pay, ad)
            torch.cuda.synchronize()
            assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < TOL, N
            if N in first:
                assert torch.equal(y, first[N]), N
            else:
                first[N] = y
    assert int(ws[:65536].count_nonzero()) == 0


@pytest.mark.parametrize("name,M", [("down", 5), ("down", 8), ("down", 16), ("gate_up", 16)])
def test_gemm_split_default_workspace(torch_gpu, name, M):
    """The Python layer's default above M = 4: gemm_fast with the call site's
    make_workspace runs the split kernels where they pay (Qwen3-8B down, and
    gate_up above M = 8), within the oracle's tolerance like the unsplit
    entry."""
    from fastllm_py import _native
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    pay, w_hat, rng = _qwen_payload(torch, name)
    N, K = QWEN3_8B[name]
    assert _native.lib().fastllm_int4_gemm_ws_bytes(M, N, K, 128) > 0
    a = rng.standard_normal((M, K)).astype(np.float16)
    ad = torch.from_numpy(a).cuda()
    ws = marlin.make_workspace(N)
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    for _ in range(2):
        y = marlin.gemm_fast(ad, pay["qweight"], pay["scales"], pay["zeros"], N, K, workspace=ws)
        torch.cuda.synchronize()
        assert Q.max_abs_rel(y.float().cpu().numpy(), ref) < TOL, (name, M)
    unsplit = torch.empty((M, N), dtype=torch.float16, device="cuda")
    assert _native.lib().FastllmCudaMarlinHalfInt4Gemm(
        ad.data_ptr(), pay["qweight"].data_ptr(), pay["scales"].data_ptr(), pay["zeros"].data_ptr(),
        unsplit.data_ptr(), M, N, K, 128, None)
    torch.cuda.synchronize()
    assert Q.max_abs_rel(unsplit.float().cpu().numpy(), ref) < TOL


@pytest.mark.parametrize("M,I,K,gs", [(1, 12288, 4096, 128), (4, 1408, 2048, 128), (8, 3072, 1024, 32),
                                      (16, 512, 4096, 128), (3, 64, 256, 128), (8, 12288, 4096, 128),
                                      (6, 1408, 8192, 128), (12, 1024, 4096, 128)])
def test_gemm_swiglu(torch_gpu, M, I, K, gs):
    """Gate/up GEMV with the SwiGLU epilogue equals the plain GEMV followed by
    swiglu of its fp16 outputs (up to the device exp), and the fp32 oracle."""
    from fastllm_py.kernels import marlin

    torch = torch_gpu
    rng = np.random.default_rng(400 + M + I + K + gs)
    W = (rng.standard_normal((2 * I, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((M, K)).astype(np.float16)
    pay, w_hat, _ = _prep(torch, W, gs)
    ad = torch.from_numpy(a).cuda()
    h = marlin.gemm_swiglu(ad, pay["qweight"], pay["scales"], pay["zeros"], 2 * I, K)
    assert h.shape == (M, I) and h.dtype == torch.float16
    gu = marlin.marlin_gemm_int4(ad, pay["qweight"], pay["scales"], pay["zeros"]).float().cpu().numpy()
    g, u = gu[:, :I], gu[:, I:]
    want = (g / (1.0 + np.exp(-g)) * u).astype(np.float16).astype(np.float32)
    got = h.float().cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-6)
    ref = Q.matmul_ref(a.astype(np.float32), w_hat)
    rg, ru = ref[:, :I], ref[:, I:]
    assert Q.max_abs_rel(got, rg / (1.0 + np.exp(-rg)) * ru) < TOL


def test_gemm_swiglu_rejects(torch_gpu):
    from fastllm_py import _native

    torch = torch_gpu
    lib = _native.lib()
    p = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda").data_ptr()
    assert lib.fastllm_int4_gemm_swiglu(p, p, p, p, p, 17, 256, 256, 128, None) == 1  # M > 16
    assert lib.fastllm_int4_gemm_swiglu(p, p, p, p, p, 1, 192, 256, 128, None) == 1   # I % 64
    assert lib.fastllm_int4_gemm_swiglu(p, p, p, p, p, 1, 256, 192, 128, None) == 1   # K % 128
    assert lib.fastllm_int4_gemm_swiglu(p, p, p, p, p, 1, 256, 256, 64, None) == 1    # group

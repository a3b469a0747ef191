"""add_rmsnorm (residual add + RMSNorm) and the captured decode layer on the
GPU, against the oracle."""
import numpy as np
import pytest

from oracle import norm as ON
from oracle import quant as Q

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,dim,xt,dt,wt", [
    (1, 4096, np.float32, np.float16, np.float16),   # decode: fp32 residual, fp16 branch output
    (5, 1024, np.float32, np.float32, np.float32),
    (17, 128, np.float16, np.float16, np.float16),   # dim < 256: 128 threads
    (3, 2048, np.float16, np.float32, np.float32),
    (2, 1000, np.float32, np.float16, np.float32),   # dim not a multiple of the thread count
    (2, 9000, np.float32, np.float16, np.float16),   # past the register path (dim > 32 x 256)
])
def test_add_rmsnorm_matches_oracle(torch_gpu, rows, dim, xt, dt, wt):
    """xnew bit-exact; h bit-exact with the oracle's fp32 sequence (same sum
    order, 1/sqrt in double), and within the reference's own test tolerance of the
    float64 formula (tests/test_fused_ops.py:10-27)."""
    from fastllm_py.kernels import ops

    torch = torch_gpu
    rng = np.random.default_rng(rows * 131 + dim)
    x = rng.standard_normal((rows, dim)).astype(xt)
    d = rng.standard_normal((rows, dim)).astype(dt)
    w = rng.standard_normal(dim).astype(wt)
    eps = 1e-6
    xnew, h = ops.add_rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(d).cuda(),
                              torch.from_numpy(w).cuda(), eps)
    assert xnew.dtype == torch.float32 and h.dtype == torch.float16
    rx, rh = ON.add_rmsnorm(x, d, w, eps)
    np.testing.assert_array_equal(xnew.cpu().numpy(), rx)
    np.testing.assert_array_equal(h.cpu().numpy().view(np.uint16), rh.view(np.uint16))
    v = x.astype(np.float64) + d.astype(np.float64)
    ref = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps) * w.astype(np.float64)
    np.testing.assert_allclose(h.float().cpu().numpy(), ref, rtol=1e-3, atol=2e-3)


def test_add_rmsnorm_rejects(torch_gpu):
    from fastllm_py import _native as nat

    lib = nat.lib()
    assert lib.fastllm_add_rmsnorm(None, 1, None, 1, None, 1, None, None, 1, 8, 1e-6, None) == 1
    torch = torch_gpu
    b = torch.zeros(64, device="cuda")
    assert lib.fastllm_add_rmsnorm(b.data_ptr(), 1, b.data_ptr(), 1, b.data_ptr(), 1, b.data_ptr(),
                                   b.data_ptr(), 0, 8, 1e-6, None) == 1


@pytest.mark.parametrize("N,K,gs,swiglu", [(6144, 4096, 128, False), (4096, 12288, 128, False),
                                           (24576, 4096, 128, True), (1536, 1024, 32, False),
                                           (512, 256, 128, True)])
def test_gemm_add_rmsnorm(torch_gpu, N, K, gs, swiglu):
    """add_rmsnorm in the GEMV prologue: xnew bit-exact, the output within
    the GEMV tolerance of the oracle (add_rmsnorm oracle, then the fp32
    dequantize-then-matmul, then swiglu) and of the two-launch path."""
    from fastllm_py.kernels import marlin, ops
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    rng = np.random.default_rng(500 + N + K + gs)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    pay = quantize_marlin_matrix_device(torch.from_numpy(W).cuda(), gs)
    q, s_, z = Q.quantize_int4_marlin(W, gs)
    s16, zp = Q.marlin_scales_zeros(s_, z)
    w_hat = Q.marlin_dequant(q, s16, zp, gs)
    x = rng.standard_normal((1, K)).astype(np.float32)
    d = (rng.standard_normal((1, K)) * 0.5).astype(np.float16)
    ln = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float16)
    xd, dd, lnd = (torch.from_numpy(a).cuda() for a in (x, d, ln))
    for _ in range(2):
        xnew, c = marlin.gemm_add_rmsnorm(xd, dd, lnd, 1e-6, pay["qweight"], pay["scales"],
                                          pay["zeros"], N, K, swiglu=swiglu)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(xnew.cpu().numpy(), x + d.astype(np.float32))
        _, h = ON.add_rmsnorm(x, d, ln, 1e-6)
        ref = Q.matmul_ref(h.astype(np.float32), w_hat)
        got = c.float().cpu().numpy()
        if swiglu:
            I = N // 2
            ref = ref[:, :I] / (1.0 + np.exp(-ref[:, :I])) * ref[:, I:]
            two = marlin.gemm_swiglu(ops.add_rmsnorm(xd, dd, lnd, 1e-6)[1], pay["qweight"],
                                     pay["scales"], pay["zeros"], N, K)
        else:
            two = marlin.gemm_fast(ops.add_rmsnorm(xd, dd, lnd, 1e-6)[1], pay["qweight"],
                                   pay["scales"], pay["zeros"], N, K)
        assert Q.max_abs_rel(got, ref) < 1e-2
        assert Q.max_abs_rel(got, two.float().cpu().numpy()) < 5e-3


def test_gemm_add_rmsnorm_rejects(torch_gpu):
    from fastllm_py import _native as nat

    lib = nat.lib()
    torch = torch_gpu
    b = torch.zeros(1 << 16, device="cuda")
    p = b.data_ptr()
    assert lib.fastllm_int4_gemm_add_rmsnorm(None, p, p, 1e-6, p, p, p, p, p, 64, 128, 128, 0, None) == 1
    assert lib.fastllm_int4_gemm_add_rmsnorm(p, p, p, 1e-6, p, p, p, p, p, 64, 192, 128, 0, None) == 1  # K % 128
    assert lib.fastllm_int4_gemm_add_rmsnorm(p, p, p, 1e-6, p, p, p, p, p, 64, 128, 128, 1, None) == 1  # swiglu N
    assert lib.fastllm_int4_gemm_add_rmsnorm(p, p, p, 1e-6, p, p, p, p, p, 64, 128, 64, 0, None) == 1  # group


def test_gemm_add_rmsnorm_rejects_aliasing(torch_gpu):
    """xnew overlapping x or delta is refused: workgroup 0 stores xnew while
    other workgroups still read x and delta."""
    from fastllm_py import _native as nat
    from fastllm_py.kernels import marlin
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    N, K = 256, 1024
    W = torch.randn((N, K), generator=torch.Generator().manual_seed(3)).mul_(0.02).cuda()
    pay = quantize_marlin_matrix_device(W, 128)
    x = torch.randn((1, K), device="cuda")
    d = torch.randn((1, K), device="cuda").half()
    ln = torch.ones(K, device="cuda").half()
    with pytest.raises(ValueError):
        marlin.gemm_add_rmsnorm(x, d, ln, 1e-6, pay["qweight"], pay["scales"], pay["zeros"], N, K,
                                xnew=x)
    c = torch.empty((1, N), device="cuda").half()
    lib = nat.lib()
    args = [pay["qweight"].data_ptr(), pay["scales"].data_ptr(), pay["zeros"].data_ptr(),
            c.data_ptr(), N, K, 128, 0, None]
    assert lib.fastllm_int4_gemm_add_rmsnorm(x.data_ptr(), d.data_ptr(), ln.data_ptr(), 1e-6,
                                             x.data_ptr(), *args) == 1
    dd = torch.empty(4 * K, device="cuda").half()  # xnew (fp32, 4K bytes) covering delta
    assert lib.fastllm_int4_gemm_add_rmsnorm(x.data_ptr(), dd[K:].data_ptr(), ln.data_ptr(), 1e-6,
                                             dd.data_ptr(), *args) == 1
    xn = torch.empty((1, K), device="cuda")
    assert lib.fastllm_int4_gemm_add_rmsnorm(x.data_ptr(), d.data_ptr(), ln.data_ptr(), 1e-6,
                                             xn.data_ptr(), *args) == 0
    torch.cuda.synchronize()


def _device_payload(torch, N, K, seed):
    from fastllm_py.moe import quantize_marlin_matrix_device

    g = torch.Generator().manual_seed(seed)
    W = (torch.randn((N, K), generator=g) * 0.02).cuda()
    return quantize_marlin_matrix_device(W, 128)


@pytest.mark.parametrize("N,K,swiglu", [(16384, 13312, False), (256, 16384, True),
                                        (256, 12288, True)])
def test_gemm_add_rmsnorm_large_k(torch_gpu, N, K, swiglu):
    """Shapes past the two-tile LDS budget: the plain GEMV drops to one tile
    per workgroup (N >= 16384, K > 12288), the SwiGLU pair falls back to the
    standalone norm + unfused kernels (K > 12288).  Checked against the
    two-launch path (oracle-tested at the other shapes)."""
    from fastllm_py.kernels import marlin, ops

    torch = torch_gpu
    pay = _device_payload(torch, N, K, 41 + K)
    g = torch.Generator().manual_seed(K)
    x = torch.randn((1, K), generator=g).cuda()
    d = (torch.randn((1, K), generator=g) * 0.5).half().cuda()
    ln = (1.0 + 0.1 * torch.randn(K, generator=g)).half().cuda()
    xnew, c = marlin.gemm_add_rmsnorm(x, d, ln, 1e-6, pay["qweight"], pay["scales"], pay["zeros"],
                                      N, K, swiglu=swiglu)
    h = ops.add_rmsnorm(x, d, ln, 1e-6)[1]
    if swiglu:
        two = marlin.gemm_swiglu(h, pay["qweight"], pay["scales"], pay["zeros"], N, K)
    else:
        two = marlin.gemm_fast(h, pay["qweight"], pay["scales"], pay["zeros"], N, K)
    torch.cuda.synchronize()
    assert torch.equal(xnew, x + d.float())
    assert Q.max_abs_rel(c.float().cpu().numpy(), two.float().cpu().numpy()) < 5e-3


@pytest.mark.parametrize("M,K", [(1, 12288), (4, 12288), (8, 12288), (1, 16384), (16, 16384)])
def test_gemm_swiglu_large_k(torch_gpu, M, K):
    """SwiGLU GEMV past four blocks per wave: fused up to K = 12288 at M <= 4,
    the GEMV + standalone swiglu beyond; both against the oracle."""
    from fastllm_py.kernels import marlin
    from fastllm_py.moe import quantize_marlin_matrix_device

    torch = torch_gpu
    N = 256
    rng = np.random.default_rng(900 + M + K)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    pay = quantize_marlin_matrix_device(torch.from_numpy(W).cuda(), 128)
    q, s_, z = Q.quantize_int4_marlin(W, 128)
    s16, zp = Q.marlin_scales_zeros(s_, z)
    w_hat = Q.marlin_dequant(q, s16, zp, 128)
    a = rng.standard_normal((M, K)).astype(np.float16)
    h = marlin.gemm_swiglu(torch.from_numpy(a).cuda(), pay["qweight"], pay["scales"], pay["zeros"],
                           N, K)
    gu = Q.matmul_ref(a.astype(np.float32), w_hat)
    g, u = gu[:, :N // 2], gu[:, N // 2:]
    ref = g / (1.0 + np.exp(-g)) * u
    assert h.shape == (M, N // 2)
    assert Q.max_abs_rel(h.float().cpu().numpy(), ref) < 1e-2


def test_swiglu_op(torch_gpu):
    """ops.swiglu on strided halves of a gate/up output vs numpy's fp32
    formula (reference ops.py:157-163), then fp16."""
    from fastllm_py.kernels import ops

    torch = torch_gpu
    rng = np.random.default_rng(5)
    gu = (rng.standard_normal((3, 2 * 1000)) * 4).astype(np.float16)
    d = torch.from_numpy(gu).cuda()
    out = ops.swiglu(d[:, :1000], d[:, 1000:])
    g, u = gu[:, :1000].astype(np.float32), gu[:, 1000:].astype(np.float32)
    ref = ((g / (1.0 + np.exp(-g))) * u).astype(np.float16).astype(np.float32)
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, rtol=2e-3, atol=1e-4)
    with pytest.raises(ValueError):
        ops.swiglu(d[:, :1000], d[:, 1000:], out=torch.empty(5, device="cuda").half())


def _layer(torch, rng, hidden, q_dim, n_qkv, inter):
    from fastllm_py.moe import quantize_marlin_matrix_device

    def mat(n, k):
        W = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        q, s, z = Q.quantize_int4_marlin(W, 128)
        s16, zp = Q.marlin_scales_zeros(s, z)
        return quantize_marlin_matrix_device(torch.from_numpy(W).cuda(), 128), Q.marlin_dequant(q, s16, zp, 128)

    w, hat = {}, {}
    for name, (n, k) in (("qkv", (n_qkv, hidden)), ("o", (hidden, q_dim)),
                         ("gate_up", (2 * inter, hidden)), ("down", (hidden, inter))):
        w[name], hat[name] = mat(n, k)
    for name in ("ln1", "ln2"):
        ln = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)
        w[name], hat[name] = torch.from_numpy(ln).cuda(), ln
    return w, hat


def _oracle_layer(hat, x, pending, q_dim, inter, eps):
    x1, h1 = ON.add_rmsnorm(x, pending, hat["ln1"], eps)
    qkv = Q.matmul_ref(h1.astype(np.float32), hat["qkv"]).astype(np.float16)
    o = Q.matmul_ref(qkv[:, :q_dim].astype(np.float32), hat["o"]).astype(np.float16)
    x2, h2 = ON.add_rmsnorm(x1, o, hat["ln2"], eps)
    gu = Q.matmul_ref(h2.astype(np.float32), hat["gate_up"])
    g, u = gu[:, :inter], gu[:, inter:]
    hh = (g / (1.0 + np.exp(-g)) * u).astype(np.float16)
    return x2, Q.matmul_ref(hh.astype(np.float32), hat["down"])


@pytest.mark.parametrize("M,fuse", [(1, True), (1, False), (4, False)])
def test_decode_layer_graph_replays(torch_gpu, M, fuse):
    """The captured layer equals the eager chain bit for bit on every replay
    (fresh inputs each time, eager work between replays) and the oracle chain
    within tolerance."""
    from fastllm_py.decode_graph import DecodeLayerGraph

    torch = torch_gpu
    rng = np.random.default_rng(77 + M)
    hidden, q_dim, n_qkv, inter = 1024, 1024, 1536, 2048
    w, hat = _layer(torch, rng, hidden, q_dim, n_qkv, inter)
    L = DecodeLayerGraph(w, M, hidden, q_dim, inter, fuse_norm=fuse).capture()
    for r in range(3):
        x = rng.standard_normal((M, hidden)).astype(np.float32)
        pend = (rng.standard_normal((M, hidden)) * 0.5).astype(np.float16)
        L.x.copy_(torch.from_numpy(x))
        L.pending.copy_(torch.from_numpy(pend))
        L.replay()
        torch.cuda.synchronize()
        gx, gp = L.x_out.cpu().numpy().copy(), L.pending_out.float().cpu().numpy().copy()
        L.step()  # eager, same buffers and inputs
        torch.cuda.synchronize()
        np.testing.assert_array_equal(gx, L.x_out.cpu().numpy(), err_msg=f"replay {r}")
        np.testing.assert_array_equal(gp, L.pending_out.float().cpu().numpy(), err_msg=f"replay {r}")
        # the residual stream is exact: x + pending, then + the o projection
        x1 = L.xnew1.cpu().numpy()
        np.testing.assert_array_equal(x1, x + pend.astype(np.float32))
        np.testing.assert_array_equal(gx, x1 + L.o.float().cpu().numpy())
        ox, op = _oracle_layer(hat, x, pend, q_dim, inter, L.eps)
        # the chain and the oracle round the same fp16 intermediates, only
        # their fp32 summation orders differ (measured: at most 2.6e-4 on x,
        # 7.1e-4 on the MLP output over 20 replays at each of these shapes)
        assert Q.max_abs_rel(gx, ox) < 5e-3, r
        assert Q.max_abs_rel(gp, op) < 5e-3, r

"""GEMV on quantize_int4_group's format vs the numpy oracle.

The weight is quantized by the product's device quantizer (bit-exact with the
oracle's restatement of fastllm_py/quantizer.py:97-117, checked here again on
the config-1 input) and the GEMV must be within max-abs-rel 1e-2 of the
oracle's ``dequantize_int4_group`` (quantizer.py:120-129) followed by an fp32
matmul, the reference's CPU path for this format.
"""
import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _case(seed, N, K, M, gs, x_dtype=np.float16):
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)  # W drawn before x
    x = rng.standard_normal((M, K)).astype(x_dtype)
    return W, x


def _check(torch, W, x, gs, out_dtype=None, out=None):
    from fastllm_py import quantizer
    from fastllm_py.kernels import int4_group

    qt = quantizer.quantize_int4_group(torch.from_numpy(W).cuda(), gs)
    p, s, z = Q.quantize_int4_group(W, gs)
    np.testing.assert_array_equal(qt.data.cpu().numpy(), p)
    np.testing.assert_array_equal(qt.scales.cpu().numpy().view(np.uint32), s.view(np.uint32))
    np.testing.assert_array_equal(qt.zeros.cpu().numpy().view(np.uint32), z.view(np.uint32))
    y = int4_group.gemv(torch.from_numpy(x).cuda(), qt, out=out, out_dtype=out_dtype)
    ref = Q.matmul_ref(x.astype(np.float32), Q.dequantize_int4_group(p, s, z, gs))
    err = Q.max_abs_rel(y.float().cpu().numpy().reshape(ref.shape), ref)
    return y, err


@pytest.mark.parametrize("M", [1, 4, 16])
def test_config1_gemv(torch_gpu, M):
    """Config 1: W 3072x1024 ~ N(0, 0.02), group 128, x (M, 1024) fp16, seed 0."""
    W, x = _case(0, 3072, 1024, M, 128)
    y, err = _check(torch_gpu, W, x, 128)
    assert y.shape == (M, 3072) and y.dtype == torch_gpu.float32
    assert err < TOL, err


GROUP_CASES = [(N, K, gs) for N, K in [(1000, 512), (48, 2048), (4096, 4096), (17, 128)]
               for gs in (32, 64, 128, 256, 512) if K % gs == 0]


@pytest.mark.parametrize("N,K,gs", GROUP_CASES)
def test_group_sizes_and_ragged_shapes(torch_gpu, N, K, gs):
    W, x = _case(100 + gs + N + K, N, K, 3, gs)
    _, err = _check(torch_gpu, W, x, gs)
    assert err < TOL, (gs, N, K, err)


def test_fp32_activations_fp16_output_and_out_buffer(torch_gpu):
    torch = torch_gpu
    W, x = _case(7, 768, 1024, 2, 128, x_dtype=np.float32)
    y, err = _check(torch, W, x, 128, out_dtype=torch.float16)
    assert y.dtype == torch.float16 and err < TOL, err
    out = torch.empty((2, 768), dtype=torch.float32, device="cuda")
    y2, err2 = _check(torch, W, x, 128, out=out)
    assert y2 is out and err2 < TOL


def test_constant_groups_and_large_m(torch_gpu):
    """Constant groups (scale 1.0 by the reference's rule, q = 0) and M > 16
    (M is taken in chunks)."""
    W, x = _case(9, 256, 1024, 40, 128)
    W[5, :128] = 0.25
    W[7, 256:384] = -0.1
    _, err = _check(torch_gpu, W, x, 128)
    assert err < TOL, err


def test_numpy_quantized_tensor_and_1d_input(torch_gpu):
    """A QuantizedTensor holding host arrays (the reference's numpy output)
    and a 1-D activation."""
    from fastllm_py import quantizer
    from fastllm_py.kernels import int4_group

    torch = torch_gpu
    W, x = _case(11, 512, 1024, 1, 128)
    p, s, z = Q.quantize_int4_group(W, 128)
    qt = quantizer.QuantizedTensor("int4_group", p, s, (512, 1024), 128, zeros=z)
    y = int4_group.gemv(torch.from_numpy(x[0]).cuda(), qt)
    assert y.shape == (512,)
    ref = Q.matmul_ref(x.astype(np.float32), Q.dequantize_int4_group(p, s, z, 128))[0]
    assert Q.max_abs_rel(y.cpu().numpy(), ref) < TOL


def test_rejects_bad_arguments(torch_gpu):
    from fastllm_py import quantizer
    from fastllm_py.kernels import int4_group

    torch = torch_gpu
    W, x = _case(13, 64, 256, 1, 128)
    qt = quantizer.quantize_int4_group(torch.from_numpy(W).cuda(), 128)
    with pytest.raises(ValueError):
        int4_group.gemv(torch.from_numpy(x).cuda(), qt, out=torch.empty(63, device="cuda"))
    with pytest.raises(ValueError):
        int4_group.gemv(torch.from_numpy(x).cuda(), qt,
                        out=torch.empty(64, dtype=torch.float64, device="cuda"))
    with pytest.raises(ValueError):
        int4_group.gemv(torch.zeros((1, 128), device="cuda"), qt)
    # a group the kernel does not take (K % 128 == 0 but group 16)
    qt16 = quantizer.quantize_int4_group(torch.from_numpy(W).cuda(), 16)
    with pytest.raises(RuntimeError):
        int4_group.gemv(torch.from_numpy(x).cuda(), qt16)

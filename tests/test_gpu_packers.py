"""GPU packers/unpackers (fastllm_py.quantizer and friends) bit-exact vs the
numpy oracle, on the reference's own test shapes and edge cases."""
import numpy as np
import pytest

from oracle import quant as Q

pytestmark = pytest.mark.gpu


def test_e4m3_codec_sweep(torch_gpu):
    from fastllm_py import quantizer

    torch = torch_gpu
    b = np.arange(0, int(np.float32(500.0).view(np.uint32)), 97, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([b.view(np.float32), -b.view(np.float32),
                        np.array([0.0, -0.0, 448.0, 1e9, -1e9], np.float32)])
    got = quantizer._fp8_e4m3_encode(x)
    np.testing.assert_array_equal(got, Q.e4m3_encode(x))
    codes = np.arange(256, dtype=np.uint8)
    np.testing.assert_array_equal(quantizer._fp8_e4m3_decode(codes), Q.e4m3_decode(codes))
    # torch tensors in -> device tensors out
    t = quantizer._fp8_e4m3_encode(torch.from_numpy(x).cuda())
    assert t.is_cuda and t.dtype == torch.uint8


@pytest.mark.parametrize("shape", [(256, 384), (100, 200), (128, 128), (1, 1000), (300, 64)])
def test_quantize_fp8_block_bit_exact(torch_gpu, shape):
    from fastllm_py import quantizer

    rng = np.random.default_rng(sum(shape))
    w = rng.standard_normal(shape).astype(np.float32)
    qt = quantizer.quantize_fp8_block(w, 128)
    q, s = Q.quantize_fp8_block(w, 128)
    np.testing.assert_array_equal(qt.data, q)
    np.testing.assert_array_equal(qt.scales, s)
    np.testing.assert_array_equal(quantizer.dequantize_fp8_block(qt), Q.dequantize_fp8_block(q, s))


def test_quantize_fp8_block_zero_block(torch_gpu):
    from fastllm_py import quantizer

    w = np.zeros((130, 130), np.float32)
    w[129, 129] = 3.0
    qt = quantizer.quantize_fp8_block(w, 128)
    assert qt.scales[0, 0] == 1.0 and qt.scales[1, 1] == np.float32(3.0 / 448.0)
    assert qt.data[129, 129] == 0x7E


@pytest.mark.parametrize("gs", [128, 32])
def test_quantize_int4_group_bit_exact(torch_gpu, gs):
    from fastllm_py import quantizer

    rng = np.random.default_rng(3)
    w = rng.standard_normal((64, 256)).astype(np.float32)
    w[2, :gs] = 1.5
    qt = quantizer.quantize_int4_group(w, gs)
    p, s, z = Q.quantize_int4_group(w, gs)
    np.testing.assert_array_equal(qt.data, p)
    np.testing.assert_array_equal(qt.scales, s)
    np.testing.assert_array_equal(qt.zeros, z)
    np.testing.assert_array_equal(quantizer.dequantize_int4_group(qt), Q.dequantize_int4_group(p, s, z, gs))


def test_quantize_int4_group_config1(torch_gpu):
    """W 3072x1024 ~ N(0, 0.02), seed 0, group 128."""
    from fastllm_py import quantizer

    rng = np.random.default_rng(0)
    W = (rng.standard_normal((3072, 1024)) * 0.02).astype(np.float32)
    qt = quantizer.quantize_int4_group(W, 128)
    p, s, z = Q.quantize_int4_group(W, 128)
    np.testing.assert_array_equal(qt.data, p)
    np.testing.assert_array_equal(qt.scales.view(np.uint32), s.view(np.uint32))
    np.testing.assert_array_equal(qt.zeros.view(np.uint32), z.view(np.uint32))

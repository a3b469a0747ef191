"""ctypes binding of native/libfastllm_kernels.so (the gfx950 HIP library).

The library is the only compute path: when it is missing, or no ROCm device
is visible, every kernel wrapper raises.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.abspath(os.path.join(_HERE, "..", "native", "libfastllm_kernels.so"))

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_B = ctypes.c_bool
_SZ = ctypes.c_size_t

# name -> (restype, argtypes).  Mirrors include/fastllm_kernels.h.
SIGNATURES: dict[str, tuple] = {
    # INT4 Marlin ABI
    "FastllmCudaGptqMarlinRepack": (_B, [_P, _P, _I, _I]),
    "FastllmCudaGptqMarlinRepackStream": (_B, [_P, _P, _I, _I, _P]),
    "FastllmCudaMarlinHalfInt4Gemm": (_B, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "FastllmCudaMarlinHalfInt4GemmStream": (_B, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P]),
    "fastllm_int4_tile_unrepack": (_B, [_P, _P, _I, _I, _P]),
    "fastllm_int4_gemm_config": (_B, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "fastllm_int4_gemm_ws_bytes": (_SZ, [_I, _I, _I, _I]),
    "fastllm_int4_gemm_ws": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P, _P]),
    "fastllm_int4_gemm_swiglu": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fastllm_add_rmsnorm": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _I, _I, _F, _P]),
    "fastllm_swiglu": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fastllm_marlin_to_moe_tile": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_int4_gemm_add_rmsnorm": (_I, [_P, _P, _P, _F, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    # packers / unpackers
    "fastllm_pack_gptq_qweight": (_I, [_P, _P, _I, _I, _P]),
    "fastllm_build_marlin_scales_zeros": (_I, [_P, _P, _P, _P, _I, _I, _P]),
    "fastllm_quantize_int4_group": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_dequantize_int4_group": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_quantize_int4_marlin": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_quantize_int4_rowmajor": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fastllm_dequantize_int4_rowmajor": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fastllm_fp8_e4m3_encode": (_I, [_P, _P, ctypes.c_long, _P]),
    "fastllm_fp8_e4m3_decode": (_I, [_P, _P, ctypes.c_long, _P]),
    "fastllm_quantize_fp8_block": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "fastllm_dequantize_fp8_block": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    # FP8 GEMV
    "fastllm_fp8_block128_quantize": (_I, [_P, _P, _I, _I, _I]),
    "fastllm_fp8_block128_quantize_stream": (_I, [_P, _P, _I, _I, _I, _P]),
    "fastllm_fp8_block128_packed_row_bytes": (_I, [_I]),
    "fastllm_fp8_block128_gemv_fp16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I]),
    "fastllm_fp8_block128_gemv_stream": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fastllm_fp8_b128x128_gemv": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P]),
    "fastllm_fp8_b128x128_gemm_ws_bytes": (_SZ, [_I, _I, _I]),
    "fastllm_fp8_b128x128_gemm_ws": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _SZ, _P]),
    # row-major INT4 / router / fused MoE
    "fastllm_int4_rowmajor_gemv": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fastllm_int4_group_gemv": (_I, [_P, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "fastllm_gate_matvec": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_route_topk": (_I, [_P, _I, _I, _I, _I, _I, _F, _P, _I, _I, _P, _P, _P, _P, _P,
                                _P, _P, _P, _P, _P, _P]),
    "fastllm_moe_build_lists": (_I, [_P, _P, _P, _I, _I, _I] + [_P] * 6),
    "fastllm_moe_int4_tile_repack": (_I, [_P, _P, _P, _P, _P, ctypes.c_long, _I, _I, _P]),
    "fastllm_moe_int4_tile_unpack": (_I, [_P, _P, _P, _P, _P, ctypes.c_long, _I, _I, _P]),
    "fastllm_moe_int4_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "fastllm_moe_int4_fused": (_I, [_P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                               [_P] * 6 + [_I, _I, _P, _SZ, _P, _P]),
    "fastllm_moe_int4_routed": (_I, [_P, _I, _I, _I, _F, _P, _I, _I, _P] + [_P] * 9 +
                                [_P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                                [_P, _SZ, _P, _P]),
    "fastllm_moe_workspace_bytes_ex": (_SZ, [_I, _I, _I, _I, _I, _I]),
    "fastllm_moe_fused_ex": (_I, [_I, _I, _P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                             [_P] * 6 + [_I, _I, _P, _SZ, _P, _P]),
    "fastllm_moe_routed_ex": (_I, [_I, _I, _P, _I, _I, _I, _F, _P, _I, _I, _P] + [_P] * 9 +
                              [_P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                              [_P, _SZ, _P, _P]),
    "fastllm_moe_int4_routed_noalloc": (_I, [_P, _I, _I, _I, _F, _P, _I, _I, _P] + [_P] * 9 +
                                        [_P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                                        [_P, _P]),
    # measurement
    "fastllm_hbm_read_probe": (_I, [_P, _SZ, _P, _I, _P]),
    "fastllm_quantize_mxfp4": (_I, [_P, _P, _P, ctypes.c_long, _I, _P]),
    "fastllm_dequantize_mxfp4": (_I, [_P, _P, _P, ctypes.c_long, _I, _P]),
    "fastllm_moe_fp8_tile_repack": (_I, [_P, _P, ctypes.c_long, _I, _P]),
    "fastllm_moe_mxfp4_tile_repack": (_I, [_P, _P, _P, _P, ctypes.c_long, _I, _P]),
    "fastllm_mxfp4_gemv": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "fastllm_moe_lowp_fused": (_I, [_I, _P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                               [_P] * 6 + [_I, _I, _P, _SZ, _P, _P]),
    "fastllm_moe_lowp_routed": (_I, [_I, _P, _I, _I, _I, _F, _P, _I, _I, _P] + [_P] * 9 +
                                [_P, _I, _I, _I, _I, _I] + [_P] * 6 + [_I] + [_P] * 6 +
                                [_P, _SZ, _P, _P]),
}


def check_rc(rc, name: str):
    """Raise on a non-zero int return code / False bool return (reference
    wrappers raise RuntimeError on failure, marlin.py:187-188, fp8.py:93-94)."""
    if rc is False or (not isinstance(rc, bool) and rc != 0):
        raise RuntimeError(f"{name} failed (rc={rc})")

_lib = None


def load():
    """Load and bind the library (raises FileNotFoundError when not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"libfastllm_kernels.so not found at {LIB_PATH}; run "
            "python fastllm-py_amd/build_native.py")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        if hasattr(lib, name):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
    _lib = lib
    return lib


def lib():
    return _lib or load()


def available() -> bool:
    try:
        load()
        return True
    except Exception:
        return False


# ---------------------------------------------------------------- tensors
def torch():
    import torch as _t
    return _t


def require_device():
    t = torch()
    if not t.cuda.is_available():
        raise RuntimeError("fastllm_py: no ROCm GPU visible; the HIP kernels are the only path")


def is_tensor(x) -> bool:
    t = torch()
    return isinstance(x, t.Tensor)


def is_device_array(x) -> bool:
    """A non-torch device array (e.g. CuPy) exposing __cuda_array_interface__."""
    return hasattr(x, "__cuda_array_interface__") and not isinstance(x, torch().Tensor)


def to_device(x, dtype=None):
    """numpy / torch / device array (e.g. CuPy, zero-copy through
    __cuda_array_interface__) -> contiguous CUDA tensor (optionally cast)."""
    t = torch()
    require_device()
    if isinstance(x, np.ndarray):
        x = t.from_numpy(np.ascontiguousarray(x))
    elif is_device_array(x):
        x = t.as_tensor(x, device="cuda")
    elif not isinstance(x, t.Tensor):
        x = t.as_tensor(np.asarray(x))
    if dtype is not None and x.dtype != dtype:
        x = x.to(dtype)
    if not x.is_cuda:
        x = x.cuda()
    return x.contiguous()


def ptr(x) -> int:
    """Device address of a torch tensor or of a __cuda_array_interface__ array."""
    if hasattr(x, "data_ptr"):
        return int(x.data_ptr())
    return int(x.__cuda_array_interface__["data"][0])


def current_stream_handle() -> int:
    t = torch()
    return int(t.cuda.current_stream().cuda_stream)


def stream_handle(stream) -> int:
    """Launch-stream handle of a torch.cuda.Stream (``.cuda_stream``), a CuPy
    stream (``.ptr``, what the reference's callers pass), a raw int handle,
    or None (the null stream) -> int."""
    if stream is None:
        return 0
    if isinstance(stream, int):
        return stream
    h = getattr(stream, "cuda_stream", None)
    if h is None:
        h = getattr(stream, "ptr", None)
    if h is None:
        raise TypeError(f"not a stream: {type(stream).__name__} has neither .cuda_stream nor .ptr")
    return int(h)


def check_out(buf, numel: int, dtypes, device, name: str = "out"):
    """Validate a caller-supplied output buffer before its pointer goes to a
    kernel: a contiguous device tensor of one of `dtypes`, on `device`, with
    exactly `numel` elements.  Raises ValueError otherwise."""
    t = torch()
    if not isinstance(buf, t.Tensor):
        raise ValueError(f"{name} must be a torch tensor")
    if buf.dtype not in tuple(dtypes):
        raise ValueError(f"{name} has dtype {buf.dtype}; expected one of {tuple(dtypes)}")
    if not buf.is_cuda or (device is not None and buf.device != t.device(device)):
        raise ValueError(f"{name} must live on {device}")
    if not buf.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if buf.numel() != numel:
        raise ValueError(f"{name} has {buf.numel()} elements; expected {numel}")


def overlaps(a, b) -> bool:
    """True when the device memory of tensors a and b intersects."""
    pa, pb = a.data_ptr(), b.data_ptr()
    na, nb = a.numel() * a.element_size(), b.numel() * b.element_size()
    return pa < pb + nb and pb < pa + na


def host_out(x, xp) -> bool:
    """The reference's xp convention: numpy (host) results exactly when the
    caller asks for xp=numpy with a host input; any other xp (CuPy, torch)
    or a device input gives device results."""
    return xp is np and not (isinstance(x, torch().Tensor) or is_device_array(x))


def as_output(x, like_numpy: bool):
    """Return x as numpy when the caller passed numpy (xp=np style)."""
    if like_numpy:
        return x.cpu().numpy()
    return x

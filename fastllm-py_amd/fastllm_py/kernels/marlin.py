"""INT4 (uint4, AWQ-style zero point) group-32/128 weight-only GEMM, Marlin ABI.

Drop-in for the reference's ``fastllm_py/kernels/marlin.py`` with PyTorch-ROCm
tensors as the buffers (reference: fastllm_py/kernels/marlin.py:1-299).  The
functions keep their names, argument order and meaning:

* ``size_m`` activation rows, ``size_k`` input features (groups run along it),
  ``size_n`` output features;
* ``C[size_m, size_n] = A[size_m, size_k] @ dequant(W).T`` with
  ``dequant(W)[n, k] = scale[g, n] * (q[n, k] - zero[g, n])``.

Every computation runs in ``native/libfastllm_kernels.so`` (gfx950 HIP).  The
host-prep helpers (``pack_gptq_qweight``, ``build_marlin_scales_zeros``)
accept numpy or torch input: numpy in (``xp=np``, the reference default) gives
numpy out, computed on the GPU and copied back; torch in gives a device tensor.
The repacked weight is this library's own tile layout (same u32 count as the
GPTQ input, as ``marlin_repack``'s callers assume).
"""
from __future__ import annotations

import numpy as np

from .. import _native as nat

# Marlin's fixed 64-column permutation tables (the caller-visible scale/zero
# layout; fastllm_py/kernels/marlin.py:41-51).
_SCALE_PERM = np.array([8 * j + i for i in range(8) for j in range(8)], dtype=np.int64)
_ZP_INTERLEAVE = np.array([0, 2, 4, 6, 1, 3, 5, 7], dtype=np.int64)


def _load():
    return nat.load()


def has_stream_gemm() -> bool:
    return hasattr(_load(), "FastllmCudaMarlinHalfInt4GemmStream")


def available() -> bool:
    try:
        _load()
        return True
    except Exception:
        return False


# --------------------------------------------------------------------------
# weight-prep helpers (GPU kernels; reference does these in numpy)
# --------------------------------------------------------------------------
def pack_gptq_qweight(q_int4, xp=np):
    """GPTQ packing (marlin.py:113-127): codes q[n, k] in 0..15, shape
    (size_n, size_k), become a uint32 array of shape (size_k // 8, size_n)
    whose word [k // 8, n] holds code k in bits 4 * (k % 8)."""
    t = nat.torch()
    size_n, size_k = q_int4.shape
    assert size_k % 8 == 0, "size_k must be a multiple of 8"
    numpy_in = nat.host_out(q_int4, xp)
    if numpy_in:
        q = nat.to_device(np.asarray(q_int4).astype(np.uint32))
    else:
        q = nat.to_device(q_int4)
        if q.dtype != t.uint32:
            q = q.to(t.int64).to(t.int32).view(t.uint32) if q.dtype != t.int32 else q.view(t.uint32)
    out = t.empty((size_k // 8, size_n), dtype=t.uint32, device=q.device)
    rc = _load().fastllm_pack_gptq_qweight(nat.ptr(q), nat.ptr(out), size_n, size_k,
                                           nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_pack_gptq_qweight")
    return nat.as_output(out, numpy_in)


def build_marlin_scales_zeros(scale, zero_int, group_size, xp=np):
    """Permute scales/zeros into the Marlin tile layout (marlin.py:130-159).

    scale [size_n, num_groups] float, zero_int [size_n, num_groups] int (0..15)
    -> (scales fp16 [num_groups, size_n], zeros u32 [num_groups, size_n//8])."""
    t = nat.torch()
    size_n, num_groups = scale.shape
    assert size_n % 64 == 0, "size_n must be a multiple of 64"
    numpy_in = nat.host_out(scale, xp)
    s = nat.to_device(np.asarray(scale).astype(np.float32) if numpy_in else scale, t.float32)
    if isinstance(zero_int, np.ndarray):
        z = nat.to_device(np.asarray(zero_int).astype(np.int64).astype(np.int32))
    else:
        z = nat.to_device(zero_int).to(t.int64).to(t.int32)
    scales = t.empty((num_groups, size_n), dtype=t.float16, device=s.device)
    zeros = t.empty((num_groups, size_n // 8), dtype=t.uint32, device=s.device)
    rc = _load().fastllm_build_marlin_scales_zeros(
        nat.ptr(s), nat.ptr(z), nat.ptr(scales), nat.ptr(zeros), size_n, num_groups,
        nat.current_stream_handle())
    nat.check_rc(rc, "fastllm_build_marlin_scales_zeros")
    return nat.as_output(scales, numpy_in), nat.as_output(zeros, numpy_in)


# Decode GEMVs above four rows split K in two or three where that pays
# (long K, or wide N above eight rows); their per-strip counters (a fixed
# 64 KiB region at offset 0, the same for every shape) and fp32 partials live
# in the workspace: 192 * size_n bytes for up to 3 splits of 16 rows after
# the counters, beside the reference's (size_n // 64) * 16 ints.
_SPLIT_COUNTER_BYTES = 16384 * 4


def _workspace_ints(size_n: int) -> int:
    split_bytes = _SPLIT_COUNTER_BYTES + 3 * 16 * size_n * 4
    return max(max(1, (size_n // 64) * 16), split_bytes // 4)


def make_workspace(size_n, xp=None):
    """Zeroed int32 workspace for one call site (marlin.py:162-167).  Besides
    the reference's max(1, (size_n//64)*16) ints it holds the split-K
    partials of the decode GEMVs above four rows (192 * size_n bytes); the
    kernels leave its counters at zero."""
    t = nat.torch()
    nat.require_device()
    return t.zeros(_workspace_ints(size_n), dtype=t.int32, device="cuda")


# --------------------------------------------------------------------------
# kernel calls
# --------------------------------------------------------------------------
def marlin_repack(std_qweight, size_k, size_n):
    """Device repack of GPTQ u32 [size_k//8, size_n] into the tile layout.

    Returns a flat uint32 device tensor with the same element count
    (marlin.py:173-189); synchronizes like the reference."""
    t = nat.torch()
    lib = _load()
    std = nat.to_device(std_qweight)
    if std.dtype != t.uint32:
        std = std.to(t.int64).to(t.int32).view(t.uint32) if std.dtype != t.int32 else std.view(t.uint32)
    out = t.empty(std.numel(), dtype=t.uint32, device=std.device)
    ok = lib.FastllmCudaGptqMarlinRepack(nat.ptr(std), nat.ptr(out), int(size_k), int(size_n))
    t.cuda.synchronize()
    if not ok:
        raise RuntimeError(f"marlin_repack: the library refused size_k={size_k}, "
                           f"size_n={size_n} (both must be multiples of 64)")
    return out


def marlin_unrepack(tile_qweight, size_k, size_n):
    """Inverse of marlin_repack: tile layout -> GPTQ u32 [size_k//8, size_n]."""
    t = nat.torch()
    src = nat.to_device(tile_qweight)
    out = t.empty((size_k // 8, size_n), dtype=t.uint32, device=src.device)
    ok = _load().fastllm_int4_tile_unrepack(nat.ptr(src), nat.ptr(out), int(size_k), int(size_n),
                                            nat.current_stream_handle())
    if not ok:
        raise RuntimeError("fastllm_int4_tile_unrepack failed")
    return out


# one zeroed workspace per (device ordinal, size_n), created on first use
_workspaces: dict = {}


def get_workspace(size_n: int):
    """Shared per-device workspace (marlin.py:195-202)."""
    t = nat.torch()
    key = (t.cuda.current_device(), size_n)
    if key not in _workspaces:
        _workspaces[key] = make_workspace(size_n)
    return _workspaces[key]


def gemm_fast(a_fp16, qweight, scales, zeros, size_n, size_k, stream=None, workspace=None,
              out=None):
    """C[M, size_n] = A @ W^T for the per-token decode loop (marlin.py:205-247),
    with no argument checks: the caller hands in an fp16 contiguous A and the
    payload that load-time code already checked, and the entry's return code
    is ignored, as the reference does.  ``stream`` (torch stream, CuPy stream
    or raw handle) selects the stream entry; None runs on the null stream.
    ``out`` may be a preallocated contiguous (M, size_n) fp16 tensor, which
    graph-captured callers keep across replays."""
    t = nat.torch()
    lib = nat.lib()
    size_m = a_fp16.shape[0]
    group_size = size_k // scales.shape[0]
    c = out if out is not None else t.empty((size_m, size_n), dtype=t.float16, device=a_fp16.device)
    ws = workspace if workspace is not None else get_workspace(size_n)
    if 4 < size_m <= 16:
        need = lib.fastllm_int4_gemm_ws_bytes(size_m, size_n, size_k, group_size)
        have = ws.numel() * ws.element_size()
        if need and have >= need:
            # split-K decode GEMV with the call site's workspace (no validation,
            # like the reference: the result code is not checked)
            lib.fastllm_int4_gemm_ws(nat.ptr(a_fp16), nat.ptr(qweight), nat.ptr(scales),
                                     nat.ptr(zeros), nat.ptr(c), size_m, size_n, size_k,
                                     group_size, nat.ptr(ws), have, None,
                                     nat.stream_handle(stream))
            return c
    if stream is not None:
        lib.FastllmCudaMarlinHalfInt4GemmStream(
            nat.ptr(a_fp16), nat.ptr(qweight), nat.ptr(scales), nat.ptr(zeros), nat.ptr(c),
            size_m, size_n, size_k, group_size, nat.ptr(ws), nat.stream_handle(stream))
    else:
        lib.FastllmCudaMarlinHalfInt4Gemm(
            nat.ptr(a_fp16), nat.ptr(qweight), nat.ptr(scales), nat.ptr(zeros), nat.ptr(c),
            size_m, size_n, size_k, group_size, nat.ptr(ws))
    return c


def gemm_swiglu(a_fp16, qweight, scales, zeros, size_n, size_k, out=None, stream=None):
    """Gate/up GEMV fused with SwiGLU for decode (M <= 16): the Marlin-format
    weight stacks gate rows [0, I) and up rows [I, 2I) (size_n = 2I); returns
    h (M, I) fp16 = swiglu(g, u) of the fp16 g, u that gemm_fast would
    return, in one launch (the reference runs gemm_fast then ops.swiglu,
    fastllm_py/kernels/ops.py:157-163)."""
    t = nat.torch()
    a = nat.to_device(a_fp16, t.float16)
    a = a.reshape(-1, size_k).contiguous()
    size_m = a.shape[0]
    group_size = size_k // scales.shape[0]
    if out is not None:
        nat.check_out(out, size_m * (size_n // 2), (t.float16,), a.device)
    h = out if out is not None else t.empty((size_m, size_n // 2), dtype=t.float16, device=a.device)
    hs = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_int4_gemm_swiglu(nat.ptr(a), nat.ptr(qweight), nat.ptr(scales),
                                            nat.ptr(zeros), nat.ptr(h), size_m, size_n, size_k,
                                            group_size, hs)
    if rc == 1:
        if size_m > 16 or size_n % 128 or size_k % 128 or group_size not in (32, 128):
            raise ValueError(f"gemm_swiglu: unsupported shape M={size_m} N={size_n} K={size_k} "
                             f"group={group_size}")
        # K beyond the fused kernel's register/LDS budget: plain GEMV, then swiglu
        gu = gemm_fast(a, qweight, scales, zeros, size_n, size_k, stream=hs,
                       workspace=get_workspace(size_n))
        inter = size_n // 2
        from . import ops
        return ops.swiglu(gu[:, :inter], gu[:, inter:], out=h, stream=hs)
    nat.check_rc(rc, "fastllm_int4_gemm_swiglu")
    return h


def gemm_add_rmsnorm(x, delta, norm_w, eps, qweight, scales, zeros, size_n, size_k, swiglu=False,
                     out=None, xnew=None, stream=None):
    """One decode row: xnew = x + delta and the Marlin GEMV of
    h = rmsnorm(xnew) * norm_w in one launch (h stays on chip); with
    ``swiglu`` the gate/up weight's SwiGLU epilogue as in ``gemm_swiglu``.
    x (1, K) fp32, delta (1, K) fp16, norm_w (K,) fp16.  Returns (xnew fp32,
    out fp16 (1, size_n) or (1, size_n/2)).  The reference issues
    add_rmsnorm then the projection (graph_decode.py:818-826, 858-866)."""
    t = nat.torch()
    xd = nat.to_device(x, t.float32).reshape(1, size_k).contiguous()
    dd = nat.to_device(delta, t.float16).reshape(1, size_k).contiguous()
    wd = nat.to_device(norm_w, t.float16).reshape(size_k).contiguous()
    n_out = size_n // 2 if swiglu else size_n
    if out is not None:
        nat.check_out(out, n_out, (t.float16,), xd.device, "out")
    if xnew is not None:
        nat.check_out(xnew, size_k, (t.float32,), xd.device, "xnew")
        if nat.overlaps(xnew, xd) or nat.overlaps(xnew, dd):
            raise ValueError("gemm_add_rmsnorm: xnew must not overlap x or delta (the kernel "
                             "stores xnew while other workgroups still read them)")
    c = out if out is not None else t.empty((1, n_out), dtype=t.float16, device=xd.device)
    xn = xnew if xnew is not None else t.empty((1, size_k), dtype=t.float32, device=xd.device)
    group_size = size_k // scales.shape[0]
    hs = nat.stream_handle(stream) if stream is not None else nat.current_stream_handle()
    rc = nat.lib().fastllm_int4_gemm_add_rmsnorm(
        nat.ptr(xd), nat.ptr(dd), nat.ptr(wd), float(eps), nat.ptr(xn), nat.ptr(qweight),
        nat.ptr(scales), nat.ptr(zeros), nat.ptr(c), size_n, size_k, group_size, int(bool(swiglu)), hs)
    if rc == 1:
        if (size_k % 128 or size_n % 64 or (swiglu and size_n % 128)
                or group_size not in (32, 128)):
            raise ValueError(f"gemm_add_rmsnorm: unsupported shape N={size_n} K={size_k} "
                             f"group={group_size}")
        # the fused prologue does not fit this shape: standalone norm, then the projection
        from . import ops
        h = t.empty((1, size_k), dtype=t.float16, device=xd.device)
        ops.add_rmsnorm(xd, dd, wd, eps, out=(xn, h), stream=hs)
        if swiglu:
            gemm_swiglu(h, qweight, scales, zeros, size_n, size_k, out=c, stream=hs)
        else:
            gemm_fast(h, qweight, scales, zeros, size_n, size_k, stream=hs,
                      workspace=get_workspace(size_n), out=c)
        return xn, c
    nat.check_rc(rc, "fastllm_int4_gemm_add_rmsnorm")
    return xn, c


def marlin_gemm_int4(a_fp16, packed_weights, scales, zeros, workspace=None, size_n=None,
                     sync=True):
    """INT4 GEMM with validation (marlin.py:250-299).

    a_fp16 [size_m, size_k] (cast to fp16), packed_weights from marlin_repack,
    scales fp16 [num_groups, size_n], zeros u32 [num_groups, size_n//8].
    Returns fp16 [size_m, size_n]; raises ValueError on bad shapes and
    RuntimeError when the library rejects the call."""
    t = nat.torch()
    lib = _load()
    a = nat.to_device(a_fp16, t.float16)
    size_m, size_k = a.shape
    num_groups = scales.shape[0]
    if size_n is None:
        size_n = scales.shape[1]
    if workspace is None:
        workspace = get_workspace(size_n)
    group_size = size_k // num_groups

    if size_n % 64 != 0 or size_k % 64 != 0:
        raise ValueError(f"marlin_gemm_int4: the tile layout needs size_n and size_k in "
                         f"multiples of 64 (got {size_n}, {size_k})")
    if group_size not in (32, 128):
        raise ValueError(f"marlin_gemm_int4: groups of 32 or 128 only (size_k / groups = "
                         f"{group_size})")
    if size_k % group_size != 0:
        raise ValueError(f"marlin_gemm_int4: size_k={size_k} is not a whole number of "
                         f"{group_size}-groups")

    scales = nat.to_device(scales, t.float16)
    zeros = nat.to_device(zeros)
    if zeros.dtype != t.uint32:
        zeros = zeros.to(t.int64).to(t.int32).view(t.uint32)
    qw = nat.to_device(packed_weights)
    c = t.empty((size_m, size_n), dtype=t.float16, device=a.device)
    have = workspace.numel() * workspace.element_size()
    need = lib.fastllm_int4_gemm_ws_bytes(size_m, size_n, size_k, group_size)
    if need and have >= need:
        ok = lib.fastllm_int4_gemm_ws(nat.ptr(a), nat.ptr(qw), nat.ptr(scales), nat.ptr(zeros),
                                      nat.ptr(c), size_m, size_n, size_k, group_size,
                                      nat.ptr(workspace), have, None, None) == 0
    else:
        ok = lib.FastllmCudaMarlinHalfInt4Gemm(
            nat.ptr(a), nat.ptr(qw), nat.ptr(scales), nat.ptr(zeros), nat.ptr(c),
            size_m, size_n, size_k, group_size, nat.ptr(workspace))
    if sync:
        t.cuda.synchronize()
    if not ok:
        raise RuntimeError("marlin_gemm_int4: the library refused the call (not a gfx950 "
                           "device, or a shape its kernels do not take)")
    return c

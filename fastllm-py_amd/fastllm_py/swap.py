"""Function-level swap of this library into the reference's ``fastllm_py``.

The reference package and this one share the package name ``fastllm_py``.
A process that runs the reference imports this one under another name
(``load_as``) and calls ``install``, which rebinds only the hot-path
functions listed in ``SWAPS`` inside the reference's own modules.  Everything
else stays the reference's: its model runner, engines, ``MoELayer``,
``SpeedEstimator``, ``ExpertPlacement``, ``GpuExpertCache``, the non-matmul
ops (``KEPT`` lists the names its callers import from the swapped modules
that are left in place).

Callers of the reference hand CuPy arrays to these functions and expect
CuPy arrays back (``xp=cupy``).  Every swapped function is wrapped so that
device arrays exposing ``__cuda_array_interface__`` enter as zero-copy torch
views (in-place ``out=`` buffers included) and device results leave as
zero-copy CuPy arrays when the call carried CuPy arrays, a CuPy stream or
``xp=cupy``.  A CuPy ``stream=`` argument is passed through untouched (the
library reads its ``.ptr``), and the call runs with torch's current stream
set to the launch stream (the given one, else CuPy's current stream), so
outputs are allocated, and default-stream launches ordered, on the stream
the caller's CuPy work uses.

``install`` also rebinds copies a reference module took with ``from X import
name`` before the swap (``moe.py:18`` binds ``route_topk`` that way).
"""
from __future__ import annotations

import dataclasses
import functools
import importlib
import importlib.util
import os
import sys

# reference module (relative to its package) -> names rebound to this library's
SWAPS = {
    "kernels.marlin": ("has_stream_gemm", "available", "pack_gptq_qweight",
                       "build_marlin_scales_zeros", "make_workspace", "marlin_repack",
                       "get_workspace", "gemm_fast", "marlin_gemm_int4"),
    "kernels.fp8": ("available", "packed_row_bytes", "quantize", "fp8_gemv"),
    "kernels.moe_int4": ("quantize_int4_rowmajor", "dequantize_int4_rowmajor",
                         "_quantize_int4_rowmajor_batched", "build_stacked_experts",
                         "gate_matvec", "fused_moe_weighted", "fused_moe_ffn2", "fused_moe_ffn",
                         "gemv_int4"),
    "quantizer": ("_fp8_e4m3_encode", "_fp8_e4m3_decode", "quantize_fp8_block",
                  "dequantize_fp8_block", "quantize_int4_group", "dequantize_int4_group"),
    "moe": ("quantize_marlin_matrix", "build_marlin_expert_payload", "_expert_ffn_marlin"),
    "expert_router": ("route_topk",),
    "graph_decode": ("_dense_gemv_kernel", "_route_topk_kernel"),
}

# where a swapped name lives here when its module or name differs
SOURCE = {
    ("graph_decode", "_dense_gemv_kernel"): ("graph_shims", "dense_gemv_kernel"),
    ("graph_decode", "_route_topk_kernel"): ("graph_shims", "route_topk_kernel"),
}

# names the reference's callers import from the swapped modules that stay the
# reference's own (model.py:243-244, moe.py:17-19, graph_decode.py:40-41)
KEPT = {
    "moe": ("MoELayer", "_expert_ffn"),
    "expert_router": ("ExpertTask", "SpeedEstimator", "ExpertPlacement"),
    "quantizer": ("QuantizedTensor", "FP8_E4M3_MAX"),
    "graph_decode": ("GraphDecoder", "graph_capable", "apply_penalties", "sample_logits"),
}

HERE = os.path.dirname(os.path.abspath(__file__))


def load_as(name: str = "fastllm_amd"):
    """Import this package under `name` (its modules use relative imports
    only), leaving ``fastllm_py`` free for the reference."""
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(HERE, "__init__.py"),
                                                  submodule_search_locations=[HERE])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def _launch_stream(torch, cp, kwargs):
    """torch stream context for the call: the caller's ``stream=`` (CuPy
    ``.ptr``, torch ``.cuda_stream`` or int), else CuPy's current stream."""
    from . import _native as nat

    s = kwargs.get("stream")
    h = nat.stream_handle(s) if s is not None else int(cp.cuda.get_current_stream().ptr)
    if h == 0:
        return torch.cuda.stream(torch.cuda.default_stream())
    return torch.cuda.stream(torch.cuda.ExternalStream(h))


def _cupy_of(v):
    m = type(v).__module__ or ""
    if m.startswith("cupy"):
        return sys.modules.get("cupy")
    return None


def _find_cupy(args, kwargs):
    xp = kwargs.get("xp")
    if xp is not None and getattr(xp, "__name__", "") == "cupy":
        return xp
    for v in list(args) + list(kwargs.values()):
        if getattr(v, "__name__", "") == "cupy" and hasattr(v, "asarray"):
            return v  # xp passed positionally
        for x in (v.values() if isinstance(v, dict) else v if isinstance(v, (list, tuple)) else (v,)):
            cp = _cupy_of(x)
            if cp is not None:
                return cp
    return None


def _map(v, fn):
    if isinstance(v, dict):
        return type(v)((k, _map(x, fn)) for k, x in v.items())
    if isinstance(v, (list, tuple)) and not hasattr(v, "_fields"):
        return type(v)(_map(x, fn) for x in v)
    if dataclasses.is_dataclass(v) and not isinstance(v, type):
        return dataclasses.replace(v, **{f.name: _map(getattr(v, f.name), fn)
                                         for f in dataclasses.fields(v)})
    return fn(v)


def adapt(fn):
    """Wrap one of this library's functions for callers that pass CuPy arrays."""

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        cp = _find_cupy(args, kwargs)
        if cp is None:
            return fn(*args, **kwargs)
        import torch

        from . import _native as nat

        def to_torch(x):
            # device arrays only: a CuPy stream is passed through as it is
            return torch.as_tensor(x, device="cuda") if nat.is_device_array(x) else x

        def to_cupy(x):
            return cp.asarray(x) if isinstance(x, torch.Tensor) and x.is_cuda else x
        if kwargs.get("xp") is cp:
            kwargs["xp"] = torch  # any non-numpy xp: device results
        with _launch_stream(torch, cp, kwargs):
            r = fn(*_map(list(args), to_torch), **_map(kwargs, to_torch))
        return _map(r, to_cupy)

    wrapper.__wrapped_amd__ = fn
    return wrapper


def install(ref_package: str = "fastllm_py", ours=None) -> list[str]:
    """Rebind SWAPS inside the (importable) reference package `ref_package`.
    Returns the rebound "module.name" list."""
    ours = ours or load_as()
    replaced, done = {}, []
    for rel, names in SWAPS.items():
        ref_mod = importlib.import_module(f"{ref_package}.{rel}")
        for name in names:
            src_mod, src_name = SOURCE.get((rel, name), (rel, name))
            ours_fn = getattr(importlib.import_module(f"{ours.__name__}.{src_mod}"), src_name)
            new = adapt(ours_fn)
            old = getattr(ref_mod, name, None)
            setattr(ref_mod, name, new)
            if old is not None:
                replaced[id(old)] = (old, new)
            done.append(f"{rel}.{name}")
    for mname, m in list(sys.modules.items()):
        if m is None or not (mname == ref_package or mname.startswith(ref_package + ".")):
            continue
        for attr, val in list(vars(m).items()):
            hit = replaced.get(id(val))
            if hit is not None and hit[0] is val:
                setattr(m, attr, hit[1])
    return done

"""The function-level swap into the reference package (CPU: name resolution).

The reference is not imported here: a stand-in package with the same module
layout holds placeholders for every name the reference's callers import from
the swapped modules (CALLER_IMPORTS, cited by file:line).  After
``swap.install`` each such name must resolve either to this library's
function (the names in ``swap.SWAPS``) or to the stand-in's own object (the
names in ``swap.KEPT``), including copies a module took with ``from X import
name`` before the swap.
"""
import importlib
import sys
import textwrap

import pytest

from fastllm_py import swap

# (reference module, name): the caller lines that import it
CALLER_IMPORTS = {
    ("kernels.marlin", "gemm_fast"): "model.py:58, graph_decode.py:770, batched.py:153, moe.py:71",
    ("kernels.marlin", "make_workspace"): "graph_decode.py:770, batched.py:153",
    ("kernels.marlin", "has_stream_gemm"): "moe.py:101-103",
    ("moe", "quantize_marlin_matrix"): "model.py:175",
    ("moe", "build_marlin_expert_payload"): "model.py:296",
    ("moe", "MoELayer"): "model.py:244",
    ("moe", "_expert_ffn_marlin"): "moe.py:135-159 (MoELayer._run_gpu_experts)",
    ("expert_router", "ExpertPlacement"): "model.py:243, moe.py:18",
    ("expert_router", "SpeedEstimator"): "model.py:243, moe.py:18",
    ("expert_router", "ExpertTask"): "moe.py:18",
    ("expert_router", "route_topk"): "moe.py:18",
    ("kernels.moe_int4", "quantize_int4_rowmajor"): "graph_decode.py:547",
    ("kernels.moe_int4", "build_stacked_experts"): "graph_decode.py:581,650-655",
    ("kernels.moe_int4", "gate_matvec"): "graph_decode.py:680,696",
    ("kernels.moe_int4", "fused_moe_weighted"): "graph_decode.py:688,692",
    ("graph_decode", "_dense_gemv_kernel"): "graph_decode.py:754",
    ("graph_decode", "_route_topk_kernel"): "graph_decode.py:682",
    ("graph_decode", "GraphDecoder"): "model.py:489, engine.py:76",
    ("graph_decode", "graph_capable"): "model.py:489, engine.py:76",
    ("graph_decode", "apply_penalties"): "model.py:507, engine.py:45",
    ("graph_decode", "sample_logits"): "model.py:507, engine.py:36",
    ("quantizer", "quantize_fp8_block"): "quantizer users (weights loading)",
    ("quantizer", "QuantizedTensor"): "quantizer users (weights loading)",
}


def _stand_in(tmp_path, name):
    """A package laid out like the reference, every name a placeholder."""
    root = tmp_path / name
    (root / "kernels").mkdir(parents=True)
    (root / "__init__.py").write_text("")
    (root / "kernels" / "__init__.py").write_text("")
    names = {}
    for (mod, n) in CALLER_IMPORTS:
        names.setdefault(mod, set()).add(n)
    for mod, ns in swap.SWAPS.items():
        names.setdefault(mod, set()).update(ns)
    for mod, ns in swap.KEPT.items():
        names.setdefault(mod, set()).update(ns)
    for mod, ns in names.items():
        body = "\n".join(f"class {n}:\n    origin = 'stand-in'\n" if n[0].isupper() or n.isupper()
                         else f"def {n}(*a, **k):\n    return 'stand-in'\n" for n in sorted(ns))
        if mod == "moe":  # module-level copy, as moe.py:18 takes it
            body = "from .expert_router import route_topk, ExpertTask\n" + body
        path = root / (mod.replace(".", "/") + ".py")
        path.write_text(textwrap.dedent(body))
    return root


def test_every_caller_import_resolves(tmp_path):
    pkg = "fastllm_ref_standin"
    _stand_in(tmp_path, pkg)
    sys.path.insert(0, str(tmp_path))
    try:
        importlib.import_module(f"{pkg}.moe")  # the copy exists before the swap
        ours = swap.load_as("fastllm_amd_swaptest")
        done = swap.install(pkg, ours=ours)
        assert len(done) == sum(len(v) for v in swap.SWAPS.values())
        for (mod, name), where in CALLER_IMPORTS.items():
            obj = getattr(importlib.import_module(f"{pkg}.{mod}"), name)
            if name in swap.SWAPS.get(mod, ()):
                inner = getattr(obj, "__wrapped_amd__", None)
                assert inner is not None, (mod, name, where)
                assert inner.__module__.startswith("fastllm_amd_swaptest"), (mod, name)
            else:
                assert name in swap.KEPT.get(mod, ()), f"{mod}.{name} ({where}) is neither swapped nor kept"
                assert getattr(obj, "origin", None) == "stand-in" or obj() == "stand-in"
        moe = importlib.import_module(f"{pkg}.moe")
        assert getattr(moe.route_topk, "__wrapped_amd__", None) is not None  # the copy was rebound
        assert moe.ExpertTask.origin == "stand-in"
    finally:
        sys.path.remove(str(tmp_path))
        for m in [m for m in sys.modules if m.startswith(pkg) or m.startswith("fastllm_amd_swaptest")]:
            del sys.modules[m]


def test_swapped_names_exist_here():
    from fastllm_py import swap as sw

    for mod, names in sw.SWAPS.items():
        for n in names:
            src_mod, src_name = sw.SOURCE.get((mod, n), (mod, n))
            m = importlib.import_module(f"fastllm_py.{src_mod}")
            assert callable(getattr(m, src_name)), (mod, n)


def test_xp_convention():
    """numpy results only for numpy input with xp=numpy; any other xp gives
    device results (graph_decode.py:563 passes xp=cupy with host weights)."""
    import numpy as np

    from fastllm_py import _native as nat

    a = np.zeros(4, np.float32)
    assert nat.host_out(a, np)
    assert not nat.host_out(a, object())
    assert nat.host_out([1.0], np)
    pytest.importorskip("torch")
    import torch

    assert not nat.host_out(torch.zeros(2), np)

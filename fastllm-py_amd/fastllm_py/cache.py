"""On-disk caches of packed weights, versioned.

The reference keeps three npz caches of finished payloads so warm starts
skip quantization (fastllm_py/model.py:179-189 ``.marlin_cache``,
fastllm_py/model.py:281-305 ``.expert_cache``, fastllm_py/graph_decode.py:
609-660 ``.rowmajor_cache``).  This library's packed layouts differ from the
reference's CUDA ones (its Marlin tile layout and its stacked-expert tile
layout), so every file written here carries a ``__format__`` tag and a
loader refuses a file whose tag is missing or different instead of feeding
foreign bytes to the kernels.

Writes go to ``<name>.tmp.npz`` and are renamed into place, as the
reference does, so a killed run leaves no truncated cache.  Loading uses
``numpy.load`` with pickles disabled.
"""
from __future__ import annotations

import os
from pathlib import Path

import numpy as np

from . import _native as nat

MARLIN_FORMAT = "fastllm-py_amd/marlin-tile/v1"
EXPERTS_FORMAT = "fastllm-py_amd/marlin-experts/v1"
STACKED_FORMAT = "fastllm-py_amd/stacked-tile/v2"  # v2: FP8 expert blocks as two 1 KB halves


def _host(v):
    if hasattr(v, "detach"):
        return v.detach().cpu().numpy()
    return np.asarray(v)


def _atomic_savez(path, arrays: dict):
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(path.name + ".tmp.npz")
    np.savez(tmp, **arrays)
    os.replace(tmp, path)


def _open(path, fmt: str):
    z = np.load(path, allow_pickle=False)
    tag = str(z["__format__"]) if "__format__" in z.files else None
    if tag != fmt:
        raise ValueError(f"{path}: cache format {tag!r}, expected {fmt!r} "
                         f"(written by another build or the reference; delete it to rebuild)")
    return z


def _to(v, device):
    if device is None:
        return v
    t = nat.torch()
    return t.from_numpy(np.ascontiguousarray(v)).to(device)


def save_marlin_payload(path, payload: dict):
    """One Marlin-ABI matrix (``quantize_marlin_matrix``'s dict: qweight,
    scales, zeros, ...) -> npz (the reference's ``.marlin_cache`` entry)."""
    out = {k: _host(v) for k, v in payload.items()}
    out["__format__"] = np.array(MARLIN_FORMAT)
    _atomic_savez(path, out)


def load_marlin_payload(path, device="cuda") -> dict:
    z = _open(path, MARLIN_FORMAT)
    return {k: _to(z[k], device) for k in z.files if k != "__format__"}


def save_expert_payloads(path, payloads: dict):
    """{expert id: Marlin payload} -> one npz with keys ``"{e}.{field}"``,
    the reference's ``.expert_cache/marlin.L{i}.npz`` schema."""
    out = {f"{e}.{k}": _host(v) for e, p in payloads.items() for k, v in p.items()}
    out["__format__"] = np.array(EXPERTS_FORMAT)
    _atomic_savez(path, out)


def load_expert_payloads(path, device="cuda") -> dict:
    z = _open(path, EXPERTS_FORMAT)
    out: dict = {}
    for key in z.files:
        if key == "__format__":
            continue
        e, rest = key.split(".", 1)
        out.setdefault(int(e), {})[rest] = _to(z[key], device)
    return out


def save_stacked(path, stacked: dict):
    """Stacked experts (``moe_int4.build_stacked_experts`` / ``stack_tiles``)
    -> npz, the reference's ``.rowmajor_cache`` schema: ``group`` as int64,
    ``*.shape`` as int64 arrays, tensors as arrays."""
    out = {}
    for k, v in stacked.items():
        if k == "group":
            out[k] = np.int64(v)
        elif k.endswith(".shape"):
            out[k] = np.asarray(v, dtype=np.int64)
        elif isinstance(v, str):
            out[k] = np.array(v)
        else:
            out[k] = _host(v)
    out["__format__"] = np.array(STACKED_FORMAT)
    _atomic_savez(path, out)


def load_stacked(path, device="cuda") -> dict:
    z = _open(path, STACKED_FORMAT)
    st = {}
    for k in z.files:
        if k == "__format__":
            continue
        if k == "group":
            st[k] = int(z[k])
        elif k.endswith(".shape"):
            st[k] = tuple(int(x) for x in z[k])
        elif z[k].dtype.kind == "U":
            st[k] = str(z[k])
        else:
            st[k] = _to(z[k], device)
    return st

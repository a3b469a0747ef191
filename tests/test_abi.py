"""The C-ABI library loads and exports every symbol include/*.h declares
(CPU only: no compute call is made)."""
import ctypes
import glob
import os
import re

import pytest

from fastllm_py import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = []
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:bool|int|void|float|size_t)\s+\**\s*(\w+)\s*\(", text, flags=re.M):
            names.append(m.group(1))
    return names


def test_header_declares_symbols():
    names = declared_symbols()
    assert "FastllmCudaMarlinHalfInt4Gemm" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"{_native.LIB_PATH} not built (run python fastllm-py_amd/build_native.py)")
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_table_matches_header():
    assert set(_native.SIGNATURES) == set(declared_symbols())


def test_moe_entry_argument_checks():
    """Shape/argument validation of the fused-MoE entry points runs before any
    device call: valid arguments reach the device check (rc 2 without a GPU,
    or launch on one), invalid ones return 1.  Fake aligned pointers only."""
    lib = _native.lib()
    p = 1 << 20  # never dereferenced: validation fails or stops at the device check
    ws = lib.fastllm_moe_int4_workspace_bytes(1, 2048, 1408, 5632, 4)
    assert ws == 256 + (4 + 1) * 5632 * 2  # the counter region, then inter_buf
    # T > 16 takes the grouped kernels (hidden % 256 == 0)
    assert lib.fastllm_moe_int4_workspace_bytes(17, 2048, 1408, 0, 68) > 0
    assert lib.fastllm_moe_int4_workspace_bytes(17, 384, 1408, 0, 68) == 0
    assert lib.fastllm_moe_int4_workspace_bytes(1, 2000, 1408, 0, 4) == 0

    def fused(T=1, hidden=2048, gs=128, inter=1408, sinter=5632, ws_bytes=ws, slots=4, entries=4):
        sh = [p] * 6 if sinter else [None] * 6
        return lib.fastllm_moe_int4_fused(p, T, hidden, gs, 60, inter, *([p] * 6), sinter, *sh,
                                          None, p, p, p, p, p, slots, entries, p, ws_bytes, p, None)

    # the deterministic combine's term rows: (max_entries + pieces T) x hidden fp32 more
    wsd = lib.fastllm_moe_workspace_bytes_ex(1, 2048, 1408, 5632, 4, 1)
    assert lib.fastllm_moe_workspace_bytes_ex(1, 2048, 1408, 5632, 4, 0) == ws
    assert wsd >= ws + (4 + 4 * 1) * 2048 * 4
    assert lib.fastllm_moe_workspace_bytes_ex(1, 2048, 1408, 5632, 4, 2) == 0  # unknown flag
    assert lib.fastllm_moe_workspace_bytes_ex(512, 2048, 768, 0, 4096, 1) >= \
        lib.fastllm_moe_int4_workspace_bytes(512, 2048, 768, 0, 4096) + 4096 * 2048 * 4

    def fused_ex(flags=1, fmt=0, ws_bytes=wsd, slots=4):
        return lib.fastllm_moe_fused_ex(fmt, flags, p, 1, 2048, 128, 60, 1408, *([p] * 6), 5632,
                                        *([p] * 6), None, p, p, p, p, p, slots, 4, p, ws_bytes, p,
                                        None)
    assert fused_ex(ws_bytes=ws) == 1     # the plain workspace is too small for the term rows
    assert fused_ex(flags=4) == 1         # unknown flag
    assert fused_ex(fmt=3) == 1           # unknown format
    assert fused_ex(slots=300) == 1       # more slots than the combine's per-token list

    import torch
    if not torch.cuda.is_available():
        assert fused() == 2
        assert fused_ex() == 2
    assert fused(gs=96) == 1
    assert fused(hidden=2000) == 1
    assert fused(ws_bytes=ws - 1) == 1
    assert fused(slots=0) == 1
    assert fused(T=17) == 1  # workspace sized for T = 1

    def routed(T=1, E=60, k=4, scoring=0, sinter=5632, ws_bytes=ws, logits=p):
        sh = [p] * 6 if sinter else [None] * 6
        return lib.fastllm_moe_int4_routed(logits, k, scoring, 0, 1.0, None, 0, 0, p, *([p] * 9),
                                           p, T, 2048, 128, E, 1408, *([p] * 6), sinter, *sh, p,
                                           ws_bytes, p, None)

    if not torch.cuda.is_available():
        assert routed() == 2
    assert routed(T=17) == 1
    assert routed(k=0) == 1
    assert routed(k=17) == 1
    assert routed(E=300) == 1
    assert routed(scoring=2) == 1
    assert routed(logits=None) == 1
    assert routed(ws_bytes=ws - 1) == 1
    assert lib.fastllm_moe_int4_tile_repack(p, p, p, p, p, 24, 256, 128, None) == 1  # rows % 16
    assert lib.fastllm_moe_int4_tile_repack(p, p, p, p, p, 32, 200, 128, None) == 1  # in % 128


def test_int4_split_workspace_sizes():
    """Split-K workspace query (host arithmetic only): above four rows the
    long-K down shape splits in two (three above eight rows) and (above eight
    rows) the wide gate_up shape in two (counters in a fixed 64 KiB region
    from offset 0 for every shape, then splits x M x N fp32 partials); qkv /
    o and four rows or fewer do not split; the Python layer's make_workspace
    covers every split shape."""
    from fastllm_py.kernels.marlin import _workspace_ints

    lib = _native.lib()
    part = lambda N: 16384 * 4  # noqa: E731
    down, gate_up = (4096, 12288), (24576, 4096)
    for M in (5, 8):
        assert lib.fastllm_int4_gemm_ws_bytes(M, *down, 128) == part(4096) + 2 * M * 4096 * 4
    for M in (9, 16):  # above eight rows: three splits
        assert lib.fastllm_int4_gemm_ws_bytes(M, *down, 128) == part(4096) + 3 * M * 4096 * 4
    assert lib.fastllm_int4_gemm_ws_bytes(16, *gate_up, 128) == part(24576) + 2 * 16 * 24576 * 4
    assert lib.fastllm_int4_gemm_ws_bytes(8, *gate_up, 128) == 0
    for N, K in ((6144, 4096), (4096, 4096)):
        assert lib.fastllm_int4_gemm_ws_bytes(16, N, K, 128) == 0
    for M in (1, 4, 17):
        assert lib.fastllm_int4_gemm_ws_bytes(M, *down, 128) == 0
    assert lib.fastllm_int4_gemm_ws_bytes(16, 4096, 12288, 32) == 0  # group 32 stays unsplit
    assert lib.fastllm_int4_gemm_ws_bytes(16, 4096, 12288, 64) == 0  # not a Marlin group
    for N in (64, 2048, 4096, 6144, 24576, 151936 // 64 * 64):
        for K in range(1024, 32768 + 1, 1024):
            for M in range(5, 17):
                assert lib.fastllm_int4_gemm_ws_bytes(M, N, K, 128) <= 4 * _workspace_ints(N)


def test_fp8_gemm_split_workspace_sizes():
    """Split-K workspace query of the FP8 prefill GEMM (host arithmetic only):
    grids under 256 64x128 tiles split (at most 4 splits of >= 4 blocks),
    larger grids and decode shapes do not."""
    lib = _native.lib()
    tile = 64 * 128 * 4
    # counters in a fixed 1 KB (every splitting grid has < 256 tiles), then partials
    # M=512, N=2048: 8 x 16 = 128 tiles -> 2 splits where K gives >= 16 blocks each
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(512, 2048, 10944) == 1024 + 2 * 128 * tile
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(512, 2048, 2048) == 0  # 16 blocks: whole
    # M=128, N=2048: 32 tiles -> 4 splits (86 blocks: 22 each)
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(128, 2048, 10944) == 1024 + 4 * 32 * tile
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(128, 2048, 4096) == 1024 + 2 * 32 * tile
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(512, 10944, 2048) == 0  # 688 tiles
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(16, 2048, 2048) == 0    # decode kernels
    assert lib.fastllm_fp8_b128x128_gemm_ws_bytes(96, 256, 320) == 0      # 3 blocks: no split

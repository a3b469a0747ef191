"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline: Qwen3-8B decode linears, INT4 group-128
in the Marlin ABI format, fp16 activations ~ N(0,1), weights ~ N(0,0.02)
before quantization.  Shapes (N x K): qkv 6144x4096, o 4096x4096, gate+up
24576x4096, down 4096x12288.  One step = the four GEMVs of one layer at batch
M; `value` = INT4 GEMV HBM GB/s at M=1 over the layer's algorithmic bytes
(packed weights + scales + zeros + activations + outputs), summed per layer.

Also measured (same JSON line, "breakdown"): M in {1,4,8,16}; FP8-E4M3
128x128-block GEMVs with bf16 activations at the DeepSeek-V2-Lite-like shapes
(configs[2]); the fused Qwen1.5-MoE-A2.7B INT4 MoE layer at 1 and 16 tokens
(configs[3]) in us/layer and against its routed-weight-bytes roofline.

Also: config 1 (the INT4 GEMV on quantize_int4_group's format, 3072x1024),
the row-major INT4 GEMV (dgemv) at the Qwen3-8B shapes, the reference ABI's
own FP8 GEMV (inline 1x128 format, fastllm_fp8_block128_gemv_fp16), the
decode MoE at the Qwen3-30B-A3B shape of the reference's one published
fused-MoE latency, the prefill GEMMs of config 5, and a streaming-read probe
(fastllm_hbm_read_probe) at every decode GEMV's byte count -- the per-launch
floor each GEMV is reported against.

The timed region of the headline is exactly --steps layer-steps (four GEMV
launches each, step i on weight copy i mod the copy count), one replay of a
HIP graph holding them; the per-GEMV figures come from graphs of >= 96
launches of one GEMV each.

Every figure is timed with HIP events around HIP-graph replays on the launch
stream.  Each graph cycles through enough weight copies (and, for the MoE,
router logits) that the bytes touched between two reads of the same weight
exceed 2.2x the 256 MB Infinity Cache, so weights stream from HBM; each leg
records its `cycle_bytes`.  `--warmup W` untimed replays, and at least 30 ms
of replays, precede each timed region.

CPU baselines: the numpy oracle on the host, 3 warm-up
runs then the median of 20; figure (i) dequantize-then-fp32-matmul per call
(the reference's CPU semantics), figure (ii) the fp32 matmul on
pre-dequantized weights (the BLAS floor); CPU model and BLAS build recorded.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "fastllm-py_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of the roofline kernel measured with rocprofv3 --pmc
# FETCH_SIZE / WRITE_SIZE (x2.000 / x1.000 copy-kernel calibration); see
# profiles/int4_gemv_gate_up_qwen3_8b_m1_traffic.md.  Keyed by (kernel, M).
MEASURED_TRAFFIC = {("int4_gemv_nb<2,4,false,0>", 1): 52_495_211}
# Average duration of the roofline kernel in the committed rocprofv3 kernel
# trace of this bench (profiles/bench_kernel_trace_full.md), beside the
# graph-timed figure the line computes live.  Keyed by (kernel, M).
ROCPROF_US = {("int4_gemv_nb<2,4,false,0>", 1): (11.48, "profiles/bench_kernel_trace_full.md")}
QWEN3_8B = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096),
            ("down", 4096, 12288)]
FP8_SHAPES = [("2048x2048", 2048, 2048), ("10944x2048", 10944, 2048), ("2048x10944", 2048, 10944)]
GS = 128
MALL_BYTES = 256 * 2 ** 20
ROTATE_BYTES = int(2.2 * MALL_BYTES)


def marlin_bytes(M, N, K, gs=GS):
    G = K // gs
    return N * K // 2 + G * N * 2 + G * N // 2 + M * K * 2 + M * N * 2


def fp8_block_bytes(M, N, K):
    return N * K + (-(-N // 128)) * (-(-K // 128)) * 4 + M * K * 2 + M * N * 2


def log(msg):
    print(msg, file=sys.stderr, flush=True)


WARMUP = [5]  # untimed replays before each timed region (--warmup)


WARM_MS = 30.0  # minimum busy time before each timed region


def graph_time(torch, stream, launches, reps, warmup=None):
    """Capture the enqueue callbacks in one HIP graph on `stream`, replay it
    `warmup` (default --warmup) times and on until the GPU has been busy for
    WARM_MS, then time `reps` replays with HIP events on that stream.
    Returns ms per replay.  (After the host-side setup of a leg -- quantizing
    and copying its weights -- the first few ms of replays run up to 30 %
    slower: 24576x4096 row-major 14.7-16.1 us, then 11.9-12.7 us.)"""
    if warmup is None:
        warmup = WARMUP[0]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        h = torch.cuda.current_stream().cuda_stream
        for fn in launches:
            fn(h)
    t_start = time.perf_counter()
    done = 0
    while done < max(1, warmup) or (time.perf_counter() - t_start) * 1e3 < WARM_MS:
        for _ in range(8):
            g.replay()
        done += 8
        torch.cuda.synchronize()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0.record(stream)
        for _ in range(reps):
            g.replay()
        t1.record(stream)
    stream.synchronize()
    return t0.elapsed_time(t1) / reps


def copies_for(nbytes):
    return max(2, -(-ROTATE_BYTES // max(1, nbytes)))


def cycle(nbytes):
    """Bytes touched between two reads of the same weight, and that over the MALL."""
    return {"cycle_bytes": int(nbytes), "cycle_over_mall": round(nbytes / MALL_BYTES, 2)}


# ------------------------------------------------------------------ INT4
def build_int4_layers(torch):
    from fastllm_py.moe import quantize_marlin_matrix_device

    gen = torch.Generator(device="cuda")
    gen.manual_seed(2000)
    base = {}
    for name, N, K in QWEN3_8B:
        W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        base[name] = quantize_marlin_matrix_device(W, GS)
        del W
    # enough copies that even the smallest matrix (o) cycles through > 2.2x MALL
    n = max(copies_for(marlin_bytes(0, N, K)) for _, N, K in QWEN3_8B)
    layers = [base] + [{k: {f: v.clone() for f, v in p.items()} for k, p in base.items()}
                       for _ in range(n - 1)]
    torch.cuda.synchronize()
    return layers


def run_int4(torch, lib, layers, M, steps, stream):
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2001 + M)
    xs = {K: torch.randn((M, K), generator=gen, device="cuda").to(torch.float16)
          for K in {k for _, _, k in QWEN3_8B}}
    outs = {name: torch.empty((M, N), dtype=torch.float16, device="cuda")
            for name, N, _ in QWEN3_8B}
    # the Python layer's entry (marlin.gemm_fast): above four rows the GEMV
    # splits K, its partials in a zeroed workspace per call site (one per
    # shape here: launches on one stream never overlap)
    wsb = {name: lib.fastllm_int4_gemm_ws_bytes(M, N, K, GS) for name, N, K in QWEN3_8B}
    wss = {name: torch.zeros(max(b, 1), dtype=torch.uint8, device="cuda") for name, b in wsb.items()}
    fn = lib.fastllm_int4_gemm_ws

    def launcher(layer, name, N, K):
        p = layer[name]
        args = (xs[K].data_ptr(), p["qweight"].data_ptr(), p["scales"].data_ptr(),
                p["zeros"].data_ptr(), outs[name].data_ptr(), M, N, K, GS,
                wss[name].data_ptr(), wsb[name], None)

        def go(h):
            if fn(*args, h) != 0:
                raise RuntimeError(f"INT4 GEMM rejected M={M} N={N} K={K}")
        return go

    L = len(layers)
    # the timed region: exactly `steps` layer-steps (step i on layer copy
    # i mod L), one replay of a graph that holds them
    seq = [launcher(layers[i % L], n, N, K) for i in range(steps) for n, N, K in QWEN3_8B]
    ms_step = graph_time(torch, stream, seq, 1) / steps
    per = {}
    r1 = max(1, -(-96 // L))
    for name, N, K in QWEN3_8B:
        seq1 = [launcher(layers[c], name, N, K) for _ in range(r1) for c in range(L)]
        per[name] = graph_time(torch, stream, seq1, 4) / (r1 * L) * 1e3
    cyc = {name: cycle(L * marlin_bytes(0, N, K)) for name, N, K in QWEN3_8B}
    cyc["layer"] = cycle(min(steps, L) * sum(marlin_bytes(0, N, K) for _, N, K in QWEN3_8B))
    return ms_step, per, steps, cyc


def run_swiglu(torch, lib, layers, stream, M_list=(1, 8)):
    """gate_up 24576x4096 with the SwiGLU epilogue in one launch
    (fastllm_int4_gemm_swiglu), beside the gate_up GEMV alone -- the unfused
    pair costs that plus a separate swiglu kernel launch."""
    N, K = 24576, 4096
    res = {}
    for M in M_list:
        x = torch.randn((M, K), device="cuda").to(torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")
        hbuf = torch.empty((M, N // 2), dtype=torch.float16, device="cuda")

        def fused(p):
            args = (x.data_ptr(), p["qweight"].data_ptr(), p["scales"].data_ptr(),
                    p["zeros"].data_ptr(), hbuf.data_ptr(), M, N, K, GS)

            def go(h):
                if lib.fastllm_int4_gemm_swiglu(*args, h) != 0:
                    raise RuntimeError("swiglu GEMV rejected")
            return go

        def gemv(p):
            args = (x.data_ptr(), p["qweight"].data_ptr(), p["scales"].data_ptr(),
                    p["zeros"].data_ptr(), y.data_ptr(), M, N, K, GS, None)

            def go(h):
                if not lib.FastllmCudaMarlinHalfInt4GemmStream(*args, h):
                    raise RuntimeError("INT4 GEMM rejected")
            return go
        L = len(layers)
        r1 = max(1, -(-48 // L))
        tf = graph_time(torch, stream, [fused(layers[c]["gate_up"]) for _ in range(r1)
                                        for c in range(L)], 4) / (r1 * L) * 1e3
        tg = graph_time(torch, stream, [gemv(layers[c]["gate_up"]) for _ in range(r1)
                                        for c in range(L)], 4) / (r1 * L) * 1e3
        res[f"M{M}"] = {"fused_us": round(tf, 3), "gemv_alone_us": round(tg, 3)}
    res.update(cycle(len(layers) * marlin_bytes(0, N, K)))
    return res


def run_layer_chain(torch, lib, layers, stream):
    """One Qwen3-8B decoder layer's quantized-matmul chain at M=1, captured in
    a HIP graph as the reference's GraphDecoder segment does
    (graph_decode.py:782-874; attention itself is outside this library): the
    input add_rmsnorm, qkv, o (on the q slice of qkv, the attention
    stand-in), the post-attention add_rmsnorm, gate_up with the SwiGLU
    epilogue and down -- six launches per layer, rotating over the layer
    copies.  Reported per layer."""
    H, NQKV, I = 4096, 6144, 12288
    f32, f16 = torch.float32, torch.float16
    z = lambda n, dt: torch.zeros(n, dtype=dt, device="cuda")  # noqa: E731
    x, pend = torch.randn(H, device="cuda"), (torch.randn(H, device="cuda") * 0.5).to(f16)
    ln1, ln2 = (1 + 0.1 * torch.randn(H, device="cuda")).to(f16), (1 + 0.1 * torch.randn(H, device="cuda")).to(f16)
    xn1, h1, qkv, o, xn2, h2 = z(H, f32), z(H, f16), z(NQKV, f16), z(H, f16), z(H, f32), z(H, f16)
    hh, out = z(I, f16), z(H, f16)
    P = lambda t: t.data_ptr()  # noqa: E731

    def chain(L):
        def go(h):
            ok = lib.fastllm_add_rmsnorm(P(x), 1, P(pend), 0, P(ln1), 0, P(xn1), P(h1), 1, H, 1e-6, h) == 0
            for a, name, c, n, k in ((h1, "qkv", qkv, NQKV, H), (qkv, "o", o, H, H)):
                p = L[name]
                ok &= bool(lib.FastllmCudaMarlinHalfInt4GemmStream(
                    P(a), P(p["qweight"]), P(p["scales"]), P(p["zeros"]), P(c), 1, n, k, GS, None, h))
            ok &= lib.fastllm_add_rmsnorm(P(xn1), 1, P(o), 0, P(ln2), 0, P(xn2), P(h2), 1, H, 1e-6, h) == 0
            p = L["gate_up"]
            ok &= lib.fastllm_int4_gemm_swiglu(P(h2), P(p["qweight"]), P(p["scales"]), P(p["zeros"]),
                                               P(hh), 1, 2 * I, H, GS, h) == 0
            p = L["down"]
            ok &= bool(lib.FastllmCudaMarlinHalfInt4GemmStream(
                P(hh), P(p["qweight"]), P(p["scales"]), P(p["zeros"]), P(out), 1, H, I, GS, None, h))
            if not ok:
                raise RuntimeError("layer chain launch rejected")
        return go

    def fused(L):
        # add_rmsnorm in the prologues of qkv and of gate_up + SwiGLU: 4 launches
        def go(h):
            p = L["qkv"]
            ok = lib.fastllm_int4_gemm_add_rmsnorm(P(x), P(pend), P(ln1), 1e-6, P(xn1), P(p["qweight"]),
                                                   P(p["scales"]), P(p["zeros"]), P(qkv), NQKV, H, GS, 0,
                                                   h) == 0
            p = L["o"]
            ok &= bool(lib.FastllmCudaMarlinHalfInt4GemmStream(
                P(qkv), P(p["qweight"]), P(p["scales"]), P(p["zeros"]), P(o), 1, H, H, GS, None, h))
            p = L["gate_up"]
            ok &= lib.fastllm_int4_gemm_add_rmsnorm(P(xn1), P(o), P(ln2), 1e-6, P(xn2), P(p["qweight"]),
                                                    P(p["scales"]), P(p["zeros"]), P(hh), 2 * I, H, GS, 1,
                                                    h) == 0
            p = L["down"]
            ok &= bool(lib.FastllmCudaMarlinHalfInt4GemmStream(
                P(hh), P(p["qweight"]), P(p["scales"]), P(p["zeros"]), P(out), 1, H, I, GS, None, h))
            if not ok:
                raise RuntimeError("fused layer chain launch rejected")
        return go

    n = len(layers)
    reps = max(1, -(-24 // n))
    nb = sum(marlin_bytes(0, N, K) for _, N, K in QWEN3_8B)
    res = {}
    for name, fn, nl in (("separate_norms", chain, 6), ("norms_in_prologues", fused, 4)):
        ms = graph_time(torch, stream, [fn(layers[c]) for _ in range(reps) for c in range(n)], 4)
        us = ms / (reps * n) * 1e3
        res[name] = {"us_per_layer": round(us, 3), "launches_per_layer": nl,
                     "weight_GB/s": round(nb / us / 1e3, 1),
                     "pct_of_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS * 100, 2)}
    res.update(cycle(n * nb))
    return res


def run_int4_group(torch, lib, stream, M_list=(1,), N=3072, K=1024, gs=128):
    """Config 1: the INT4 GEMV on quantize_int4_group's format (u8 nibbles,
    fp32 scale and minimum per 128-group), 3072x1024, fp16 x -> fp32 y,
    rotated over copies (1.77 MB each) past 2.2x MALL."""
    from fastllm_py import quantizer

    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    qt = quantizer.quantize_int4_group(W, gs)
    del W
    wb = N * K // 2 + 2 * N * (K // gs) * 4
    n = copies_for(wb)
    cps = [(qt.data, qt.scales, qt.zeros)] + [(qt.data.clone(), qt.scales.clone(),
                                               qt.zeros.clone()) for _ in range(n - 1)]
    res = {}
    for M in M_list:
        x = torch.randn((M, K), generator=gen, device="cuda").to(torch.float16)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")

        def mk(d, sc, z, x=x, y=y, M=M):
            def go(h):
                if lib.fastllm_int4_group_gemv(x.data_ptr(), 0, d.data_ptr(), sc.data_ptr(),
                                               z.data_ptr(), y.data_ptr(), 1, M, N, K, gs, h):
                    raise RuntimeError("int4 group gemv failed")
            return go
        seq = [mk(*c) for c in cps]
        us = graph_time(torch, stream, seq, 3) / len(seq) * 1e3
        nb = wb + M * K * 2 + M * N * 4
        res[f"M{M}"] = {"us_per_call": round(us, 3), "bytes": nb, "GB/s": round(nb / us / 1e3, 1),
                        "pct_of_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS * 100, 2)}
    res.update(cycle(n * wb))
    del cps
    torch.cuda.empty_cache()
    return res


def rowmajor_bytes(M, N, K, gs=GS):
    return N * K // 2 + 2 * N * (K // gs) * 2 + M * K * 2 + M * N * 2


def run_rowmajor(torch, lib, stream, M=1):
    """The row-major INT4 GEMV (the reference's dgemv format: u8 nibbles, fp16
    scale and zero per group) at the Qwen3-8B shapes, fp16 in and out, each
    matrix rotated over copies past 2.2x MALL; per call and summed per layer."""
    from fastllm_py.kernels import moe_int4

    gen = torch.Generator(device="cuda")
    gen.manual_seed(2100)
    res, total_us, total_b = {}, 0.0, 0
    for name, N, K in QWEN3_8B:
        W = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
        qw, sc, ze, _ = moe_int4._quantize_int4_rowmajor_batched(W, GS)
        del W
        n = copies_for(rowmajor_bytes(0, N, K))
        cps = [(qw, sc, ze)] + [(qw.clone(), sc.clone(), ze.clone()) for _ in range(n - 1)]
        x = torch.randn((M, K), generator=gen, device="cuda").to(torch.float16)
        y = torch.empty((M, N), dtype=torch.float16, device="cuda")

        def mk(q, s_, z, x=x, y=y, N=N, K=K):
            def go(h):
                if lib.fastllm_int4_rowmajor_gemv(x.data_ptr(), 0, q.data_ptr(), s_.data_ptr(),
                                                  z.data_ptr(), y.data_ptr(), 0, M, N, K, GS, h):
                    raise RuntimeError("row-major gemv failed")
            return go
        seq = [mk(*c) for c in cps]
        us = graph_time(torch, stream, seq, 3) / len(seq) * 1e3
        nb = rowmajor_bytes(M, N, K)
        res[name] = {"us_per_call": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                     **cycle(n * rowmajor_bytes(0, N, K))}
        total_us += us
        total_b += nb
        del cps, qw, sc, ze
        torch.cuda.empty_cache()
    res["layer"] = {"M": M, "us": round(total_us, 3), "GB/s": round(total_b / total_us / 1e3, 1),
                    "pct_of_hbm_peak": round(total_b / total_us / 1e3 / HBM_PEAK_GBS * 100, 2)}
    return res


# ------------------------------------------------------------------- FP8
def run_fp8(torch, lib, stream, M_list=(1, 8)):
    from fastllm_py import quantizer

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3000)
    res = {}
    for name, N, K in FP8_SHAPES:
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        qt = quantizer.quantize_fp8_block(W, 128)
        del W
        n = copies_for(N * K)
        cps = [(qt.data, qt.scales)] + [(qt.data.clone(), qt.scales.clone()) for _ in range(n - 1)]
        for M in M_list:
            x = torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16)
            y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
            f = lib.fastllm_fp8_b128x128_gemv

            def mk(q, s, x=x, y=y, M=M):
                def go(h):
                    if f(x.data_ptr(), q.data_ptr(), s.data_ptr(), None, y.data_ptr(), M, N, K, 1, h):
                        raise RuntimeError("fp8 gemv failed")
                return go
            rounds = max(1, -(-96 // n))
            seq = [mk(q, s) for _ in range(rounds) for q, s in cps]
            us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
            nb = fp8_block_bytes(M, N, K)
            res[f"{name}/M{M}"] = {"us_per_call": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                   "bytes": nb, **cycle(n * fp8_block_bytes(0, N, K))}
        del cps, qt
        torch.cuda.empty_cache()
    for M in M_list:
        tb = sum(res[f"{n}/M{M}"]["bytes"] for n, _, _ in FP8_SHAPES)
        tt = sum(res[f"{n}/M{M}"]["us_per_call"] for n, _, _ in FP8_SHAPES)
        res[f"sum/M{M}"] = {"us": round(tt, 3), "GB/s": round(tb / tt / 1e3, 1),
                            "pct_of_hbm_peak": round(tb / tt / 1e3 / HBM_PEAK_GBS * 100, 2)}
    return res


def run_fp8_prefill(torch, lib, stream, M=512):
    """The config-3 shapes at prefill size (M=512, bf16): the FP8 MFMA GEMM,
    with its MFMA utilisation against the dense bf16 peak."""
    from fastllm_py import quantizer

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3100)
    res = {}
    for name, N, K in FP8_SHAPES:
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        qt = quantizer.quantize_fp8_block(W, 128)
        del W
        x = torch.randn((M, K), generator=gen, device="cuda").to(torch.bfloat16)
        y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        # the Python layer's entry (kernels.fp8.fp8_gemv_block): split-K for
        # grids under 256 tiles, partials in a zeroed workspace
        f = lib.fastllm_fp8_b128x128_gemm_ws
        wsb = lib.fastllm_fp8_b128x128_gemm_ws_bytes(M, N, K)
        ws = torch.zeros(max(wsb, 1), dtype=torch.uint8, device="cuda")
        n = copies_for(N * K)
        cps = [(qt.data, qt.scales)] + [(qt.data.clone(), qt.scales.clone()) for _ in range(n - 1)]

        def mk(q, s, x=x, y=y, N=N, K=K, ws=ws, wsb=wsb):
            def go(h):
                if f(x.data_ptr(), q.data_ptr(), s.data_ptr(), None, y.data_ptr(), M, N, K, 1,
                     ws.data_ptr(), wsb, h):
                    raise RuntimeError("fp8 gemm failed")
            return go
        seq = [mk(q, s) for q, s in cps]
        us = graph_time(torch, stream, seq, 3) / len(seq) * 1e3
        tf = 2.0 * M * N * K / us / 1e6
        res[f"{name}/M{M}"] = {"us_per_call": round(us, 3), "TFLOP/s": round(tf, 1),
                               "mfma_util_bf16_dense": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                               **cycle(n * fp8_block_bytes(0, N, K))}
        del qt, cps
        torch.cuda.empty_cache()
    return res


def run_fp8_inline(torch, lib, stream, M_list=(1, 8), shapes=(("2048x2048", 2048, 2048),
                                                               ("10944x2048", 10944, 2048))):
    """The reference ABI's own FP8 GEMV, fastllm_fp8_block128_gemv_fp16
    (native/fastllm_fp8_block128.cu:273-287): the inline 1x128 format (per row
    [128 e4m3][fp32 scale] x K/128, quantized by fastllm_fp8_block128_quantize),
    fp16 activations, at the configs[2] shapes the format takes (K % 128 == 0).
    Launched through its stream entry, which runs the same kernels, so it can
    be graph-timed (the reference's entry synchronizes after every call)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3100)
    res = {}
    for name, N, K in shapes:
        W = (torch.randn((N, K), generator=gen, device="cuda") * 0.02).half()
        per = lib.fastllm_fp8_block128_packed_row_bytes(K)
        q = torch.empty((N, per), dtype=torch.uint8, device="cuda")
        h0 = torch.cuda.current_stream().cuda_stream
        if lib.fastllm_fp8_block128_quantize_stream(W.data_ptr(), q.data_ptr(), N, K, 0, h0):
            raise RuntimeError("fp8 inline quantize failed")
        del W
        n = copies_for(N * per)
        cps = [q] + [q.clone() for _ in range(n - 1)]
        for M in M_list:
            x = torch.randn((M, K), generator=gen, device="cuda").half()
            y = torch.empty((M, N), dtype=torch.float16, device="cuda")
            f = lib.fastllm_fp8_block128_gemv_stream

            def mk(w, x=x, y=y, M=M):
                def go(h):
                    if f(x.data_ptr(), w.data_ptr(), y.data_ptr(), None, M, K, N, per, 0, h):
                        raise RuntimeError("fp8 inline gemv failed")
                return go
            rounds = max(1, -(-96 // n))
            seq = [mk(w) for _ in range(rounds) for w in cps]
            us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
            nb = N * per + M * K * 2 + M * N * 2
            res[f"{name}/M{M}"] = {"us_per_call": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                   "pct_of_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS * 100, 2),
                                   "bytes": nb, **cycle(n * N * per)}
        del cps, q
        torch.cuda.empty_cache()
    return res


def mxfp4_bytes(M, N, K):
    """Bytes one dense MXFP4 GEMV call moves: codes (N K / 2), E8M0 scale
    words (N K / 32), fp16 A and C."""
    return N * K // 2 + N * K // 32 + 2 * M * K + 2 * M * N


def run_mxfp4(torch, lib, stream, M_list=(1, 8, 16)):
    """Dense MXFP4 GEMV (fastllm_mxfp4_gemv) at the Qwen3-8B decode shapes,
    weights quantized on the GPU (OCP MXFP4) into the MoE tile layout and
    rotated through HBM; the per-call times and one layer's sum."""
    from fastllm_py.kernels import mxfp4

    gen = torch.Generator(device="cuda")
    gen.manual_seed(3200)
    res = {}
    layer = {M: 0.0 for M in M_list}
    layer_bytes = {M: 0 for M in M_list}
    for name, N, K in QWEN3_8B:
        W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
        base = mxfp4.quantize(W)
        del W
        wb = N * K // 2 + N * K // 32
        n = copies_for(wb)
        cps = [base] + [{"qtile": base["qtile"].clone(), "e8w": base["e8w"].clone(), "shape": base["shape"]}
                        for _ in range(n - 1)]
        for M in M_list:
            x = torch.randn((M, K), generator=gen, device="cuda").half()
            y = torch.empty((M, N), dtype=torch.float16, device="cuda")
            f = lib.fastllm_mxfp4_gemv

            def mk(w, x=x, y=y, M=M):
                def go(h):
                    if f(x.data_ptr(), w["qtile"].data_ptr(), w["e8w"].data_ptr(), y.data_ptr(), M, N, K, h):
                        raise RuntimeError("mxfp4 gemv failed")
                return go
            rounds = max(1, -(-96 // n))
            seq = [mk(w) for _ in range(rounds) for w in cps]
            us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
            nb = mxfp4_bytes(M, N, K)
            res[f"{name}/M{M}"] = {"us_per_call": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                   "pct_of_hbm_peak": round(nb / us / 1e3 / HBM_PEAK_GBS * 100, 2),
                                   "bytes": nb, **cycle(n * wb)}
            layer[M] += us
            layer_bytes[M] += nb
        del cps, base
        torch.cuda.empty_cache()
    for M in M_list:
        res[f"layer/M{M}"] = {"us": round(layer[M], 3), "GB/s": round(layer_bytes[M] / layer[M] / 1e3, 1),
                              "pct_of_hbm_peak": round(layer_bytes[M] / layer[M] / 1e3 / HBM_PEAK_GBS * 100, 2)}
    # the prefill GEMM (M > 64: mx4_gemm_mfma) at the dense INT4 GEMM's shape
    M, N, K = 512, 8192, 2048
    W = torch.randn((N, K), generator=gen, device="cuda") * 0.02
    base = mxfp4.quantize(W)
    del W
    wb = N * K // 2 + N * K // 32
    n = copies_for(wb)
    cps = [base] + [{"qtile": base["qtile"].clone(), "e8w": base["e8w"].clone(), "shape": base["shape"]}
                    for _ in range(n - 1)]
    x = torch.randn((M, K), generator=gen, device="cuda").half()
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")

    def mkp(w):
        def go(h):
            if lib.fastllm_mxfp4_gemv(x.data_ptr(), w["qtile"].data_ptr(), w["e8w"].data_ptr(), y.data_ptr(),
                                      M, N, K, h):
                raise RuntimeError("mxfp4 gemm failed")
        return go
    rounds = max(1, -(-64 // n))
    us = graph_time(torch, stream, [mkp(w) for _ in range(rounds) for w in cps], 4) / (rounds * n) * 1e3
    tf = 2.0 * M * N * K / (us * 1e-6) / 1e12
    res["prefill_gemm"] = {"shape": f"M{M} N{N} K{K}", "us_per_call": round(us, 3), "TFLOP/s": round(tf, 1),
                           "mfma_util_fp16_dense": round(tf / MFMA_F16_PEAK_TFLOPS, 4), **cycle(n * wb)}
    del cps, base
    torch.cuda.empty_cache()
    return res


def run_stream_probe(torch, lib, stream, sizes):
    """Per-launch floor of a streaming read of each byte count: the library's
    HBM read probe (fastllm_hbm_read_probe: every wave load a contiguous 1 KB,
    non-temporal, all loads issued before the first use, nothing computed or
    stored), graph-timed like the GEMVs, each launch at its own offset of a
    buffer larger than 2.2x the MALL so every launch reads HBM.  Best of 4, 8
    and 16 loads per lane.  `sizes`: name -> bytes."""
    big = max(sizes.values())
    stride_of = {k: -(-v // 4096) * 4096 for k, v in sizes.items()}
    buf_bytes = max(ROTATE_BYTES + big, 2 * big) + 4096
    buf = torch.empty(buf_bytes, dtype=torch.uint8, device="cuda")
    buf.random_(0, 256)
    sink = torch.zeros(1024, dtype=torch.int32, device="cuda")
    base = buf.data_ptr()
    res = {}
    for name, nb in sizes.items():
        nb16 = -(-nb // 16) * 16
        st = stride_of[name]
        slots = max(1, (buf_bytes - nb16) // st + 1)
        n = min(slots, max(copies_for(nb16), 2))
        offs = [i * st for i in range(n)]
        best = None
        for nl in (4, 8, 16):
            def mk(off, nl=nl):
                def go(h):
                    if lib.fastllm_hbm_read_probe(base + off, nb16, sink.data_ptr(), nl, h):
                        raise RuntimeError("hbm read probe failed")
                return go
            rounds = max(1, -(-96 // n))
            seq = [mk(o) for _ in range(rounds) for o in offs]
            us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
            if best is None or us < best[0]:
                best = (us, nl)
        # the same reads ending in one dependent store per workgroup (as a
        # GEMV's workgroups end): the part of a GEMV's gap that any kernel
        # with outputs pays
        nl = best[1]
        seq = [(lambda off: (lambda h: lib.fastllm_hbm_read_probe(base + off, nb16, sink.data_ptr(),
                                                                   nl | 64, h)))(o)
               for _ in range(max(1, -(-96 // n))) for o in offs]
        us_st = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
        res[name] = {"bytes": int(nb16), "us_per_launch": round(best[0], 3),
                     "GB/s": round(nb16 / best[0] / 1e3, 1),
                     "pct_of_hbm_peak": round(nb16 / best[0] / 1e3 / HBM_PEAK_GBS * 100, 2),
                     "loads_per_lane": best[1], "us_per_launch_with_store": round(us_st, 3),
                     **cycle(n * nb16)}
    del buf, sink
    torch.cuda.empty_cache()
    return res


# ------------------------------------------------------------------- MoE
# Decode MoE layers: Qwen1.5-MoE-A2.7B and the
# Qwen3-30B-A3B layer of the reference's only published fused-MoE latency
# (fused_moe_weighted, 36 us/layer at M=1 on an RTX 5090,
# fastllm_py/kernels/moe_int4.py:179).
MOE_SHAPES = {
    "qwen15_a27b": {"E": 60, "hidden": 2048, "inter": 1408, "sinter": 5632, "K": 4, "norm": False},
    "qwen3_30b_a3b": {"E": 128, "hidden": 2048, "inter": 768, "sinter": 0, "K": 8, "norm": True},
}


def moe_weight_bytes(fmt, out_f, in_f):
    """Packed bytes of one (out, in) expert matrix: INT4 g128 (nibbles + fp16
    scale and zero per group), FP8 (codes + fp32 per 128x128 block), MXFP4
    (nibbles + one E8M0 byte per 32)."""
    n = out_f * in_f
    return {"int4": n // 2 + n // 128 * 4, "fp8": n + n // (128 * 128) * 4,
            "mxfp4": n // 2 + n // 32}[fmt]


def run_moe(torch, lib, stream, T_list=(1, 16), fmt="int4", shape="qwen15_a27b", deterministic=False):
    """Fused decode MoE layer with `fmt` expert weights (INT4 g128, FP8
    128x128-block e4m3 or MXFP4) at MOE_SHAPES[shape]: router from fp16
    logits ~ N(0,1) (top-K softmax; Qwen1.5: no renorm, plus the shared
    expert with its sigmoid gate; Qwen3-30B-A3B: renormalised top-8, no shared
    expert) + routed experts.  Timed unit = one layer: every launch of
    moe_route_forward (router, gate/up, down; with ``deterministic`` also
    the ordered combine)."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    sp = MOE_SHAPES[shape]
    E, hidden, inter, sinter, K, norm = (sp[k] for k in ("E", "hidden", "inter", "sinter", "K", "norm"))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4000 if shape == "qwen15_a27b" else 4100)

    def stacked(d, proj, n, out_f, in_f):
        w = (torch.randn((n, out_f, in_f), generator=gen, device="cuda") * 0.02).half()
        if fmt == "int4":
            qw, sc, ze, _ = moe_int4._quantize_int4_rowmajor_batched(w, 128)
            d.update(moe_int4.stack_tiles(proj, qw, sc, ze, 128))
        else:
            d.update(moe_int4.stack_lowp(fmt, proj, w.float()))

    def layer():
        meta = {"group": 128} if fmt == "int4" else {"group": moe_int4.LOWP_FORMATS[fmt][1],
                                                     "format": fmt}
        st, sh = dict(meta), (dict(meta) if sinter else None)
        for d, n, inn in ((st, E, inter), (sh, 1, sinter)):
            if d is None:
                continue
            for proj, (o, i) in (("gate", (inn, hidden)), ("up", (inn, hidden)),
                                 ("down", (hidden, inn))):
                stacked(d, proj, n, o, i)
        return st, sh
    expert_bytes = 3 * moe_weight_bytes(fmt, inter, hidden)
    shared_bytes = 3 * moe_weight_bytes(fmt, sinter, hidden) if sinter else 0
    # layer copies: one token's routed set + the shared expert, over 2.2x MALL
    nl = copies_for(K * expert_bytes + shared_bytes)
    layers = [layer() for _ in range(nl)]
    res = {}
    for T in T_list:
        # every launch of the cycle routes its own logits (tokens differ per
        # layer and step), so consecutive launches touch different experts
        rounds = max(1, -(-48 // nl))
        n_ent = rounds * nl
        logits = torch.randn((n_ent, T, E), generator=gen, device="cuda").half().float()
        xs = torch.randn((n_ent, T, hidden), generator=gen, device="cuda").half().float()
        slog = torch.randn((n_ent, T), generator=gen, device="cuda") if sinter else None
        bufs = {}
        touched, per_layer = set(), []
        for i in range(n_ent):
            route_topk_device(logits[i], K, norm_topk_prob=norm,
                              shared_logit=slog[i] if sinter else None, out=bufs)
            ids = np.unique(bufs["topk_ids"].cpu().numpy())
            per_layer.append(len(ids) * expert_bytes + shared_bytes)
            touched.update((i % nl, int(e)) for e in ids)
        y = torch.empty((T, hidden), device="cuda")
        ws = torch.empty((moe_int4.moe_workspace_bytes(T, hidden, inter, sinter, T * K,
                                                       deterministic),),
                         dtype=torch.uint8, device="cuda")

        def mk(i, st, sh, bufs=bufs, y=y, ws=ws, T=T):
            def go(h):
                moe_int4.moe_route_forward(xs[i], logits[i], st, K, E, hidden, inter,
                                           norm_topk_prob=norm, shared=sh, shared_inter=sinter,
                                           shared_logit=slog[i] if sinter else None, route=bufs,
                                           out=y, workspace=ws, stream=h,
                                           deterministic=deterministic)
            return go
        seq = [mk(i, *layers[i % nl]) for i in range(n_ent)]
        us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
        routed = float(np.mean(per_layer))
        res[f"T{T}"] = {"us_per_layer": round(us, 3),
                        "distinct_experts_mean": round((routed - shared_bytes) / expert_bytes, 2),
                        "routed_weight_bytes_mean": int(routed),
                        "roofline_us": round(routed / HBM_PEAK_GBS / 1e3, 3),
                        "frac_of_roofline": round(routed / HBM_PEAK_GBS / 1e3 / us, 4),
                        "launch_cycle": f"{n_ent} layers: {nl} weight copies x {rounds} logits sets",
                        **cycle(len(touched) * expert_bytes + nl * shared_bytes)}
    del layers
    torch.cuda.empty_cache()
    return res


# ----------------------------------------------------------- prefill GEMM
MFMA_F16_PEAK_TFLOPS = 2500.0


def run_gemm_prefill(torch, lib, stream, M=512, N=8192, K=2048):
    """Config 5's dense INT4 GEMM on the matrix cores: M=512 fp16 rows against an
    8192x2048 INT4 g128 Marlin-format weight (rotated through HBM)."""
    from fastllm_py.moe import quantize_marlin_matrix_device

    gen = torch.Generator(device="cuda")
    gen.manual_seed(5000)
    W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
    base = quantize_marlin_matrix_device(W, GS)
    del W
    n = copies_for(marlin_bytes(0, N, K))
    cps = [base] + [{f: v.clone() for f, v in base.items()} for _ in range(n - 1)]
    x = torch.randn((M, K), generator=gen, device="cuda").to(torch.float16)
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    fn = lib.FastllmCudaMarlinHalfInt4GemmStream

    def mk(p):
        args = (x.data_ptr(), p["qweight"].data_ptr(), p["scales"].data_ptr(),
                p["zeros"].data_ptr(), y.data_ptr(), M, N, K, GS, None)

        def go(h):
            if not fn(*args, h):
                raise RuntimeError("INT4 GEMM rejected")
        return go
    rounds = max(1, -(-64 // n))
    seq = [mk(p) for _ in range(rounds) for p in cps]
    us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
    flops = 2.0 * M * N * K
    tflops = flops / (us * 1e-6) / 1e12
    del cps
    torch.cuda.empty_cache()
    return {"shape": f"M{M} N{N} K{K}", "us_per_call": round(us, 3), "TFLOP/s": round(tflops, 1),
            "mfma_util_fp16_dense": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "weight_GB/s": round(marlin_bytes(M, N, K) / us / 1e3, 1),
            **cycle(n * marlin_bytes(0, N, K))}


def run_moe_prefill(torch, lib, stream, T=512, fmt="int4", deterministic=False, routed=True):
    """Config 5's grouped MoE layer (Qwen3-30B-A3B): 128 experts, hidden 2048,
    inter 768, top-8 softmax with renormalisation from fp16 logits ~ N(0,1),
    M=512 tokens, `fmt` expert weights.  Timed unit = one layer: router +
    gate/up + down launches (``routed``: moe_route_forward, one native call
    whose router also builds the lists and the fp16 copy of x; else
    route_topk_device + moe_forward, five launches); HBM-bound on the routed
    experts' packed weights."""
    from fastllm_py.expert_router import route_topk_device
    from fastllm_py.kernels import moe_int4

    E, hidden, inter, K = 128, 2048, 768, 8
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5100)

    def layer():
        st = {"group": 128} if fmt == "int4" else {"group": moe_int4.LOWP_FORMATS[fmt][1],
                                                   "format": fmt}
        for proj, (o, i) in (("gate", (inter, hidden)), ("up", (inter, hidden)),
                             ("down", (hidden, inter))):
            w = (torch.randn((E, o, i), generator=gen, device="cuda") * 0.02).half()
            if fmt == "int4":
                qw, sc, ze, _ = moe_int4._quantize_int4_rowmajor_batched(w, 128)
                st.update(moe_int4.stack_tiles(proj, qw, sc, ze, 128))
            else:
                st.update(moe_int4.stack_lowp(fmt, proj, w.float()))
            del w
        return st
    expert_bytes = moe_weight_bytes(fmt, inter, hidden) * 2 + moe_weight_bytes(fmt, hidden, inter)
    nl = copies_for(E * expert_bytes)
    layers = [layer() for _ in range(nl)]
    logits = torch.randn((T, E), generator=gen, device="cuda").half().float()
    x = torch.randn((T, hidden), generator=gen, device="cuda").half().float()
    bufs = {}
    route_topk_device(logits, K, norm_topk_prob=True, out=bufs)
    torch.cuda.synchronize()
    distinct = len(np.unique(bufs["topk_ids"].cpu().numpy()))
    y = torch.empty((T, hidden), device="cuda")
    ws = torch.zeros((moe_int4.moe_workspace_bytes(T, hidden, inter, 0, T * K, deterministic),),
                     dtype=torch.uint8, device="cuda")  # zero-filled: the router's counter

    def mk(st):
        def go(h):
            if routed:
                moe_int4.moe_route_forward(x, logits, st, K, E, hidden, inter, norm_topk_prob=True,
                                           route=bufs, out=y, workspace=ws, stream=h,
                                           deterministic=deterministic)
                return
            route_topk_device(logits, K, norm_topk_prob=True, out=bufs, stream=h)
            moe_int4.moe_forward(x, st, E, hidden, inter, bufs, max_slots=E, max_entries=T * K,
                                 out=y, workspace=ws, stream=h, deterministic=deterministic)
        return go
    rounds = max(1, -(-16 // nl))
    seq = [mk(st) for _ in range(rounds) for st in layers]
    us = graph_time(torch, stream, seq, 4) / len(seq) * 1e3
    routed = distinct * expert_bytes
    flops = 2.0 * T * K * 3 * inter * hidden
    del layers
    torch.cuda.empty_cache()
    return {"T": T, "us_per_layer": round(us, 3), "distinct_experts": distinct,
            "entry": "moe_route_forward" if routed else "route_topk_device + moe_forward",
            "routed_weight_bytes": routed, "weight_GB/s": round(routed / us / 1e3, 1),
            "pct_of_hbm_peak": round(routed / us / 1e3 / HBM_PEAK_GBS * 100, 2),
            "TFLOP/s": round(flops / (us * 1e-6) / 1e12, 1), **cycle(nl * routed)}


# ------------------------------------------------------------- CPU baseline
def host_info():
    """CPU model, core count and the numpy BLAS build the baselines ran on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas, threads = "unknown", None
    try:
        import threadpoolctl

        for lib_ in threadpoolctl.threadpool_info():
            if lib_.get("user_api") == "blas":
                threads = lib_.get("num_threads")
                blas = (f"{lib_.get('internal_api')} {lib_.get('version')} "
                        f"({lib_.get('architecture')}, {threads} threads)")
                break
    except Exception:  # threadpoolctl missing: report the build only
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "numpy": np.__version__,
            "blas": blas, "blas_threads": threads}


def time_median(fn, warmups=3, runs=20):
    """3 warm-ups, then the median of `runs` timed calls (seconds)."""
    for _ in range(warmups):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _figures(name, nbytes, fn_i, fn_ii, info, sample, scale=1.0):
    """Figure (i) dequantize-then-matmul and (ii) the matmul on pre-dequantized
    fp32 weights, each 3 warm-ups + median of 20, times `scale` (a sample of
    the unit's work scaled to the whole unit)."""
    t1 = time_median(fn_i) * scale
    t2 = time_median(fn_ii) * scale
    return {"value": round(nbytes / t1 / 1e9, 4), "unit": "GB/s", "us": round(t1 * 1e6, 1),
            "blas_floor": {"us": round(t2 * 1e6, 1), "GB/s": round(nbytes / t2 / 1e9, 3)},
            "cores": info["blas_threads"] or os.cpu_count(), "kind": "port",
            "sample": f"{name}; {sample}; numpy oracle, 3 warm-ups + median of 20; "
                      f"(i) dequantize-then-fp32 matmul per call (elementwise numpy on 1 thread, "
                      f"BLAS on {info['blas_threads']}), blas_floor = (ii) fp32 matmul on "
                      f"pre-dequantized weights; {info['cpu_model']}, {info['blas']}"}


def cpu_baseline_int4(info):
    """Config 2 at M=1 (one Qwen3-8B layer, 4 GEMVs) on the Marlin-format
    weights: the headline's CPU baseline."""
    from oracle import quant as Q

    rng = np.random.default_rng(3000)
    layer = []
    for name, N, K in QWEN3_8B:
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        q, s, z = Q.quantize_int4_marlin(W, GS)
        s16, zp = Q.marlin_scales_zeros(s, z)
        layer.append((N, K, q, s16, zp))
        del W
    x = {K: rng.standard_normal((1, K)).astype(np.float16).astype(np.float32)
         for K in {k for _, _, k in QWEN3_8B}}
    hats = [Q.marlin_dequant(q, s16, zp, GS) for _, _, q, s16, zp in layer]

    def fi():
        for N, K, q, s16, zp in layer:
            Q.matmul_ref(x[K], Q.marlin_dequant(q, s16, zp, GS))

    def fii():
        for (N, K, *_), w in zip(layer, hats):
            Q.matmul_ref(x[K], w)
    nbytes = sum(marlin_bytes(1, N, K) for _, N, K in QWEN3_8B)
    r = _figures("config 2: one Qwen3-8B layer (qkv, o, gate_up, down) at M=1, Marlin format",
                 nbytes, fi, fii, info, "unit = one layer")
    r["us_per_layer"] = r.pop("us")
    return r


def cpu_baseline_int4_group(info, N=3072, K=1024, gs=128):
    """Config 1 on the host: dequantize_int4_group then the fp32 GEMV."""
    from oracle import quant as Q

    rng = np.random.default_rng(0)
    W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, K)).astype(np.float16).astype(np.float32)
    p, sc, z = Q.quantize_int4_group(W, gs)
    w = Q.dequantize_int4_group(p, sc, z, gs)
    nbytes = N * K // 2 + 2 * N * (K // gs) * 4 + K * 2 + N * 4
    return _figures("config 1: 3072x1024 int4_group GEMV at M=1", nbytes,
                    lambda: Q.matmul_ref(x, Q.dequantize_int4_group(p, sc, z, gs)),
                    lambda: Q.matmul_ref(x, w), info, "unit = one call")


def cpu_baseline_fp8(info):
    """Config 3 at M=1 on the host: the three 128x128-block e4m3 shapes, summed."""
    from oracle import quant as Q

    rng = np.random.default_rng(3100)
    mats = []
    for _, N, K in FP8_SHAPES:
        W = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        q, sc = Q.quantize_fp8_block(W, 128)
        mats.append((q, sc, rng.standard_normal((1, K)).astype(np.float32),
                     Q.dequantize_fp8_block(q, sc, 128)))
        del W
    nbytes = sum(fp8_block_bytes(1, N, K) for _, N, K in FP8_SHAPES)

    def fi():
        for q, sc, x, _ in mats:
            Q.matmul_ref(x, Q.dequantize_fp8_block(q, sc, 128))

    def fii():
        for _, _, x, w in mats:
            Q.matmul_ref(x, w)
    return _figures("config 3: the 3 FP8 128x128-block shapes at M=1, summed", nbytes, fi, fii,
                    info, "unit = the sum of the three calls")


def _moe_expert(rng, hidden, n_inter, n_exp=1):
    from oracle import quant as Q

    d = {}
    for p, shp in (("gate", (n_inter, hidden)), ("up", (n_inter, hidden)),
                   ("down", (hidden, n_inter))):
        w = (rng.standard_normal((n_exp,) + shp) * 0.02).astype(np.float16).astype(np.float32)
        d.update(zip((f"{p}.qweight", f"{p}.scales", f"{p}.zeros"),
                     Q.quantize_int4_rowmajor(w, 128)))
    return d


def cpu_baseline_moe(info):
    """Config 4 at T=1 on the host, the reference's CPU semantics
    (fastllm_py/moe.py:161-175): route_topk, then per routed expert and for
    the shared expert dequantize the row-major INT4 weights to fp32 and run
    the FFN.  The four routed experts are built once and stand for whichever
    the router picks (the cost does not depend on which)."""
    from oracle import moe as OM
    from oracle import router as R

    E, hidden, inter, sinter, K = 60, 2048, 1408, 5632, 4
    rng = np.random.default_rng(3200)
    routed = [_moe_expert(rng, hidden, inter) for _ in range(K)]
    shared = _moe_expert(rng, hidden, sinter)
    x = rng.standard_normal((1, hidden)).astype(np.float16).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float16).astype(np.float32)
    deq = [OM.dequant_stacked(d, 128) for d in routed + [shared]]

    def run(dequantize):
        _, idx, w = R.route_topk(logits, K, return_arrays=True)
        y = np.zeros((1, hidden), np.float32)
        for j, d in enumerate(routed + [shared]):
            dd = OM.dequant_stacked(d, 128) if dequantize else deq[j]
            c = w[0, j] if j < K else 1.0
            y += c * OM.expert_ffn(x, dd["gate"][0], dd["up"][0], dd["down"][0])
        return y
    expert_bytes = 3 * inter * hidden // 2 + 3 * inter * hidden // 128 * 4
    shared_bytes = 3 * sinter * hidden // 2 + 3 * sinter * hidden // 128 * 4
    r = _figures("config 4: Qwen1.5-MoE layer at T=1 (route_topk + 4 routed experts + shared)",
                 K * expert_bytes + shared_bytes, lambda: run(True), lambda: run(False), info,
                 "unit = one layer")
    r["us_per_layer_T1"] = r.pop("us")
    return r


def cpu_baseline_moe_prefill(info, T=512, n_sample=16):
    """Config 5's grouped MoE layer on the host (Qwen3-30B-A3B, T=512, top-8
    of 128 with renormalisation): route_topk over all 512 tokens, then the
    expert-grouped FFN (fastllm_py/moe.py:135-175) of `n_sample` experts with
    their routed tokens, scaled by 128 / n_sample to the whole layer."""
    from oracle import moe as OM
    from oracle import router as R

    E, hidden, inter, K = 128, 2048, 768, 8
    rng = np.random.default_rng(3300)
    logits = rng.standard_normal((T, E)).astype(np.float16).astype(np.float32)
    x = rng.standard_normal((T, hidden)).astype(np.float16).astype(np.float32)
    _, idx, w = R.route_topk(logits, K, norm_topk_prob=True, return_arrays=True)
    experts = [_moe_expert(rng, hidden, inter) for _ in range(n_sample)]
    deq = [OM.dequant_stacked(d, 128) for d in experts]
    rows = [np.nonzero(idx == e) for e in range(n_sample)]

    def run(dequantize):
        R.route_topk(logits, K, norm_topk_prob=True, return_arrays=True)
        y = np.zeros((T, hidden), np.float32)
        for e in range(n_sample):
            t_i, k_i = rows[e]
            if len(t_i) == 0:
                continue
            d = OM.dequant_stacked(experts[e], 128) if dequantize else deq[e]
            y[t_i] += w[t_i, k_i][:, None] * OM.expert_ffn(x[t_i], d["gate"][0], d["up"][0],
                                                           d["down"][0])
        return y
    expert_bytes = 3 * inter * hidden // 2 + 3 * inter * hidden // 128 * 4
    r = _figures(f"config 5: Qwen3-30B-A3B grouped MoE layer, T={T}", E * expert_bytes,
                 lambda: run(True), lambda: run(False), info,
                 f"unit = one layer, sampled as routing + {n_sample} of the 128 experts "
                 f"scaled x{E // n_sample}", scale=E / n_sample)
    r["us_per_layer"] = r.pop("us")
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ms", default="1,4,8,16")
    ap.add_argument("--only", default="int4,swiglu,layer,probe,group,rm,fp8,fp8i,fp8p,mx4,moe,moelp,"
                                      "moe30,moedet,gemm,moelpp")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first copy a 64 MiB buffer 5 times (a known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    WARMUP[0] = max(1, args.warmup)
    import torch

    from fastllm_py import _native as nat

    lib = nat.load()
    torch.cuda.init()
    stream = torch.cuda.Stream()
    if args.calib_copy:
        src = torch.ones(16 * 2 ** 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("calibration copy: 5 x 64 MiB (67108864 B read + written per launch)")
        del src, dst
    only = set(args.only.split(","))
    breakdown = {}

    ms_list = [int(m) for m in args.ms.split(",")]
    layers = build_int4_layers(torch)
    log(f"INT4: {len(layers)} Qwen3-8B layer copies")
    per_m = {}
    steps_run = args.steps
    cyc = {}
    for M in ms_list:
        ms_step, per, done, cyc = run_int4(torch, lib, layers, M, args.steps, stream)
        if M == ms_list[0]:
            steps_run = done
        nbytes = sum(marlin_bytes(M, N, K) for _, N, K in QWEN3_8B)
        gbs = nbytes / (ms_step * 1e-3) / 1e9
        per_m[M] = {"ms_per_layer": ms_step, "GB/s": gbs, "us_per_call": per}
        log(f"INT4 M={M}: {ms_step * 1e3:.2f} us/layer {gbs:.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s) per call "
            f"{ {k: round(v, 2) for k, v in per.items()} }")
    breakdown["int4_qwen3_8b"] = {
        str(m): {"GB/s": round(v["GB/s"], 1),
                 "pct_of_hbm_peak": round(v["GB/s"] / HBM_PEAK_GBS * 100, 2),
                 "us_per_layer": round(v["ms_per_layer"] * 1e3, 3),
                 "us_per_call": {k: round(u, 3) for k, u in v["us_per_call"].items()}}
        for m, v in per_m.items()}
    breakdown["int4_qwen3_8b"]["cycle"] = cyc
    if "swiglu" in only:
        breakdown["int4_gate_up_swiglu"] = run_swiglu(torch, lib, layers, stream)
    if "layer" in only:
        breakdown["int4_layer_chain_graph_M1"] = run_layer_chain(torch, lib, layers, stream)
        log(f"gate_up + SwiGLU: {breakdown['int4_gate_up_swiglu']}")
    del layers
    torch.cuda.empty_cache()

    if "group" in only:
        breakdown["int4_group_config1"] = run_int4_group(torch, lib, stream, M_list=(1, 16))
        log(f"config 1: {breakdown['int4_group_config1']}")
    if "rm" in only:
        breakdown["int4_rowmajor_dgemv_qwen3_8b_M1"] = run_rowmajor(torch, lib, stream)
        log(f"row-major: {breakdown['int4_rowmajor_dgemv_qwen3_8b_M1']}")
    if "gemm" in only:
        breakdown["int4_gemm_prefill"] = run_gemm_prefill(torch, lib, stream)
        log(f"GEMM: {breakdown['int4_gemm_prefill']}")
        breakdown["moe_prefill_qwen3_30b_a3b_int4"] = run_moe_prefill(torch, lib, stream)
        log(f"MoE prefill: {breakdown['moe_prefill_qwen3_30b_a3b_int4']}")
    if "moelpp" in only:
        for fmt in ("fp8", "mxfp4"):
            key = f"moe_prefill_qwen3_30b_a3b_{fmt}"
            breakdown[key] = run_moe_prefill(torch, lib, stream, fmt=fmt)
            log(f"MoE prefill {fmt}: {breakdown[key]}")
    if "fp8" in only:
        breakdown["fp8_b128x128_bf16"] = run_fp8(torch, lib, stream)
        log(f"FP8: {breakdown['fp8_b128x128_bf16']}")
    if "fp8p" in only:
        breakdown["fp8_prefill_gemm_M512"] = run_fp8_prefill(torch, lib, stream)
        log(f"FP8 prefill: {breakdown['fp8_prefill_gemm_M512']}")
    if "fp8i" in only:
        breakdown["fp8_inline_1x128_abi_fp16"] = run_fp8_inline(torch, lib, stream)
        log(f"FP8 inline ABI: {breakdown['fp8_inline_1x128_abi_fp16']}")
    if "mx4" in only:
        breakdown["mxfp4_gemv_qwen3_8b"] = run_mxfp4(torch, lib, stream)
        log(f"MXFP4 GEMV: {breakdown['mxfp4_gemv_qwen3_8b']}")
    if "moe" in only:
        breakdown["moe_qwen15_a27b_int4"] = run_moe(torch, lib, stream)
        log(f"MoE: {breakdown['moe_qwen15_a27b_int4']}")
    if "moelp" in only:
        for fmt in ("fp8", "mxfp4"):
            breakdown[f"moe_qwen15_a27b_{fmt}"] = run_moe(torch, lib, stream, fmt=fmt)
            log(f"MoE {fmt}: {breakdown[f'moe_qwen15_a27b_{fmt}']}")
    if "moedet" in only:
        # the ordered (bit-reproducible) combine, beside the atomic legs above
        key = "moe_qwen15_a27b_int4_deterministic"
        breakdown[key] = run_moe(torch, lib, stream, deterministic=True)
        log(f"MoE deterministic: {breakdown[key]}")
        key = "moe_prefill_qwen3_30b_a3b_int4_deterministic"
        breakdown[key] = run_moe_prefill(torch, lib, stream, deterministic=True)
        log(f"MoE prefill deterministic: {breakdown[key]}")
    if "moe30" in only:
        for fmt in ("int4", "fp8", "mxfp4"):
            key = f"moe_decode_qwen3_30b_a3b_{fmt}"
            breakdown[key] = run_moe(torch, lib, stream, T_list=(1,), fmt=fmt, shape="qwen3_30b_a3b")
            breakdown[key]["reference_published"] = {
                "us_per_layer": 36.0, "hardware": "RTX 5090", "kernel": "fused_moe_weighted, INT4 g128",
                "source": "fastllm_py/kernels/moe_int4.py:179"}
            log(f"MoE decode Qwen3-30B-A3B {fmt}: {breakdown[key]}")
    if "probe" in only:
        # the streaming-read floor at each decode GEMV's byte count, and the
        # GEMVs as a fraction of it
        sizes = {f"int4_{n}_M1": marlin_bytes(1, N, K) for n, N, K in QWEN3_8B}
        sizes.update({f"fp8_{n}_M1": fp8_block_bytes(1, N, K) for n, N, K in FP8_SHAPES})
        sizes.update({f"mxfp4_{n}_M1": mxfp4_bytes(1, N, K) for n, N, K in QWEN3_8B})
        sizes["peak_512MiB"] = 512 * 2 ** 20
        pr = run_stream_probe(torch, lib, stream, sizes)
        if 1 in per_m:
            for n, N, K in QWEN3_8B:
                g = per_m[1]["us_per_call"][n]
                pr[f"int4_{n}_M1"]["gemv_us"] = round(g, 3)
                pr[f"int4_{n}_M1"]["gemv_pct_of_probe"] = round(pr[f"int4_{n}_M1"]["us_per_launch"] / g * 100, 1)
                pr[f"int4_{n}_M1"]["gemv_minus_probe_us"] = round(g - pr[f"int4_{n}_M1"]["us_per_launch"], 3)
                pr[f"int4_{n}_M1"]["gemv_minus_probe_with_store_us"] = round(
                    g - pr[f"int4_{n}_M1"]["us_per_launch_with_store"], 3)
            lay = sum(pr[f"int4_{n}_M1"]["us_per_launch"] for n, _, _ in QWEN3_8B)
            pr["int4_layer_M1"] = {"probe_us": round(lay, 3),
                                   "probe_pct_of_hbm_peak": round(
                                       sum(marlin_bytes(1, N, K) for _, N, K in QWEN3_8B) / lay / 1e3
                                       / HBM_PEAK_GBS * 100, 2),
                                   "gemv_us": round(per_m[1]["ms_per_layer"] * 1e3, 3),
                                   "gemv_pct_of_probe": round(lay / (per_m[1]["ms_per_layer"] * 1e3) * 100, 1)}
        if "fp8_b128x128_bf16" in breakdown:
            for n, N, K in FP8_SHAPES:
                g = breakdown["fp8_b128x128_bf16"][f"{n}/M1"]["us_per_call"]
                pr[f"fp8_{n}_M1"]["gemv_us"] = g
                pr[f"fp8_{n}_M1"]["gemv_pct_of_probe"] = round(pr[f"fp8_{n}_M1"]["us_per_launch"] / g * 100, 1)
                pr[f"fp8_{n}_M1"]["gemv_minus_probe_us"] = round(g - pr[f"fp8_{n}_M1"]["us_per_launch"], 3)
                pr[f"fp8_{n}_M1"]["gemv_minus_probe_with_store_us"] = round(
                    g - pr[f"fp8_{n}_M1"]["us_per_launch_with_store"], 3)
        if "mxfp4_gemv_qwen3_8b" in breakdown:
            for n, N, K in QWEN3_8B:
                g = breakdown["mxfp4_gemv_qwen3_8b"][f"{n}/M1"]["us_per_call"]
                pr[f"mxfp4_{n}_M1"]["gemv_us"] = g
                pr[f"mxfp4_{n}_M1"]["gemv_pct_of_probe"] = round(pr[f"mxfp4_{n}_M1"]["us_per_launch"] / g * 100, 1)
                pr[f"mxfp4_{n}_M1"]["gemv_minus_probe_us"] = round(g - pr[f"mxfp4_{n}_M1"]["us_per_launch"], 3)
        breakdown["hbm_read_probe"] = pr
        log(f"HBM read probe: {pr}")

    head = per_m[ms_list[0]]
    M0 = ms_list[0]
    # roofline of the dominant kernel: the gate_up INT4 GEMV (24576x4096, 52% of
    # the layer's bytes) at the headline M, timed alone.
    bpl = marlin_bytes(M0, 24576, 4096)
    dur_us = head["us_per_call"]["gate_up"]
    achieved = bpl / (dur_us * 1e-6) / 1e9
    kname = "int4_gemv_nb<2,4,false,0>"
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": MEASURED_TRAFFIC.get((kname, M0)),
                "kernel": f"{kname} (gate_up 24576x4096, M={M0})",
                "bytes_per_launch": int(bpl), "us_per_launch": round(dur_us, 3),
                "us_per_launch_source": "HIP events around graph replays of >= 96 launches on "
                                        "the launch stream (this run)"}
    rp = ROCPROF_US.get((kname, M0))
    if rp is not None:
        roofline["us_per_launch_rocprof"] = rp[0]
        roofline["frac_rocprof"] = round(bpl / (rp[0] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
        roofline["rocprof_summary"] = rp[1]
    if "hbm_read_probe" in breakdown and M0 == 1:
        pg = breakdown["hbm_read_probe"]["int4_gate_up_M1"]
        roofline["stream_probe_us"] = pg["us_per_launch"]
        roofline["frac_of_stream_probe"] = round(pg["us_per_launch"] / dur_us, 4)

    cpu = None
    if not args.no_cpu_baseline:
        info = host_info()
        log(f"timing CPU baselines (numpy oracle) on {info}")
        cpu = cpu_baseline_int4(info)
        cpu["host"] = info
        log(f"CPU config 2: {cpu}")
        legs = (("int4_group_config1", cpu_baseline_int4_group),
                ("fp8_b128x128_bf16", cpu_baseline_fp8),
                ("moe_qwen15_a27b_int4", cpu_baseline_moe),
                ("moe_prefill_qwen3_30b_a3b_int4", cpu_baseline_moe_prefill))
        for key, fn in legs:
            if key in breakdown:
                breakdown[key]["cpu_baseline"] = fn(info)
                log(f"CPU {key}: {breakdown[key]['cpu_baseline']}")

    out = {
        "metric": "INT4/FP8 GEMV HBM GB/s (% of peak) at Qwen3-8B shapes; fused-MoE us/layer",
        "value": round(head["GB/s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_run,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_layer"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic: N(0,0.02) weights quantized by the product packers, N(0,1) activations",
        "config": {"workload": "Qwen3-8B decode linears (qkv/o/gate_up/down), INT4 g128 Marlin ABI, "
                               "one step = one layer's 4 GEMVs", "M": M0,
                   "pct_of_hbm_peak": round(head["GB/s"] / HBM_PEAK_GBS * 100, 2)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown": breakdown,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

"""Benchmark of the quantized-weight matmul path on one MI355X.

Workload: Qwen3-8B decode linears, INT4 group-128 in
the Marlin ABI format, fp16 activations ~ N(0,1), weights ~ N(0,0.02) before
quantization.  Shapes (N x K): qkv 6144x4096, o 4096x4096, gate+up 24576x4096,
down 4096x12288.  One step = the four GEMVs of one layer at batch M; layers
rotate over enough weight copies (> 2 x the 256 MB Infinity Cache) that every
step streams its weights from HBM.

value = INT4 GEMV HBM GB/s at M=1 over the layer's algorithmic bytes (packed
weights + scales + zeros + activations + outputs).  Per-M figures, the FP8 and
fused-MoE figures and the roofline/cpu_baseline objects ride on the same line.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
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
QWEN3_8B = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096),
            ("down", 4096, 12288)]
GS = 128
MALL_BYTES = 256 * 2 ** 20


def marlin_bytes(M, N, K, gs=GS):
    G = K // gs
    return N * K // 2 + G * N * 2 + G * N // 2 + M * K * 2 + M * N * 2


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ INT4 GPU
def build_int4_layers(torch, copies):
    """Quantize one random Qwen3-8B layer through the product packers and
    clone its packed tensors `copies` times (distinct HBM copies)."""
    from fastllm_py.moe import quantize_marlin_matrix_device

    gen = torch.Generator(device="cuda")
    gen.manual_seed(2000)
    base = {}
    for name, N, K in QWEN3_8B:
        W = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        base[name] = quantize_marlin_matrix_device(W, GS)
        del W
    layers = [base] + [{n: {k: v.clone() for k, v in p.items()} for n, p in base.items()}
                       for _ in range(copies - 1)]
    torch.cuda.synchronize()
    return layers


def _graph_time(torch, stream, launch_seq, reps, warmup):
    """Capture launch_seq() (a list of enqueue callbacks) in one HIP graph on
    `stream`, replay it warmup times, then time `reps` replays with HIP
    events on that stream.  Returns ms per replay."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        h = torch.cuda.current_stream().cuda_stream
        for fn in launch_seq:
            fn(h)
    for _ in range(max(1, warmup)):
        g.replay()
    stream.synchronize()
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


def run_int4(torch, lib, layers, M, steps, warmup, stream):
    """Time `steps` layer passes at batch M.  One HIP graph holds a pass over
    every layer copy (4 GEMVs each); replays are timed with HIP events on the
    launch stream.  Also times each shape alone (a graph of back-to-back
    launches over the copies) for per-call figures.
    Returns (ms_per_step, {shape: us_per_call})."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(2001 + M)
    xs = {K: torch.randn((M, K), generator=gen, device="cuda").to(torch.float16)
          for K in {k for _, _, k in QWEN3_8B}}
    outs = {name: torch.empty((M, N), dtype=torch.float16, device="cuda")
            for name, N, _ in QWEN3_8B}
    fn = lib.FastllmCudaMarlinHalfInt4GemmStream

    def launcher(layer, name, N, K):
        p = layer[name]
        args = (xs[K].data_ptr(), p["qweight"].data_ptr(), p["scales"].data_ptr(),
                p["zeros"].data_ptr(), outs[name].data_ptr(), M, N, K, GS, None)

        def go(h):
            if not fn(*args, h):
                raise RuntimeError(f"INT4 GEMM rejected M={M} N={N} K={K}")
        return go

    # every timed graph holds >= 96 launches so graph-launch cost is amortised
    L = len(layers)
    rounds = max(1, -(-24 // L))
    seq = [launcher(layers[c], name, N, K)
           for _ in range(rounds) for c in range(L) for name, N, K in QWEN3_8B]
    per_graph = rounds * L
    reps = max(1, -(-steps // per_graph))
    ms_step = _graph_time(torch, stream, seq, reps, max(1, warmup // per_graph)) / per_graph
    per = {}
    rounds1 = max(1, -(-96 // L))
    for name, N, K in QWEN3_8B:
        seq1 = [launcher(layers[c], name, N, K) for _ in range(rounds1) for c in range(L)]
        per[name] = _graph_time(torch, stream, seq1, max(2, reps // 4), 1) / (rounds1 * L)
    return ms_step, per, reps * per_graph


# ------------------------------------------------------------- CPU baseline
def cpu_baseline_int4(budget_s=15.0):
    """The reference's CPU semantics through the numpy oracle: per call,
    dequantize the packed Marlin-format weight to fp32, then the fp32 GEMV.
    Sample: the four Qwen3-8B GEMVs at M=1 (one layer) repeated until ~budget_s."""
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
    nbytes = sum(marlin_bytes(1, N, K) for _, N, K in QWEN3_8B)
    reps, t_total = 0, 0.0
    while t_total < budget_s and reps < 50:
        t0 = time.perf_counter()
        for N, K, q, s16, zp in layer:
            w_hat = Q.marlin_dequant(q, s16, zp, GS)
            _ = Q.matmul_ref(x[K], w_hat)
        t_total += time.perf_counter() - t0
        reps += 1
    us_per_layer = t_total / reps * 1e6
    return {
        "value": round(nbytes / (us_per_layer * 1e-6) / 1e9, 3),
        "unit": "GB/s",
        "us_per_layer": round(us_per_layer, 1),
        "cores": os.cpu_count(),
        "kind": "port",
        "sample": f"numpy dequantize-then-fp32-GEMV of one Qwen3-8B layer (4 GEMVs, M=1), "
                  f"{reps} reps, {t_total:.1f}s; BLAS threads = all host cores",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ms", default="1,4,8,16")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import torch

    from fastllm_py import _native as nat

    lib = nat.load()
    torch.cuda.init()
    layer_bytes_w = sum(marlin_bytes(0, N, K) for _, N, K in QWEN3_8B)
    copies = max(2, int(np.ceil(2.2 * MALL_BYTES / layer_bytes_w)))
    log(f"building {copies} INT4 Qwen3-8B layer copies ({copies * layer_bytes_w / 1e6:.0f} MB)")
    layers = build_int4_layers(torch, copies)
    stream = torch.cuda.Stream()

    per_m = {}
    ms_list = [int(m) for m in args.ms.split(",")]
    for M in ms_list:
        ms_step, per, steps_done = run_int4(torch, lib, layers, M, args.steps, args.warmup, stream)
        if M == ms_list[0]:
            steps_run = steps_done
        nbytes = sum(marlin_bytes(M, N, K) for _, N, K in QWEN3_8B)
        gbs = nbytes / (ms_step * 1e-3) / 1e9
        per_m[M] = {"ms_per_layer": ms_step, "GB/s": gbs,
                    "us_per_call": {k: round(v * 1e3, 3) for k, v in per.items()},
                    "bytes_per_layer": nbytes}
        log(f"INT4 M={M}: {ms_step * 1e3:.1f} us/layer  {gbs:.0f} GB/s "
            f"({gbs / HBM_PEAK_GBS * 100:.1f}% of 8 TB/s)  per call us: "
            f"{ {k: round(v * 1e3, 2) for k, v in per.items()} }")

    head = per_m[ms_list[0]]
    # roofline of the dominant kernel: the gate_up GEMV (24576x4096, 52% of the
    # layer's bytes) at the headline M, timed alone as a graph of back-to-back
    # launches over the rotating weight copies.
    M0 = ms_list[0]
    bytes_per_launch = marlin_bytes(M0, 24576, 4096)
    dur_us = head["us_per_call"]["gate_up"]
    achieved = bytes_per_launch / (dur_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "int4_gemv_nb<2,4,false,true> (gate_up 24576x4096, M=%d)" % M0,
                "bytes_per_launch": int(bytes_per_launch),
                "us_per_launch": round(dur_us, 3)}

    cpu = None
    if not args.no_cpu_baseline:
        log("timing CPU baseline (numpy oracle) ...")
        cpu = cpu_baseline_int4()

    out = {
        "metric": "INT4 GEMV HBM GB/s at Qwen3-8B decode shapes (M=1, summed per layer)",
        "value": round(head["GB/s"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_run,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_layer"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-w/fp16-a (fp32 accumulate)",
        "data": "synthetic (random N(0,0.02) weights quantized by the product packers, "
                "N(0,1) fp16 activations)",
        "config": {"workload": "Qwen3-8B decode linears qkv/o/gate_up/down, INT4 g128 Marlin ABI",
                   "M": M0, "layer_copies": copies, "pct_of_hbm_peak": round(head["GB/s"] / HBM_PEAK_GBS * 100, 2),
                   "int4_per_M": {str(m): {"GB/s": round(v["GB/s"], 1),
                                           "us_per_layer": round(v["ms_per_layer"] * 1e3, 2),
                                           "us_per_call": v["us_per_call"]}
                                  for m, v in per_m.items()}},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark: Phi-4-shaped batch-1 projection GEMVs (preq2 Q4, gs=32) on one MI355X.

One step = the four projection GEMVs of one Phi-4 decoder layer at batch 1,
each quantizing its fp32 activation to int8 inside the kernel as the
reference's gemv_preq2_fused_avx2 does:
    qkv 5120x3072, o_proj 3072x3072, gate_up 16384x3072, down 3072x8192.
Steps rotate over --layers distinct weight sets (default 16, ~1 GB) so that the
256 MB Infinity Cache cannot serve the weights: every step streams its
62.9 MB from HBM.  Inputs are resident in HBM before the timed region.

value = algorithmic bytes per step (packed weights + fp32 x + fp32 y) / step time.
roofline = the gate_up kernel (the largest GEMV), timed with HIP events on its
stream inside the timed region.  cpu_baseline = the reference's own
gemv_preq2_fused_avx2 (compiled from its sources into oracle/_ref) on one
layer's four GEMVs, on the host cores, for ~10 s.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path[:0] = [str(REPO / "asdsl-framework_amd")]

METRIC = "Q4 GEMV achieved HBM GB/s (% of peak); Phi-4-shape batch-1 decode tok/s"
HBM_PEAK_GBS = 8000.0
# (name, out_features M, in_features K)
LAYER = [("qkv", 5120, 3072), ("o_proj", 3072, 3072), ("gate_up", 16384, 3072), ("down", 3072, 8192)]
GS = 32


def gemv_bytes(M: int, K: int, gs: int = GS) -> int:
    G = K // gs
    return M * G * 4 + ((M + 3) // 4) * G * 4 * (gs // 2) + 4 * K + 4 * M


def build_layers(n_layers: int, seed: int):
    import torch

    from asdsl.quantization.synthetic import preq2_from_weights_torch

    gen = torch.Generator(device="cuda").manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        mats = {}
        for name, M, K in LAYER:
            w = torch.randn((M, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
            mats[name] = preq2_from_weights_torch(w, GS)
            del w
        layers.append(mats)
    xs = {name: torch.randn(K, generator=gen, device="cuda", dtype=torch.float32) for name, M, K in LAYER}
    ys = {name: torch.empty(M, device="cuda", dtype=torch.float32) for name, M, K in LAYER}
    torch.cuda.synchronize()
    return layers, xs, ys


def cpu_baseline(layer0, xs, ys_gpu, seconds: float):
    """Reference CPU path (oracle/_ref) on one layer; also a parity spot check."""
    sys.path.insert(0, str(REPO))
    import oracle

    host = {n: (m.cpu().numpy(), q.cpu().numpy()) for n, (m, q) in layer0.items()}
    xh = {n: x.cpu().numpy() for n, x in xs.items()}
    if oracle.reference_available("_native_gemv"):
        ng = oracle.load_reference("_native_gemv")
        kind = "reference"

        def run(n, M, K, y):
            ng.gemv_preq2_fused_avx2(host[n][0], host[n][1], xh[n], y, M, K, GS)
    else:
        kind = "port"

        def run(n, M, K, y):
            y[:] = oracle.gemv_preq2_fused(host[n][0], host[n][1], xh[n], M, K, GS)
    ys = {n: np.zeros(M, np.float32) for n, M, K in LAYER}
    for n, M, K in LAYER:  # warm-up + parity
        run(n, M, K, ys[n])
    parity = {}
    for n, M, K in LAYER:
        g = ys_gpu[n]
        parity[n] = float(np.linalg.norm(g - ys[n]) / np.linalg.norm(ys[n]))
    t0 = time.perf_counter()
    steps = 0
    while True:
        for n, M, K in LAYER:
            run(n, M, K, ys[n])
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    step_bytes = sum(gemv_bytes(M, K) for _, M, K in LAYER)
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)) if kind == "reference" else 1
    return {
        "value": round(step_bytes * steps / el / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{steps} steps of one layer's 4 preq2 GEMVs (gemv_preq2_fused_avx2) in {el:.1f} s, "
                  f"ms_per_step={1e3 * el / steps:.2f}",
    }, parity


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the GEMV path has no "
              "multi-GPU mode.", file=sys.stderr)
        return 2

    import torch

    from asdsl import _hip

    layers, xs, ys = build_layers(args.layers, seed=42)
    lib = _hip.LIB
    stream = torch.cuda.current_stream()
    sh = int(stream.cuda_stream)
    ptrs = [{n: (_hip.ptr(m), _hip.ptr(q)) for n, (m, q) in L.items()} for L in layers]
    xp = {n: _hip.ptr(x) for n, x in xs.items()}
    yp = {n: _hip.ptr(y) for n, y in ys.items()}

    def step(i, ev=None):
        p = ptrs[i % len(ptrs)]
        for n, M, K in LAYER:
            if ev is not None and n == "gate_up":
                ev[0].record(stream)
            st = lib.asdsl_gemv_preq2_fused(p[n][0], p[n][1], xp[n], yp[n], M, K, GS, sh)
            if ev is not None and n == "gate_up":
                ev[1].record(stream)
            if st:
                raise RuntimeError(_hip.last_error())

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    for i in range(args.steps):
        step(i, evs[i])
    t_end.record(stream)
    torch.cuda.synchronize()
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / args.steps
    gu_ms = float(np.mean([a.elapsed_time(b) for a, b in evs]))

    step_bytes = sum(gemv_bytes(M, K) for _, M, K in LAYER)
    value = step_bytes / (ms_step * 1e-3) / 1e9
    gu_bytes = gemv_bytes(16384, 3072)
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9

    # per-GEMV event timing (separate, untimed pass) for the report
    per = {}
    for n, M, K in LAYER:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        reps = 200
        e0.record(stream)
        for i in range(reps):
            p = ptrs[i % len(ptrs)]
            lib.asdsl_gemv_preq2_fused(p[n][0], p[n][1], xp[n], yp[n], M, K, GS, sh)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        per[n] = {"us": round(us, 2), "GB/s": round(gemv_bytes(M, K) / (us * 1e-6) / 1e9, 1)}

    # outputs of layer 0 for the parity spot check
    step(0)
    torch.cuda.synchronize()
    ys_host = {n: y.cpu().numpy() for n, y in ys.items()}

    cpu, parity = (None, None)
    if not args.no_cpu:
        cpu, parity = cpu_baseline(layers[0], xs, ys_host, args.cpu_seconds)

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: W~N(0,0.02) fp32 quantized to preq2 Q4 gs=32 (asymmetric, fp16 scale/zero), "
                "x~N(0,1) fp32, seeded; weights resident in HBM",
        "config": {
            "workload": "phi4_layer_projection_gemvs_preq2_g32",
            "gemvs": {n: [M, K] for n, M, K in LAYER},
            "batch": 1,
            "layers_rotated": args.layers,
            "bytes_per_step": step_bytes,
        },
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "kernel": "preq2_gemv_kernel (gate_up 16384x3072)",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_us": round(gu_ms * 1e3, 3),
            "bytes_per_launch": gu_bytes,
        },
        "per_gemv": per,
        "cpu_baseline": cpu,
        "parity_rel_l2_vs_cpu": parity,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

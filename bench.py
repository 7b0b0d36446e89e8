#!/usr/bin/env python3
"""Benchmark: Phi-4-shaped batch-1 projection GEMVs (preq2 Q4, gs=32) on one MI355X.

One step = the four projection GEMVs of one Phi-4 decoder layer at batch 1,
each quantizing its fp32 activation to int8 inside the kernel as the
reference's gemv_preq2_fused_avx2 does:
    qkv 5120x3072, o_proj 3072x3072, gate_up 16384x3072, down 3072x8192.
Steps rotate over --layers distinct weight sets (default 16, ~1 GB) so that the
256 MB Infinity Cache cannot serve the weights: every step streams its
62.9 MB from HBM.  Inputs are resident in HBM before the timed region.

value    = algorithmic bytes per step (packed weights + fp16 meta + fp32 x + fp32 y)
           / wall time per step (HIP events around the K timed steps).
           The K steps run as replays of HIP graphs (one graph = one rotation
           cycle of 16 steps = 64 GEMV launches), as a decode engine launches.
roofline = the gate_up GEMV kernel: its algorithmic bytes / its average
           launch duration, from HIP events around replays of a graph of 64
           back-to-back gate_up launches over the rotated weights (the dispatch
           gaps between graph nodes are included, so this bounds the kernel
           duration from above).
cpu_baseline = the reference's own gemv_preq2_fused_avx2 (compiled from its
           sources into oracle/_ref) on one layer's four GEMVs on the host
           cores for ~10 s (OpenMP, OMP_NUM_THREADS threads).
extra    = lm_head 200064x3072 preq2-g128 GEMV (untimed phase, same graph
           method, two alternating copies of 327 MB).

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
LM_HEAD = (200064, 3072, 128)
# HBM bytes per gate_up launch measured by rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE on `bench.py --pmc-probe`, each scaled by the same counter on a
# 64 MiB device copy (fetch x1.9993, write x1.0); see
# profiles/preq2_gemv_phi4_layer_g32.md.  A property of the kernel's access
# pattern: re-measure when the kernel's loads change.
GATE_UP_TRAFFIC_BYTES = 31_681_704


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
        "sample": f"{steps} steps of one layer's 4 preq2 g32 GEMVs (gemv_preq2_fused_avx2, OpenMP) "
                  f"in {el:.1f} s, ms_per_step={1e3 * el / steps:.3f}",
    }, parity


def lm_head_kernel(lib, capture, timed_replays):
    """lm_head preq2-g128 GEMV: a graph of 8 back-to-back launches alternating
    between two 327 MB weight copies, replayed; time per launch."""
    import torch

    from asdsl import _hip
    from asdsl.quantization.synthetic import preq2_from_weights_torch

    M, K, gs = LM_HEAD
    gen = torch.Generator(device="cuda").manual_seed(7)
    copies = []
    for _ in range(2):
        w = torch.randn((M, K), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        copies.append(preq2_from_weights_torch(w, gs))
        del w
    x = torch.randn(K, generator=gen, device="cuda", dtype=torch.float32)
    y = torch.empty(M, device="cuda", dtype=torch.float32)
    ptrs = [(_hip.ptr(m), _hip.ptr(q)) for m, q in copies]

    def calls(h):
        for i in range(8):
            if lib.asdsl_gemv_preq2_fused(ptrs[i % 2][0], ptrs[i % 2][1], _hip.ptr(x), _hip.ptr(y), M, K, gs, h):
                raise RuntimeError(_hip.last_error())
    g = capture(calls)
    reps = 12
    us = 1e3 * timed_replays(g, reps) / (reps * 8)
    nbytes = gemv_bytes(M, K, gs)
    del g, copies
    torch.cuda.empty_cache()
    return {"shape": [M, K], "group_size": gs, "kernel_us": round(us, 2), "bytes": nbytes,
            "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
            "frac_of_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-lm-head", action="store_true")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc runs: 50 gate_up GEMVs over rotated weights, then 50 plain "
                         "64 MiB device copies (the counter scale reference); prints nothing else")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}): this GEMV path runs on a "
              "single MI355X and has no multi-GPU mode.", file=sys.stderr)
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
    if args.pmc_probe:
        n, M, K = LAYER[2]
        for i in range(50):
            p = ptrs[i % len(ptrs)]
            lib.asdsl_gemv_preq2_fused(p[n][0], p[n][1], xp[n], yp[n], M, K, GS, sh)
        src = torch.ones(16 << 20, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(50):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "gate_up preq2 g32 x50 then copy 64 MiB x50",
                          "gemv_bytes": gemv_bytes(M, K), "copy_bytes": src.numel() * 4}), flush=True)
        return 0
    L = len(layers)

    def step(i, stream_handle):
        p = ptrs[i % L]
        for n, M, K in LAYER:
            st = lib.asdsl_gemv_preq2_fused(p[n][0], p[n][1], xp[n], yp[n], M, K, GS, stream_handle)
            if st:
                raise RuntimeError(_hip.last_error())

    def capture(calls):
        """HIP graph of `calls(stream_handle)` (torch's capture stream)."""
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up on the side stream before capture
            calls(int(side.cuda_stream))
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            calls(int(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return g

    def timed_replays(g, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    # One rotation cycle (L steps) per graph, plus the remainder, so that
    # exactly --steps steps run back to back with no host launch gaps.
    cycle = capture(lambda h: [step(i, h) for i in range(L)])
    rem = args.steps % L
    tail = capture(lambda h: [step(i, h) for i in range(rem)]) if rem else None
    for _ in range(max(1, args.warmup // L)):
        cycle.replay()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(args.steps // L):
        cycle.replay()
    if tail is not None:
        tail.replay()
    t_end.record()
    torch.cuda.synchronize()
    ms_step = t_start.elapsed_time(t_end) / args.steps

    step_bytes = sum(gemv_bytes(M, K) for _, M, K in LAYER)
    value = step_bytes / (ms_step * 1e-3) / 1e9

    # Per-GEMV kernel time: a graph of 4*L back-to-back launches of one GEMV
    # over the rotated weights, replayed; time / launches.  Includes the
    # (small) dispatch gaps between graph nodes, so it bounds the kernel
    # duration from above.
    per = {}
    for n, M, K in LAYER:
        def calls(h, n=n, M=M, K=K):
            for i in range(4 * L):
                p = ptrs[i % L]
                if lib.asdsl_gemv_preq2_fused(p[n][0], p[n][1], xp[n], yp[n], M, K, GS, h):
                    raise RuntimeError(_hip.last_error())
        g = capture(calls)
        reps = 25
        us = 1e3 * timed_replays(g, reps) / (reps * 4 * L)
        per[n] = {"kernel_us": round(us, 3), "GB/s": round(gemv_bytes(M, K) / (us * 1e-6) / 1e9, 1)}
        del g
    gu_us = per["gate_up"]["kernel_us"]
    gu_bytes = gemv_bytes(16384, 3072)
    gu_gbs = gu_bytes / (gu_us * 1e-6) / 1e9

    # outputs of layer 0 for the parity spot check
    step(0, int(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ys_host = {n: y.cpu().numpy() for n, y in ys.items()}
    del cycle, tail

    extra = {}
    if not args.no_lm_head:
        extra["lm_head_preq2_g128"] = lm_head_kernel(lib, capture, timed_replays)

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
            "kernel": "preq2_gemv_kernel (gate_up 16384x3072, gs=32)",
            "achieved": round(gu_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
            "traffic": GATE_UP_TRAFFIC_BYTES,
            "avg_us": round(gu_us, 3),
            "timing": "HIP events around replays of a HIP graph of 64 back-to-back gate_up launches "
                      "over 16 rotated weight sets; per-launch average",
            "bytes_per_launch": gu_bytes,
        },
        "per_gemv": per,
        "extra": extra,
        "cpu_baseline": cpu,
        "parity_rel_l2_vs_cpu": parity,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

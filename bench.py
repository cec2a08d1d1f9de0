#!/usr/bin/env python3
"""Benchmark of the sparse-ternary GEMV hot path on one MI355X.

Workload (FFN shapes at bs=1): the decode-time FFN GEMVs
of a 30-layer BitNet-2B-4T-shape model, each layer with its own weights:
gate 6912x2560, up 6912x2560 and down 2560x6912, int8 activations in, exact
int32 accumulators out.  One step = one pass over all 90 matrices (298.6 MB
of packed weights, more than the 256 MB Infinity Cache, so the pass streams
from HBM), launched back to back on one stream and replayed as a HIP graph.

The JSON line reports
  value      algorithmic GB/s of the whole step (weights + x + y bytes per
             launch, summed, divided by the step time; inputs resident in HBM)
  roofline   the bit-plane GEMV kernel: algorithmic bytes per launch / its
             average launch duration (HIP events around each launch, on the
             launch stream), against the 8 TB/s HBM peak
  cpu_baseline  the reference's CPU GEMV (its own unpack_to_int8 + int32 MAC,
             built from the reference sources into oracle/_ref) on the
             6912x2560 matrix, single thread, on this host
plus per-shape single-launch times (cold: Infinity Cache and L2 flushed by a
1 GiB write; warm: same buffers back to back) and a one-launch streamed figure
(160 stacked copies of 6912x2560, 531 MB) under "detail".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
H, I = 2560, 6912


def gemv_bytes(rows: int, cols: int) -> int:
    """Algorithmic bytes of one int8->int32 GEMV launch: meta (cols/8 per row)
    + signs (cols/16 per row) + x (cols) + y (4 per row)."""
    return rows * cols // 8 + rows * cols // 16 + cols + 4 * rows


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-graph", action="store_true", help="time eager launches instead")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the reference is "
              "single-GPU; see DESIGN.md for how the GEMV would shard). Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from spbitnet_amd import _lib
    from spbitnet_amd import kernels as K
    from spbitnet_amd import weights as W

    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    # ---- synthetic weights: 3 generated matrices, copied into distinct buffers per layer
    log("generating weights")
    base = {
        "gate": W.random_layer(I, H, W.seed_for("bench", "gate")),
        "up": W.random_layer(I, H, W.seed_for("bench", "up")),
        "down": W.random_layer(H, I, W.seed_for("bench", "down")),
    }

    def to_dev(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(dev)

    dev_base = {k: (to_dev(L.meta), to_dev(L.values)) for k, L in base.items()}
    layers = []
    for _ in range(args.layers):
        layers.append({k: (m.clone(), v.clone()) for k, (m, v) in dev_base.items()})

    a_in = W.normal_f32(W.seed_for("bench", "x"), H)
    g = W.normal_f32(W.seed_for("bench", "g"), I)
    u = W.normal_f32(W.seed_for("bench", "u"), I)
    x_h, _ = W.quantize_absmax_host(a_in)
    x_i, _ = W.quantize_absmax_host((np.maximum(g, 0) ** 2 * u).astype(np.float32))
    d_xh = torch.from_numpy(x_h).to(dev)
    d_xi = torch.from_numpy(x_i).to(dev)
    ys = [{k: torch.empty(base[k].rows, dtype=torch.int32, device=dev) for k in base}
          for _ in range(args.layers)]

    launches = []  # (meta, values, x, y, rows, cols, ms, vs)
    for l in range(args.layers):
        for k in ("gate", "up", "down"):
            L = base[k]
            m, v = layers[l][k]
            x = d_xh if k != "down" else d_xi
            launches.append((m, v, x, ys[l][k], L.rows, L.cols, L.meta_stride, L.values_stride))
    step_bytes = sum(gemv_bytes(r, c) for (_, _, _, _, r, c, _, _) in launches)

    stream = torch.cuda.current_stream()

    def run_step():
        for (m, v, x, y, r, c, ms, vs) in launches:
            K.sparse_ternary_gemv_gpu(m, v, x, y, r, c, ms, vs, stream=stream)

    # correctness spot check against the integer product (host, exact)
    run_step()
    torch.cuda.synchronize()
    for k, xx in (("gate", x_h), ("down", x_i)):
        L = base[k]
        dense = W.unpack(L.meta, L.values, L.rows, L.cols).astype(np.int64)
        want = (dense @ xx.astype(np.int64)).astype(np.int32)
        got = ys[-1][k].cpu().numpy()
        if not (got == want).all():
            log(f"MISMATCH in {k}")
            return 1
    log("spot check passed")

    # ---- timed step: graph replay (default) or eager
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run_step()
        torch.cuda.synchronize()

    def step():
        if graph is not None:
            graph.replay()
        else:
            run_step()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- per-launch kernel durations (events bracketing each launch)
    log("per-launch event timing")
    per = {"gate": [], "up": [], "down": []}
    kinds = ["gate", "up", "down"] * args.layers
    reps = max(2, min(args.steps, 5))
    for _ in range(reps):
        evs = []
        for (m, v, x, y, r, c, ms, vs) in launches:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            K.sparse_ternary_gemv_gpu(m, v, x, y, r, c, ms, vs, stream=stream)
            b.record(stream)
            evs.append((a, b))
        torch.cuda.synchronize()
        for kind, (a, b) in zip(kinds, evs):
            per[kind].append(a.elapsed_time(b) * 1e3)  # us
    all_us = [t for k in per for t in per[k]]
    avg_us = sum(all_us) / len(all_us)
    avg_bytes = step_bytes / len(launches)
    kernel_gbs = avg_bytes / (avg_us * 1e-6) / 1e9

    # ---- single-launch cold / warm per shape
    detail = {"per_launch_avg_us": {k: round(sum(v) / len(v), 3) for k, v in per.items()}}
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    shapes = {"6912x2560": ("gate", d_xh), "2560x6912": ("down", d_xi)}
    for name, (k, xx) in shapes.items():
        m, v = dev_base[k]
        L = base[k]
        y = torch.empty(L.rows, dtype=torch.int32, device=dev)

        def one():
            K.sparse_ternary_gemv_gpu(m, v, xx, y, L.rows, L.cols, L.meta_stride, L.values_stride,
                                      stream=stream)

        warm, cold = [], []
        for i in range(40):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            one()
            b.record(stream)
            torch.cuda.synchronize()
            warm.append(a.elapsed_time(b) * 1e3)
        for i in range(20):
            flush.fill_(i & 0xFF)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            one()
            b.record(stream)
            torch.cuda.synchronize()
            cold.append(a.elapsed_time(b) * 1e3)
        warm.sort()
        cold.sort()
        nb = gemv_bytes(L.rows, L.cols)
        detail[name] = {
            "warm_us_median": round(warm[len(warm) // 2], 3),
            "cold_us_median": round(cold[len(cold) // 2], 3),
            "warm_GBs": round(nb / (warm[len(warm) // 2] * 1e-6) / 1e9, 1),
            "cold_GBs": round(nb / (cold[len(cold) // 2] * 1e-6) / 1e9, 1),
            "bytes": nb,
        }
    del flush

    # ---- streamed, one launch: 160 stacked copies of 6912x2560 (531 MB)
    copies = 160
    m, v = dev_base["gate"]
    Lg = base["gate"]
    sm = m.repeat(copies, 1)
    sv = v.repeat(copies, 1)
    sy = torch.empty(Lg.rows * copies, dtype=torch.int32, device=dev)
    rows_total = Lg.rows * copies
    for _ in range(2):
        K.sparse_ternary_gemv_gpu(sm, sv, d_xh, sy, rows_total, Lg.cols, Lg.meta_stride,
                                  Lg.values_stride, stream=stream)
    torch.cuda.synchronize()
    ts = []
    for _ in range(5):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        K.sparse_ternary_gemv_gpu(sm, sv, d_xh, sy, rows_total, Lg.cols, Lg.meta_stride,
                                  Lg.values_stride, stream=stream)
        b.record(stream)
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) * 1e3)
    ts.sort()
    sb = rows_total * Lg.cols * 3 // 16 + Lg.cols + 4 * rows_total
    detail["streamed_one_launch_160x6912x2560"] = {
        "us_median": round(ts[len(ts) // 2], 2),
        "GBs": round(sb / (ts[len(ts) // 2] * 1e-6) / 1e9, 1),
        "frac_of_peak": round(sb / (ts[len(ts) // 2] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes": sb,
    }
    del sm, sv, sy
    detail["wall_s_timed_region"] = round(wall, 4)
    detail["graph"] = graph is not None

    # ---- CPU baseline: the reference's CPU GEMV on this host, single thread
    cpu = None
    if not args.no_cpu_baseline:
        try:
            from oracle import oracle as O
            if O.ref_available():
                L = base["gate"]
                fn, kind = (lambda: O.ref_cpu_sparse_gemv(L.meta, L.values, x_h, L.rows, L.cols)), "reference"
            else:
                L = base["gate"]
                fn, kind = (lambda: O.gemv(L.meta, L.values, x_h, L.rows, L.cols)), "port"
            n = 0
            t0 = time.perf_counter()
            while time.perf_counter() - t0 < args.cpu_seconds:
                fn()
                n += 1
            dt = time.perf_counter() - t0
            cpu = {
                "value": round(n * gemv_bytes(L.rows, L.cols) / dt / 1e9, 4),
                "unit": "GB/s",
                "cores": 1,
                "kind": kind,
                "sample": f"{n} calls of cpu_sparse_gemv (unpack_to_int8 + int32 MAC) on the "
                          f"6912x2560 gate matrix, {dt:.1f} s, {dt / n * 1e3:.1f} ms/call; "
                          f"host has {os.cpu_count()} logical CPUs",
            }
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline skipped: {e}")

    out = {
        "metric": "bs=1 decode tok/s (2.4B ternary 2:4); GEMV achieved HBM GB/s as % of peak",
        "value": round(value_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic (seeded N(0,1) latent weights, 2:4 top-2 mask, ternary signs; "
                "int8 absmax-quantised N(0,1) / relu2-gated activations)",
        "config": {
            "workload": f"config1 FFN GEMVs at bs=1: {args.layers} layers x (gate 6912x2560, "
                        f"up 6912x2560, down 2560x6912), distinct weights per layer, int8->int32",
            "launches_per_step": len(launches),
            "bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value_gbs / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_bitplane_kernel",
            "achieved": round(kernel_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(avg_us, 3),
            "bytes_per_launch": int(avg_bytes),
        },
        "cpu_baseline": cpu,
        "detail": detail,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

#!/usr/bin/env python3
"""Benchmark of the sparse-ternary GEMV hot path on one MI355X.

Workload (FFN shapes at bs=1, int8 activations in, exact
int32 accumulators out): the gate/up shape 6912x2560 and the down shape
2560x6912.  The timed step is the streamed cold-cache protocol: for each
shape, 80 distinct weight copies (separate HBM memory, 265 MB per shape,
531 MB per step: more than twice the 256 MB Infinity Cache, so every step
streams from HBM) reduced by one launch of the drop-in GEMV entry point
(spb_sparse_ternary_gemv) over the stacked copies; 2 launches per step.

The JSON line reports
  value      algorithmic GB/s of the step (packed weight bytes + x + y per
             launch, divided by the step time; inputs resident in HBM; the
             K timed steps are back-to-back replays of a 10-step HIP graph)
  roofline   the streaming GEMV kernel: algorithmic bytes per launch / its
             average launch duration over the timed region (HIP events on
             the launch stream around the K steps, 2K launches), against
             the 8 TB/s HBM peak; traffic from the committed rocprofv3 PMC
             summary when it was taken on the present kernel sources
  cpu_baseline  the reference's CPU GEMV (its own unpack_to_int8 + int32 MAC,
             built from the reference sources into oracle/_ref) on the
             6912x2560 matrix, single thread, on this host
and under "detail":
  protocol_b2b     BASELINE's protocol literally: 160 distinct copies of each
                   FFN shape as 160 separate launches in one HIP graph (one
                   serial chain, and four independent chains)
  mall_resident    48 and 24 stacked copies (160 / 80 MB, below the 256 MB
                   Infinity Cache) re-streamed back to back, with the
                   non-temporal and the default load policy
  shapes           every config 0/1/4 shape: one cold launch (caches flushed
                   by a 1 GiB write) and warm launches back to back from a
                   graph (the 1-4 MB matrix stays in the caches)
  decode_step_*    30 layers x gate/up/down as 90 separate launches (graph)
  gemm_config2     the batched GEMM at N = 16 / 64 / 256 (matrix cores vs
                   the add/sub kernel)
  decode_config3 / decode_config4_bs1 / decode_config4_b8 / _b32
                   end-to-end greedy decode of the 2.4B-parameter
                   BitNet-b1.58-2B-4T shape (random-init weights) through
                   the HIP engines, tokens/s over the decode steps
  cpu_baselines    the reference CPU GEMV with and without its per-call
                   unpack (1 thread) and the PyTorch CPU BitLinear of
                   python/baseline_pytorch.py at all cores and at 1 thread,
                   per shape, with the host's core count and CPU model
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
H, I = 2560, 6912
# BASELINE configs 0, 1 and 4: the bs=1 GEMV shapes (rows x cols)
SHAPES = [(2560, 2560), (6912, 2560), (2560, 6912), (2048, 2048), (5632, 2048), (2048, 5632),
          (8192, 2560)]
PMC_JSON = os.path.join(ROOT, "profiles", "gemv_stream_config1.pmc.json")
GOLDEN_DECODE = os.path.join(ROOT, "tests", "golden", "decode_2b4t_tokens.json")


def gemv_bytes(rows: int, cols: int) -> int:
    """Algorithmic bytes of one int8->int32 GEMV launch: meta (cols/8 per row)
    + signs (cols/16 per row) + x (cols) + y (4 per row)."""
    return rows * cols // 8 + rows * cols // 16 + cols + 4 * rows


def kernel_sources_sha() -> str:
    """Hash of the sources the streamed GEMV kernel is compiled from."""
    h = hashlib.sha256()
    for f in ("bitplane.hpp", "sparse_ternary.hip", "common.hpp"):
        with open(os.path.join(ROOT, "spbitnet_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def read_traffic():
    """HBM bytes per launch of the streamed GEMV from the committed rocprofv3
    PMC summary (FETCH_SIZE and WRITE_SIZE runs, scaled by a copy of known
    size), only when it was taken on the present kernel sources; else None
    and the reason."""
    try:
        with open(PMC_JSON) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None, "no PMC summary"
    if d.get("kernel_sources_sha") != kernel_sources_sha():
        return None, "PMC summary taken on other kernel sources"
    return {"bytes_per_launch": int(d["traffic_bytes_per_launch_avg"]),
            "source": os.path.relpath(PMC_JSON, ROOT)}, None


# Bytes one decode step must read at minimum: every packed projection of the
# 30 layers plus the bf16 LM head (tied embedding), config 3.
def decode_bytes_per_token(cfg) -> int:
    H, I, kvd = cfg.hidden_size, cfg.intermediate_size, cfg.num_key_value_heads * cfg.head_dim
    per_layer = sum(r * c * 3 // 16 for r, c in
                    [(H, H), (kvd, H), (kvd, H), (H, H), (I, H), (I, H), (H, I)])
    return cfg.num_hidden_layers * per_layer + cfg.vocab_size * H * 2


def kv_bytes_per_position(cfg) -> int:
    """KV-cache bytes one decode step reads per cached position (bf16 K and V
    of every layer)."""
    return cfg.num_hidden_layers * 2 * cfg.num_key_value_heads * cfg.head_dim * 2


def host_info() -> dict:
    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    import torch
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None
    quota = None  # CPUs the cgroup's CPU quota allows (cgroup v2 cpu.max, else v1)
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()[:2]
        if q != "max":
            quota = int(q) / int(per)
    except (OSError, ValueError):
        try:
            with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f:
                q = int(f.read())
            with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
                per = int(f.read())
            if q > 0:
                quota = q / per
        except (OSError, ValueError):
            pass
    usable = affinity or os.cpu_count() or 1
    if quota is not None:
        usable = max(1, min(usable, int(quota)))
    return {"nproc": os.cpu_count(), "sched_affinity_cpus": affinity,
            "cgroup_cpu_quota": None if quota is None else round(quota, 2),
            "usable_cores": usable, "lscpu_model": model,
            "torch_threads_default": torch.get_num_threads()}


def golden_decode():
    try:
        with open(GOLDEN_DECODE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


class Bench:
    def __init__(self, args):
        import torch
        from spbitnet_amd import _lib
        self.args = args
        self.torch = torch
        _lib.load()
        self.dev = torch.device("cuda:0")
        torch.cuda.set_device(self.dev)
        self.stream = torch.cuda.current_stream()

    def log(self, msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    def ev(self):
        return self.torch.cuda.Event(enable_timing=True)

    def to_dev(self, a):
        import numpy as np
        return self.torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(self.dev)

    def graph_of(self, fn):
        g = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(g):
            fn()
        return g

    def time_replays(self, g, reps):
        """ms per replay of graph g over `reps` back-to-back replays."""
        torch = self.torch
        g.replay()
        torch.cuda.synchronize()
        a, b = self.ev(), self.ev()
        a.record(self.stream)
        for _ in range(reps):
            g.replay()
        b.record(self.stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--prewarm-ms", type=float, default=30.0,
                    help="run the step this long before the warmup steps (clock ramp)")
    ap.add_argument("--copies", type=int, default=80, help="distinct weight copies per shape")
    ap.add_argument("--layers", type=int, default=30, help="layers of the decode-shaped step")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="seconds of the reference CPU GEMV sample")
    ap.add_argument("--no-detail", action="store_true")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip every end-to-end decode measurement")
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--no-long-decode", action="store_true",
                    help="skip the config-4 (2048-token prompt, 4096 KV) batch-1 decode")
    ap.add_argument("--no-short-decode", action="store_true",
                    help="skip the config-3 decode (keep config 4)")
    ap.add_argument("--no-batch-decode", action="store_true",
                    help="skip the config-4 decode at batch 8 and 32")
    ap.add_argument("--batches", default="8,32", help="config-4 decode batch sizes")
    ap.add_argument("--no-stepwise-prefill", action="store_true",
                    help="config 4: skip timing the prefill as one decode step per token")
    ap.add_argument("--only-batch-decode", action="store_true",
                    help="profiling: run only the config-4 batched decode and print its results")
    ap.add_argument("--only-mall-resident", action="store_true",
                    help="profiling: run only the Infinity-Cache-resident GEMV protocol "
                         "(for a rocprofv3 FETCH_SIZE pass) and print its timings")
    ap.add_argument("--only-decode", action="store_true",
                    help="profiling: run only the end-to-end decode measurements and print them")
    ap.add_argument("--only-gemm", action="store_true",
                    help="profiling: run only the config-2 batched GEMMs and print their timings")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 256 MiB once (known bytes, for scaling rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--pmc-summary", metavar="DIR",
                    help="write profiles/gemv_stream_config1.pmc.json from the rocprofv3 "
                         "databases under DIR/{fetch,write,calib_f,calib_w} and exit")
    args = ap.parse_args()

    if args.pmc_summary:
        return pmc_summary(args.pmc_summary)

    if args.copy_calibration:
        import torch
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda:0").fill_(1)
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        b.copy_(a)
        torch.cuda.synchronize()
        print("copied 268435456 bytes", flush=True)
        return 0

    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the reference is "
              "single-GPU; the GEMV would shard by rows, or by 128-column K slices with an "
              "exact int32 all-reduce). Run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from spbitnet_amd import kernels as K
    from spbitnet_amd import weights as W

    B = Bench(args)
    dev, stream, log, ev = B.dev, B.stream, B.log, B.ev

    if args.only_batch_decode or args.only_decode:
        print(json.dumps(decode_runs(B, args, batch_only=args.only_batch_decode)), flush=True)
        return 0

    log("generating weights")
    base = {
        "gate": W.random_layer(I, H, W.seed_for("bench", "gate")),
        "up": W.random_layer(I, H, W.seed_for("bench", "up")),
        "down": W.random_layer(H, I, W.seed_for("bench", "down")),
    }
    dev_base = {k: (B.to_dev(L.meta), B.to_dev(L.values)) for k, L in base.items()}
    a_in = W.normal_f32(W.seed_for("bench", "x"), H)
    g = W.normal_f32(W.seed_for("bench", "g"), I)
    u = W.normal_f32(W.seed_for("bench", "u"), I)
    x_h, _ = W.quantize_absmax_host(a_in)
    x_i, _ = W.quantize_absmax_host((np.maximum(g, 0) ** 2 * u).astype(np.float32))
    d_x = {"gate": torch.from_numpy(x_h).to(dev), "up": torch.from_numpy(x_h).to(dev),
           "down": torch.from_numpy(x_i).to(dev)}

    def exact(L, xx):
        dense = W.unpack(L.meta, L.values, L.rows, L.cols).astype(np.int64)
        return (dense @ xx.astype(np.int64)).astype(np.int32)

    want = {"gate": exact(base["gate"], x_h), "down": exact(base["down"], x_i)}

    if args.only_mall_resident:
        print(json.dumps(mall_resident(B, base, dev_base, d_x, want)), flush=True)
        return 0
    if args.only_gemm:
        print(json.dumps(gemm_config2(B, base, dev_base, W, K)), flush=True)
        return 0

    # ---- the timed step: streamed, one launch per shape over stacked copies
    launches = []
    for k in ("gate", "down"):
        L = base[k]
        m, v = dev_base[k]
        sm = m.repeat(args.copies, 1)
        sv = v.repeat(args.copies, 1)
        rows = L.rows * args.copies
        sy = torch.empty(rows, dtype=torch.int32, device=dev)
        launches.append((k, sm, sv, d_x[k], sy, rows, L.cols, L.meta_stride, L.values_stride))
    step_bytes = sum(gemv_bytes(r, c) for (_, _, _, _, _, r, c, _, _) in launches)

    def launch(item):
        # torch's current stream: the capture stream inside torch.cuda.graph()
        _, sm, sv, xx, sy, rows, cols, ms, vs = item
        K.sparse_ternary_gemv_gpu(sm, sv, xx, sy, rows, cols, ms, vs)

    def step():
        for item in launches:
            launch(item)

    step()
    torch.cuda.synchronize()
    for (k, _, _, _, sy, rows, _, _, _) in launches:
        got = sy.cpu().numpy().reshape(args.copies, -1)
        if not (got == want[k][None, :]).all():
            log(f"MISMATCH in streamed {k}")
            return 1
    log("streamed outputs exact")

    # The GPU's clocks settle only after ~2 ms of sustained load following an
    # idle period (launches of this step measured 55-64 us at first, then
    # ~47-51 us), so the step first runs for --prewarm-ms from a one-step
    # graph.  The W warmup steps and the K timed steps then run as replays of
    # a graph of kGraphSteps steps (and one graph of the remainder), back to
    # back: the ~8 us a replay adds at its start is spread over 20 launches,
    # the host's per-launch cost stays out of the GPU timeline, and the graph
    # stays small (one graph of 200 steps measured ~5 % slower per launch
    # than replays of a 10-step graph on the same box).
    def step_graph(n):
        return B.graph_of(lambda: [step() for _ in range(n)])

    kGraphSteps = 10

    def run_steps(k):
        """Launch k steps as replays of kGraphSteps-step graphs (no host sync)."""
        for _ in range(k // kGraphSteps):
            g_block.replay()
        if k % kGraphSteps:
            g_rem[k % kGraphSteps].replay()

    g_block = step_graph(kGraphSteps)
    g_rem = {r: step_graph(r) for r in {args.steps % kGraphSteps, args.warmup % kGraphSteps} if r}
    g_one = step_graph(1)
    t_pre = time.perf_counter()
    while time.perf_counter() - t_pre < args.prewarm_ms * 1e-3:
        for _ in range(8):
            g_one.replay()
        torch.cuda.synchronize()
    del g_one
    run_steps(args.warmup)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    e0, e1 = ev(), ev()
    e0.record(stream)
    run_steps(args.steps)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    value_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9
    del g_block, g_rem

    # Average launch duration of the GEMV kernel over the timed region: the
    # events bracket its 2K launches (back to back; the average includes the
    # gaps between consecutive graph kernels and between replays).
    avg_us = ms_per_step * 1e3 / len(launches)
    avg_bytes = step_bytes / len(launches)
    kernel_gbs = avg_bytes / (avg_us * 1e-6) / 1e9
    detail = {"copies_per_shape": args.copies, "prewarm_ms": args.prewarm_ms}
    del launches

    if not args.no_detail:
        detail["protocol_b2b"] = protocol_b2b(B, base, dev_base, d_x, want)
        detail["mall_resident"] = mall_resident(B, base, dev_base, d_x, want)
        detail["shapes"], shape_layers = shape_timings(B, W, K)
        detail.update(decode_shaped_steps(B, args, base, dev_base, d_x, want, K))
        detail["gemm_config2_6912x2560_warm_b2b"] = gemm_config2(B, base, dev_base, W, K)
    else:
        shape_layers = None

    if not args.no_decode:
        detail.update(decode_runs(B, args))

    # ---- CPU baselines on this host
    cpu = None
    if not args.no_cpu_baseline:
        try:
            cpu, detail["cpu_baselines"] = cpu_baselines(B, args, base, x_h, shape_layers, W)
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
                "int8 absmax-quantised N(0,1) and relu2-gated activations)",
        "config": {
            "workload": f"config1 FFN-shape 2:4 sparse-ternary GEMVs at bs=1, streamed cold: "
                        f"{args.copies} distinct copies each of 6912x2560 and 2560x6912, one "
                        f"launch per shape over the stacked copies, int8->int32 "
                        f"(160 separate launches per shape: detail.protocol_b2b)",
            "bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value_gbs / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_stream_kernel",
            "achieved": round(kernel_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(avg_us, 2),
            "bytes_per_launch": int(avg_bytes),
        },
        "cpu_baseline": cpu,
        "detail": detail,
    }
    traffic, why = read_traffic()
    if traffic is not None:
        out["roofline"]["traffic"] = traffic["bytes_per_launch"]
        out["roofline"]["traffic_source"] = traffic["source"]
    else:
        out["roofline"]["traffic_note"] = why
    print(json.dumps(out), flush=True)
    return 0


# ---- detail measurements ------------------------------------------------------------------

def protocol_b2b(B, base, dev_base, d_x, want, copies=160):
    """BASELINE's streamed protocol taken literally: `copies` distinct copies
    of each FFN shape (530 MB per shape, twice the Infinity Cache) as that many
    separate launches of the drop-in GEMV, captured in one HIP graph; one
    serial chain (every launch waits for the previous one, as consecutive
    projections of a decode step do) and four independent chains (launches
    that may overlap).  Sum of algorithmic bytes over the graph's time."""
    import numpy as np
    from spbitnet_amd import kernels as K
    torch = B.torch
    res = {}
    for name, k in (("6912x2560", "gate"), ("2560x6912", "down")):
        L = base[k]
        m, v = dev_base[k]
        sm = m.repeat(copies, 1)
        sv = v.repeat(copies, 1)
        ys = torch.empty((copies, L.rows), dtype=torch.int32, device=B.dev)
        ms, vs = L.meta_stride, L.values_stride

        def one(i):
            K.sparse_ternary_gemv_gpu(sm[i * L.rows:(i + 1) * L.rows], sv[i * L.rows:(i + 1) * L.rows],
                                      d_x[k], ys[i], L.rows, L.cols, ms, vs)

        row = {"copies": copies, "launches": copies}
        side_streams = [torch.cuda.Stream() for _ in range(4)]  # default priority
        for chains in (1, 4):
            def body():
                if chains == 1:
                    for i in range(copies):
                        one(i)
                    return
                main = torch.cuda.current_stream()
                side = side_streams[:chains]
                for s in side:
                    s.wait_stream(main)
                for i in range(copies):
                    with torch.cuda.stream(side[i % chains]):
                        one(i)
                for s in side:
                    main.wait_stream(s)
            ys.fill_(-1)
            g = B.graph_of(body)
            ms_rep = B.time_replays(g, 5)
            ok = bool((ys.cpu().numpy() == want[k][None, :]).all())
            us = ms_rep * 1e3 / copies
            gbs = gemv_bytes(L.rows, L.cols) / (us * 1e-6) / 1e9
            row[f"chains{chains}"] = {"us_per_launch": round(us, 3), "GBs": round(gbs, 1),
                                      "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                                      "exact": ok}
            del g
        res[name] = row
        del sm, sv, ys
    B.log("protocol_b2b done")
    return res


def mall_resident(B, base, dev_base, d_x, want, copies=(48, 24), reps=20):
    """Stacked copies of each FFN shape small enough to stay in the 256 MB
    Infinity Cache (48 copies = 160 MB, 24 = 80 MB per shape), re-streamed by
    one launch each, `reps` launches back to back from a graph, with two load
    policies: "nt" (the drop-in entry point's non-temporal weight loads, the
    cold stream's policy) and "default" (spb_sparse_ternary_gemv_resident: the
    default cache policy, which lets the set stay in the cache)."""
    from spbitnet_amd import kernels as K
    torch = B.torch
    res = {"copies": list(copies), "policies": {
        "nt": "spb_sparse_ternary_gemv (non-temporal weight loads)",
        "default": "spb_sparse_ternary_gemv_resident (default cache policy)"}}
    for name, k in (("6912x2560", "gate"), ("2560x6912", "down")):
        L = base[k]
        m, v = dev_base[k]
        for nc in copies:
            sm = m.repeat(nc, 1)
            sv = v.repeat(nc, 1)
            rows = L.rows * nc
            y = torch.empty(rows, dtype=torch.int32, device=B.dev)
            for pol in ("nt", "default"):
                def body():
                    for _ in range(reps):
                        K.sparse_ternary_gemv_gpu(sm, sv, d_x[k], y, rows, L.cols,
                                                  L.meta_stride, L.values_stride,
                                                  resident=(pol == "default"))
                g = B.graph_of(body)
                for _ in range(3):
                    g.replay()
                ms_rep = B.time_replays(g, 3)
                ok = bool((y.cpu().numpy().reshape(nc, -1) == want[k][None, :]).all())
                us = ms_rep * 1e3 / reps
                nb = gemv_bytes(rows, L.cols)
                res[f"{name}_x{nc}_{pol}"] = {
                    "MB": round(nb / 1e6, 1), "us_per_launch": round(us, 2),
                    "GBs": round(nb / (us * 1e-6) / 1e9, 1),
                    "frac_of_hbm_peak": round(nb / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "exact": ok}
                del g
            del sm, sv, y
        # the rate per added byte between the two set sizes: a launch has a
        # fixed cost (~2 us: launch, first loads' latency, tail) that the
        # smaller sets amortise over fewer bytes
        lo, hi = min(copies), max(copies)
        for pol in ("nt", "default"):
            a, b = res[f"{name}_x{lo}_{pol}"], res[f"{name}_x{hi}_{pol}"]
            dus = b["us_per_launch"] - a["us_per_launch"]
            dmb = b["MB"] - a["MB"]
            res[f"{name}_marginal_{pol}_GBs"] = round(dmb * 1e6 / (dus * 1e-6) / 1e9, 1) if dus > 0 else None
    B.log("mall_resident done")
    return res


def shape_timings(B, W, K, reps=20):
    """Every config 0/1/4 GEMV shape: one launch with the caches flushed by a
    1 GiB write first (cold, median of 15), and `reps` launches of the same
    matrix back to back from a graph (warm: the 1-4 MB matrix stays in the
    caches; per-launch time).  Outputs checked against the exact product."""
    import numpy as np
    torch = B.torch
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=B.dev)
    res, layers = {}, {}
    for rows, cols in SHAPES:
        L = W.random_layer(rows, cols, W.seed_for("bench-shape", rows, cols))
        layers[(rows, cols)] = L
        m, v = B.to_dev(L.meta), B.to_dev(L.values)
        xq, _ = W.quantize_absmax_host(W.normal_f32(W.seed_for("bench-shape-x", rows, cols), cols))
        x = torch.from_numpy(xq).to(B.dev)
        y = torch.empty(rows, dtype=torch.int32, device=B.dev)

        def call():
            K.sparse_ternary_gemv_gpu(m, v, x, y, rows, cols, L.meta_stride, L.values_stride)
        ts = []
        for i in range(15):
            flush.fill_(i & 0xFF)
            a, b = B.ev(), B.ev()
            a.record(B.stream)
            call()
            b.record(B.stream)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e3)
        cold = sorted(ts)[len(ts) // 2]
        dense = W.unpack(L.meta, L.values, rows, cols).astype(np.int64)
        ok = bool((y.cpu().numpy() == (dense @ xq.astype(np.int64))).all())
        g = B.graph_of(lambda: [call() for _ in range(reps)])
        warm = B.time_replays(g, 5) * 1e3 / reps
        nb = gemv_bytes(rows, cols)
        res[f"{rows}x{cols}"] = {"bytes": nb, "cold_us": round(cold, 3),
                                 "cold_GBs": round(nb / (cold * 1e-6) / 1e9, 1),
                                 "warm_graph_us": round(warm, 3),
                                 "warm_GBs": round(nb / (warm * 1e-6) / 1e9, 1), "exact": ok}
        del g
    del flush
    B.log("shape timings done")
    return res, layers


def decode_shaped_steps(B, args, base, dev_base, d_x, want, K):
    """30 layers x (gate, up, down) as separate launches replayed from a
    graph, with int8 activations and with precomputed activation planes."""
    torch = B.torch
    layers = [{k: (m.clone(), v.clone()) for k, (m, v) in dev_base.items()}
              for _ in range(args.layers)]
    ys = [{k: torch.empty(base[k].rows, dtype=torch.int32, device=B.dev) for k in base}
          for _ in range(args.layers)]
    planes = {k: torch.empty(K.planes_words(base[k].cols), dtype=torch.int32, device=B.dev)
              for k in ("gate", "down")}

    def decode_step(use_planes):
        for l in range(args.layers):
            if use_planes:
                K.activation_planes_gpu(d_x["gate"], planes["gate"], H)
            for k in ("gate", "up", "down"):
                L = base[k]
                m, v = layers[l][k]
                if use_planes:
                    if k == "down":
                        K.activation_planes_gpu(d_x["down"], planes["down"], I)
                    K.sparse_ternary_gemv_planes_gpu(
                        m, v, planes["gate" if k != "down" else "down"], ys[l][k], L.rows,
                        L.cols, L.meta_stride, L.values_stride)
                else:
                    K.sparse_ternary_gemv_gpu(m, v, d_x[k], ys[l][k], L.rows, L.cols,
                                              L.meta_stride, L.values_stride)

    dec_bytes = args.layers * (2 * gemv_bytes(I, H) + gemv_bytes(H, I))
    out = {}
    for use_planes in (False, True):
        gph = B.graph_of(lambda: decode_step(use_planes))
        for _ in range(3):
            gph.replay()
        t = B.time_replays(gph, 10)
        ok = all((ys[-1][k].cpu().numpy() == want["gate" if k != "down" else "down"]).all()
                 for k in ("gate", "down"))
        out["decode_step_int8" if not use_planes else "decode_step_planes"] = {
            "launches": args.layers * (3 if not use_planes else 5),
            "ms": round(t, 4), "GBs": round(dec_bytes / (t * 1e-3) / 1e9, 1), "exact": bool(ok)}
        del gph
    return out


def gemm_config2(B, base, dev_base, W, K):
    """Config 2: the batched GEMM, matrix-core (SMFMAC) vs add/sub kernel, 20
    back-to-back launches captured in a graph."""
    import numpy as np
    torch = B.torch
    L = base["gate"]
    m, v = dev_base["gate"]
    g2 = {}
    for n in (16, 64, 256):
        X = torch.from_numpy(np.stack([W.quantize_absmax_host(
            W.normal_f32(W.seed_for("bench-gemm", t), H))[0] for t in range(n)])).to(B.dev)
        Y = torch.empty((n, L.rows), dtype=torch.int32, device=B.dev)
        row = {}
        for kern in ("auto", "addsub"):
            K.sparse_ternary_gemm_gpu(m, v, X, Y, L.rows, L.cols, n, L.meta_stride,
                                      L.values_stride, kernel=kern)
            torch.cuda.synchronize()
            if kern == "auto":
                dense = W.unpack(L.meta, L.values, L.rows, L.cols).astype(np.float64)
                want2 = (X.cpu().numpy().astype(np.float64) @ dense.T).astype(np.int32)
                row["exact"] = bool((Y.cpu().numpy() == want2).all())
            gph = B.graph_of(lambda: [K.sparse_ternary_gemm_gpu(
                m, v, X, Y, L.rows, L.cols, n, L.meta_stride, L.values_stride, kernel=kern)
                for _ in range(20)])
            us = B.time_replays(gph, 5) * 1e3 / 20
            del gph
            name = "smfmac" if kern == "auto" else "addsub"
            nb = L.rows * L.cols * 3 // 16 + n * L.cols + 4 * n * L.rows
            row[f"{name}_us"] = round(us, 2)
            row[f"{name}_GBs"] = round(nb / (us * 1e-6) / 1e9, 1)
            row[f"{name}_dense_equiv_TOPS"] = round(2.0 * L.rows * L.cols * n / (us * 1e-6) / 1e12, 2)
        g2[f"n{n}"] = row
    # the cuSPARSELt backend's drop-in (CuSparseLtGemm: any-int8 weights pruned
    # to 2:4 and compressed, then D = A_pruned * B) on the same shape, with
    # int8 weights over the whole range
    rng = np.random.default_rng(2)
    A = torch.from_numpy(rng.integers(-128, 128, (L.rows, L.cols)).astype(np.int8)).to(B.dev)
    for n in (16, 64, 256):
        ctx = K.CuSparseLtGemm(L.rows, L.cols, n, device=B.dev)
        ctx.prepare(A)
        Xb = torch.from_numpy(rng.integers(-128, 128, (n, L.cols)).astype(np.int8)).to(B.dev)
        D = torch.empty((n, L.rows), dtype=torch.int32, device=B.dev)
        ctx.execute(Xb, D)
        P = torch.empty_like(A)
        ctx.get_pruned_weights(P)
        torch.cuda.synchronize()
        want = (Xb.cpu().numpy().astype(np.float64) @
                P.cpu().numpy().astype(np.float64).T).astype(np.int32)
        gph = B.graph_of(lambda: [ctx.execute(Xb, D) for _ in range(20)])
        us = B.time_replays(gph, 5) * 1e3 / 20
        del gph
        nb = K.sparse_i8_compressed_size(L.rows, L.cols) + n * L.cols + 4 * n * L.rows
        g2[f"n{n}"]["i8_sparse_us"] = round(us, 2)
        g2[f"n{n}"]["i8_sparse_GBs"] = round(nb / (us * 1e-6) / 1e9, 1)
        g2[f"n{n}"]["i8_sparse_dense_equiv_TOPS"] = round(
            2.0 * L.rows * L.cols * n / (us * 1e-6) / 1e12, 2)
        g2[f"n{n}"]["i8_sparse_exact"] = bool((D.cpu().numpy() == want).all())
        del ctx, P, D
    return g2


def decode_runs(B, args, batch_only=False):
    """End-to-end greedy decode of the BitNet-b1.58-2B-4T shape with
    random-init weights generated on the device (one model for every run):
    config 3 (33-token prompt, max_seq 256), config 4 at batch 1 (2048-token
    prompt, 4096-position cache) and at batch 8 and 32 (2048-token prompts).
    Tokens/s over the decode steps only (the reference's convention,
    src/main.cpp:175-215); the prefill's wall time reported beside it."""
    import numpy as np
    torch = B.torch
    from spbitnet_amd.model import BatchInferenceEngine, InferenceEngine, Model, ModelConfig
    cfg = ModelConfig.bitnet_b158_2b4t()
    B.log("decode: generating the random 2.4B-parameter model")
    model = Model.random(cfg, seed=2025)
    torch.cuda.synchronize()
    nbytes = decode_bytes_per_token(cfg)
    golden = golden_decode()
    out = {}
    desc = ("BitNet-b1.58-2B-4T shape, random init (30 layers, hidden 2560, 20/5 heads, "
            "FFN 6912, vocab 128256, bf16 tied embedding / LM head, bf16 KV cache)")

    def prompt_of(n, seed):
        return [cfg.bos_token_id] + [int(t) for t in np.random.default_rng(seed).integers(
            0, cfg.vocab_size, n - 1)]

    def bs1(max_seq, prompt_len, key, stepwise):
        n = args.decode_tokens
        eng = InferenceEngine(model, max_seq=max_seq)
        prompt = prompt_of(prompt_len, 2025)
        runs, pre = [], []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            eng.generate(prompt, 0, stop_at_eos=False)  # reset + prefill
            torch.cuda.synchronize()
            pre.append((time.perf_counter() - t0) * 1e3)
            a, b = B.ev(), B.ev()
            a.record(B.stream)
            eng.decode_steps(n)
            b.record(B.stream)
            torch.cuda.synchronize()
            runs.append(a.elapsed_time(b))
        ms = sorted(runs)[1]
        pre_ms = sorted(pre)[1]
        toks = eng.generate(prompt, n, stop_at_eos=False)
        again = eng.generate(prompt, n, stop_at_eos=False)
        r = {"model": desc, "max_seq": max_seq, "prompt_tokens": len(prompt), "decode_tokens": n,
             "tok_per_s": round(n / (ms * 1e-3), 1), "us_per_token": round(ms * 1e3 / n, 1),
             "ms_runs": [round(x, 3) for x in runs], "min_bytes_per_token": nbytes,
             "effective_GBs": round(nbytes * n / (ms * 1e-3) / 1e9, 1),
             "frac_of_hbm_peak": round(nbytes * n / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
             "kernels_per_token": 5 * cfg.num_hidden_layers + 1,
             "greedy_repeatable": toks == again, "first_tokens": toks[:8],
             "prefill_ms": round(pre_ms, 2),
             "prefill_tok_per_s": round((len(prompt) - 1) / (pre_ms * 1e-3), 1)}
        gold = golden.get(key)
        if gold is not None:
            m = min(len(gold["tokens"]), len(toks))
            r["oracle_tokens_match"] = gold["prompt_len"] == len(prompt) and toks[:m] == gold["tokens"][:m]
            r["oracle_tokens_checked"] = m
        if stepwise:
            eng.set_prefill_batch(0)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            eng.generate(prompt, 0, stop_at_eos=False)
            torch.cuda.synchronize()
            r["prefill_stepwise_ms"] = round((time.perf_counter() - t0) * 1e3, 1)
            r["stepwise_prefill_same_tokens"] = eng.generate(prompt, n, stop_at_eos=False) == toks
            eng.set_prefill_batch(16)
        B.log(f"decode {key}: {r['tok_per_s']} tok/s")
        eng.close()
        torch.cuda.empty_cache()
        return r

    def batched(bsz):
        n = args.decode_tokens
        eng = BatchInferenceEngine(model, max_seq=4096, batch=bsz)
        # sequence 0 is config4_bs1's prompt (its oracle tokens are committed)
        prompts = [prompt_of(2048, 2025 if b == 0 else 4000 + b) for b in range(bsz)]
        runs, pre = [], []
        for _ in range(3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            eng.generate(prompts, 0, stop_at_eos=False)  # prefill every sequence
            torch.cuda.synchronize()
            pre.append((time.perf_counter() - t0) * 1e3)
            a, b = B.ev(), B.ev()
            a.record(B.stream)
            eng.decode_steps(n)
            b.record(B.stream)
            torch.cuda.synchronize()
            runs.append(a.elapsed_time(b))
        ms = sorted(runs)[1]
        toks = eng.generate(prompts, n, stop_at_eos=False)
        # two sequences decoded alone by the bs=1 engine
        one = InferenceEngine(model, max_seq=4096)
        same = all(one.generate(prompts[b], n, stop_at_eos=False) == toks[b]
                   for b in (0, bsz - 1))
        one.close()
        kv = kv_bytes_per_position(cfg) * sum(2048 + i for i in range(n)) / n  # per sequence
        r = {"model": desc, "batch": bsz, "max_seq": 4096, "prompt_tokens": 2048,
             "decode_steps": n, "tok_per_s": round(bsz * n / (ms * 1e-3), 1),
             "us_per_step": round(ms * 1e3 / n, 1), "ms_runs": [round(x, 3) for x in runs],
             "weight_bytes_per_step": nbytes, "kv_bytes_per_step": int(kv * bsz),
             "min_GBs": round((nbytes + kv * bsz) / (ms * 1e-3 / n) / 1e9, 1),
             "prefill_ms": round(sorted(pre)[1], 1),
             "prefill_tok_per_s": round(bsz * 2047 / (sorted(pre)[1] * 1e-3), 1),
             "tokens_equal_bs1_engine": same}
        # every sequence of the batch with committed oracle tokens (sequence 0
        # is config4_bs1's prompt; sequence b > 0 is config4_seq{4000 + b})
        checked, match = [], True
        for b in range(bsz):
            gold = golden.get("config4_bs1" if b == 0 else f"config4_seq{4000 + b}")
            if gold is None or gold["prompt_len"] != 2048:
                continue
            m = min(len(gold["tokens"]), len(toks[b]))
            match = match and toks[b][:m] == gold["tokens"][:m]
            checked.append(b)
        if checked:
            r["oracle_tokens_match"] = match
            r["oracle_tokens_checked"] = min(n, 128)
            r["oracle_sequences_checked"] = checked
        B.log(f"decode config4 batch {bsz}: {r['tok_per_s']} tok/s")
        eng.close()
        torch.cuda.empty_cache()
        return r

    if not batch_only:
        if not args.no_short_decode:
            out["decode_config3"] = bs1(256, 33, "config3", False)
        if not args.no_long_decode:
            out["decode_config4_bs1"] = bs1(4096, 2048, "config4_bs1",
                                            not args.no_stepwise_prefill)
    if batch_only or not args.no_batch_decode:
        for bsz in [int(b) for b in args.batches.split(",") if b]:
            out[f"decode_config4_b{bsz}"] = batched(bsz)
    del model
    torch.cuda.empty_cache()
    return out


def cpu_baselines(B, args, base, x_h, shape_layers, W):
    """The CPU path timed on this host, as reported baselines:
      * A10, the reference's CPU GEMV (tests/test_sparse_ternary.cu:17-33): its
        own unpack_to_int8 + int32 MAC (oracle/_ref, or the oracle's
        restatement when the reference build is absent), single thread, on
        6912x2560 for args.cpu_seconds; and the MAC alone on a pre-unpacked
        matrix (the baseline without the per-call unpack);
      * A11, the PyTorch CPU BitLinear of python/baseline_pytorch.py:56-107
        (oracle/cpu_bitlinear.py): dense float32 {-1,0,+1} weight @ the
        absmax-quantised input, per shape, at torch's default thread count
        and at 1 thread (median of a bounded sample per shape)."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from oracle.cpu_bitlinear import TorchSparseBitLinear
    info = host_info()
    L = base["gate"]
    if O.ref_available():
        fn, kind = (lambda: O.ref_cpu_sparse_gemv(L.meta, L.values, x_h, L.rows, L.cols)), "reference"
    else:
        fn, kind = (lambda: O.gemv(L.meta, L.values, x_h, L.rows, L.cols)), "port"
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < args.cpu_seconds:
        fn()
        n += 1
    dt = time.perf_counter() - t0
    nb = gemv_bytes(L.rows, L.cols)
    primary = {
        "value": round(n * nb / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": kind,
        "sample": f"{n} calls of cpu_sparse_gemv (unpack_to_int8 + int32 MAC) on the 6912x2560 "
                  f"gate matrix, {dt:.1f} s, {dt / n * 1e3:.1f} ms/call; host: {info['nproc']} "
                  f"logical CPUs, {info['usable_cores']} usable by this process (affinity "
                  f"{info['sched_affinity_cpus']}, cgroup quota {info['cgroup_cpu_quota']}), "
                  f"{info['lscpu_model']}"}
    dense = O.unpack(L.meta, L.values, L.rows, L.cols)
    n2, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 2.0 or n2 < 3:
        O.dense_mac(dense, x_h)
        n2 += 1
    dt2 = time.perf_counter() - t0
    detail = {"host": info,
              "A10_cpu_gemv_6912x2560": {"kind": kind, "threads": 1,
                                         "ms_with_unpack": round(dt / n * 1e3, 2),
                                         "ms_mac_only": round(dt2 / n2 * 1e3, 2)},
              "A11_torch_bitlinear": {}}
    threads_default = torch.get_num_threads()
    threads_all = info["usable_cores"]  # the cores this process may actually run on
    layers = shape_layers or {(r, c): W.random_layer(r, c, W.seed_for("bench-shape", r, c))
                              for r, c in SHAPES}
    for (rows, cols), Lx in layers.items():
        m = TorchSparseBitLinear(Lx.meta, Lx.values, Lx.gamma, rows, cols)
        x = torch.from_numpy(W.normal_f32(W.seed_for("bench-cpu-x", rows, cols), cols)).half()
        row = {}
        for label, nt in (("all_cores", threads_all), ("one_thread", 1)):
            torch.set_num_threads(nt)
            m(x)
            ts, t0 = [], time.perf_counter()
            while (time.perf_counter() - t0 < 0.6 or len(ts) < 5) and len(ts) < 200:
                t1 = time.perf_counter()
                m(x)
                ts.append(time.perf_counter() - t1)
            med = sorted(ts)[len(ts) // 2]
            row[f"{label}_us"] = round(med * 1e6, 1)
            row[f"{label}_threads"] = nt
        torch.set_num_threads(threads_default)
        detail["A11_torch_bitlinear"][f"{rows}x{cols}"] = row
    B.log("cpu baselines done")
    return primary, detail


def pmc_summary(d):
    """profiles/gemv_stream_config1.pmc.json from four rocprofv3 --pmc runs
    under d: FETCH_SIZE and WRITE_SIZE of the timed step (d/fetch, d/write)
    and of a 256 MiB copy (d/calib_f, d/calib_w, from --copy-calibration),
    whose readings scale the counters to bytes."""
    import collections
    import glob
    import sqlite3

    def per_kernel(sub, counter, filt):
        dbs = glob.glob(os.path.join(d, sub, "**", "*.db"), recursive=True)
        if not dbs:
            raise SystemExit(f"no rocprofv3 database under {os.path.join(d, sub)}")
        c = sqlite3.connect(dbs[0])
        rows = c.execute("select kernel_name, counter_name, value, lds_block_size from "
                         "counters_collection where counter_name=?", (counter,)).fetchall()
        out = collections.defaultdict(list)
        for kn, _, v, lds in rows:
            if filt in kn:
                out[lds].append(v)
        return out

    fetch = per_kernel("fetch", "FETCH_SIZE", "gemv_stream_kernel")
    write = per_kernel("write", "WRITE_SIZE", "gemv_stream_kernel")
    cf = per_kernel("calib_f", "FETCH_SIZE", "copy")
    cw = per_kernel("calib_w", "WRITE_SIZE", "copy")
    cal_f = max(v for vs in cf.values() for v in vs)
    cal_w = max(v for vs in cw.values() for v in vs)
    fs, ws = 268435456 / 1024 / cal_f, 268435456 / 1024 / cal_w
    alg = sorted([gemv_bytes(6912 * 80, 2560), gemv_bytes(2560 * 80, 6912)])
    out = {"kernel": "gemv_stream_kernel<BuildPlanes<Int8Src>, Int32Sink>",
           "workload": "bench.py streamed step: 80 stacked copies of 6912x2560 and of 2560x6912, "
                       "one launch each",
           "kernel_sources_sha": kernel_sources_sha(),
           "commands": [
               "rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_stream/fetch -o f -- python3 -u "
               "bench.py --steps 2 --warmup 1 --prewarm-ms 5 --no-cpu-baseline --no-detail --no-decode",
               "rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_stream/write -o w -- python3 -u "
               "bench.py --steps 2 --warmup 1 --prewarm-ms 5 --no-cpu-baseline --no-detail --no-decode",
               "rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_stream/calib_f -o c -- python3 -u "
               "bench.py --copy-calibration",
               "rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_stream/calib_w -o c -- python3 -u "
               "bench.py --copy-calibration",
               "python3 bench.py --pmc-summary gpurun_out/pmc_stream"],
           "calibration": {"copy_bytes_each_way": 268435456, "FETCH_SIZE_kib": cal_f,
                           "WRITE_SIZE_kib": cal_w, "fetch_scale": round(fs, 5),
                           "write_scale": round(ws, 5)},
           "per_launch": {}}
    tot_t = 0
    keys = sorted(fetch)
    for lds in keys:
        f = sum(fetch[lds]) / len(fetch[lds])
        w = sum(write[lds]) / len(write[lds])
        t = int((f * fs + w * ws) * 1024)
        out["per_launch"][f"lds{lds}"] = {"dispatches": len(fetch[lds]), "fetch_kib_raw": f,
                                          "write_kib_raw": w, "traffic_bytes": t}
        tot_t += t
    out["traffic_bytes_per_launch_avg"] = tot_t // len(keys)
    out["algorithmic_bytes_per_launch_avg"] = sum(alg) // 2
    out["traffic_over_algorithmic"] = round(out["traffic_bytes_per_launch_avg"] /
                                            out["algorithmic_bytes_per_launch_avg"], 4)
    # Infinity-Cache-resident protocol (48 copies re-streamed), when its
    # FETCH_SIZE pass (d/mall) is present.  FETCH_SIZE counts the bytes the L2
    # fetches from the fabric, whether the Infinity Cache or HBM serves them:
    # it shows that each launch moves its algorithmic bytes once; the
    # residency itself shows in the launch time.
    mdbs = glob.glob(os.path.join(d, "mall", "**", "*.db"), recursive=True)
    if mdbs:
        import re
        c = sqlite3.connect(mdbs[0])
        rows = c.execute("select kernel_name, value, lds_block_size from counters_collection "
                         "where counter_name='FETCH_SIZE'").fetchall()
        mall = collections.defaultdict(list)
        for kn, v, lds in rows:
            if "gemv_stream_kernel" not in kn:
                continue
            pol = re.findall(r",\s*(\d+)\s*>\s*\(", kn)  # the load policy: last template argument
            name = {"2": "nt", "0": "default"}.get(pol[-1] if pol else "", "?")
            mall[f"lds{lds}_{name}"].append(v)
        out["mall_resident"] = {
            "command": "rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_stream/mall -o m -- python3 "
                       "-u bench.py --only-mall-resident",
            "algorithmic_bytes": {f"{shape}x{nc}": gemv_bytes(r * nc, k)
                                  for shape, r, k in (("6912x2560", 6912, 2560),
                                                      ("2560x6912", 2560, 6912))
                                  for nc in (48, 24)},
            "per_launch": {key: {"dispatches": len(v),
                                 "fetch_bytes": int(sum(v) / len(v) * fs * 1024)}
                           for key, v in sorted(mall.items())}}
        out["commands"].insert(4, out["mall_resident"]["command"])
    with open(PMC_JSON, "w") as fh:
        json.dump(out, fh, indent=1)
    print(json.dumps(out, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())

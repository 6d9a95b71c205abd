#!/usr/bin/env python3
"""Decode benchmark of the GGUF quantized-matmul path on one MI355X.

Workload (one "step" = one decode token, batch 1): the Llama-3-8B Q4_K_M
projection set -- 32 layers of q/k/v/o/gate/up in Q4_K and down in Q6_K, plus
the 128256 x 4096 Q6_K lm_head -- run as fused dequant-GEMVs over weights
resident in HBM in their packed GGUF layout (4 841 250 816 weight bytes per
step), bf16 input activations, float32 accumulation, captured as one HIP graph.
Weights are synthetic: N(0, 0.02) with 1 % of rows x4, drawn from a fixed seed
and quantized on the device.  Attention and norms are outside the path; the
step streams exactly the projection weights.

Printed (one JSON line on stdout):
  value      weight-streaming throughput of the whole step, GB/s
  roofline   the dominant kernel (Q4_K GEMV, 14336 x 4096, M = 1) timed with
             HIP events on its launch stream over a rotation of the 64 distinct
             gate/up matrices (2.1 GB, beyond the 256 MB Infinity Cache),
             algorithmic bytes per launch / average launch time, vs 8 TB/s
  cpu_baseline  the reference CPU path (numpy dequant + float32 x @ W.T,
             as the oracle restates it) on the host cores, warm fp32-weight
             cache, one layer + 1/8 of lm_head timed and scaled to a step
Usage: python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K dequant-GEMV HBM GB/s (% of peak); 8B-shape decode tokens/s at 1 GPU"
PEAK_HBM_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_14336x4096_m1_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_launches(fns, reps):
    """Average ms per launch of the launches in ``fns``, captured once into a
    HIP graph and replayed ``reps`` times back to back; HIP events are recorded
    on the stream the replays (and so the kernels) run on."""
    import torch

    for f in fns:
        f()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for f in fns:
            f()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for f in fns:
            f()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / (reps * len(fns))


def dominant_kernel_roofline(ls, reps):
    import torch

    from dracort_amd.kernels import gguf_gemv

    mats = [layer[p] for layer in ls.layers for p in ("gate", "up")]
    n, k = mats[0].shape
    x = torch.randn((1, k), device="cuda").to(torch.bfloat16)
    y = torch.empty((1, n), device="cuda", dtype=torch.float32)
    fns = [lambda w=w: gguf_gemv(x, w.data, w.ggml_type, w.shape, out=y) for w in mats]
    ms = time_launches(fns, reps)
    alg_bytes = mats[0].nbytes + k * 2 + n * 4
    achieved = alg_bytes / (ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    return {
        "kernel": "gemv_x1_kernel<Q4_K> (decode GEMV, M = 1, bf16 x) on a 14336 x 4096 Q4_K weight",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "traffic": traffic,
        "alg_bytes_per_launch": alg_bytes,
        "avg_launch_us": round(ms * 1e3, 3),
        "launches_timed": reps * len(fns),
        "rotation": f"{len(mats)} distinct weights, {len(mats) * mats[0].nbytes / 1e9:.2f} GB (> 256 MB Infinity Cache)",
    }


def cpu_baseline(ls, step_bytes):
    """The reference CPU path on a bounded sample of the same workload."""
    import numpy as np
    import torch
    from threadpoolctl import threadpool_limits

    from oracle import gguf_ref, matmul_ref

    cores = len(os.sched_getaffinity(0))
    layer = {p: (w.data.cpu().numpy(), w.ggml_type, w.shape) for p, w in ls.layers[0].items()}
    lm = ls.lm_head
    rows = lm.shape[0] // 8
    rb = lm.nbytes // lm.shape[0]
    lm_part = (lm.data[: rows * rb].cpu().numpy(), lm.ggml_type, (rows, lm.shape[1]))
    x = torch.randn((1, ls.shape.hidden)).to(torch.bfloat16).float().numpy()
    xi = torch.randn((1, ls.shape.inter)).to(torch.bfloat16).float().numpy()

    def dq(spec):
        b, t, shp = spec
        return gguf_ref.dequantize_matrix(t, b, shp)

    def timed(fn, budget_s):
        """Mean seconds per call of fn, repeated until budget_s has passed (at least twice)."""
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if n >= 2 and el >= budget_s:
                return el / n

    with threadpool_limits(limits=cores):
        t0 = time.perf_counter()
        wl = {p: dq(spec) for p, spec in layer.items()}
        t_dq_layer = time.perf_counter() - t0
        t0 = time.perf_counter()
        wlm = dq(lm_part)
        t_dq_lm = time.perf_counter() - t0

        def layer_fn():
            for p, w in wl.items():
                matmul_ref.cpu_linear_f32(xi if p == "down" else x, w)

        t_layer = timed(layer_fn, 6.0)
        t_lm = timed(lambda: matmul_ref.cpu_linear_f32(x, wlm), 3.0)
    # one step = 32 layers + the full lm_head (8 x the timed 1/8 of its rows)
    step_warm = ls.shape.n_layers * t_layer + 8 * t_lm
    step_cold = step_warm + ls.shape.n_layers * t_dq_layer + 8 * t_dq_lm
    return {
        "value": round(step_bytes / step_warm / 1e9, 2),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            "numpy restatement of the reference _dequantize + float32 x @ W.T (OpenBLAS, threads pinned to "
            f"{cores}) on 1 decoder layer (7 projections) and 1/8 of the lm_head rows, M = 1, warm fp32-weight "
            f"cache, each timed for >= 3-6 s; step = {ls.shape.n_layers} x layer + 8 x lm_head part"
        ),
        "ms_per_step_warm": round(step_warm * 1e3, 2),
        "tokens_per_s_warm": round(1.0 / step_warm, 3),
        "tokens_per_s_cold": round(1.0 / step_cold, 4),
        "dequant_s_layer": round(t_dq_layer, 3),
        "dequant_s_lm_part": round(t_dq_lm, 3),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=1, help="decode batch (tokens per step), <= 16")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of one HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--roofline-reps", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one MI355X: this path runs on a single GPU (no collectives are built); "
            "run with --gpus 1.")
        return 2

    import torch

    from dracort_amd import _native
    from dracort_amd.runtime.decode import DecodeStep, LlamaShape, layer_set_bytes, synthetic_layer_set

    _native.load()  # fail loudly if the HIP library is missing
    if not torch.cuda.is_available():
        log("no GPU visible")
        return 1
    torch.cuda.set_device(0)
    shape = LlamaShape()
    t0 = time.time()
    ls = synthetic_layer_set(shape, seed=args.seed, device="cuda")
    torch.cuda.synchronize()
    step_bytes = ls.weight_bytes
    assert step_bytes == layer_set_bytes(shape)
    log(f"generated {step_bytes / 1e9:.3f} GB of GGUF weights in {time.time() - t0:.1f} s")

    step = DecodeStep(ls, m=args.batch)
    if args.no_graph:
        run = step.run
    else:
        step.capture()
        run = step.replay
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = ev0.elapsed_time(ev1) / args.steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"decode step: {ms:.3f} ms (wall {wall / args.steps * 1e3:.3f} ms), {gbs:.1f} GB/s, "
        f"{args.batch * 1e3 / ms:.1f} tokens/s")

    roof = dominant_kernel_roofline(ls, args.roofline_reps)
    log(f"roofline: {roof}")

    cpu = None
    if not args.no_cpu_baseline:
        t0 = time.time()
        cpu = cpu_baseline(ls, step_bytes)
        log(f"cpu baseline ({time.time() - t0:.1f} s): {cpu}")

    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b-q4_k_m-decode-projection-set",
            "layers": shape.n_layers,
            "batch": args.batch,
            "hidden": shape.hidden,
            "inter": shape.inter,
            "kv_dim": shape.kv_dim,
            "vocab": shape.vocab,
            "weights": "Q4_K q/k/v/o/gate/up, Q6_K down + lm_head",
            "weight_bytes_per_step": step_bytes,
            "activations": "bf16",
            "hip_graph": not args.no_graph,
        },
        "tokens_per_s": round(args.batch * 1e3 / ms, 2),
        "pct_of_peak_hbm": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

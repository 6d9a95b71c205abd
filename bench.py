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
  roofline_step_dominant  the same measurement for the launch that dominates
             the step: the fused gate + up + SiLU.up GEMV (2 x 14336 x 4096)
  cpu_baseline  the reference CPU path (numpy dequant + float32 x @ W.T,
             as the oracle restates it) on the host cores, warm fp32-weight
             cache, one layer + 1/8 of lm_head timed and scaled to a step
  configs    configurations 1, 2, 4 and 5 at full size on the GPU, each with
             the reference CPU path timed beside it (warm, cold, one thread)
  full_decode  the complete decode step (norms, RoPE, KV cache, attention)
  batch16    the projection step and the full step for 16 sequences at once
Modes: --stream-probe (read-only kernel at each launch size: the per-launch
ceiling), --suite / --types / --traffic-probe / --mfma-probe / --moe-probe.
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
PEAK_BF16_TFLOPS = 2516.6  # dense bf16 MFMA, 256 CU x 4096 FLOP/clk x 2.4 GHz
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
        "kernel": "gemv_x1p_kernel<Q4_K> (persistent decode GEMV, M = 1, bf16 x) on a 14336 x 4096 Q4_K weight",
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


def step_dominant_roofline(ls, reps):
    """The launch that dominates the timed step: gate + up + SiLU.up of one
    layer (2 x 14336 x 4096 Q4_K, M = 1, bf16 x) in one fused launch, timed
    like the roofline kernel over the 32 layers' distinct gate/up pairs
    (2.1 GB).  Reported beside ``roofline`` (the single 14336 x 4096 GEMV)."""
    import torch

    from dracort_amd.kernels import gguf_gemv_swiglu

    pairs = [(layer["gate"], layer["up"]) for layer in ls.layers]
    n, k = pairs[0][0].shape
    x = torch.randn((1, k), device="cuda").to(torch.bfloat16)
    y = torch.empty((1, n), device="cuda", dtype=torch.float32)
    fns = [lambda g=g, u=u: gguf_gemv_swiglu(x, g.data, u.data, g.ggml_type, g.shape, out=y) for g, u in pairs]
    ms = time_launches(fns, reps)
    alg_bytes = 2 * pairs[0][0].nbytes + k * 2 + n * 4
    achieved = alg_bytes / (ms * 1e-3) / 1e9
    return {
        "kernel": "gemv_x1p_kernel<Q4_K, kSwiGLU> (fused gate + up + SiLU.up, M = 1, bf16 x), 2 x 14336 x 4096 Q4_K",
        "bound": "hbm",
        "achieved": round(achieved, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(achieved / PEAK_HBM_GBS, 4),
        "alg_bytes_per_launch": alg_bytes,
        "avg_launch_us": round(ms * 1e3, 3),
        "launches_timed": reps * len(fns),
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
    # the same layer on one thread (the reference's default is OpenBLAS's own
    # thread count; one thread is its floor)
    with threadpool_limits(limits=1):
        t_layer_1 = timed(layer_fn, 3.0)
    layer_bytes = sum(w.nbytes for w in ls.layers[0].values())
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
        "one_thread_layer_GB_s": round(layer_bytes / t_layer_1 / 1e9, 2),
    }


def full_decode(ls, batch: int, context: int, steps: int, warmup: int):
    """The full decode step (RMSNorms, RoPE + KV-cache attention, projections,
    lm_head) on the same layer set, ``context`` tokens already cached per
    sequence, one HIP graph per step; positions advance every step."""
    import torch

    from dracort_amd.runtime.decode import AttentionShape, DecodeStep

    attn = AttentionShape(max_positions=context + warmup + steps + 2)
    step = DecodeStep(ls, m=batch, attention=attn, start_position=context)
    step.capture()
    for _ in range(warmup):
        step.replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step.replay()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / steps
    kv_bytes = 2 * len(ls.layers) * batch * attn.n_kv_heads * attn.head_dim * 2 * (context + warmup + steps // 2)
    out = {"batch": batch, "context": context, "ms_per_step": round(ms, 4),
           "tokens_per_s": round(batch * 1e3 / ms, 2), "kv_cache_bytes_read_per_step": kv_bytes,
           "note": "per layer: RMSNorm, q/k/v, RoPE + float16 KV append + GQA attention, o + residual, RMSNorm, "
                   "gate/up SwiGLU, down + residual; final RMSNorm, lm_head"}
    del step
    torch.cuda.empty_cache()
    return out


def rotation(make, nbytes, min_total=1 << 30):
    """Distinct copies of a synthetic weight so that a timed rotation streams
    >= min_total bytes (beyond the 256 MB Infinity Cache)."""
    import torch

    first = make()
    n = max(2, -(-min_total // nbytes))
    return [first] + [torch.empty_like(first).copy_(first) for _ in range(n - 1)]


def suite(reps: int, gemv_only: bool = False):
    """The other configurations of the path, one JSON line each (stdout);
    ``gemv_only``: configurations 1 and 2 only (kernel traces)."""
    import torch

    from dracort_amd.format.gguf import tensor_bytes
    from dracort_amd.kernels import gguf_gemm, gguf_gemv, gguf_moe, moe_workspace_bytes
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    lines = []

    def gemv_line(cfg, t, n, k, m, xdtype):
        nb = tensor_bytes(t, (n, k))
        mats = rotation(lambda: synthetic_weight(n, k, t, gen, "cuda").data, nb)
        x = torch.randn((m, k), device="cuda").to(xdtype)
        y = torch.empty((m, n), device="cuda")
        ms = time_launches([lambda w=w: gguf_gemv(x, w, t, (n, k), out=y) for w in mats], reps)
        alg = nb + x.numel() * x.element_size() + y.numel() * 4
        del mats
        return {"config": cfg, "kernel": "decode GEMV", "ggml_type": t, "shape": [n, k], "m": m,
                "x_dtype": str(xdtype).replace("torch.", ""), "us_per_launch": round(ms * 1e3, 3),
                "GB_s": round(alg / (ms * 1e-3) / 1e9, 1), "frac_hbm_peak": round(alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "alg_bytes": alg}

    # 1: Q8_0 GEMV 4096 x 4096, float32 activations
    lines.append(gemv_line(1, 8, 4096, 4096, 1, torch.float32))
    # 2: Q4_0 GEMV at the Llama-3-8B projection shapes, batch 1 / 4 / 8, float32 activations
    for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
        for m in (1, 4, 8):
            lines.append(gemv_line(2, 2, n, k, m, torch.float32))
    if gemv_only:
        return lines
    # 3 (single kernels): Q4_K / Q6_K GEMVs at M = 1 and 16, bf16 activations
    for t, n, k in ((12, 14336, 4096), (12, 4096, 4096), (14, 4096, 14336), (14, 128256, 4096)):
        for m in (1, 16):
            lines.append(gemv_line(3, t, n, k, m, torch.bfloat16))
    # 3 (full step): norms + RoPE / KV-cache attention + projections, contexts 1024 / 4096, batch 1 / 16
    from dracort_amd.runtime.decode import LlamaShape, synthetic_layer_set

    ls = synthetic_layer_set(LlamaShape(n_layers=32), seed=0, device="cuda")
    for batch, context in ((1, 1024), (1, 4096), (16, 1024)):
        d = full_decode(ls, batch, context, 20, 2)
        d.update({"config": 3, "kernel": "full decode step (HIP graph)"})
        lines.append(d)
        log(json.dumps(d))
    del ls
    torch.cuda.empty_cache()
    # 4: prefill GEMM, Q4_K weights, bf16 activations, M = 512 / 2048
    for n, k in ((14336, 4096), (4096, 14336)):
        w = synthetic_weight(n, k, 12, gen, "cuda")
        for m in (512, 2048):
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), device="cuda")
            ms = time_launches([lambda: gguf_gemm(x, w.data, 12, (n, k), out=y)], reps)
            flops = 2.0 * m * n * k
            lines.append({"config": 4, "kernel": "prefill GEMM (bf16 MFMA)", "ggml_type": 12, "shape": [n, k], "m": m,
                          "us_per_launch": round(ms * 1e3, 2), "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1),
                          "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
        del w
    # 5: Mixtral-8x7B MoE FFN, Q4_K experts, 64 tokens, top-2
    hid, inter, ne, tok = 4096, 14336, 8, 64
    wg = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wu = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wd = [synthetic_weight(hid, inter, 12, gen, "cuda").data for _ in range(ne)]
    # seeded like the weights: the routing (and so the number of 16-token tiles) is the same every run
    x = torch.randn((tok, hid), generator=gen, device="cuda").to(torch.bfloat16)
    logits = torch.randn((tok, ne), generator=gen, device="cuda")
    ws = torch.empty(moe_workspace_bytes(tok, hid, inter, ne, 2), dtype=torch.uint8, device="cuda")
    y = torch.empty((tok, hid), device="cuda")
    ms = time_launches([lambda: gguf_moe(x, logits, wg, wu, wd, 12, inter, top_k=2, workspace=ws, out=y)], reps)
    wbytes = sum(t.numel() for t in wg + wu + wd)
    lines.append({"config": 5, "kernel": "MoE FFN (route + grouped expert GEMVs + combine)", "experts": ne, "tokens": tok,
                  "top_k": 2, "us_per_call": round(ms * 1e3, 2), "weight_bytes": wbytes,
                  "GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1), "frac_hbm_peak": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
    return lines


def types_suite(reps: int):
    """Decode GEMV of every GGUF block type at two Llama-3-8B shapes, M = 1
    (bf16 and float32 activations) and M = 4, one JSON line each (stdout)."""
    import torch

    from dracort_amd.format.gguf import TYPE_NAMES, tensor_bytes
    from dracort_amd.kernels import gguf_gemv
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda")
    gen.manual_seed(11)
    lines = []
    for t in sorted(TYPE_NAMES):
        for n, k in ((14336, 4096), (4096, 14336)):
            nb = tensor_bytes(t, (n, k))
            mats = rotation(lambda: synthetic_weight(n, k, t, gen, "cuda").data, nb)
            for m, xdtype in ((1, torch.bfloat16), (1, torch.float32), (4, torch.bfloat16)):
                x = torch.randn((m, k), device="cuda").to(xdtype)
                y = torch.empty((m, n), device="cuda")
                ms = time_launches([lambda w=w: gguf_gemv(x, w, t, (n, k), out=y) for w in mats], reps)
                alg = nb + x.numel() * x.element_size() + y.numel() * 4
                lines.append({"kernel": "decode GEMV", "ggml_type": TYPE_NAMES[t], "shape": [n, k], "m": m,
                              "x_dtype": str(xdtype).replace("torch.", ""), "us_per_launch": round(ms * 1e3, 3),
                              "GB_s": round(alg / (ms * 1e-3) / 1e9, 1),
                              "frac_hbm_peak": round(alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "alg_bytes": alg})
                log(json.dumps(lines[-1]))
            del mats
    return lines


def traffic_probe(reps: int):
    """The roofline kernel's rotation plus a plain copy of known size, for the
    FETCH_SIZE / WRITE_SIZE counter runs (the copy calibrates the counters)."""
    import torch

    from dracort_amd.runtime.decode import LlamaShape, synthetic_layer_set

    shape = LlamaShape(n_layers=32)
    ls = synthetic_layer_set(shape, seed=0, device="cuda")
    dominant_kernel_roofline(ls, reps)
    src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"traffic probe: {reps} copies of {src.numel()} bytes")


def mfma_probe(reps: int):
    """The prefill GEMMs of configuration 4, launched eagerly ``reps`` times
    each, for the matrix-core counter runs."""
    import torch

    from dracort_amd.kernels import gemm_workspace_bytes, gguf_gemm
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    for n, k in ((14336, 4096), (4096, 14336)):
        w = synthetic_weight(n, k, 12, gen, "cuda")
        for m in (512, 2048):
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), device="cuda")
            ws = torch.empty(gemm_workspace_bytes(12, m, k), dtype=torch.uint8, device="cuda")
            for _ in range(reps):
                gguf_gemm(x, w.data, 12, (n, k), out=y, workspace=ws)
            torch.cuda.synchronize()
            log(f"mfma probe: [{n},{k}] m={m} x{reps}")


def moe_probe(reps: int):
    """Configuration 5's MoE FFN launched eagerly ``reps`` times (kernel traces)."""
    import torch

    from dracort_amd.kernels import gguf_moe, moe_workspace_bytes
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    hid, inter, ne, tok = 4096, 14336, 8, 64
    wg = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wu = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wd = [synthetic_weight(hid, inter, 12, gen, "cuda").data for _ in range(ne)]
    # seeded like the weights: the routing (and so the number of 16-token tiles) is the same every run
    x = torch.randn((tok, hid), generator=gen, device="cuda").to(torch.bfloat16)
    logits = torch.randn((tok, ne), generator=gen, device="cuda")
    ws = torch.empty(moe_workspace_bytes(tok, hid, inter, ne, 2), dtype=torch.uint8, device="cuda")
    y = torch.empty((tok, hid), device="cuda")
    for _ in range(reps):
        gguf_moe(x, logits, wg, wu, wd, 12, inter, top_k=2, workspace=ws, out=y)
    torch.cuda.synchronize()
    log(f"moe probe: x{reps}")


PROBE_LIB = os.path.join(ROOT, "dracort_amd", "lib", "libdraco_probe.so")


def stream_probe(reps: int):
    """The single-launch ceiling: a kernel that only reads (16-byte loads,
    four in flight per thread) one buffer of each decode-step launch size,
    timed like the roofline kernel (HIP events around graph replays of a
    rotation of distinct buffers beyond the Infinity Cache), over several grid
    sizes.  One JSON line per (size, grid) and one summary line per size."""
    import ctypes

    import torch

    lib = ctypes.CDLL(PROBE_LIB)
    lib.draco_probe_stream_read.restype = ctypes.c_int
    lib.draco_probe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_void_p, ctypes.c_void_p]
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    sizes = {"o 4096x4096 Q4_K": 9437184, "q/k/v 6144x4096 Q4_K": 14155776, "gate 14336x4096 Q4_K": 33030144,
             "down 4096x14336 Q6_K": 48168960, "gate+up 2x14336x4096 Q4_K": 66060288}
    lines = []
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for what, nbytes in sizes.items():
        bufs = rotation(lambda: torch.empty(nbytes, dtype=torch.uint8, device="cuda").random_(0, 255), nbytes)
        best = None
        for per_cu in (1, 2, 4, 8):
            for loads in (4, 8, 16):
                blocks = cus * per_cu

                def launch(b=None, blocks=blocks, loads=loads):
                    rc = lib.draco_probe_stream_read(b.data_ptr(), nbytes, blocks, loads, sink.data_ptr(),
                                                     torch.cuda.current_stream().cuda_stream)
                    assert rc == 0, rc

                ms = time_launches([lambda b=b: launch(b) for b in bufs], reps)
                gbs = nbytes / (ms * 1e-3) / 1e9
                line = {"probe": "stream_read", "launch": what, "bytes": nbytes, "workgroups": blocks,
                        "loads_in_flight": loads, "us_per_launch": round(ms * 1e3, 3), "GB_s": round(gbs, 1),
                        "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4), "rotation_bytes": nbytes * len(bufs)}
                log(json.dumps(line))
                lines.append(line)
                if best is None or ms < best["us_per_launch"] / 1e3:
                    best = dict(line)
        lines.append({"probe": "stream_read best", "launch": what, "bytes": nbytes,
                      "us_per_launch": best["us_per_launch"], "GB_s": best["GB_s"],
                      "frac_hbm_peak": best["frac_hbm_peak"], "workgroups": best["workgroups"],
                      "loads_in_flight": best["loads_in_flight"]})
        del bufs
        torch.cuda.empty_cache()
    return lines


def chain_probe(reps: int):
    """Read-only chains with the decode step's launch sizes (32 x [q/k/v, o,
    gate + up, down] + lm_head, 4 841 250 816 B, one buffer beyond the
    Infinity Cache): one launch per phase, with and without a page-translation
    warm-up of the next phase (one 16-byte word per 64 KB touched in each
    launch's last step), against one persistent cooperative launch over all
    phases with no synchronisation (the bound) and with a grid-wide barrier
    between phases (relaxed, or with release / acquire fences).  HIP events
    around `reps` back-to-back chains.  One JSON line per variant."""
    import ctypes

    import torch

    lib = ctypes.CDLL(PROBE_LIB)
    lib.draco_probe_chain_launches.restype = ctypes.c_int
    lib.draco_probe_chain_launches.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
    lib.draco_probe_chain_persistent.restype = ctypes.c_int
    lib.draco_probe_chain_persistent.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                 ctypes.c_void_p]
    sizes = [14155776, 9437184, 66060288, 48168960] * 32 + [430940160]
    offs, tot = [], 0
    for nb in sizes:
        offs += [tot // 16, nb // 16]
        tot += nb
    buf = torch.empty(tot, dtype=torch.uint8, device="cuda").random_(0, 255)
    ph_host = (ctypes.c_int64 * len(offs))(*offs)
    ph_dev = torch.tensor(offs, dtype=torch.int64, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream()
    n = len(sizes)

    def timed(run):
        run()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            run()
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) / reps

    lines = []

    def emit(variant, ms, **kw):
        line = {"probe": "launch_chain", "variant": variant, "phases": n, "bytes": tot,
                "us_per_chain": round(ms * 1e3, 1), "GB_s": round(tot / (ms * 1e-3) / 1e9, 1), **kw}
        log(json.dumps(line))
        lines.append(line)

    for stride_kb in (0, 64, 2048):
        def run(stride_kb=stride_kb):
            rc = lib.draco_probe_chain_launches(buf.data_ptr(), ph_host, n, 8 * cus, stride_kb * 1024 // 16,
                                                sink.data_ptr(), stream.cuda_stream)
            assert rc == 0, rc
        emit("one launch per phase" + (f", next-phase pages touched every {stride_kb} KB" if stride_kb else ""),
             timed(run), workgroups=8 * cus)
    names = {0: "persistent, no synchronisation", 1: "persistent, relaxed grid barrier per phase",
             2: "persistent, release/acquire grid barrier per phase"}
    for mode in (0, 1, 2):
        counters = [torch.zeros(32 * 32, dtype=torch.int32, device="cuda") for _ in range(reps + 1)]
        it = iter(counters)

        def run(mode=mode):
            rc = lib.draco_probe_chain_persistent(buf.data_ptr(), ph_dev.data_ptr(), n, 2 * cus, mode,
                                                  next(it).data_ptr(), err.data_ptr(), sink.data_ptr(),
                                                  stream.cuda_stream)
            assert rc == 0, rc
        ms = timed(run)
        torch.cuda.synchronize()
        emit(names[mode], ms, workgroups=2 * cus, timed_out_waits=int(err.item()))
    base = lines[3]["us_per_chain"]
    for line in lines[4:]:
        line["us_per_barrier"] = round((line["us_per_chain"] - base) / (n - 1), 3)
    return lines


def _timed_cpu(fn, budget_s):
    """Mean seconds per call of fn, repeated until budget_s has passed (at least twice, after one warm call)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if n >= 2 and el >= budget_s:
            return el / n


def config_suite(reps: int, cpu: bool = True):
    """Configurations 1, 2, 4 and 5 at their full sizes on the GPU, each with
    the reference CPU path (the numpy restatement of _dequantize + float32
    x @ W.T, or the float32 MoE) timed beside it on the host cores: warm
    (float32 weights cached, the reference's steady state) and cold
    (dequantization + matmul, its first use), plus one OpenBLAS thread for
    the warm figure; configuration 1 also checks the GPU dequantization
    bit-exact against the oracle's."""
    import numpy as np
    import torch

    from dracort_amd.format.gguf import tensor_bytes
    from dracort_amd.kernels import gguf_dequantize, gguf_gemm, gguf_gemv, gguf_moe, moe_workspace_bytes
    from dracort_amd.runtime.decode import synthetic_weight

    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    cores = len(os.sched_getaffinity(0))
    out = {"cpu_cores": cores, "1": [], "2": [], "4": [], "5": []}
    if cpu:
        from threadpoolctl import threadpool_limits

        from oracle import gguf_ref, matmul_ref

    def cpu_gemv(t, n, k, blocks_dev, ms_list, xs, flops=False):
        """{warm, cold, 1-thread} for the given activations xs (one per GPU line)."""
        blocks = blocks_dev.cpu().numpy()
        res = []
        with threadpool_limits(limits=cores):
            t0 = time.perf_counter()
            w = gguf_ref.dequantize_matrix(t, blocks, (n, k))
            t_dq = time.perf_counter() - t0
            for x in xs:
                t_mm = _timed_cpu(lambda: matmul_ref.cpu_linear_f32(x, w), 0.4)
                res.append({"warm_s": t_mm, "cold_s": t_mm + t_dq})
        with threadpool_limits(limits=1):
            t1 = _timed_cpu(lambda: matmul_ref.cpu_linear_f32(xs[0], w), 0.4)
        return w, res, t1

    def gemv_gpu(t, n, k, m, xdtype):
        nb = tensor_bytes(t, (n, k))
        mats = rotation(lambda: synthetic_weight(n, k, t, gen, "cuda").data, nb, min_total=640 << 20)
        x = torch.randn((m, k), device="cuda").to(xdtype)
        y = torch.empty((m, n), device="cuda")
        ms = time_launches([lambda w=w: gguf_gemv(x, w, t, (n, k), out=y) for w in mats], reps)
        alg = nb + x.numel() * x.element_size() + y.numel() * 4
        return mats, ms, alg

    # 1: Q8_0 4096 x 4096, float32 x, M = 1; GPU dequant bit-exact vs the oracle's
    mats, ms, alg = gemv_gpu(8, 4096, 4096, 1, torch.float32)
    line = {"kernel": "decode GEMV", "ggml_type": "Q8_0", "shape": [4096, 4096], "m": 1, "x_dtype": "float32",
            "us_per_launch": round(ms * 1e3, 3), "GB_s": round(alg / (ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "alg_bytes": alg}
    if cpu:
        xh = np.random.default_rng(1).standard_normal((1, 4096)).astype(np.float32)
        w, res, t1 = cpu_gemv(8, 4096, 4096, mats[0], None, [xh])
        gpu_w = gguf_dequantize(mats[0], 8, (4096, 4096)).cpu().numpy()
        line["cpu"] = {"warm_GB_s": round(alg / res[0]["warm_s"] / 1e9, 2),
                       "cold_GB_s": round(alg / res[0]["cold_s"] / 1e9, 3),
                       "one_thread_warm_GB_s": round(alg / t1 / 1e9, 2), "cores": cores,
                       "dequant_bit_exact": bool(np.array_equal(gpu_w.view(np.uint32), w.view(np.uint32)))}
    out["1"].append(line)
    del mats
    # 2: Q4_0 at the four Llama-3-8B projection shapes, float32 x, M = 1 / 4 / 8
    for n, k in ((4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)):
        lines = []
        for m in (1, 4, 8):
            mats, ms, alg = gemv_gpu(2, n, k, m, torch.float32)
            lines.append({"kernel": "decode GEMV", "ggml_type": "Q4_0", "shape": [n, k], "m": m,
                          "x_dtype": "float32", "us_per_launch": round(ms * 1e3, 3),
                          "GB_s": round(alg / (ms * 1e-3) / 1e9, 1),
                          "frac_hbm_peak": round(alg / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4), "alg_bytes": alg})
            first = mats[0]
            del mats
        if cpu:
            xs = [np.random.default_rng(m).standard_normal((m, k)).astype(np.float32) for m in (1, 4, 8)]
            _, res, t1 = cpu_gemv(2, n, k, first, None, xs)
            for ln, r in zip(lines, res):
                ln["cpu"] = {"warm_GB_s": round(ln["alg_bytes"] / r["warm_s"] / 1e9, 2),
                             "cold_GB_s": round(ln["alg_bytes"] / r["cold_s"] / 1e9, 3), "cores": cores}
            lines[0]["cpu"]["one_thread_warm_GB_s"] = round(lines[0]["alg_bytes"] / t1 / 1e9, 2)
        out["2"] += lines
        torch.cuda.empty_cache()
    # 4: prefill GEMM, Q4_K, bf16 x, M = 512 / 2048
    for n, k in ((14336, 4096), (4096, 14336)):
        wq = synthetic_weight(n, k, 12, gen, "cuda")
        lines, xs = [], []
        for m in (512, 2048):
            x = torch.randn((m, k), device="cuda").to(torch.bfloat16)
            y = torch.empty((m, n), device="cuda")
            ms = time_launches([lambda: gguf_gemm(x, wq.data, 12, (n, k), out=y)], reps)
            flops = 2.0 * m * n * k
            lines.append({"kernel": "prefill GEMM", "ggml_type": "Q4_K", "shape": [n, k], "m": m,
                          "us_per_launch": round(ms * 1e3, 2), "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1),
                          "frac_mfma_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)})
            xs.append(x.float().cpu().numpy())
        if cpu:
            blocks = wq.data.cpu().numpy()
            with threadpool_limits(limits=cores):
                t0 = time.perf_counter()
                w = gguf_ref.dequantize_matrix(12, blocks, (n, k))
                t_dq = time.perf_counter() - t0
                for ln, x in zip(lines, xs):
                    t_mm = _timed_cpu(lambda: matmul_ref.cpu_linear_f32(x, w), 0.5)
                    fl = 2.0 * x.shape[0] * n * k
                    ln["cpu"] = {"warm_GFLOP_s": round(fl / t_mm / 1e9, 1),
                                 "cold_GFLOP_s": round(fl / (t_mm + t_dq) / 1e9, 1), "cores": cores}
            with threadpool_limits(limits=1):
                x0 = xs[0][:64]
                t1 = _timed_cpu(lambda: matmul_ref.cpu_linear_f32(x0, w), 0.5)
                lines[0]["cpu"]["one_thread_warm_GFLOP_s"] = round(2.0 * 64 * n * k / t1 / 1e9, 1)
                lines[0]["cpu"]["one_thread_sample"] = "64 of the 512 rows"
            del w
        out["4"] += lines
        del wq
        torch.cuda.empty_cache()
    # 5: Mixtral-8x7B-shaped MoE FFN, 8 Q4_K experts, 64 bf16 tokens, top-2
    hid, inter, ne, tok = 4096, 14336, 8, 64
    wg = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wu = [synthetic_weight(inter, hid, 12, gen, "cuda").data for _ in range(ne)]
    wd = [synthetic_weight(hid, inter, 12, gen, "cuda").data for _ in range(ne)]
    # seeded like the weights: the routing (and so the number of 16-token tiles) is the same every run
    x = torch.randn((tok, hid), generator=gen, device="cuda").to(torch.bfloat16)
    logits = torch.randn((tok, ne), generator=gen, device="cuda")
    ws = torch.empty(moe_workspace_bytes(tok, hid, inter, ne, 2), dtype=torch.uint8, device="cuda")
    y = torch.empty((tok, hid), device="cuda")
    ms = time_launches([lambda: gguf_moe(x, logits, wg, wu, wd, 12, inter, top_k=2, workspace=ws, out=y)], reps)
    wbytes = sum(t.numel() for t in wg + wu + wd)
    line = {"kernel": "MoE FFN (route + grouped expert GEMVs + combine)", "experts": ne, "tokens": tok, "top_k": 2,
            "us_per_call": round(ms * 1e3, 2), "weight_bytes": wbytes, "GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
            "frac_hbm_peak": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    if cpu:
        # a bounded sample: experts 0 and 1 with the tokens routed to them, scaled to the 8 experts
        xh, lg = x.float().cpu().numpy(), logits.cpu().numpy()
        idx, _ = matmul_ref.route_ref(lg, 2)
        with threadpool_limits(limits=cores):
            t0 = time.perf_counter()
            exps = [(gguf_ref.dequantize_matrix(12, wg[e].cpu().numpy(), (inter, hid)),
                     gguf_ref.dequantize_matrix(12, wu[e].cpu().numpy(), (inter, hid)),
                     gguf_ref.dequantize_matrix(12, wd[e].cpu().numpy(), (hid, inter))) for e in range(2)]
            t_dq = time.perf_counter() - t0
            # the real routing; only experts 0 and 1 carry weights, so exactly their token sets are computed
            t_mm = _timed_cpu(lambda: matmul_ref.cpu_moe_f32(xh, lg, exps, 2), 1.0)
        share = (idx < 2).sum() / idx.size  # the sample's fraction of the 128 (token, expert) pairs
        scale = 1.0 / max(share, 1e-9)
        line["cpu"] = {"warm_GB_s": round(wbytes / (t_mm * scale) / 1e9, 2),
                       "cold_GB_s": round(wbytes / ((t_mm + t_dq) * scale) / 1e9, 3), "cores": cores,
                       "sample": f"experts 0-1 ({int((idx < 2).sum())} of 128 token-expert pairs), scaled to all 8"}
        del exps
    out["5"].append(line)
    del wg, wu, wd
    torch.cuda.empty_cache()
    return out


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
    ap.add_argument("--full-context", type=int, default=1024,
                    help="also time the full decode step (norms + attention) at this context (0: skip)")
    ap.add_argument("--suite", action="store_true", help="measure configurations 1, 2, 4, 5 (one JSON line each)")
    ap.add_argument("--gemv-probe", action="store_true", help="configurations 1 and 2 only (kernel traces)")
    ap.add_argument("--types", action="store_true", help="decode GEMV of every GGUF block type (one JSON line each)")
    ap.add_argument("--traffic-probe", action="store_true", help="run only the roofline rotation + a 256 MB copy")
    ap.add_argument("--mfma-probe", action="store_true", help="run only the configuration-4 GEMMs (counter runs)")
    ap.add_argument("--moe-probe", action="store_true", help="run only the configuration-5 MoE FFN (kernel traces)")
    ap.add_argument("--chain-probe", action="store_true",
                    help="read-only chains of the step's launch sizes: launches vs one persistent kernel with barriers")
    ap.add_argument("--stream-probe", action="store_true",
                    help="time a read-only kernel on each decode-launch size (the single-launch ceiling)")
    ap.add_argument("--no-batch16", action="store_true", help="skip the batch-16 decode steps of the default line")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip configurations 1, 2, 4, 5 (GPU and CPU) in the default run")
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
    if args.suite or args.gemv_probe:
        for line in suite(args.roofline_reps, gemv_only=args.gemv_probe):
            print(json.dumps(line), flush=True)
        return 0
    if args.types:
        for line in types_suite(args.roofline_reps):
            print(json.dumps(line), flush=True)
        return 0
    if args.traffic_probe:
        traffic_probe(args.roofline_reps)
        return 0
    if args.mfma_probe:
        mfma_probe(3)
        return 0
    if args.moe_probe:
        moe_probe(3)
        return 0
    if args.chain_probe:
        for line in chain_probe(10):
            print(json.dumps(line), flush=True)
        return 0
    if args.stream_probe:
        for line in stream_probe(args.roofline_reps):
            print(json.dumps(line), flush=True)
        return 0
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

    full = None
    if args.full_context > 0:
        full = full_decode(ls, args.batch, args.full_context, max(10, args.steps // 2), 2)
        log(f"full decode step: {full}")

    # the same layer set decoded for 16 sequences at once (one token each):
    # the projection step and the full step, reported beside the batch-1 value
    batch16 = None
    if args.batch == 1 and not args.no_batch16:
        b16 = DecodeStep(ls, m=16)
        b16.capture()
        for _ in range(3):
            b16.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n16 = max(10, args.steps // 2)
        e0.record(stream)
        for _ in range(n16):
            b16.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        ms16 = e0.elapsed_time(e1) / n16
        del b16
        torch.cuda.empty_cache()
        batch16 = {"batch": 16, "ms_per_step": round(ms16, 4), "tokens_per_s": round(16e3 / ms16, 2),
                   "weight_GB_s": round(step_bytes / (ms16 * 1e-3) / 1e9, 1), "steps": n16,
                   "full_decode": full_decode(ls, 16, args.full_context, n16, 2) if args.full_context > 0 else None}
        log(f"batch-16 decode: {batch16}")

    roof = dominant_kernel_roofline(ls, args.roofline_reps)
    log(f"roofline: {roof}")
    dom = step_dominant_roofline(ls, args.roofline_reps)
    log(f"step-dominant launch: {dom}")

    configs = None
    if not args.no_configs:
        t0 = time.time()
        configs = config_suite(max(5, args.roofline_reps // 2), cpu=not args.no_cpu_baseline)
        log(f"configurations 1, 2, 4, 5 ({time.time() - t0:.1f} s): {json.dumps(configs)}")

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
        "full_decode": full,
        "batch16": batch16,
        "roofline": roof,
        "roofline_step_dominant": dom,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

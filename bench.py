"""Decode / verify attention over the Q8_0 paged KV pool on one MI355X.

Default workload: BASELINE config 1 (the metric's config that fits one GPU): 4 sequences at contexts 8K / 16K / 32K /
64K sharing one pool of 256-token pages with a seeded random page interleaving, each running a speculative-verify
step of T = 3 query tokens, through all 12 full-attention layers (16 Q heads, 2 KV heads, d 256). A step = for each
layer, one fnkv_attn_decode launch that appends the step's 3 new K/V cells per sequence (Q8_0) and attends over the
whole context (split-K over pages + log-sum-exp merge). Steps repeat at the same positions (a verify step whose draft
is rejected overwrites the same cells next time), so the pool does not grow; the step is captured once in a HIP graph
and replayed. K/V/Q are synthetic, seeded, BASELINE's distribution (N(0,1), 4 of 256 channels x8).

Prints one JSON line: tokens/s (query tokens of all sequences through all 12 layers per second), with GB/s of
algorithmic HBM bytes, the roofline of the attention launch, and the CPU baseline (the oracle's ggml-semantics flash
attention, multithreaded, on a bounded sample) measured in the same run.
"""
import argparse
import csv
import glob
import json
import os
import shutil
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "fnfl-v100_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

HQ, HKV, D = 16, 2, 256
BYTES_PER_CELL_LAYER = 2 * HKV * (D + 2 * (D // 32))  # K and V, both heads: codes + fp16 scales = 1,088 B
PEAK_HBM_GBS = 8000.0

CONFIGS = {
    "cfg1": dict(ctxs=[8192, 16384, 32768, 65536], T=3, layers=12,
                 workload="cfg1: 4 seqs 8K/16K/32K/64K, verify T=3, 12 layers, shared Q8_0 pool, permuted pages"),
    "cfg1kv8": dict(ctxs=[8192, 16384, 32768, 65536], T=3, layers=12, fmt="kv8",
                    workload="cfg1 on a KV8 pool (FNFL's group-64 8-bit format, fn/quant/kv_q8_ref.cpp): 4 seqs "
                             "8K/16K/32K/64K, verify T=3, 12 layers, permuted pages"),
    "cfg2": dict(ctxs=[262144], T=1, layers=1, copies=4,
                 workload="cfg2: 1 seq 262,144 cells, decode T=1, 1 layer, scattered pages"),
    "cfg2v": dict(ctxs=[262144], T=5, layers=1, copies=4,
                  workload="cfg2: 1 seq 262,144 cells, verify T=5, 1 layer, scattered pages"),
    "cfg0": dict(ctxs=[4096], T=1, layers=1, copies=64, workload="cfg0: 1 seq 4,096 cells, decode T=1, 1 layer"),
    "cfg3": dict(ctxs=[131072 + 2048], T=2048, layers=1, prefill=True,
                 workload="cfg3: 2,048-token fp16 chunk appended at depth 131,072 and attended causally over 133,120 "
                          "cells (chunked prefill, matrix cores), 1 layer"),
    "qsa3": dict(depth=196608 - 3, T=3, layers=12, sparse=True,
                 workload="qsa3: sparse (QSA) attention, 3 rows at 196,608 cells, each over its own 512 blocks + tail "
                          "(random, rows disjoint: the reference's QA2 shape), 12 layers"),
    "qsa1": dict(depth=196608 - 1, T=1, layers=12, sparse=True,
                 workload="qsa1: sparse (QSA) attention, 1 row at 196,608 cells over 512 blocks + tail, 12 layers"),
    "qa2b3": dict(depth=196608 - 3, T=3, layers=12, attend=True,
                  workload="qa2b3: attn::attend over the Q8_0 pool at the reference's QA2 shape: 12 query heads on one "
                           "KV head, 3 rows at 196,608 cells, each over its own 512 blocks + tail, prepare (norm, IMROPE) "
                           "and gate included, 12 layers"),
    "qa2b1": dict(depth=196608 - 1, T=1, layers=12, attend=True,
                  workload="qa2b1: the same with 1 row"),
    "datc": dict(cells=196608, datc=True,
                 workload="datc: DA-TC draft step row (prepare with q, dense attention, gate) at 196,608 cells of F16 "
                          "K/V, 12 query heads, the reference's deepest draft-bench point"),
    "datc4k": dict(cells=4096, datc=True,
                   workload="datc4k: DA-TC draft step row at 4,096 cells of F16 K/V (the reference's shallowest point)"),
}
PEAK_MFMA_F16_TFLOPS = 2500.0  # dense fp16 matrix-core peak


def prefill_flops(ctx, rows):
    """4 d flops a visible (query, key) pair and query head: QK^T and PV, 2 d each"""
    pairs = sum(ctx - rows + t + 1 for t in range(rows))
    return 4 * D * HQ * pairs


def algorithmic_bytes(ctxs, T):
    """Per layer: K+V read over every cell (the T new ones included), Q in and O out (fp16), the T new cells'
    Q8_0 write and their fp16 K/V read."""
    kv_read = sum(ctxs) * BYTES_PER_CELL_LAYER
    qo = len(ctxs) * T * HQ * D * 2 * 2
    append = len(ctxs) * T * (BYTES_PER_CELL_LAYER + 2 * HKV * D * 2)
    return kv_read + qo + append


def make_pool(torch, fnkv, cases, ctxs, T, layers, seed, h_kv=HKV, fmt=None):
    n_pages = sum(-(-c // 256) for c in ctxs) + 16
    pool = fnkv.Pool(len(ctxs) + 1, n_pages, layers, h_kv, **({} if fmt is None else {"fmt": fmt}))
    slots = list(range(len(ctxs)))
    cases.scatter_ensure(pool, slots, ctxs, seed, churn=0.2)
    g = torch.Generator(device="cuda")
    for layer in range(layers):
        g.manual_seed(seed * 1000 + layer)
        for s, c in zip(slots, ctxs):
            kv = []
            for _ in range(2):
                x = torch.randn((c, h_kv, D), generator=g, device="cuda", dtype=torch.float32)
                ch = torch.randperm(D, generator=g, device="cuda")[:4]
                x[:, :, ch] *= 8.0
                kv.append(x.half())
            pool.append(s, layer, 0, kv[0], kv[1])
    torch.cuda.synchronize()
    return pool, slots


def cpu_baseline(ctxs, T, layers, seed, threads):
    """The oracle's ggml-semantics CPU flash attention (fp32 Q) on one layer of the workload (all sequences),
    scaled to tokens/s of the whole step; returns the dict for the JSON line."""
    import numpy as np

    import cases
    import oracle as O

    t_layer = 0.0
    for i, c in enumerate(ctxs):
        k16, v16 = cases.kv_rows(seed + i, c, HKV)
        (kq, kd, _), (vq, vd, _) = cases.decoded(O, k16, v16)
        kb, vb = O.to_block_q8_0(kq, kd), O.to_block_q8_0(vq, vd)
        q16 = cases.queries(seed + i, (T, HQ, D)).view(np.uint16)
        O.attn_ggml(q16, kb, vb, min(c, 2048), threads=threads)  # warm the threads and caches
        t0 = time.perf_counter()
        O.attn_ggml(q16, kb, vb, c, threads=threads)
        t_layer += time.perf_counter() - t0
    tokens = len(ctxs) * T
    tok_s = tokens / (t_layer * layers)
    return {
        "value": round(tok_s, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 of {layers} layers, all {len(ctxs)} sequences at full context, T={T}, fp32-Q ggml-semantics "
                  f"flash attention over Q8_0 K/V (oracle/fnkv_oracle.c or_attn_ggml), {threads} threads; "
                  f"layer time {t_layer * 1e3:.1f} ms x {layers} layers",
        "gb_s": round(algorithmic_bytes(ctxs, T) / t_layer / 1e9, 3),
    }


COPY_BYTES = 1 << 30  # the calibration copy: 1 GiB read, 1 GiB written


def traffic_child(args, torch, run_step):
    """The child of a counter pass: the workload's launches (eager, a few steps), then a plain elementwise copy of
    COPY_BYTES (torch.neg into a second buffer) three times, whose counter readings calibrate the counter's unit."""
    for _ in range(3):
        run_step()
    torch.cuda.synchronize()
    src = torch.ones(COPY_BYTES // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def _counter_means(out_dir):
    """rocprofv3 counter CSV -> {kernel name: mean counter value per dispatch}"""
    sums, counts = {}, {}
    for f in glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for row in csv.DictReader(fh):
                k = row.get("Kernel_Name", "")
                sums[k] = sums.get(k, 0.0) + float(row.get("Counter_Value", 0.0))
                counts[k] = counts.get(k, 0) + 1
    return {k: sums[k] / counts[k] for k in sums}


def measure_traffic(argv, kernels=("decode", "merge_kernel")):
    """HBM bytes of one fnkv_attn_decode launch (decode + merge kernels) from two rocprofv3 counter passes over a child
    run of the same workload: FETCH_SIZE, then WRITE_SIZE (KiB a dispatch), each scaled by bytes / reading of the
    same counter for the calibration copy of known size in the same child. Runs before this process touches the GPU.
    Returns (traffic bytes, detail dict) or (None, reason)."""
    rocprof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not os.path.exists(rocprof):
        return None, "rocprofv3 not found"
    env = dict(os.environ, TMPDIR="/tmp")
    detail = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        out_dir = tempfile.mkdtemp(prefix="fnkv_pmc_", dir="/tmp")
        cmd = [rocprof, "--pmc", counter, "--output-format", "csv", "-d", out_dir, "-o", "run", "--",
               sys.executable, os.path.abspath(__file__), "--traffic-child", *argv]
        try:
            r = subprocess.run(cmd, timeout=180, capture_output=True, text=True, env=env, cwd="/tmp")
        except subprocess.TimeoutExpired:
            return None, f"{counter} pass timed out"
        means = _counter_means(out_dir)
        shutil.rmtree(out_dir, ignore_errors=True)
        if r.returncode != 0 or not means:
            return None, f"{counter} pass failed ({r.returncode})"
        # the launch's kernels (one dispatch each a launch): the fnkv kernels whose names hold one of `kernels`
        launch = sum(v for k, v in means.items() if "fnkv" in k and any(n in k for n in kernels))
        copy = [v for k, v in means.items() if "neg" in k.lower()]
        if not copy or copy[0] <= 0 or launch <= 0:
            return None, f"{counter}: kernels not found in the counter output"
        factor = COPY_BYTES / (copy[0] * 1024.0)
        detail[counter] = {"kib_per_launch": round(launch, 1), "copy_kib": round(copy[0], 1),
                           "scale_bytes_per_kib": round(factor, 2), "bytes_per_launch": int(launch * 1024 * factor)}
    total = detail["FETCH_SIZE"]["bytes_per_launch"] + detail["WRITE_SIZE"]["bytes_per_launch"]
    return total, detail


def run_prefill(args, cfg):
    """one step = the chunk's Q8_0 append (fnkv_q8_append) + its causal attention over the whole
    context (fnkv_attn_prefill), captured in a HIP graph; the roofline is the matrix cores' (algorithmic flops)."""
    import numpy as np
    import torch

    import cases
    import fnkv

    ctx, rows = cfg["ctxs"][0], cfg["T"]
    depth = ctx - rows
    torch.cuda.set_device(0)
    pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, HKV)
    cases.scatter_ensure(pool, [0], [ctx], args.seed, churn=0.2)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    kv = []
    for _ in range(2):
        x = torch.randn((ctx, HKV, D), generator=g, device="cuda", dtype=torch.float32)
        ch = torch.randperm(D, generator=g, device="cuda")[:4]
        x[:, :, ch] *= 8.0
        kv.append(x.half())
    pool.append(0, 0, 0, kv[0][:depth].contiguous(), kv[1][:depth].contiguous())
    kc, vc = kv[0][depth:].contiguous(), kv[1][depth:].contiguous()
    q = torch.randn((rows, HQ, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws_n = pool.prefill_ws_bytes(ctx, rows, HQ)
    ws = torch.empty(max(ws_n, 16), dtype=torch.uint8, device="cuda") if ws_n > 0 else False

    def step():
        pool.append(0, 0, depth, kc, vc)
        pool.prefill(0, 0, ctx, q, out, ws=ws)

    step()
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
    run = graph.replay if graph is not None else step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"
    flops = prefill_flops(ctx, rows)
    step_s = gpu_s / args.steps
    tflops = flops / step_s / 1e12
    line = {
        "metric": "chunked-prefill attention over the Q8_0 paged KV: tokens/s and matrix-core TFLOP/s",
        "value": round(rows * args.steps / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 KV dequantized to fp16 hi + lo, fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q)",
        "config": {"workload": cfg["workload"], "context": ctx, "chunk": rows, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "page_tokens": 256, "hip_graph": graph is not None},
        "roofline": {
            "kernel": "fnkv_q8_append + fnkv_attn_prefill (append_kernel + prefill_kernel + prefill_merge_kernel), per step",
            "bound": "mfma",
            "achieved": round(tflops, 3),
            "peak": PEAK_MFMA_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_MFMA_F16_TFLOPS, 4),
            "traffic": None,
            "flops_per_step": flops,
            "step_us": round(step_s * 1e6, 3),
        },
    }
    if not args.no_cpu:
        import oracle as O
        threads = max(1, min(16, os.cpu_count() or 1))
        sample = 16
        (kq, kd, _), (vq, vd, _) = cases.decoded(O, kv[0].cpu().numpy(), kv[1].cpu().numpy())
        kb, vb = O.to_block_q8_0(kq, kd), O.to_block_q8_0(vq, vd)
        q16 = q[-sample:].cpu().numpy().view(np.uint16)
        O.attn_ggml(q16[:1], kb, vb, 2048, threads=threads)
        t1 = time.perf_counter()
        O.attn_ggml(q16, kb, vb, ctx, threads=threads)
        dt = time.perf_counter() - t1
        sample_flops = 4 * D * HQ * sum(ctx - sample + t + 1 for t in range(sample))
        cpu_step = dt * flops / sample_flops
        line["cpu_baseline"] = {
            "value": round(rows / cpu_step, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the chunk's last {sample} of {rows} query rows over the full context, fp32-Q ggml-semantics "
                      f"flash attention (oracle/fnkv_oracle.c or_attn_ggml), {threads} threads, {dt:.2f} s, scaled "
                      f"by visible pairs to the chunk",
            "tflops": round(sample_flops / dt / 1e12, 4),
        }
    print(json.dumps(line), flush=True)
    pool.close()


def run_sparse(args, cfg):
    """Sparse (QSA) attention: one step = for each of the 12 layers one fnkv_attn_sparse launch (the rows' own cells
    written, each row attending to its 512 selected blocks and tail), captured in a HIP graph. Algorithmic bytes: the
    selected cells' K and V (both heads), Q in and O out, the new cells' write."""
    import numpy as np
    import torch

    import cases
    import fnkv
    import oracle as O

    depth, T, layers = cfg["depth"], cfg["T"], cfg["layers"]
    ctx = depth + T
    torch.cuda.set_device(0)
    pool, slots = make_pool(torch, fnkv, cases, [ctx], T, layers, args.seed)
    bodies, cells = [], []
    for layer in range(layers):
        w, o, c = O.qsa_body(depth, T, args.seed + layer)
        bodies.append((torch.from_numpy(w.view(np.int32)).cuda(), torch.from_numpy(o).cuda()))
        cells.append(c)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    q = torch.randn((layers, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers, T, HKV, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.empty(pool.sparse_ws_bytes(depth, T, HQ), dtype=torch.uint8, device="cuda")

    def step():
        for layer in range(layers):
            pool.sparse(0, depth, layer, q[layer], bodies[layer][0], bodies[layer][1], out[layer], ws=ws,
                        k_new=kn[layer], v_new=vn[layer])

    step()
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
    run = graph.replay if graph is not None else step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"
    sel = sum(sum(c.size for c in cl) for cl in cells) / layers  # selected cells a layer, all rows
    bytes_layer = int(sel * BYTES_PER_CELL_LAYER + T * HQ * D * 2 * 2 + T * (BYTES_PER_CELL_LAYER + 2 * HKV * D * 2))
    launch_s = gpu_s / (args.steps * layers)
    achieved = bytes_layer / launch_s / 1e9
    tiles = len(np.unique(np.concatenate([c // 32 for c in cells[0]])))
    line = {
        "metric": "sparse (QSA) decode attention over the Q8_0 pool: tokens/s + achieved GB/s of the selected cells",
        "value": round(T * args.steps / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 KV (int8 codes + fp16 scales), fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q; random selections)",
        "config": {"workload": cfg["workload"], "cells": ctx, "rows": T, "layers": layers, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "selected_cells_per_layer": int(sel),
                   "tiles_read_per_layer_per_head": tiles, "hip_graph": graph is not None},
        "roofline": {
            "kernel": "fnkv_attn_sparse launch (sparse_plan_kernel + decode kernel + merge_kernel), per layer",
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": None,
            "traffic_note": f"whole 17,408 B tiles are read: {tiles} a head a layer for {int(sel)} selected cells",
            "bytes_per_launch": bytes_layer,
            "launch_us": round(launch_s * 1e6, 3),
        },
    }
    if not args.no_cpu:
        threads = max(1, min(16, os.cpu_count() or 1))
        k16, v16 = cases.kv_rows(args.seed, ctx, HKV)
        q16 = cases.queries(args.seed, (T, HQ, D)).view(np.uint16)
        t_layer = 0.0
        for t in range(T):
            c = cells[0][t]
            (kq, kd, _), (vq, vd, _) = cases.decoded(O, k16[c], v16[c])
            kb, vb = O.to_block_q8_0(kq, kd), O.to_block_q8_0(vq, vd)
            O.attn_ggml(q16[t:t + 1], kb, vb, c.size, threads=threads)
            t1 = time.perf_counter()
            O.attn_ggml(q16[t:t + 1], kb, vb, c.size, threads=threads)
            t_layer += time.perf_counter() - t1
        line["cpu_baseline"] = {
            "value": round(T / (t_layer * layers), 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"1 of {layers} layers: each row's selected cells gathered, fp32-Q ggml-semantics flash attention "
                      f"over them (oracle/fnkv_oracle.c or_attn_ggml), {threads} threads, {t_layer * 1e3:.2f} ms a "
                      f"layer x {layers}",
        }
    print(json.dumps(line), flush=True)
    pool.close()


def run_attend(args, cfg):
    """fnkv_qsa_attend (attn::attend, fn/kernels/qsa/attend.h:57-141) at the reference's QA2 shape: one step = for
    each of the 12 layers one call that prepares the rows' q and k (RMS norm, IMROPE), writes the new cells, attends
    each row over its selection and gates the output (F32 + int8 activation format), captured in a HIP graph. The
    reference measured its BF16 kernel for this shape at 29.2 us (B = 3) and 22.5 us (B = 1) warm on a V100
    (attend.h:47-48)."""
    import numpy as np
    import torch

    import cases
    import fnkv
    import oracle as O

    depth, T, layers = cfg["depth"], cfg["T"], cfg["layers"]
    hq, h_kv = 12, 1
    ctx = depth + T
    torch.cuda.set_device(0)
    pool, slots = make_pool(torch, fnkv, cases, [ctx], T, layers, args.seed, h_kv=h_kv)
    bodies, cells = [], []
    for layer in range(layers):
        w, o, c = O.qsa_body(depth, T, args.seed + layer)
        bodies.append((torch.from_numpy(w.view(np.int32)).cuda(), torch.from_numpy(o).cuda()))
        cells.append(c)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    qfull = torch.empty((layers, T, hq, 512), device="cuda").uniform_(-3.0, 3.0, generator=g)
    kv = torch.empty((layers, 2, T, h_kv, D), device="cuda").uniform_(-2.0, 2.0, generator=g)
    norms = torch.empty((2, D), device="cuda").uniform_(0.3, 1.8, generator=g)
    pos = torch.arange(depth, ctx, dtype=torch.int32, device="cuda").repeat(4, 1).contiguous()
    out = torch.empty((layers, T, hq, D), device="cuda")
    codes = torch.empty((layers, T, hq * D), dtype=torch.int8, device="cuda")
    scales = torch.empty((layers, T, hq * 8, 2), device="cuda")
    ws = torch.empty(pool.qsa_ws_bytes(depth, T, hq), dtype=torch.uint8, device="cuda")

    def step():
        for layer in range(layers):
            pool.qsa_attend(0, depth, layer, qfull[layer], kv[layer, 0], kv[layer, 1], norms[0], norms[1], pos,
                            bodies[layer][0], bodies[layer][1], out[layer], codes[layer], scales[layer], ws=ws)

    step()
    torch.cuda.synchronize()
    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
    run = graph.replay if graph is not None else step
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out).all().item(), "non-finite attention output"
    cell_bytes = h_kv * 2 * (D + 2 * (D // 32))  # K and V of the one KV head: 544 B a cell
    sel = sum(sum(c.size for c in cl) for cl in cells) / layers
    bytes_layer = int(sel * cell_bytes + T * hq * 512 * 4 + T * h_kv * D * 4 * 2 + T * hq * D * (4 + 1)
                      + T * hq * 8 * 8 + T * cell_bytes)
    launch_s = gpu_s / (args.steps * layers)
    achieved = bytes_layer / launch_s / 1e9
    tiles = len(np.unique(np.concatenate([c // 32 for c in cells[0]])))
    line = {
        "metric": "attn::attend over the Q8_0 pool at the reference's QA2 shape: tokens/s and us an attend call",
        "value": round(T * args.steps / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 KV (int8 codes + fp16 scales), fp16 q operand, fp32 prepare / softmax / accumulate / out",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8; uniform q / k / v / gates / norms; random "
                "selections)",
        "config": {"workload": cfg["workload"], "cells": ctx, "rows": T, "layers": layers, "q_heads": hq,
                   "kv_heads": h_kv, "head_dim": D, "selected_cells_per_layer": int(sel),
                   "tiles_read_per_layer": tiles, "hip_graph": graph is not None},
        "roofline": {
            "kernel": "fnkv_qsa_attend call (qsa_prepare_kernel + decode kernel (sparse) + merge_kernel (gated)), "
                      "a layer",
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": None,
            "traffic_note": f"whole 17,408 B tiles are read: {tiles} a layer for {int(sel)} selected cells",
            "bytes_per_launch": bytes_layer,
            "launch_us": round(launch_s * 1e6, 3),
            "reference_v100_us": 29.2 if T == 3 else 22.5 if T == 1 else None,
        },
    }
    print(json.dumps(line), flush=True)
    pool.close()


def run_datc(args, cfg):
    """DA-TC's draft step row (fn/kernels/draft/draft.h:47-83): one step = fnkv_datc_prepare (the row's 12 query heads
    and its new cell's K / V) then fnkv_datc_attend (the attention over every cell, the fold, the gate), one HIP graph
    a step. Every cell comes from HBM: the steps rotate over copies of the caches totalling over 1 GB (the reference's
    warm bench rotates over 200 MB for the V100's 6 MB L2; MI355X's last-level cache is 256 MB). Algorithmic bytes a
    step: K and V of the cells (1,024 B a cell), the prepare's inputs and outputs, the attend's q16, gates and outputs."""
    traffic, traffic_detail = None, "skipped (--no-traffic)"
    if not args.traffic_child and not args.no_traffic:
        passthrough = [x for x in sys.argv[1:] if x not in ("--no-cpu",)]
        traffic, traffic_detail = measure_traffic(passthrough, ("datc_attend_kernel", "datc_fold_kernel",
                                                                "datc_prepare_kernel"))
    import numpy as np
    import torch

    import fnkv
    import oracle as O

    n = cfg["cells"]
    nb, NHd, HDd = n - 1, fnkv.DATC_HEADS, 256
    max_cells = n + 8
    copy_bytes = max_cells * HDd * 2 * 2
    copies = max(2, min(512, -(-1_200_000_000 // copy_bytes)))
    torch.cuda.set_device(0)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed)
    caches = torch.randn((copies, 2, max_cells, HDd), generator=g, device="cuda").half().view(torch.int16)
    qfull = torch.empty((1, NHd, 512), device="cuda").uniform_(-3.0, 3.0, generator=g)
    kv = torch.empty((2, 1, HDd), device="cuda").uniform_(-2.0, 2.0, generator=g)
    norms = torch.empty((2, HDd), device="cuda").uniform_(0.3, 1.8, generator=g)
    ints = torch.tensor([nb, 1], dtype=torch.int32, device="cuda")
    pos = torch.full((4, 1), nb, dtype=torch.int32, device="cuda")
    q16 = torch.empty((1, NHd, HDd), dtype=torch.int16, device="cuda")
    part = torch.empty(fnkv.datc_part_bytes() // 4, dtype=torch.float32, device="cuda")
    out = torch.empty(NHd * HDd, dtype=torch.float32, device="cuda")
    codes = torch.empty(NHd * HDd, dtype=torch.int8, device="cuda")
    scales = torch.empty(NHd * HDd // 16, dtype=torch.float32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")

    fused = not args.datc_two_call

    def step(i):
        kc, vc = caches[i][0], caches[i][1]
        if fused:
            fnkv.datc_step(kv_k=kv[0], kv_v=kv[1], k_norm=norms[1], n_before=ints[0:1], pos=pos, stride=ints[1:2],
                           k_cache=kc, v_cache=vc, err=err, qfull=qfull, q_norm=norms[0], q16=q16, part=part,
                           out=out, codes=codes, scales=scales)
            return
        fnkv.datc_prepare(1, kv_k=kv[0], kv_v=kv[1], k_norm=norms[1], n_before=ints[0:1], pos=pos, stride=ints[1:2],
                          k_cache=kc, v_cache=vc, err=err, qfull=qfull, q_norm=norms[0], q16=q16)
        fnkv.datc_attend(q16=q16, qfull=qfull, k_cache=kc, v_cache=vc, n_before=ints[0:1], part=part, out=out,
                         codes=codes, scales=scales, err=err)

    for i in range(copies):
        step(i)
    torch.cuda.synchronize()
    if args.traffic_child:
        traffic_child(args, torch, lambda: step(0))
        return
    # one graph holds `copies` steps, one on each copy of the caches (the reference's bench times graphs of n_copy
    # steps, fn/kernels/draft/draft_bench.cu:250-292); K steps = ceil(K / copies) replays
    replays = max(1, -(-args.steps // copies))
    warm = max(1, -(-args.warmup // copies))
    run = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step(0)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(copies):
                step(i)
        torch.cuda.synchronize()
        run = graph.replay
    else:
        def run():
            for i in range(copies):
                step(i)
    for _ in range(warm):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(replays):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    n_steps = replays * copies
    assert int(err.item()) == 0, "DA-TC error word set"
    assert torch.isfinite(out).all().item(), "non-finite attention output"
    step_s = gpu_s / n_steps
    bytes_step = (n * HDd * 2 * 2  # K and V of every cell
                  + NHd * 512 * 4 + 2 * HDd * 4 + 2 * HDd * 4 + 4 * 4  # prepare: qfull, k / v, norms, positions
                  + NHd * HDd * 2 + 2 * HDd * 2  # q16 and the new cell written
                  + (0 if fused else NHd * HDd * 2) + NHd * HDd * 4  # attend: q16 (two calls) and the gates read
                  + NHd * HDd * 4 + NHd * HDd + NHd * HDd // 16 * 4)  # out, codes, scales written
    achieved = bytes_step / step_s / 1e9
    line = {
        "metric": "DA-TC draft step row (prepare + dense F16 attention + gate): steps/s and achieved GB/s",
        "value": round(n_steps / wall, 3),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": n_steps,
        "warmup": warm * copies,
        "ms_per_step": round(wall / n_steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 K/V and q, f32 accumulate and softmax, f16 P",
        "data": "synthetic (seeded N(0,1) F16 caches, uniform q / k / v / gates / norms)",
        "config": {"workload": cfg["workload"], "cells": n, "q_heads": NHd, "head_dim": HDd,
                   "cache_copies_rotated": copies, "rotated_mb": round(copies * copy_bytes / 1e6),
                   "steps_per_graph": copies, "hip_graph": not args.no_graph,
                   "entry": "fnkv_datc_step" if fused else "fnkv_datc_prepare + fnkv_datc_attend"},
        "roofline": {
            "kernel": ("fnkv_datc_step (datc_attend_kernel, datc_fold_kernel with the prepare folded in)" if fused
                       else "fnkv_datc_prepare + fnkv_datc_attend (datc_prepare_kernel, datc_attend_kernel, "
                            "datc_fold_kernel)") + ", a step",
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_detail": traffic_detail,
            "bytes_per_launch": bytes_step,
            "launch_us": round(step_s * 1e6, 3),
            "reference_floor_v100_us": round(1.95 + n * 1024 / 1021.6e3, 2),
        },
    }
    if not args.no_cpu:
        from threadpoolctl import threadpool_limits
        threads = max(1, min(16, os.cpu_count() or 1))
        kh = caches[0][0].cpu().numpy().view(np.uint16)
        vh = caches[0][1].cpu().numpy().view(np.uint16)
        qh = q16[0].cpu().numpy().view(np.uint16)
        gate = qfull[0, :, 256:].cpu().numpy()
        cells = np.arange(n)
        with threadpool_limits(limits=threads):
            O.datc_attn_f64(qh, gate, kh, vh, cells)
            reps, t1 = 0, time.perf_counter()
            while reps < 3 or time.perf_counter() - t1 < 2.0:
                O.datc_attn_f64(qh, gate, kh, vh, cells)
                reps += 1
            cpu_s = (time.perf_counter() - t1) / reps
        line["cpu_baseline"] = {
            "value": round(1.0 / cpu_s, 3), "unit": "steps/s", "cores": threads, "kind": "port",
            "sample": f"the attention of one step row over all {n} cells in fp64 numpy (oracle/oracle.py "
                      f"datc_attn_f64, BLAS threads capped at {threads}), {reps} reps, {cpu_s * 1e3:.1f} ms each; the "
                      f"reference has no CPU path for DA-TC",
        }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="cfg1", choices=sorted(CONFIGS))
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--T", type=int, default=None, help="override the config's query tokens a sequence")
    ap.add_argument("--ctxs", default=None, help="override the config's contexts (comma-separated cells)")
    ap.add_argument("--no-append", action="store_true", help="attend only (the step's cells appended beforehand)")
    ap.add_argument("--datc-two-call", action="store_true",
                    help="DA-TC: time fnkv_datc_prepare then fnkv_datc_attend instead of fnkv_datc_step")
    ap.add_argument("--no-traffic", action="store_true", help="skip the two rocprofv3 counter passes (traffic: null)")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the path is measured on one MI355X); --gpus must be 1",
              file=sys.stderr)
        sys.exit(2)
    if CONFIGS[args.config].get("prefill"):
        run_prefill(args, CONFIGS[args.config])
        return
    if CONFIGS[args.config].get("sparse"):
        run_sparse(args, CONFIGS[args.config])
        return
    if CONFIGS[args.config].get("datc"):
        run_datc(args, CONFIGS[args.config])
        return
    if CONFIGS[args.config].get("attend"):
        run_attend(args, CONFIGS[args.config])
        return

    traffic, traffic_detail = None, "skipped (--no-traffic)"
    if not args.traffic_child and not args.no_traffic:
        passthrough = [a for a in sys.argv[1:] if a not in ("--no-cpu",)]
        traffic, traffic_detail = measure_traffic(passthrough)

    import torch

    import cases
    import fnkv

    cfg = CONFIGS[args.config]
    ctxs, T, layers = cfg["ctxs"], cfg["T"], cfg["layers"]
    if args.T is not None:
        T = args.T
    if args.ctxs is not None:
        ctxs = [int(c) for c in args.ctxs.split(",")]
    workload = cfg["workload"] if (args.T is None and args.ctxs is None) else f"custom: contexts {ctxs}, T={T}, {layers} layers"
    # a single-layer step is one short launch pair: the graph then holds `copies` steps, each over its own layer of the
    # pool (over 1 GB of caches in all, beyond the 256 MB last-level cache), so one replay's idle gap is spread over
    # several steps as it is over a many-layer step (cfg1's 12 layers)
    copies = cfg.get("copies", 1) if not args.no_graph else 1
    torch.cuda.set_device(0)
    fmt = fnkv.FMT_KV8 if cfg.get("fmt") == "kv8" else None
    pool, slots = make_pool(torch, fnkv, cases, ctxs, T, layers * copies, args.seed, fmt=fmt)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    n = len(ctxs)
    q = torch.randn((layers * copies, n, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers * copies, n, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers * copies, n, T, HKV, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.empty(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")

    def step():
        for layer in range(layers * copies):
            pool.decode(slots, ctxs, T, layer, q[layer], out[layer], ws, k_new=None if args.no_append else kn[layer],
                        v_new=None if args.no_append else vn[layer])

    step()  # first call sets up the kernels' attributes outside any capture
    torch.cuda.synchronize()
    if args.traffic_child:
        traffic_child(args, torch, step)
        pool.close()
        return
    graph = None
    if not args.no_graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
    run = graph.replay if graph is not None else step

    replays = max(1, -(-args.steps // copies))
    warm = max(1, -(-args.warmup // copies))
    n_steps = replays * copies
    for _ in range(warm):
        run()
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(replays):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"

    ms_per_step = wall / n_steps * 1e3
    tokens = n * T * n_steps
    bytes_layer = algorithmic_bytes(ctxs, T)
    launch_s = gpu_s / (n_steps * layers)  # one layer's attention launch (decode_kernel + merge_kernel)
    achieved = bytes_layer / launch_s / 1e9
    line = {
        "metric": "decode-attn tokens/s + achieved HBM GB/s over Q8_0 paged KV, 64K-262K ctx",
        "value": round(tokens / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n_steps,
        "warmup": warm * copies,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("kv8 KV (int8 codes + fp16 group-64 scales)" if fmt is not None else
                  "q8_0 KV (int8 codes + fp16 scales)") + ", fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q)",
        "config": {"workload": workload, "contexts": ctxs, "T": T, "layers": layers, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "page_tokens": 256, "hip_graph": graph is not None,
                   "pool_format": cfg.get("fmt", "q8_0"),
                   "steps_per_graph": copies, "layers_rotated": layers * copies},
        "gb_s": round(bytes_layer * layers * n_steps / wall / 1e9, 3),
        "roofline": {
            "kernel": "fnkv_attn_decode launch (decode_kernel + merge_kernel), per layer",
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_detail": traffic_detail,
            "bytes_per_launch": bytes_layer,
            "launch_us": round(launch_s * 1e6, 3),
        },
    }
    if not args.no_cpu:
        threads = max(1, min(16, os.cpu_count() or 1))
        line["cpu_baseline"] = cpu_baseline(ctxs, T, layers, args.seed, threads)
    print(json.dumps(line), flush=True)
    pool.close()


if __name__ == "__main__":
    main()

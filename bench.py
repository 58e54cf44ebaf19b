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
    "cfg4": dict(layers=12, T=5, chunk=4096, mixed=True,
                 workload="cfg4: mixed 8-sequence pool step with page churn: 3 finished sequences free their pages, 2 "
                          "sequences append and attend a 4,096-token chunk, 6 verify T=5 at contexts U[1K, 196K], 12 "
                          "layers"),
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


def make_pool(torch, fnkv, cases, ctxs, T, layers, seed, h_kv=HKV, fmt=None, map_to=None):
    """A pool holding the sequences' first ctxs cells of every layer (seeded K/V, BASELINE's distribution), their pages
    scattered; map_to (optional, >= ctxs): the cells each slot has mapped (room for the steps' new cells)."""
    mapped = list(ctxs) if map_to is None else list(map_to)
    n_pages = sum(-(-c // 256) for c in mapped) + 16
    pool = fnkv.Pool(len(ctxs) + 1, n_pages, layers, h_kv, **({} if fmt is None else {"fmt": fmt}))
    slots = list(range(len(ctxs)))
    cases.scatter_ensure(pool, slots, mapped, seed, churn=0.2)
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


def host_info():
    """The host the CPU baseline runs on: logical CPUs (nproc), the CPUs this process may run on, the model name, and
    the thread count used: every CPU the process may use, capped by OMP_NUM_THREADS where the environment sets one (the
    GPU box sets it to its per-GPU CPU share)."""
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cap = os.environ.get("OMP_NUM_THREADS", "")
    threads = min(affinity, int(cap)) if cap.isdigit() and int(cap) > 0 else affinity
    return {"nproc": os.cpu_count(), "affinity_cpus": affinity, "cpu_model": model, "threads": threads,
            "thread_cap": f"OMP_NUM_THREADS={cap}" if cap else None}


def _best_of(fn, reps=5):
    fn()  # warmup (threads, caches)
    best = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
    return best


def _cpu_case(O, cases, seed, ctx, T, threads, q_seed=None):
    """ggml-semantics CPU flash attention (Q as Q8_0 with an integer dot, as ggml-cpu runs Q8_0 K; V widened to F32)
    of T query rows over ctx cells of one layer: best-of-5 seconds after a warmup."""
    import numpy as np

    k16, v16 = cases.kv_rows(seed, ctx, HKV)
    (kq, kd, _), (vq, vd, _) = cases.decoded(O, k16, v16)
    kb, vb = O.to_block_q8_0(kq, kd), O.to_block_q8_0(vq, vd)
    del k16, v16, kq, vq
    q16 = cases.queries(seed if q_seed is None else q_seed, (T, HQ, D)).view(np.uint16)
    return kb, vb, _best_of(lambda: O.attn_ggml(q16, kb, vb, ctx, q_as_q8=True, threads=threads))


def cpu_baseline(ctxs, T, layers, seed, extra=True):
    """The CPU path timed beside the GPU: the oracle's ggml-semantics flash attention over Q8_0 K/V (Q as Q8_0, integer
    K dot, F32 V accumulate: ggml-cpu's path for Q8_0 caches), multithreaded over (query row, head), on one of the
    layers of the workload (all sequences at full context), best-of-5 after a warmup, scaled to tokens/s of the whole
    step. With `extra`, cfg0 (4,096 cells, T = 1) and cfg2 (262,144 cells, T = 1 and T = 5) are timed the same way.
    Returns the dict for the JSON line."""
    import cases
    import oracle as O

    info = host_info()
    threads = info["threads"]
    t_layer = 0.0
    for i, c in enumerate(ctxs):
        t_layer += _cpu_case(O, cases, seed + i, c, T, threads)[2]
    tokens = len(ctxs) * T
    tok_s = tokens / (t_layer * layers)
    out = {
        "value": round(tok_s, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 of {layers} layers, all {len(ctxs)} sequences at full context, T={T}, ggml-semantics flash "
                  f"attention over Q8_0 K/V (Q as Q8_0, integer K dot, F32 V; oracle/fnkv_oracle.c or_attn_ggml), "
                  f"{threads} threads, best of 5 after a warmup; layer time {t_layer * 1e3:.1f} ms x {layers} layers",
        "gb_s": round(algorithmic_bytes(ctxs, T) / t_layer / 1e9, 3),
        "host": info,
    }
    if extra:
        timings = {}
        _, _, s0 = _cpu_case(O, cases, seed + 100, 4096, 1, threads)
        timings["cfg0"] = {"ctx": 4096, "T": 1, "seconds": round(s0, 6), "tokens_s": round(1 / s0, 3),
                           "gb_s": round(algorithmic_bytes([4096], 1) / s0 / 1e9, 3)}
        kb, vb, s1 = _cpu_case(O, cases, seed + 200, 262144, 1, threads)
        timings["cfg2_T1"] = {"ctx": 262144, "T": 1, "seconds": round(s1, 6), "tokens_s": round(1 / s1, 3),
                              "gb_s": round(algorithmic_bytes([262144], 1) / s1 / 1e9, 3)}
        import numpy as np
        q16 = cases.queries(seed + 201, (5, HQ, D)).view(np.uint16)
        s5 = _best_of(lambda: O.attn_ggml(q16, kb, vb, 262144, q_as_q8=True, threads=threads))
        timings["cfg2_T5"] = {"ctx": 262144, "T": 5, "seconds": round(s5, 6), "tokens_s": round(5 / s5, 3),
                              "gb_s": round(algorithmic_bytes([262144], 5) / s5 / 1e9, 3)}
        out["configs"] = timings
    return out


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


def measure_traffic(argv, kernels=("stream_kernel", "merge_row_kernel", "merge_kernel")):
    """HBM bytes of one fnkv_attn_decode launch (stream + merge kernels) from two rocprofv3 counter passes over a child
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


def time_prefill(args, cfg, steps, warmup):
    """BASELINE config 3's step (the chunk's Q8_0 append + its causal attention over the whole context) captured in a
    HIP graph and replayed: returns (wall seconds, GPU seconds between HIP events, the pool's K/V, q) of `steps`
    replays after `warmup`."""
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
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"
    del graph
    pool.close()
    return wall, gpu_s, kv, q


def run_prefill(args, cfg):
    """one step = the chunk's Q8_0 append (fnkv_q8_append) + its causal attention over the whole
    context (fnkv_attn_prefill), captured in a HIP graph; the roofline is the matrix cores' (algorithmic flops)."""
    import numpy as np

    import cases

    ctx, rows = cfg["ctxs"][0], cfg["T"]
    wall, gpu_s, kv, q = time_prefill(args, cfg, args.steps, args.warmup)
    graph = not args.no_graph
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
                   "head_dim": D, "page_tokens": 256, "hip_graph": graph},
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
        threads = host_info()["threads"]
        sample = 16
        (kq, kd, _), (vq, vd, _) = cases.decoded(O, kv[0].cpu().numpy(), kv[1].cpu().numpy())
        kb, vb = O.to_block_q8_0(kq, kd), O.to_block_q8_0(vq, vd)
        q16 = q[-sample:].cpu().numpy().view(np.uint16)
        dt = _best_of(lambda: O.attn_ggml(q16, kb, vb, ctx, q_as_q8=True, threads=threads), reps=3)
        sample_flops = 4 * D * HQ * sum(ctx - sample + t + 1 for t in range(sample))
        cpu_step = dt * flops / sample_flops
        line["cpu_baseline"] = {
            "value": round(rows / cpu_step, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"the chunk's last {sample} of {rows} query rows over the full context, ggml-semantics flash "
                      f"attention (Q as Q8_0; oracle/fnkv_oracle.c or_attn_ggml), {threads} threads, best of 3: "
                      f"{dt:.2f} s, scaled by visible pairs to the chunk",
            "host": host_info(),
            "tflops": round(sample_flops / dt / 1e12, 4),
        }
    print(json.dumps(line), flush=True)


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
        threads = host_info()["threads"]
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
        "dtype": "q8_0 KV (int8 codes + fp16 scales), q as fp16 hi + lo operands, fp32 prepare / softmax / accumulate / out",
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
        threads = host_info()["threads"]
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


def run_mixed(args, cfg):
    line, extra = time_mixed(args, cfg)
    if not args.no_cpu:
        line["cpu_baseline"] = mixed_cpu_baseline(args, cfg, extra)
    print(json.dumps(line), flush=True)


def time_mixed(args, cfg):
    """a mixed 8-sequence pool step with page churn. Beforehand three finished sequences take
    interleaved pages and free them (holes in the free list), then the eight sequences grow page by page in a seeded
    random order (a fragmented page table). A step = for each of the 12 layers: two sequences each append a 4,096-token
    fp16 chunk (fnkv_q8_append) and attend it causally over their whole context (fnkv_attn_prefill), then one
    fnkv_attn_decode launch runs the six other sequences' T = 5 verify (their new cells appended by the launch). The
    step is one HIP graph; the prefill half and the decode half are also captured and timed on their own, giving the
    prefill's matrix-core rate (algorithmic flops) and the decode's HBM rate (algorithmic bytes)."""
    import numpy as np
    import torch

    import cases
    import fnkv

    layers, T, chunk = cfg["layers"], cfg["T"], cfg["chunk"]
    rng = np.random.default_rng([args.seed, 4])
    pf_slots, vf_slots = [0, 1], [2, 3, 4, 5, 6, 7]
    pf_depth = [int(rng.integers(1024, 196 * 1024 + 1)) for _ in pf_slots]
    vf_ctx = [int(rng.integers(1024, 196 * 1024 + 1)) for _ in vf_slots]
    ctx_of = dict(zip(pf_slots, [d + chunk for d in pf_depth]))
    ctx_of.update(zip(vf_slots, vf_ctx))
    finished = {5: int(rng.integers(64, 256)), 6: int(rng.integers(64, 256)), 7: int(rng.integers(64, 256))}
    n_pages = sum(-(-c // 256) for c in ctx_of.values()) + 32
    torch.cuda.set_device(0)
    pool = fnkv.Pool(9, n_pages, layers, HKV)
    have = {s: 0 for s in finished}
    while any(have[s] < finished[s] for s in finished):
        s = int(rng.choice([x for x in finished if have[x] < finished[x]]))
        have[s] += 1
        assert pool.ensure(s, have[s] * 256)[0] == 0
    for s in finished:
        assert pool.trim(s, 0) == 0
    order = pf_slots + vf_slots
    cases.scatter_ensure(pool, order, [ctx_of[s] for s in order], args.seed)
    g = torch.Generator(device="cuda")
    chunks = {}
    for layer in range(layers):
        g.manual_seed(args.seed * 1000 + layer)
        for s in order:
            c = ctx_of[s]
            kv = []
            for _ in range(2):
                x = torch.randn((c, HKV, D), generator=g, device="cuda", dtype=torch.float32)
                ch = torch.randperm(D, generator=g, device="cuda")[:4]
                x[:, :, ch] *= 8.0
                kv.append(x.half())
            upto = c - chunk if s in pf_slots else c - T
            pool.append(s, layer, 0, kv[0][:upto].contiguous(), kv[1][:upto].contiguous())
            if s in pf_slots:
                chunks[(s, layer)] = (kv[0][upto:].contiguous(), kv[1][upto:].contiguous())
            del kv
    torch.cuda.synchronize()
    g.manual_seed(args.seed + 7)
    qp = {(s, l): torch.randn((chunk, HQ, D), generator=g, device="cuda").half() for s in pf_slots
          for l in range(layers)}
    outp = {k: torch.empty_like(v) for k, v in qp.items()}
    wsp = {}
    for s in pf_slots:
        n = pool.prefill_ws_bytes(ctx_of[s], chunk, HQ)
        wsp[s] = torch.empty(max(n, 16), dtype=torch.uint8, device="cuda") if n > 0 else False
    nv = len(vf_slots)
    qv = torch.randn((layers, nv, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers, nv, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers, nv, T, HKV, D), generator=g, device="cuda").half()
    outv = torch.empty_like(qv)
    ctxs = [ctx_of[s] for s in vf_slots]
    wsv = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")

    def prefill_half(layer):
        for s in pf_slots:
            kc, vc = chunks[(s, layer)]
            pool.append(s, layer, ctx_of[s] - chunk, kc, vc)
            pool.prefill(s, layer, ctx_of[s], qp[(s, layer)], outp[(s, layer)], ws=wsp[s])

    def decode_half(layer):
        pool.decode(vf_slots, ctxs, T, layer, qv[layer], outv[layer], wsv, k_new=kn[layer], v_new=vn[layer])

    def whole():
        for layer in range(layers):
            prefill_half(layer)
            decode_half(layer)

    def pre_only():
        for layer in range(layers):
            prefill_half(layer)

    def dec_only():
        for layer in range(layers):
            decode_half(layer)

    whole()
    torch.cuda.synchronize()

    def capture(fn):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            fn()
        torch.cuda.synchronize()
        return gr

    def timed(gr, steps, warmup):
        for _ in range(warmup):
            gr.replay()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(steps):
            gr.replay()
        ev1.record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, ev0.elapsed_time(ev1) / 1e3

    steps, warm = max(1, args.steps), max(1, args.warmup)
    g_whole = capture(whole)
    wall, gpu_whole = timed(g_whole, steps, warm)
    del g_whole
    g_dec = capture(dec_only)
    _, gpu_dec = timed(g_dec, max(steps, 20), warm)
    gpu_dec /= max(steps, 20)
    del g_dec
    g_pre = capture(pre_only)
    _, gpu_pre = timed(g_pre, steps, warm)
    gpu_pre /= steps
    del g_pre
    assert torch.isfinite(outv.float()).all().item(), "non-finite verify output"
    assert all(torch.isfinite(o.float()).all().item() for o in outp.values()), "non-finite prefill output"

    tokens = (len(pf_slots) * chunk + nv * T) * steps
    flops = layers * sum(prefill_flops(ctx_of[s], chunk) for s in pf_slots)
    dec_bytes = layers * algorithmic_bytes(ctxs, T)
    pre_tflops = flops / gpu_pre / 1e12
    dec_gbs = dec_bytes / gpu_dec / 1e9
    line = {
        "metric": "decode-attn tokens/s + achieved HBM GB/s over Q8_0 paged KV, 64K-262K ctx",
        "value": round(tokens / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 KV (int8 codes + fp16 scales), fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q)",
        "config": {"workload": cfg["workload"], "prefill_depths": pf_depth, "chunk": chunk,
                   "verify_contexts": vf_ctx, "T": T, "layers": layers, "q_heads": HQ, "kv_heads": HKV,
                   "head_dim": D, "page_tokens": 256, "finished_pages_freed": sum(finished.values()),
                   "hip_graph": True},
        "step_us": round(gpu_whole / steps * 1e6, 3),
        "roofline": {
            "kernel": "prefill half (fnkv_q8_append + fnkv_attn_prefill of both chunks), per step",
            "bound": "mfma",
            "achieved": round(pre_tflops, 3),
            "peak": PEAK_MFMA_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(pre_tflops / PEAK_MFMA_F16_TFLOPS, 4),
            "traffic": None,
            "flops_per_step": flops,
            "prefill_us_per_step": round(gpu_pre * 1e6, 3),
        },
        "decode_part": {
            "kernel": "fnkv_attn_decode launch over the six verify sequences (T = 5), 12 a step",
            "bound": "hbm",
            "achieved": round(dec_gbs, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(dec_gbs / PEAK_HBM_GBS, 4),
            "bytes_per_step": dec_bytes,
            "launch_us": round(gpu_dec / layers * 1e6, 3),
        },
    }
    pool.close()
    return line, dict(vf_ctx=vf_ctx, pf_slots=pf_slots, ctx_of=ctx_of, flops=flops, nv=nv, chunk=chunk, T=T,
                      layers=layers)


def mixed_cpu_baseline(args, cfg, x):
    """config 4's CPU baseline (the ggml-semantics port), sampled: see the record's "sample"."""
    import numpy as np

    import cases
    import oracle as O

    vf_ctx, pf_slots, ctx_of, flops = x["vf_ctx"], x["pf_slots"], x["ctx_of"], x["flops"]
    nv, chunk, T, layers = x["nv"], x["chunk"], x["T"], x["layers"]
    info = host_info()
    threads = info["threads"]
    # decode half: one layer, the six verify sequences; prefill half: the last 16 rows of one chunk, scaled by
    # visible pairs to both chunks
    t_dec = 0.0
    for i, c in enumerate(vf_ctx):
        t_dec += _cpu_case(O, cases, args.seed + i, c, T, threads)[2]
    s0 = pf_slots[0]
    c0 = ctx_of[s0]
    kb, vb, _ = _cpu_case(O, cases, args.seed + 50, c0, 1, threads)
    sample = 16
    q16 = cases.queries(args.seed + 51, (sample, HQ, D)).view(np.uint16)
    t_s = _best_of(lambda: O.attn_ggml(q16, kb, vb, c0, q_as_q8=True, threads=threads), reps=3)
    sample_flops = 4 * D * HQ * sum(c0 - sample + t + 1 for t in range(sample))
    t_pre = t_s * (flops / layers) / sample_flops
    cpu_step = layers * (t_dec + t_pre)
    return {
        "value": round((len(pf_slots) * chunk + nv * T) / cpu_step, 3), "unit": "tokens/s", "cores": threads,
        "kind": "port",
        "sample": f"one layer's six verify sequences (T={T}, best of 5) and the last {sample} rows of one chunk "
                  f"(best of 3, scaled by visible pairs to both chunks), ggml-semantics flash attention (Q as "
                  f"Q8_0; oracle/fnkv_oracle.c or_attn_ggml), {threads} threads, x {layers} layers",
        "host": info,
    }


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
    ap.add_argument("--no-extra", action="store_true", help="cfg1: skip the cfg2 / cfg2v launches timed beside it")
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
    if CONFIGS[args.config].get("mixed"):
        run_mixed(args, CONFIGS[args.config])
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
    custom = args.T is not None or args.ctxs is not None
    workload = cfg["workload"] if not custom else f"custom: contexts {ctxs}, T={T}, {layers} layers"
    torch.cuda.set_device(0)
    fmt = fnkv.FMT_KV8 if cfg.get("fmt") == "kv8" else None
    r = time_decode(args, torch, fnkv, cases, ctxs, T, layers, cfg.get("copies", 1), fmt, args.steps, args.warmup)
    if r is None:  # the counter pass's child
        return
    line = {
        "metric": "decode-attn tokens/s + achieved HBM GB/s over Q8_0 paged KV, 64K-262K ctx",
        "value": r["tokens_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": r["n_steps"],
        "warmup": r["warmup"],
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("kv8 KV (int8 codes + fp16 group-64 scales)" if fmt is not None else
                  "q8_0 KV (int8 codes + fp16 scales)") + ", fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q)",
        "config": {"workload": workload, "contexts": ctxs, "T": T, "layers": layers, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "page_tokens": 256, "hip_graph": r["graph"],
                   "pool_format": cfg.get("fmt", "q8_0"),
                   "steps_per_graph": r["copies"], "layers_rotated": layers * r["copies"]},
        "gb_s": r["gb_s"],
        "roofline": {
            "kernel": "fnkv_attn_decode launch (stream_kernel + merge_row_kernel), per layer",
            "bound": "hbm",
            "achieved": r["achieved"],
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": r["frac"],
            "traffic": traffic,
            "traffic_detail": traffic_detail,
            "bytes_per_launch": r["bytes_per_launch"],
            "launch_us": r["launch_us"],
        },
    }
    # the default run also times BASELINE config 2 (262,144 cells, decode T = 1 and verify T = 5), the metric's
    # deep-context end, on the same box: the same launch, figures per launch
    if args.config == "cfg1" and not custom and not args.no_extra:
        also = {}
        for name in ("cfg2", "cfg2v"):
            c2 = CONFIGS[name]
            x = time_decode(args, torch, fnkv, cases, c2["ctxs"], c2["T"], c2["layers"], c2["copies"], None, 8, 4)
            also[name] = {"workload": c2["workload"], "launch_us": x["launch_us"], "achieved_gb_s": x["achieved"],
                          "frac": x["frac"], "tokens_s": x["tokens_s"], "bytes_per_launch": x["bytes_per_launch"],
                          "steps": x["n_steps"]}
        # the engine's own call: device contexts advancing by T every replay of one captured step
        xd = time_decode_dev(args, torch, fnkv, cases, ctxs, T, layers, 20, 5)
        also["cfg1_dev"] = {"workload": "cfg1 through fnkv_attn_decode_dev: one captured graph of the 12 launches "
                                        "and a context advance, replayed as contexts grow by T",
                            **xd}
        c0 = CONFIGS["cfg0"]
        x0 = time_decode(args, torch, fnkv, cases, c0["ctxs"], c0["T"], c0["layers"], c0["copies"], None, 64, 64)
        also["cfg0"] = {"workload": c0["workload"], "launch_us": x0["launch_us"], "achieved_gb_s": x0["achieved"],
                        "frac": x0["frac"], "tokens_s": x0["tokens_s"], "bytes_per_launch": x0["bytes_per_launch"],
                        "steps": x0["n_steps"], "bound": "latency (4,096 cells: fixed costs dominate)"}
        c4 = CONFIGS["cfg4"]
        a4 = argparse.Namespace(**{**vars(args), "steps": 2, "warmup": 1})
        l4, _ = time_mixed(a4, c4)
        also["cfg4"] = {"workload": c4["workload"], "step_us": l4["step_us"],
                        "prefill_tflops": l4["roofline"]["achieved"], "prefill_frac": l4["roofline"]["frac"],
                        "decode_launch_us": l4["decode_part"]["launch_us"],
                        "decode_gb_s": l4["decode_part"]["achieved"], "decode_frac": l4["decode_part"]["frac"],
                        "tokens_s": l4["value"]}
        c3 = CONFIGS["cfg3"]
        _, gpu_s, _, _ = time_prefill(args, c3, 10, 2)
        step_s = gpu_s / 10
        tf = prefill_flops(c3["ctxs"][0], c3["T"]) / step_s / 1e12
        also["cfg3"] = {"workload": c3["workload"], "step_us": round(step_s * 1e6, 3), "achieved_tflops": round(tf, 3),
                        "frac": round(tf / PEAK_MFMA_F16_TFLOPS, 4), "bound": "mfma"}
        line["configs_also"] = also
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(ctxs, T, layers, args.seed, extra=args.config == "cfg1" and not custom)
    print(json.dumps(line), flush=True)


def time_decode(args, torch, fnkv, cases, ctxs, T, layers, copies, fmt, steps, warmup):
    """One fnkv_attn_decode launch a layer over `layers` layers (each appending its T new cells per sequence and
    attending over the whole context), captured in a HIP graph of `copies` steps over separate layers of the pool (a
    single-layer step is one short launch pair: the graph then holds several steps, each over its own layer, over 1 GB
    of caches in all, beyond the 256 MB last-level cache, so one replay's idle gap is spread over several steps as it
    is over cfg1's 12 layers); W replays untimed, then the timed ones between HIP events on the graph's stream.
    Returns the figures, or None in a counter pass's child (which only runs the launches)."""
    copies = copies if not args.no_graph else 1
    pool, slots = make_pool(torch, fnkv, cases, ctxs, T, layers * copies, args.seed, fmt=fmt)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    n = len(ctxs)
    q = torch.randn((layers * copies, n, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers * copies, n, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers * copies, n, T, HKV, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")

    def step():
        for layer in range(layers * copies):
            pool.decode(slots, ctxs, T, layer, q[layer], out[layer], ws, k_new=None if args.no_append else kn[layer],
                        v_new=None if args.no_append else vn[layer])

    step()  # first call sets up the kernels' attributes outside any capture
    torch.cuda.synchronize()
    if args.traffic_child:
        traffic_child(args, torch, step)
        pool.close()
        return None
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

    replays = max(1, -(-steps // copies))
    warm = max(1, -(-warmup // copies))
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
    del graph
    pool.close()

    bytes_layer = algorithmic_bytes(ctxs, T)
    launch_s = gpu_s / (n_steps * layers)  # one layer's attention launch (decode_kernel + merge_kernel)
    achieved = bytes_layer / launch_s / 1e9
    return {"tokens_s": round(n * T * n_steps / wall, 3), "n_steps": n_steps, "warmup": warm * copies,
            "ms_per_step": round(wall / n_steps * 1e3, 4), "graph": not args.no_graph, "copies": copies,
            "gb_s": round(bytes_layer * layers * n_steps / wall / 1e9, 3), "achieved": round(achieved, 3),
            "frac": round(achieved / PEAK_HBM_GBS, 4), "bytes_per_launch": bytes_layer,
            "launch_us": round(launch_s * 1e6, 3)}


def time_decode_dev(args, torch, fnkv, cases, ctxs, T, layers, steps, warmup):
    """The engine's own call (host/engine_step.cpp's pattern, the reference's TG1 depth, attend.h:108): one captured
    graph of the step's fnkv_attn_decode_dev launches (one a layer; contexts read from device words by the launch,
    the grid fixed by a host bound) followed by a device add that advances every sequence's context by T, replayed
    W times untimed and then K times between HIP events: each replay attends over T more cells than the last and
    appends its own new cells. Returns the per-launch figures at the timed replays' mean context."""
    n_adv = warmup + steps + 1  # the eager run advances too
    bound = [c + T * n_adv for c in ctxs]
    pool, slots = make_pool(torch, fnkv, cases, ctxs, T, layers, args.seed, map_to=bound)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    n = len(ctxs)
    q = torch.randn((layers, n, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers, n, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers, n, T, HKV, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.zeros(pool.decode_ws_bytes(bound, T, HQ), dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx_dev = torch.tensor(ctxs, dtype=torch.int64, device="cuda")

    def step():
        for layer in range(layers):
            pool.decode_dev(slots, ctx_dev, bound, T, layer, q[layer], out[layer], ws, err, k_new=kn[layer],
                            v_new=vn[layer])
        ctx_dev.add_(T)

    step()  # the library's one-time set-up outside the capture (and the first advance)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    first = ctx_dev.cpu().tolist()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        graph.replay()
    ev1.record(stream)
    torch.cuda.synchronize()
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert int(err.item()) == 0, "a launch refused its context"
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"
    del graph
    pool.close()
    mean_ctx = [c + T * (steps - 1) / 2.0 for c in first]
    bytes_layer = algorithmic_bytes([int(round(c)) for c in mean_ctx], T)
    launch_s = gpu_s / (steps * layers)  # a layer's launch pair (the context add spread over the step's 12)
    achieved = bytes_layer / launch_s / 1e9
    return {"launch_us": round(launch_s * 1e6, 3), "achieved_gb_s": round(achieved, 3),
            "frac": round(achieved / PEAK_HBM_GBS, 4), "tokens_s": round(n * T * steps / gpu_s, 3),
            "bytes_per_launch": bytes_layer, "steps": steps, "contexts_first": first,
            "step_us": round(gpu_s / steps * 1e6, 3)}


if __name__ == "__main__":
    main()

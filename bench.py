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
import json
import os
import sys
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
    "cfg2": dict(ctxs=[262144], T=1, layers=1,
                 workload="cfg2: 1 seq 262,144 cells, decode T=1, 1 layer, scattered pages"),
    "cfg2v": dict(ctxs=[262144], T=5, layers=1,
                  workload="cfg2: 1 seq 262,144 cells, verify T=5, 1 layer, scattered pages"),
    "cfg0": dict(ctxs=[4096], T=1, layers=1, workload="cfg0: 1 seq 4,096 cells, decode T=1, 1 layer"),
}


def algorithmic_bytes(ctxs, T):
    """Per layer: K+V read over every cell (the T new ones included), Q in and O out (fp16), the T new cells'
    Q8_0 write and their fp16 K/V read."""
    kv_read = sum(ctxs) * BYTES_PER_CELL_LAYER
    qo = len(ctxs) * T * HQ * D * 2 * 2
    append = len(ctxs) * T * (BYTES_PER_CELL_LAYER + 2 * HKV * D * 2)
    return kv_read + qo + append


def make_pool(torch, fnkv, cases, ctxs, T, layers, seed):
    n_pages = sum(-(-c // 256) for c in ctxs) + 16
    pool = fnkv.Pool(len(ctxs) + 1, n_pages, layers, HKV)
    slots = list(range(len(ctxs)))
    cases.scatter_ensure(pool, slots, ctxs, seed, churn=0.2)
    g = torch.Generator(device="cuda")
    for layer in range(layers):
        g.manual_seed(seed * 1000 + layer)
        for s, c in zip(slots, ctxs):
            kv = []
            for _ in range(2):
                x = torch.randn((c, HKV, D), generator=g, device="cuda", dtype=torch.float32)
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
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (the path is measured on one MI355X); --gpus must be 1",
              file=sys.stderr)
        sys.exit(2)

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
    torch.cuda.set_device(0)
    pool, slots = make_pool(torch, fnkv, cases, ctxs, T, layers, args.seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(args.seed + 7)
    n = len(ctxs)
    q = torch.randn((layers, n, T, HQ, D), generator=g, device="cuda").half()
    kn = torch.randn((layers, n, T, HKV, D), generator=g, device="cuda").half()
    vn = torch.randn((layers, n, T, HKV, D), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.empty(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")

    def step():
        for layer in range(layers):
            pool.decode(slots, ctxs, T, layer, q[layer], out[layer], ws, k_new=None if args.no_append else kn[layer],
                        v_new=None if args.no_append else vn[layer])

    step()  # first call sets up the kernels' attributes outside any capture
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
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        run()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) / 1e3
    assert torch.isfinite(out.float()).all().item(), "non-finite attention output"

    ms_per_step = wall / args.steps * 1e3
    tokens = n * T * args.steps
    bytes_layer = algorithmic_bytes(ctxs, T)
    launch_s = gpu_s / (args.steps * layers)  # one layer's attention launch (decode_kernel + merge_kernel)
    achieved = bytes_layer / launch_s / 1e9
    line = {
        "metric": "decode-attn tokens/s + achieved HBM GB/s over Q8_0 paged KV, 64K-262K ctx",
        "value": round(tokens / wall, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 KV (int8 codes + fp16 scales), fp16 Q/O, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) K/V with 4 of 256 channels x8, N(0,1) Q)",
        "config": {"workload": workload, "contexts": ctxs, "T": T, "layers": layers, "q_heads": HQ,
                   "kv_heads": HKV, "head_dim": D, "page_tokens": 256, "hip_graph": graph is not None},
        "gb_s": round(bytes_layer * layers * args.steps / wall / 1e9, 3),
        "roofline": {
            "kernel": "fnkv_attn_decode launch (decode_kernel + merge_kernel), per layer",
            "bound": "hbm",
            "achieved": round(achieved, 3),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": None,
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

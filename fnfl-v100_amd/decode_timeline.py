"""Per-workgroup timeline and wave-0 phase clocks of one dense decode launch (stream_kernel), from an instrumented
build of the library (-DFNKV_TIMING: every workgroup stamps the real-time counter at five points and every wave its
loop's end; with -DFNKV_TIMING_PHASES as well, wave 0 also sums its shader-clock cycles per loop phase, in a build of
its own because the clock reads reshape the loop's schedule).

    FNKV_EXTRA_FLAGS=-DFNKV_TIMING FNKV_LIB_OUT=/tmp/fnkv_timing/libfnkv.so python3 fnfl-v100_amd/build_lib.py
    FNKV_LIB_PATH=/tmp/fnkv_timing/libfnkv.so python3 fnfl-v100_amd/decode_timeline.py --ctxs 8192,16384,32768,65536 --T 3

Times are microseconds after the first workgroup's "entry" stamp (its first instruction once its kernel arguments
are in); "page table in" is the landing of its walk's page-table entries and Q rows, "start" its first stamp after
them.
A product build has no stamps: this tool refuses to run on one."""
import argparse
import ctypes
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "fnfl-v100_amd"), os.path.join(ROOT, "tests"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

STAMPS = ["start", "q + first tile in", "loop end + barrier", "LDS fold done", "end", "entry", "page table in"]
PHASES = ["wait K", "scores + issue K", "softmax", "wait V", "PV + issue V", "-", "loop back"]
MAX_WG = 4096


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ctxs", default="8192,16384,32768,65536")
    ap.add_argument("--T", type=int, default=3)
    ap.add_argument("--reps", type=int, default=6)
    ap.add_argument("--dev", type=int, default=0, metavar="SLACK",
                    help="launch through fnkv_attn_decode_dev: contexts in a device word, the host bound SLACK cells "
                         "above them (0: fnkv_attn_decode with host contexts)")
    args = ap.parse_args()
    import torch

    import bench
    import cases
    import fnkv
    L = fnkv.lib()
    if not hasattr(L, "fnkv_debug_timing"):
        sys.exit("decode_timeline: the loaded library has no timing stamps (build it with -DFNKV_TIMING)")
    L.fnkv_debug_timing.argtypes = [ctypes.c_void_p]
    ctxs = [int(x) for x in args.ctxs.split(",")]
    bound = [c + args.dev for c in ctxs]
    pool, slots = bench.make_pool(torch, fnkv, cases, ctxs, args.T, 1, 1234, map_to=bound)
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    q = torch.randn((len(ctxs), args.T, 16, 256), generator=g, device="cuda").half()
    out = torch.empty_like(q)
    ws = torch.zeros(pool.decode_ws_bytes(bound, args.T, 16), dtype=torch.uint8, device="cuda")
    ctx_dev = torch.tensor(ctxs, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ts = torch.zeros(MAX_WG * 24, dtype=torch.int64, device="cuda")
    for _ in range(args.reps):  # the last launch's stamps are kept
        ts.zero_()
        L.fnkv_debug_timing(ctypes.c_void_p(ts.data_ptr()))
        if args.dev > 0:
            pool.decode_dev(slots, ctx_dev, bound, args.T, 0, q, out, ws, err)
        else:
            pool.decode(slots, ctxs, args.T, 0, q, out, ws)
        torch.cuda.synchronize()
    if int(err.item()) != 0:
        sys.exit("decode_timeline: the launch refused a context")
    L.fnkv_debug_timing(ctypes.c_void_p(0))
    a = ts.cpu().numpy()
    st = a[:MAX_WG * 16].reshape(MAX_WG, 16)
    used = st[:, 0] != 0
    s = st[used]
    if not used.any():
        sys.exit("decode_timeline: no stamps were written")
    t0 = s[:, 5].min() if (s[:, 5] != 0).all() else s[:, 0].min()  # the first workgroup's entry
    us = lambda v: (v - t0) * 10 / 1000.0  # noqa: E731 (real-time ticks of 10 ns)
    how = f", device contexts (host bound + {args.dev})" if args.dev > 0 else ""
    print(f"contexts {ctxs}, T = {args.T}{how}: {int(used.sum())} workgroups")
    for k, nm in enumerate(STAMPS):
        v = s[:, k]
        v = v[v != 0]
        if v.size:
            r = us(v)
            print(f"  {nm:20s} min {r.min():6.2f} median {np.median(r):6.2f} max {r.max():6.2f} us")
    for wv in range(8):
        v = s[:, 8 + wv]
        v = v[v != 0]
        if v.size:
            r = us(v)
            print(f"  wave {wv} loop end       min {r.min():6.2f} median {np.median(r):6.2f} max {r.max():6.2f} us")
    # workgroups are dealt to the 8 XCDs round-robin in launch order (x fastest, then y)
    idx = np.nonzero(used)[0]
    loop_end = us(s[:, 2])
    print("loop end + barrier by XCD (workgroup index mod 8): median / max us")
    print("  " + "  ".join(f"{x}: {np.median(loop_end[idx % 8 == x]):5.2f}/{loop_end[idx % 8 == x].max():5.2f}"
                           for x in range(8)))
    ph = a[MAX_WG * 16:MAX_WG * 24].reshape(MAX_WG, 8)[used]
    if not ph.any():
        print("(no phase clocks: a build without -DFNKV_TIMING_PHASES)")
        pool.close()
        return
    print("wave 0's phase cycles summed over its tiles (median over workgroups):")
    for p, nm in enumerate(PHASES):
        if nm != "-":
            print(f"  {nm:18s} {np.median(ph[:, p]):9.0f}")
    pool.close()


if __name__ == "__main__":
    main()

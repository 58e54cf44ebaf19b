"""Builds libfnkv.so (the HIP library behind include/fnkv.h) for gfx950, in-tree, and the C++ host harness
engine_step (host/engine_step.cpp: the reference engine's calling pattern over the C-ABI) linked against it.

hipcc compiles each source to an object (in parallel) and links the shared library next to this file. Every HIP
source is compiled with packed-fp32 instructions disabled (their hand-written forms are avoided on this target) and
with per-file flags (below).

Measurement builds: FNKV_EXTRA_FLAGS adds flags to every source (e.g. -DFNKV_TIMING, the decode kernels' real-time
stamps read by decode_timeline.py) and FNKV_LIB_OUT names the library to write instead of the in-tree one (its objects
go to a build folder beside it; the harness is not built).
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_OUT = os.environ.get("FNKV_LIB_OUT")
BUILD = os.path.join(os.path.dirname(os.path.abspath(LIB_OUT)), "_build") if LIB_OUT else os.path.join(HERE, "_build")
LIB = os.path.abspath(LIB_OUT) if LIB_OUT else os.path.join(HERE, "libfnkv.so")
HARNESS = os.path.join(HERE, "engine_step")
SOURCES = ["pool.hip", "append.hip", "decode.hip", "stream.hip", "prefill.hip", "sparse.hip", "datc.hip", "qsa.hip", "qsp.hip"]
ARCH = os.environ.get("FNKV_ARCH", "gfx950")

COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if c and (os.path.isabs(c) and os.path.exists(c) or not os.path.isabs(c)):
            return c
    return "hipcc"


# per-file flags: the quantizer must not fuse x * id into the rounding test (ggml rounds the product first); the
# attention kernels run two waves a SIMD and keep their matrix-core accumulators in ordinary registers (VGPR form)
VGPR_MFMA = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
EXTRA = {"append.hip": ["-ffp-contract=off"], "decode.hip": VGPR_MFMA, "stream.hip": VGPR_MFMA, "prefill.hip": VGPR_MFMA,
         "sparse.hip": ["-ffp-contract=off"], "qsa.hip": ["-ffp-contract=off"], "qsp.hip": ["-ffp-contract=off"]}


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    extra_env = os.environ.get("FNKV_EXTRA_FLAGS", "").split()
    cmd = [hipcc(), *COMMON, *EXTRA.get(src, []), *extra_env, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if LIB_OUT:
        return LIB
    # the host harness: host code only, linked against the library next to it
    tmp = HARNESS + ".tmp"
    cmd = [hipcc(), "-O2", "-std=c++17", "-Wall", "-I", os.path.join(HERE, "..", "include"),
           os.path.join(HERE, "host", "engine_step.cpp"), "-L", HERE, "-lfnkv", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on host/engine_step.cpp:\n{r.stderr}")
    os.replace(tmp, HARNESS)
    if verbose:
        print(f"built {LIB} and {HARNESS}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

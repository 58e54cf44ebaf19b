"""The C++ host harness (fnfl-v100_amd/host/engine_step.cpp) run as its own process: the reference engine's calling
pattern over the C-ABI with no Python on the path (runtime.cpp:1483-1537 ensure_cells with the reclaim retry, the
prompt append, layer.cpp:660-695's per-layer decode as one captured HIP graph replayed while the device contexts
advance, a refused context). The harness checks its own results (graph replays bitwise equal to the eager launches,
within 1e-3 plus one fp16 ulp of the host-context launch, the refused-depth bit with nothing written) and exits
non-zero otherwise."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HARNESS = os.path.join(os.path.dirname(__file__), "..", "fnfl-v100_amd", "engine_step")


def test_engine_step_harness():
    assert os.path.exists(HARNESS), "engine_step is not built: run __graft_entry__.build() first"
    print("engine_step 12", flush=True)
    r = subprocess.run([HARNESS, "12"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    print(r.stderr)
    assert r.returncode == 0, r.stderr
    assert "engine_step ok" in r.stdout
    assert "reservation:" in r.stdout and "refusal:" in r.stdout

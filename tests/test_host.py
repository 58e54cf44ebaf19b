"""Host-side checks of the C-ABI library, CPU only: it loads, exports every entry point include/fnkv.h declares,
and its pure host logic (the page rounding and the reclaim choice) gives the reference's known answers
(fn/runtime/slots_test.cpp:26-84). No GPU call is made here."""
import ctypes
import os
import re

import fnkv

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "fnkv.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(fnkv_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = fnkv.lib()
    names = declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert missing == []
    assert sorted(fnkv.EXPORTS) == names


def test_pages_for_known_answers():
    pc, n = 16384, 16
    assert [fnkv.pages_for(c, pc, n) for c in (0, 1, pc, pc + 1, 262144, 262144 + 5)] == [0, 1, 1, 2, 16, 16]
    assert fnkv.pages_for(32768 + 128 + 69, pc, n) == 3
    assert fnkv.pages_for(131072 + 32 + 69, pc, n) == 9
    assert fnkv.pages_for(-5, pc, n) == 0 and fnkv.pages_for(5, 0, n) == 0
    assert fnkv.pages_for(262144, 256, 1 << 20) == 1024


def test_reclaim_victim_known_answers():
    v = [[False, 3, 7], [False, 2, 4], [True, 5, 1], [False, 0, 2]]
    a = fnkv.reclaim_victim(v, 0)
    b = fnkv.reclaim_victim(v, 1)
    v[1][0] = True
    c = fnkv.reclaim_victim(v, 0)
    v[0][2] = 0
    d = fnkv.reclaim_victim(v, 3)
    assert (a, b, c, d) == (1, 0, -1, 0)
    # ties on the release order go to the lower slot (strict <)
    assert fnkv.reclaim_victim([[False, 1, 5], [False, 1, 5]], -1) == 0


def test_page_block_bytes():
    assert fnkv.lib().fnkv_page_block_bytes() == 8 * 17408


def test_draft_entries_refuse_missing_arguments_on_the_host():
    # the DA-TC entries check their arguments before any device call: null structs, or structs with null pointers,
    # are refused with the contract error and a message (draft.h:47-78: rejected, nothing enqueued)
    L = fnkv.lib()
    assert L.fnkv_datc_prepare(1, None, None) == fnkv.ERR_ARG
    assert L.fnkv_datc_attend(None, None) == fnkv.ERR_ARG
    assert L.fnkv_datc_step(None, None, None) == fnkv.ERR_ARG
    assert "fnkv_datc_step" in fnkv.last_error()
    p = fnkv.DatcPrepareArgs()
    a = fnkv.DatcAttendArgs()
    p.row0, a.row0 = 0, 1
    assert L.fnkv_datc_step(ctypes.byref(p), ctypes.byref(a), None) == fnkv.ERR_ARG


def test_rope_theta_scale_is_the_f32_power():
    # theta_scale = powf(1e7, -2 / 64) (attend.cu:830-832), the F32 rounding of the exact value
    import numpy as np
    got = np.float32(fnkv.rope_theta_scale())
    want = np.float32(10000000.0 ** (-2.0 / 64.0))
    assert abs(float(got) - float(want)) <= float(np.spacing(want))


def test_bench_refuses_more_than_one_gpu():
    # the bench contract: N > 1 exits with a message (one GPU only), before touching a device
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)

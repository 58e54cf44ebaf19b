"""DA-TC, the draft block's dense F16 attention (fn/kernels/draft/draft.h:47-83), on the GPU against the oracle: the
reference's own checker's cases and bounds (fn/kernels/draft/draft_test.cpp:710-887):
  prepare  the F32 q and k within 1e-6 (max |error| / max |ref|) of the FP64 norm + IMROPE; the K cache bitwise
           f16(the launch's F32 k) and within one F16 ulp of the FP64 k (values of at least 1e-3 of the row's largest);
           V bitwise f16(kv_v); q16 bitwise f16(q / 16)
  attend   each head within 2e-3 of FP64 over the stored F16 inputs (q16, K, V), gated; the codes and scales bitwise
           the activation rule of the F32 output; bitwise reruns
Cases: steps at n_before 0 .. 196,607 (the reference's list, through the 58,581 / 131,072 / 196,608-cell bench
depths), chained rows with distinct rope planes, catch-ups (K and V only) at B_c 1..5, SP2 sparse bodies at depths
1 .. 196,600, a body whose K is not this depth's, cells past the cache (the error word, nothing written), and the host
refusals."""
import numpy as np
import pytest

import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

NH, HD, QS = 12, 256, 512
MAX_N = 196608
CELLS = MAX_N + 16
ATTN_BOUND, F32_BOUND = 2e-3, 1e-6
ERR = fnkv.DEV_ERR_DRAFT_DEPTH


@pytest.fixture(scope="module")
def card():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    rng = np.random.default_rng(0x44415443)
    k = rng.uniform(-2.0, 2.0, (CELLS, HD)).astype(np.float16)
    v = rng.uniform(-1.5, 1.5, (CELLS, HD)).astype(np.float16)
    band = min(1000, MAX_N // 3)  # a band of large keys deep in the history
    k[band:band + 3] = (k[band:band + 3].astype(np.float32) * 6.0).astype(np.float16)
    c = {
        "rng": rng,
        "k": k.view(np.uint16).copy(), "v": v.view(np.uint16).copy(),
        "q_norm": rng.uniform(0.3, 1.8, HD).astype(np.float32),
        "k_norm": rng.uniform(0.3, 1.8, HD).astype(np.float32),
        "ts": fnkv.rope_theta_scale(),
    }
    dev = {
        "kc": torch.from_numpy(c["k"].view(np.int16)).cuda(), "vc": torch.from_numpy(c["v"].view(np.int16)).cuda(),
        "qn": torch.from_numpy(c["q_norm"]).cuda(), "kn": torch.from_numpy(c["k_norm"]).cuda(),
        "part": torch.empty(fnkv.datc_part_bytes() // 4, dtype=torch.float32, device="cuda"),
        "out": torch.empty(NH * HD, dtype=torch.float32, device="cuda"),
        "codes": torch.empty(NH * HD, dtype=torch.int8, device="cuda"),
        "scales": torch.empty(NH * HD // 16, dtype=torch.float32, device="cuda"),
        "err": torch.zeros(1, dtype=torch.int32, device="cuda"),
        "q16": torch.empty((5, NH, HD), dtype=torch.int16, device="cuda"),
        "qf32": torch.empty((5, NH, HD), dtype=torch.float32, device="cuda"),
        "kf32": torch.empty((5, HD), dtype=torch.float32, device="cuda"),
    }
    c["dev"] = dev
    return c


def make_inputs(c, n_before, rows, stride, planes, sparse, row0, bad_k=0):
    rng = c["rng"]
    inp = {
        "qfull": rng.uniform(-3.0, 3.0, (rows, NH, QS)).astype(np.float32),
        "kv_k": rng.uniform(-2.0, 2.0, (rows, HD)).astype(np.float32),
        "kv_v": rng.uniform(-1.5, 1.5, (rows, HD)).astype(np.float32),
    }
    pos = np.zeros((4, stride), np.int32)
    for t in range(stride):
        p = n_before + t
        for pl in range(4):
            pos[pl, t] = p + 17 * pl - (3 * p // 4 if pl == 3 else 0) if planes else p
    inp["pos"] = pos
    inp["body"] = None
    if sparse:
        n_vis = n_before // 4
        K = min(n_vis, 512)
        blocks = np.sort(rng.choice(n_vis, K, replace=False)) if n_vis > 512 else np.arange(n_vis)
        tail = np.arange(4 * n_vis, n_before)
        inp["body"] = np.concatenate([[K + bad_k, n_before % 4], blocks, tail]).astype(np.uint32)
    inp["cells"] = O.datc_cells(n_before, row0, None if inp["body"] is None else np.concatenate(
        [[min(n_before // 4, 512), 0], inp["body"][2:]]))
    return inp


def run(c, n_before, rows, row0, stride, step, inp, max_cells=CELLS):
    d = c["dev"]
    nb = torch.tensor([n_before], dtype=torch.int32, device="cuda")
    st = torch.tensor([stride], dtype=torch.int32, device="cuda")
    pos = torch.from_numpy(inp["pos"]).cuda()
    qfull = torch.from_numpy(inp["qfull"]).cuda()
    kvk = torch.from_numpy(inp["kv_k"]).cuda()
    kvv = torch.from_numpy(inp["kv_v"]).cuda()
    body = torch.from_numpy(inp["body"].view(np.int32)).cuda() if inp["body"] is not None else None
    d["out"].view(torch.int32).fill_(-1)
    d["err"].zero_()
    cell = n_before + row0
    if cell + rows <= max_cells:  # the new cells hold junk: prepare must write them
        d["kc"][cell:cell + rows] = 0x7F7F
        d["vc"][cell:cell + rows] = 0x7F7F
    fnkv.datc_prepare(rows, kv_k=kvk, kv_v=kvv, k_norm=d["kn"], n_before=nb, pos=pos, stride=st, k_cache=d["kc"],
                      v_cache=d["vc"], err=d["err"], row0=row0, qfull=qfull if step else None, q_norm=d["qn"],
                      q16=d["q16"], q_f32=d["qf32"], k_f32=d["kf32"], theta_scale=c["ts"])
    if step:
        fnkv.datc_attend(q16=d["q16"], qfull=qfull, k_cache=d["kc"], v_cache=d["vc"], n_before=nb, part=d["part"],
                         out=d["out"], codes=d["codes"], scales=d["scales"], err=d["err"], row0=row0, body=body)
    torch.cuda.synchronize()
    o = {"err": int(d["err"].item()) & 0xFFFFFFFF, "out": d["out"].cpu().numpy().copy()}
    o["codes"] = d["codes"].cpu().numpy().copy()
    o["scales"] = d["scales"].cpu().numpy().copy()
    o["q16"] = d["q16"][:rows].cpu().numpy().view(np.uint16).copy()
    o["qf32"] = d["qf32"][:rows].cpu().numpy().copy()
    o["kf32"] = d["kf32"][:rows].cpu().numpy().copy()
    if cell + rows <= max_cells:
        o["k_new"] = d["kc"][cell:cell + rows].cpu().numpy().view(np.uint16).copy()
        o["v_new"] = d["vc"][cell:cell + rows].cpu().numpy().view(np.uint16).copy()
    return o


def f16_ulp(y):
    y = np.abs(np.asarray(y, np.float64))
    e = np.where(y > 0, np.floor(np.log2(np.where(y > 0, y, 1.0))), -24.0)
    return np.where(y > 0, 2.0 ** (np.maximum(e, -14) - 10), 2.0**-24)


def check(c, n_before, rows, row0, stride, step, inp, o):
    assert o["err"] == 0, f"error word {o['err']:#x}"
    for r in range(rows):
        col = row0 + r
        p4 = [int(inp["pos"][pl, col]) for pl in range(4)]
        y = O.norm_rope_f64(inp["kv_k"][r], c["k_norm"], p4, c["ts"])
        assert O.norm_err(y, o["kf32"][r]) <= F32_BOUND
        kb = o["k_new"][r]
        assert np.array_equal(kb, o["kf32"][r].astype(np.float16).view(np.uint16)), "K is not f16(the F32 k)"
        big = np.abs(y) >= 1e-3 * np.abs(y).max()
        kv = kb.view(np.float16).astype(np.float64)
        assert (np.abs(kv - y) / f16_ulp(y))[big].max() <= 1.0, "K more than one F16 ulp from the FP64 k"
        assert np.array_equal(o["v_new"][r], inp["kv_v"][r].astype(np.float16).view(np.uint16)), "V is not f16(v)"
        cellr = n_before + col
        c["k"][cellr] = kb
        c["v"][cellr] = o["v_new"][r]
    if not step:
        return
    p4 = [int(inp["pos"][pl, row0]) for pl in range(4)]
    for h in range(NH):
        qd = O.norm_rope_f64(inp["qfull"][0, h, :HD], c["q_norm"], p4, c["ts"])
        assert O.norm_err(qd, o["qf32"][0, h]) <= F32_BOUND
    q16_want = (o["qf32"][0] * np.float32(0.0625)).astype(np.float16).view(np.uint16)
    assert np.array_equal(o["q16"][0], q16_want), "q16 is not f16(q / 16)"
    gate = inp["qfull"][0, :, HD:]
    ref = O.datc_attn_f64(o["q16"][0], gate, c["k"], c["v"], inp["cells"])
    out = o["out"].reshape(NH, HD)
    errs = [O.norm_err(ref[h], out[h]) for h in range(NH)]
    assert max(errs) <= ATTN_BOUND, errs
    codes, scales = O.act_quantize(o["out"])
    assert np.array_equal(codes, o["codes"]), "codes are not the activation rule of the output"
    assert np.array_equal(scales.reshape(-1).view(np.uint32), o["scales"].view(np.uint32))


def same(a, b):
    return all(np.array_equal(np.asarray(a[k]).view(np.uint8), np.asarray(b[k]).view(np.uint8))
               for k in ("out", "codes", "scales", "q16", "k_new", "v_new"))


STEPS = [0, 1, 62, 63, 64, 127, 200, 4095, 9215, 9216, 9217, 58580, 131071, 196607]


@pytest.mark.parametrize("n_before", STEPS)
def test_step_row(card, n_before):
    print(f"datc step n_before {n_before}", flush=True)
    inp = make_inputs(card, n_before, 1, 1, False, False, 0)
    o = run(card, n_before, 1, 0, 1, True, inp)
    check(card, n_before, 1, 0, 1, True, inp, o)
    again = run(card, n_before, 1, 0, 1, True, inp)
    assert same(o, again), "a rerun is not bitwise identical"


@pytest.mark.parametrize("n_before,row0,stride,planes", [(300, 1, 3, False), (300, 2, 3, True),
                                                          (MAX_N - 2, 1, 2, False), (300, 3, 4, True)])
def test_chained_step(card, n_before, row0, stride, planes):
    print(f"datc chain n_before {n_before} row0 {row0}", flush=True)
    inp = make_inputs(card, n_before, 1, stride, planes, False, row0)
    o = run(card, n_before, 1, row0, stride, True, inp)
    check(card, n_before, 1, row0, stride, True, inp, o)


@pytest.mark.parametrize("rows", [1, 2, 3, 4, 5])
def test_catch_up(card, rows):
    print(f"datc catch-up rows {rows}", flush=True)
    inp = make_inputs(card, 500 + 7 * rows, rows, rows, rows == 3, False, 0)
    o = run(card, 500 + 7 * rows, rows, 0, rows, False, inp)
    check(card, 500 + 7 * rows, rows, 0, rows, False, inp, o)


def test_catch_up_at_the_cache_end(card):
    nb = MAX_N + 11
    inp = make_inputs(card, nb, 5, 5, False, False, 0)
    o = run(card, nb, 5, 0, 5, False, inp)
    check(card, nb, 5, 0, 5, False, inp, o)


SPARSE = [1, 7, 64, 2048, 2051, 2052, 2055, 9217, 58581, 131070, 196600]


@pytest.mark.parametrize("i,n_before", list(enumerate(SPARSE)))
def test_sparse_step(card, i, n_before):
    row0 = i % 4
    print(f"datc sparse n_before {n_before} row0 {row0}", flush=True)
    inp = make_inputs(card, n_before, 1, 4, row0 == 2, True, row0)
    o = run(card, n_before, 1, row0, 4, True, inp)
    check(card, n_before, 1, row0, 4, True, inp, o)
    again = run(card, n_before, 1, row0, 4, True, inp)
    assert same(o, again)


def test_sparse_full_body_equals_dense(card):
    # at N / 4 <= 512 the body lists every whole block: the same cells as the dense row, in the same order
    n_before, row0 = 1500, 2
    inp = make_inputs(card, n_before, 1, 4, False, True, row0)
    o_sp = run(card, n_before, 1, row0, 4, True, inp)
    dense = dict(inp, body=None)
    o_d = run(card, n_before, 1, row0, 4, True, dense)
    assert np.array_equal(o_sp["out"].view(np.uint32), o_d["out"].view(np.uint32))


def test_sparse_body_of_another_depth(card):
    inp = make_inputs(card, 3000, 1, 4, False, True, 1, bad_k=1)
    o = run(card, 3000, 1, 1, 4, True, inp)
    assert o["err"] == ERR
    assert np.all(o["out"].view(np.uint32) == 0xFFFFFFFF), "output written"


def test_cells_past_the_cache(card):
    d = card["dev"]
    before = d["kc"][CELLS - 1].clone()
    inp = make_inputs(card, CELLS - 1, 2, 2, False, False, 0)
    o = run(card, CELLS - 1, 2, 0, 2, False, inp)
    assert o["err"] == ERR
    assert torch.equal(before, d["kc"][CELLS - 1]), "prepare wrote past its contract"
    inp = make_inputs(card, CELLS - 1, 1, 2, False, False, 1)
    o = run(card, CELLS - 1, 1, 1, 2, True, inp)
    assert o["err"] == ERR
    assert np.all(o["out"].view(np.uint32) == 0xFFFFFFFF), "output written"


def test_host_refusals(card):
    d = card["dev"]
    nb = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.ones(1, dtype=torch.int32, device="cuda")
    pos = torch.zeros((4, 5), dtype=torch.int32, device="cuda")
    kv = torch.zeros((5, HD), dtype=torch.float32, device="cuda")
    common = dict(kv_k=kv, kv_v=kv, k_norm=d["kn"], n_before=nb, pos=pos, stride=st, k_cache=d["kc"],
                  v_cache=d["vc"], err=d["err"])
    for rows, row0 in ((0, 0), (6, 0), (3, 3)):
        with pytest.raises(fnkv.FnkvError):
            fnkv.datc_prepare(rows, row0=row0, **common)
    qfull = torch.zeros((NH, QS), dtype=torch.float32, device="cuda")
    att = dict(q16=d["q16"], qfull=qfull, k_cache=d["kc"], v_cache=d["vc"], n_before=nb, part=d["part"],
               out=d["out"], codes=d["codes"], scales=d["scales"], err=d["err"])
    with pytest.raises(fnkv.FnkvError):
        fnkv.datc_attend(row0=5, **att)
    body = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(fnkv.FnkvError):
        fnkv.datc_attend(row0=4, body=body, **att)
    with pytest.raises(fnkv.FnkvError):  # 32-bit cache offsets
        fnkv.datc_attend(max_cells=1 << 22, **att)


def run_step(c, n_before, row0, stride, inp, fused):
    """The step row: fnkv_datc_step, or prepare then attend (the reference's sequence)."""
    d = c["dev"]
    nb = torch.tensor([n_before], dtype=torch.int32, device="cuda")
    st = torch.tensor([stride], dtype=torch.int32, device="cuda")
    pos = torch.from_numpy(inp["pos"]).cuda()
    qfull = torch.from_numpy(inp["qfull"]).cuda()
    kvk = torch.from_numpy(inp["kv_k"]).cuda()
    kvv = torch.from_numpy(inp["kv_v"]).cuda()
    body = torch.from_numpy(inp["body"].view(np.int32)).cuda() if inp["body"] is not None else None
    d["out"].view(torch.int32).fill_(-1)
    d["q16"].zero_()
    d["err"].zero_()
    cell = n_before + row0
    if cell < CELLS:
        d["kc"][cell] = 0x7F7F
        d["vc"][cell] = 0x7F7F
    common = dict(kv_k=kvk, kv_v=kvv, k_norm=d["kn"], n_before=nb, pos=pos, stride=st, k_cache=d["kc"],
                  v_cache=d["vc"], err=d["err"], row0=row0, theta_scale=c["ts"])
    if fused:
        fnkv.datc_step(q_norm=d["qn"], qfull=qfull, q16=d["q16"], part=d["part"], out=d["out"], codes=d["codes"],
                       scales=d["scales"], q_f32=d["qf32"], k_f32=d["kf32"], body=body, **common)
    else:
        fnkv.datc_prepare(1, qfull=qfull, q_norm=d["qn"], q16=d["q16"], q_f32=d["qf32"], k_f32=d["kf32"], **common)
        fnkv.datc_attend(q16=d["q16"], qfull=qfull, k_cache=d["kc"], v_cache=d["vc"], n_before=nb, part=d["part"],
                         out=d["out"], codes=d["codes"], scales=d["scales"], err=d["err"], row0=row0, body=body)
    torch.cuda.synchronize()
    o = {"err": int(d["err"].item()) & 0xFFFFFFFF}
    for k in ("out", "codes", "scales", "q16", "qf32", "kf32"):
        o[k] = d[k].cpu().numpy().copy()
    o["q16"] = o["q16"][:1]
    o["qf32"] = o["qf32"][:1]
    o["kf32"] = o["kf32"][:1]
    if cell < CELLS:
        o["k_new"] = d["kc"][cell].cpu().numpy().copy()
        o["v_new"] = d["vc"][cell].cpu().numpy().copy()
    return o


@pytest.mark.parametrize("n_before,row0,sparse", [(0, 0, False), (63, 1, False), (4095, 0, False),
                                                   (58580, 2, False), (196607, 0, False), (7, 1, True),
                                                   (9217, 3, True), (131070, 2, True)])
def test_fused_step_matches_prepare_then_attend(card, n_before, row0, sparse):
    print(f"datc fused step n_before {n_before} row0 {row0} sparse {sparse}", flush=True)
    inp = make_inputs(card, n_before, 1, 4, True, sparse, row0)
    two = run_step(card, n_before, row0, 4, inp, fused=False)
    one = run_step(card, n_before, row0, 4, inp, fused=True)
    assert two["err"] == 0 and one["err"] == 0
    for k in ("out", "codes", "scales", "q16", "qf32", "kf32", "k_new", "v_new"):
        assert np.array_equal(np.asarray(one[k]).view(np.uint8), np.asarray(two[k]).view(np.uint8)), k


def test_fused_step_refusals(card):
    # the row's cell past the caches, row0 past the round's rows, a body not made at this depth: the error bit, no
    # output, no cell written
    for n_before, row0, stride, sparse, bad_k in ((CELLS - 1, 1, 4, False, 0), (100, 2, 2, False, 0),
                                                  (3000, 1, 4, True, 1)):
        inp = make_inputs(card, n_before, 1, stride, False, sparse, row0, bad_k=bad_k)
        o = run_step(card, n_before, row0, stride, inp, fused=True)
        assert o["err"] == ERR
        assert np.all(o["out"].view(np.uint32) == 0xFFFFFFFF), "output written"
        if "k_new" in o:
            assert np.all(o["k_new"].view(np.uint16) == 0x7F7F), "cell written"


def test_fused_step_host_refusals(card):
    d = card["dev"]
    nb = torch.zeros(1, dtype=torch.int32, device="cuda")
    st = torch.ones(1, dtype=torch.int32, device="cuda")
    pos = torch.zeros((4, 1), dtype=torch.int32, device="cuda")
    kv = torch.zeros((1, HD), dtype=torch.float32, device="cuda")
    qfull = torch.zeros((NH, QS), dtype=torch.float32, device="cuda")
    args = dict(kv_k=kv, kv_v=kv, k_norm=d["kn"], q_norm=d["qn"], n_before=nb, pos=pos, stride=st, k_cache=d["kc"],
                v_cache=d["vc"], q16=d["q16"], part=d["part"], out=d["out"], codes=d["codes"], scales=d["scales"],
                err=d["err"])
    d["out"].view(torch.int32).fill_(-1)
    with pytest.raises(fnkv.FnkvError):  # no q rows
        fnkv.datc_step(qfull=None, **args)
    with pytest.raises(fnkv.FnkvError):  # row0 past the attend's rows
        fnkv.datc_step(qfull=qfull, row0=5, **args)
    misaligned = torch.zeros(HD + 1, dtype=torch.float32, device="cuda")[1:]
    with pytest.raises(fnkv.FnkvError):  # k rows off a 16-byte boundary
        fnkv.datc_step(qfull=qfull, **{**args, "kv_k": misaligned})
    torch.cuda.synchronize()
    assert np.all(d["out"].cpu().numpy().view(np.uint32) == 0xFFFFFFFF), "a refusal enqueued work"

"""One captured HIP graph serving every decode step: the launches that read their context or depth from device memory
(fnkv_attn_decode_dev, fnkv_attn_sparse_dev, fnkv_attend; the reference's device depth, fn/kernels/qsa/attend.h:108,
"read by the launch (TG1)") are captured once and replayed while the context advances by T a step, every step checked
against the oracle's fp64 attention (max-abs 2e-3, the fp16 output rounding aside). A context or depth outside the
launch's contract writes nothing (no cells, no outputs) and sets the caller-cleared error word's refused-depth bit (2,
attend.h:91-92); the other sequences of the launch run. attend_lanes: each lane bitwise its lone call."""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2e-3
HQ, HKV, D = 16, 2, 256


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def capture(fn):
    """fn() run once eagerly on a side stream (warm-up), then captured into one graph"""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


class DecodeLoop:
    """Sequences in a pool, their fp16 K/V for every position up to the bound, and the oracle's decoded copy."""

    def __init__(self, ctx0, T, steps, seed, fmt=fnkv.FMT_Q8_0):
        self.T, self.steps = T, steps
        self.ctx0 = list(ctx0)
        self.cap = [c + T * steps for c in ctx0]
        self.pool = fnkv.Pool(len(ctx0) + 1, sum(-(-c // 256) for c in self.cap) + 8, 1, HKV, fmt=fmt)
        self.slots = list(range(len(ctx0)))
        cases.scatter_ensure(self.pool, self.slots, self.cap, seed, churn=0.3)
        self.kv, self.dec = [], []
        for s, c0 in zip(self.slots, self.ctx0):
            k16, v16 = cases.kv_rows(seed * 10 + s, self.cap[s], HKV)
            first = c0 - T  # cells before the first step's new ones
            if first:
                self.pool.append(s, 0, 0, torch.from_numpy(k16[:first]).cuda(), torch.from_numpy(v16[:first]).cuda())
            self.kv.append((k16, v16))
            if fmt == fnkv.FMT_KV8:
                (_, _, kf), (_, _, vf) = cases.decoded_kv8(O, k16, v16)
            else:
                (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
            self.dec.append((kf, vf))
        torch.cuda.synchronize()


@pytest.mark.parametrize("T,ctx0", [(1, [517, 3000, 9001]), (3, [700, 3000, 9000]), (5, [1290, 20000])])
def test_decode_one_graph_advancing_context(T, ctx0):
    steps = 8
    L = DecodeLoop(ctx0, T, steps, seed=40 + T)
    n = len(ctx0)
    ctx_dev = torch.tensor(ctx0, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q = torch.empty((n, T, HQ, D), dtype=torch.float16, device="cuda")
    kn = torch.empty((n, T, HKV, D), dtype=torch.float16, device="cuda")
    vn = torch.empty_like(kn)
    out = torch.empty_like(q)
    ws = torch.zeros(L.pool.decode_ws_bytes(L.cap, T, HQ), dtype=torch.uint8, device="cuda")

    def launch():
        L.pool.decode_dev(L.slots, ctx_dev, L.cap, T, 0, q, out, ws, err, k_new=kn, v_new=vn)

    # inputs of step 0 staged before the warm-up run (which performs step 0's append, redone identically by replay 0)
    def stage(i):
        for s in range(n):
            c = ctx0[s] + i * T
            k16, v16 = L.kv[s]
            kn[s].copy_(torch.from_numpy(k16[c - T:c]))
            vn[s].copy_(torch.from_numpy(v16[c - T:c]))
        ctx_dev.copy_(torch.tensor([c + i * T for c in ctx0], dtype=torch.int64))
        q16 = cases.queries(1000 + i, (n, T, HQ, D))
        q.copy_(torch.from_numpy(q16))
        return q16

    stage(0)
    graph = capture(launch)
    worst = 0.0
    for i in range(steps):
        q16 = stage(i)
        graph.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for s in range(n):
            c = ctx0[s] + i * T
            kf, vf = L.dec[s]
            ref = O.attn_f64(q16[s].view(np.uint16), kf, vf, c)
            e = cases.out_err(got[s], ref)
            worst = max(worst, e)
            assert e <= TOL, (i, s, c, e)
    assert err.item() == 0
    # the appended cells are the oracle's Q8_0 blocks of the step's K / V, at the advancing positions
    for s in range(n):
        c_end = ctx0[s] + (steps - 1) * T
        blocks = L.pool.export(s, 0, 1, 0, ctx0[s] - T, c_end - ctx0[s] + T)
        torch.cuda.synchronize()
        k16 = L.kv[s][0][ctx0[s] - T:c_end, 1]
        kq, kd = O.q8_0_quantize(k16.astype(np.float32))
        qs, dd = O.from_block_q8_0(blocks.cpu().numpy().reshape(-1, 34))
        assert np.array_equal(qs.reshape(kq.shape), kq) and np.array_equal(dd.reshape(kd.shape), kd)


@pytest.mark.parametrize("T", [1, 3, 5])
def test_decode_dev_context_far_below_bound(T):
    # the grid and the strided splits come from the host bound (~9,000 cells above each context here), the walks'
    # tile counts from the device word: most splits hold no tile of their sequence and the merge skips them
    steps = 3000
    L = DecodeLoop([T + 40, 2000, 5003], T, steps, seed=70 + T)
    n = len(L.ctx0)
    ctx_dev = torch.tensor(L.ctx0, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q16 = cases.queries(90 + T, (n, T, HQ, D))
    q = torch.from_numpy(q16).cuda()
    kn = torch.from_numpy(np.stack([L.kv[s][0][c - T:c] for s, c in enumerate(L.ctx0)])).cuda()
    vn = torch.from_numpy(np.stack([L.kv[s][1][c - T:c] for s, c in enumerate(L.ctx0)])).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(L.pool.decode_ws_bytes(L.cap, T, HQ), dtype=torch.uint8, device="cuda")
    L.pool.decode_dev(L.slots, ctx_dev, L.cap, T, 0, q, out, ws, err, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert err.item() == 0
    got = out.cpu().numpy()
    for s, c in enumerate(L.ctx0):
        kf, vf = L.dec[s]
        ref = O.attn_f64(q16[s].view(np.uint16), kf, vf, c)
        assert cases.out_err(got[s], ref) <= TOL, (s, c)


@pytest.mark.parametrize("case", range(6))
def test_seeded_random_device_context_launches(case):
    # seeded shapes through fnkv_attn_decode_dev: 1-8 sequences, T 1-6, contexts log-uniform in [T + 1, 40,000], each
    # sequence's host bound 0-3,000 steps of T above its context (so the grid's strided splits hold from all to few
    # of its tiles), the step's new cells written by the launch
    rng = np.random.default_rng([case, 5151])
    n = int(rng.integers(1, 9))
    T = int(rng.integers(1, 7))
    ctx0 = [int(max(T + 1, round(np.exp(rng.uniform(np.log(T + 2), np.log(40000)))))) for _ in range(n)]
    steps = int(rng.integers(0, 3001))
    print(f"case {case}: n {n} T {T} ctxs {ctx0} slack {T * steps}", flush=True)
    L = DecodeLoop(ctx0, T, steps, seed=500 + case)
    ctx_dev = torch.tensor(ctx0, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q16 = cases.queries(600 + case, (n, T, HQ, D))
    q = torch.from_numpy(q16).cuda()
    kn = torch.from_numpy(np.stack([L.kv[s][0][c - T:c] for s, c in enumerate(ctx0)])).cuda()
    vn = torch.from_numpy(np.stack([L.kv[s][1][c - T:c] for s, c in enumerate(ctx0)])).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(L.pool.decode_ws_bytes(L.cap, T, HQ), dtype=torch.uint8, device="cuda")
    L.pool.decode_dev(L.slots, ctx_dev, L.cap, T, 0, q, out, ws, err, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert err.item() == 0
    got = out.cpu().numpy()
    for s, c in enumerate(ctx0):
        kf, vf = L.dec[s]
        assert cases.out_err(got[s], O.attn_f64(q16[s].view(np.uint16), kf, vf, c)) <= TOL, (case, s, c)


def test_decode_dev_matches_host_context_launch():
    # T = 1 (16 query rows a KV head): the host-value launch splits the same way, so the outputs are bitwise equal
    L = DecodeLoop([4100, 777], 1, 0, seed=3)
    for s in range(2):
        k16, v16 = L.kv[s]
        L.pool.append(s, 0, L.ctx0[s] - 1, torch.from_numpy(k16[-1:]).cuda(), torch.from_numpy(v16[-1:]).cuda())
    q = torch.from_numpy(cases.queries(5, (2, 1, HQ, D))).cuda()
    ws = torch.zeros(L.pool.decode_ws_bytes(L.cap, 1, HQ), dtype=torch.uint8, device="cuda")
    a, b = torch.empty_like(q), torch.empty_like(q)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    L.pool.decode(L.slots, L.cap, 1, 0, q, a, ws)
    L.pool.decode_dev(L.slots, torch.tensor(L.cap, dtype=torch.int64, device="cuda"), L.cap, 1, 0, q, b, ws, err)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)) and err.item() == 0


@pytest.mark.parametrize("bad", ["past_bound", "below_T"])
def test_decode_refused_context_writes_nothing(bad):
    T = 3
    L = DecodeLoop([1000, 5000], T, 2, seed=9)
    cap = L.cap
    ctx = [cap[0] + 1 if bad == "past_bound" else T - 1, 5000]
    ctx_dev = torch.tensor(ctx, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q16 = cases.queries(8, (2, T, HQ, D))
    q = torch.from_numpy(q16).cuda()
    # sequence 0's rows (refused) are its first cells' values; sequence 1's are its own new cells
    kn = torch.from_numpy(np.stack([L.kv[0][0][:T], L.kv[1][0][ctx[1] - T:ctx[1]]])).cuda()
    vn = torch.from_numpy(np.stack([L.kv[0][1][:T], L.kv[1][1][ctx[1] - T:ctx[1]]])).cuda()
    out = torch.full_like(q, 7.0)
    ws = torch.zeros(L.pool.decode_ws_bytes(cap, T, HQ), dtype=torch.uint8, device="cuda")
    before = [L.pool.export(0, 0, h, kv, 0, cap[0]).cpu() for h in range(HKV) for kv in range(2)]
    L.pool.decode_dev(L.slots, ctx_dev, cap, T, 0, q, out, ws, err, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert err.item() == fnkv.DEV_ERR_DEPTH
    assert bool((out[0] == 7.0).all())  # the refused sequence's rows untouched
    after = [L.pool.export(0, 0, h, kv, 0, cap[0]).cpu() for h in range(HKV) for kv in range(2)]
    assert all(torch.equal(x, y) for x, y in zip(before, after))  # and its cells
    kf, vf = L.dec[1]  # the other sequence ran (its new cells are the ones kn[1] holds: its own positions)
    ref = O.attn_f64(q16[1].view(np.uint16), kf, vf, ctx[1])
    assert cases.out_err(out[1].cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("T", [1, 3])
def test_replay_after_trim_reads_no_unmapped_page(T):
    # Outside the contract (a slot must stay mapped up to the bound while a captured launch can run): the slot of
    # sequence 1 is trimmed below the context its captured launch reads, so the tail of its page-table row is
    # unmapped (-1). The replay reads nothing through those entries (the walk takes page 0 instead), writes nothing
    # for that sequence (no outputs, no new cells) and sets the refused-depth bit; sequence 0 is computed as before.
    # T = 1 walks strided splits, T = 3 contiguous ones.
    ctx = [3000, 5000]
    L = DecodeLoop(ctx, T, 0, seed=21 + T)
    ctx_dev = torch.tensor(ctx, dtype=torch.int64, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q = torch.from_numpy(cases.queries(5, (2, T, HQ, D))).cuda()
    kn = torch.from_numpy(np.stack([L.kv[i][0][c - T:c] for i, c in enumerate(ctx)])).cuda()
    vn = torch.from_numpy(np.stack([L.kv[i][1][c - T:c] for i, c in enumerate(ctx)])).cuda()
    out = torch.full_like(q, 7.0)
    ws = torch.zeros(L.pool.decode_ws_bytes(ctx, T, HQ), dtype=torch.uint8, device="cuda")
    g = capture(lambda: L.pool.decode_dev(L.slots, ctx_dev, ctx, T, 0, q, out, ws, err, k_new=kn, v_new=vn))
    g.replay()
    torch.cuda.synchronize()
    assert err.item() == 0
    ref = out.clone()
    assert L.pool.trim(1, 1024) == 0  # the engine would drain and re-capture first; this replay runs regardless
    assert L.pool.mapped_cells(1) == 1024
    out.fill_(7.0)
    for _ in range(2):
        g.replay()
        torch.cuda.synchronize()
        assert err.item() == fnkv.DEV_ERR_DEPTH
        assert bool((out[1] == 7.0).all())  # nothing written for the trimmed sequence
        assert torch.equal(out[0].view(torch.int16), ref[0].view(torch.int16))  # the other one as before
        err.zero_()


def test_decode_dev_host_refusals_enqueue_nothing():
    L = DecodeLoop([600], 1, 1, seed=2)
    q = torch.zeros((1, 1, HQ, D), dtype=torch.float16, device="cuda")
    out = torch.full_like(q, 3.0)
    ws = torch.zeros(L.pool.decode_ws_bytes(L.cap, 1, HQ), dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ctx_dev = torch.tensor([600], dtype=torch.int64, device="cuda")
    with pytest.raises(fnkv.FnkvError):  # a bound past the slot's mapped cells
        L.pool.decode_dev(L.slots, ctx_dev, [L.pool.mapped_cells(0) + 1], 1, 0, q, out, ws, err)
    with pytest.raises(fnkv.FnkvError):  # no error word
        L.pool.decode_dev(L.slots, ctx_dev, L.cap, 1, 0, q, out, ws, None)
    torch.cuda.synchronize()
    assert bool((out == 3.0).all()) and err.item() == 0


def test_decode_duplicate_slot_with_append_refused():
    L = DecodeLoop([600], 1, 1, seed=2)
    q = torch.zeros((2, 1, HQ, D), dtype=torch.float16, device="cuda")
    kn = torch.zeros((2, 1, HKV, D), dtype=torch.float16, device="cuda")
    out = torch.empty_like(q)
    ws = torch.zeros(L.pool.decode_ws_bytes([600, 600], 1, HQ), dtype=torch.uint8, device="cuda")
    with pytest.raises(fnkv.FnkvError):
        L.pool.decode([0, 0], [600, 600], 1, 0, q, out, ws, k_new=kn, v_new=kn)
    L.pool.decode([0, 0], [600, 600], 1, 0, q, out, ws)  # reading one slot twice is fine
    torch.cuda.synchronize()


@pytest.mark.parametrize("T,depth0", [(1, 3000), (3, 16100)])
def test_sparse_one_graph_advancing_depth(T, depth0):
    steps = 8
    bound = depth0 + T * steps + 5  # depth + T <= bound at every step
    hq = HQ
    pool = fnkv.Pool(2, -(-bound // 256) + 8, 1, HKV)
    cases.scatter_ensure(pool, [0], [bound], 11, churn=0.3)
    k16, v16 = cases.kv_rows(77, bound, HKV)
    pool.append(0, 0, 0, torch.from_numpy(k16[:depth0]).cuda(), torch.from_numpy(v16[:depth0]).cuda())
    (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
    depth_dev = torch.tensor([depth0], dtype=torch.int32, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    q = torch.empty((T, hq, D), dtype=torch.float16, device="cuda")
    kn = torch.empty((T, HKV, D), dtype=torch.float16, device="cuda")
    vn = torch.empty_like(kn)
    out = torch.empty_like(q)
    body = torch.zeros(T * (2 + 512 + 3) + 8, dtype=torch.int32, device="cuda")
    offs = torch.zeros(T + 1, dtype=torch.int32, device="cuda")
    ws = torch.empty(pool.sparse_ws_bytes(bound - T, T, hq), dtype=torch.uint8, device="cuda")

    def stage(i):
        d = depth0 + i * T
        words, o, cells = O.qsa_body(d, T, 500 + i, clustered=i % 2 == 1)
        body[:words.size].copy_(torch.from_numpy(words.view(np.int32)))
        offs.copy_(torch.from_numpy(o))
        kn.copy_(torch.from_numpy(k16[d:d + T]))
        vn.copy_(torch.from_numpy(v16[d:d + T]))
        depth_dev.fill_(d)
        q16 = cases.queries(700 + i, (T, hq, D))
        q.copy_(torch.from_numpy(q16))
        return q16, cells

    stage(0)
    graph = capture(lambda: pool.sparse_dev(0, depth_dev, bound, 0, q, body, offs, out, ws, err, k_new=kn,
                                            v_new=vn))
    for i in range(steps):
        q16, cells = stage(i)
        graph.replay()
        torch.cuda.synchronize()
        ref = O.attn_f64_cells(q16.view(np.uint16), kf, vf, cells)
        e = cases.out_err(out.cpu().numpy(), ref)
        assert e <= TOL, (i, e)
    assert err.item() == 0
    # a depth past the bound: nothing written, the bit set
    out.fill_(5.0)
    depth_dev.fill_(bound - T + 1)
    graph.replay()
    torch.cuda.synchronize()
    assert err.item() == fnkv.DEV_ERR_DEPTH and bool((out == 5.0).all())


class AttendCase:
    """fnkv_attend's inputs for one sequence of a pool (the reference's card: hq query heads on h_kv KV heads)."""

    def __init__(self, pool, slot, T, hq, h_kv, bound, seed):
        self.pool, self.slot, self.T, self.hq, self.h_kv, self.bound = pool, slot, T, hq, h_kv, bound
        self.seed = seed
        z = lambda *s, **k: torch.zeros(s, device="cuda", **k)  # noqa: E731
        self.qfull, self.kv_k, self.kv_v = z(T, hq, 512), z(T, h_kv, 256), z(T, h_kv, 256)
        self.q_norm, self.k_norm = z(256), z(256)
        self.pos = z(4, T, dtype=torch.int32)
        self.body = z(T * (2 + 512 + 3) + 8, dtype=torch.int32)
        self.offs = z(T + 1, dtype=torch.int32)
        self.depth = z(1, dtype=torch.int32)
        self.err = z(1, dtype=torch.int32)
        self.out = z(T, hq, 256)
        self.codes = z(T, hq * 256, dtype=torch.int8)
        self.scales = z(T, hq * 8, 2)
        self.k_f32 = z(T, h_kv, 256)
        self.ws = torch.empty(pool.attend_ws_bytes(bound, T, hq), dtype=torch.uint8, device="cuda")
        self.args = pool.attend_args(slot, 0, self.depth, bound, self.qfull, self.kv_k, self.kv_v, self.q_norm,
                                     self.k_norm, self.pos, self.body, self.offs, self.out, self.codes, self.scales,
                                     self.ws, self.err, k_f32=self.k_f32)

    def stage(self, depth, step):
        rng = np.random.default_rng([self.seed, step])
        T = self.T
        words, o, cells = O.qsa_body(depth, T, self.seed + step)
        self.body.zero_()
        self.body[:words.size].copy_(torch.from_numpy(words.view(np.int32)))
        self.offs.copy_(torch.from_numpy(o))
        x = dict(qfull=rng.uniform(-3, 3, (T, self.hq, 512)), kv_k=rng.uniform(-2, 2, (T, self.h_kv, 256)),
                 kv_v=rng.uniform(-1.5, 1.5, (T, self.h_kv, 256)), q_norm=rng.uniform(0.3, 1.8, 256),
                 k_norm=rng.uniform(0.3, 1.8, 256))
        x = {k: v.astype(np.float32) for k, v in x.items()}
        for k, v in x.items():
            getattr(self, k).copy_(torch.from_numpy(v))
        pos = np.array([[depth + t] * 4 for t in range(T)], np.int32).T.copy()
        self.pos.copy_(torch.from_numpy(pos))
        self.depth.fill_(depth)
        return x, pos, cells


def attend_reference(c, depth, x, pos, cells, kdec, vdec, fmt=fnkv.FMT_Q8_0):
    """the oracle's gated output for case c at this depth; kdec, vdec: the decoded cache, cells depth.. replaced by
    the pool's rule applied to the launch's own F32 k (read back) and to v"""
    ts = fnkv.rope_theta_scale()
    T = c.T
    q64 = np.stack([[O.norm_rope_f64(x["qfull"][t, h, :256], x["q_norm"], list(pos[:, t]), ts)
                     for h in range(c.hq)] for t in range(T)])
    kf = c.k_f32.cpu().numpy()
    kc, kd = O.q8_0_quantize(kf)
    vc, vd = O.q8_0_quantize(x["kv_v"])
    kdec, vdec = kdec.copy(), vdec.copy()
    kdec[depth:depth + T] = O.q8_0_dequantize(kc, kd)
    vdec[depth:depth + T] = O.q8_0_dequantize(vc, vd)
    return O.attn_f64_cells(q64, kdec, vdec, cells) / (1.0 + np.exp(-x["qfull"][:, :, 256:].astype(np.float64)))


@pytest.mark.parametrize("T", [1, 3])
def test_attend_one_graph_advancing_depth(T):
    steps, depth0, hq, h_kv = 8, 9000, 12, 1
    bound = depth0 + T * steps
    pool = fnkv.Pool(2, -(-bound // 256) + 8, 1, h_kv)
    cases.scatter_ensure(pool, [0], [bound], 5, churn=0.3)
    k16, v16 = cases.kv_rows(31, bound, h_kv)
    pool.append(0, 0, 0, torch.from_numpy(k16[:depth0]).cuda(), torch.from_numpy(v16[:depth0]).cuda())
    (_, _, kdec), (_, _, vdec) = cases.decoded(O, k16, v16)
    c = AttendCase(pool, 0, T, hq, h_kv, bound, seed=60 + T)
    c.stage(depth0, 0)
    graph = capture(lambda: fnkv.attend(T, c.args))
    for i in range(steps):
        d = depth0 + i * T
        x, pos, cells = c.stage(d, i)
        graph.replay()
        torch.cuda.synchronize()
        ref = attend_reference(c, d, x, pos, cells, kdec, vdec)
        got = c.out.cpu().numpy()
        e = float(np.abs(got.astype(np.float64) - ref).max())
        assert np.isfinite(got).all() and e <= TOL, (i, e)
        ne = max(O.norm_err(ref[t, h], got[t, h]) for t in range(T) for h in range(c.hq))
        assert ne <= 1e-5, (i, ne)  # the reference checker's bound, qa2_test.cpp:58
        # the cells the step wrote become the cache the next steps read
        kdec[d:d + T] = O.q8_0_dequantize(*O.q8_0_quantize(c.k_f32.cpu().numpy()))
        vdec[d:d + T] = O.q8_0_dequantize(*O.q8_0_quantize(x["kv_v"]))
    assert c.err.item() == 0
    # a refused depth: nothing written (outputs and cells), the bit set
    c.out.fill_(9.0)
    before = pool.export(0, 0, 0, 0, 0, bound).cpu()
    c.depth.fill_(bound - T + 1)
    graph.replay()
    torch.cuda.synchronize()
    assert c.err.item() == fnkv.DEV_ERR_DEPTH and bool((c.out == 9.0).all())
    assert torch.equal(before, pool.export(0, 0, 0, 0, 0, bound).cpu())


@pytest.mark.parametrize("lanes,T", [(2, 1), (3, 3), (4, 5)])
def test_attend_lanes_bitwise_their_lone_calls(lanes, T):
    hq, h_kv = 12, 1
    depths = [3000 + 1111 * u for u in range(lanes)]
    bounds = [d + T for d in depths]
    pool = fnkv.Pool(lanes + 1, sum(-(-b // 256) for b in bounds) + 8, 1, h_kv)
    cases.scatter_ensure(pool, list(range(lanes)), bounds, 17, churn=0.3)
    cs = []
    for u in range(lanes):
        k16, v16 = cases.kv_rows(90 + u, bounds[u], h_kv)
        pool.append(u, 0, 0, torch.from_numpy(k16[:depths[u]]).cuda(), torch.from_numpy(v16[:depths[u]]).cuda())
        c = AttendCase(pool, u, T, hq, h_kv, bounds[u], seed=200 + 7 * u)
        c.stage(depths[u], 0)
        cs.append(c)

    def snapshot():
        torch.cuda.synchronize()
        r = []
        for u, c in enumerate(cs):
            r += [c.out.cpu().clone(), c.codes.cpu().clone(), c.scales.cpu().clone(), c.k_f32.cpu().clone(),
                  pool.export(u, 0, 0, 0, depths[u], T).cpu(), pool.export(u, 0, 0, 1, depths[u], T).cpu()]
        return r

    for c in cs:
        fnkv.attend(T, c.args)
    lone = snapshot()
    for c in cs:
        c.out.zero_(), c.codes.zero_(), c.scales.zero_(), c.k_f32.zero_()
    fnkv.attend_lanes(T, [c.args for c in cs])
    joint = snapshot()
    assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(lone, joint))
    # a lane at a refused depth writes nothing; the others run
    cs[0].depth.fill_(bounds[0] + 1)
    cs[0].out.fill_(4.0)
    fnkv.attend_lanes(T, [c.args for c in cs])
    again = snapshot()
    torch.cuda.synchronize()
    assert cs[0].err.item() == fnkv.DEV_ERR_DEPTH and bool((cs[0].out == 4.0).all())
    assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(lone[6:], again[6:]))
    # two lanes on one slot, or one lane outside the contract: nothing enqueued
    with pytest.raises(fnkv.FnkvError):
        fnkv.attend_lanes(T, [cs[1].args, cs[1].args])
    with pytest.raises(fnkv.FnkvError):
        fnkv.attend_lanes(T, [cs[1].args])

"""Decode / speculative-verify attention on the GPU against the oracle (max-abs 2e-3 against the fp64 attention over
the decoded cache, fp32-Q), plus the properties the reference's own tests hold (qa2_test.cpp:532-643): bitwise
reruns, and here also bitwise invariance under a different physical page placement."""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2e-3
HQ, HKV = 16, 2


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


class Setup:
    """Sequences appended into a pool, with the oracle's decoded copy of their caches."""

    def __init__(self, ctxs, seed, layers=1, n_pages=None, churn=0.0, order_seed=None):
        n_pages = n_pages or sum(-(-c // 256) for c in ctxs) + 8
        self.pool = fnkv.Pool(len(ctxs) + 1, n_pages, layers, HKV)
        self.slots = list(range(len(ctxs)))
        self.ctxs = list(ctxs)
        cases.scatter_ensure(self.pool, self.slots, self.ctxs, seed if order_seed is None else order_seed, churn)
        self.dec = {}
        for s, c in zip(self.slots, self.ctxs):
            for layer in range(layers):
                k16, v16 = cases.kv_rows(seed * 100 + s, c, HKV, layer)
                self.pool.append(s, layer, 0, torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda())
                (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
                self.dec[(s, layer)] = (kf, vf)
        torch.cuda.synchronize()

    def run(self, q16, T, layer=0, slots=None, ctxs=None):
        slots = self.slots if slots is None else slots
        ctxs = self.ctxs if ctxs is None else ctxs
        q = torch.from_numpy(q16).cuda()
        out = torch.empty_like(q)
        ws = torch.zeros(self.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
        self.pool.decode(slots, ctxs, T, layer, q, out, ws)
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def check(self, q16, got, T, layer=0, slots=None, ctxs=None):
        slots = self.slots if slots is None else slots
        ctxs = self.ctxs if ctxs is None else ctxs
        worst = 0.0
        for i, (s, c) in enumerate(zip(slots, ctxs)):
            kf, vf = self.dec[(s, layer)]
            ref = O.attn_f64(q16[i].view(np.uint16), kf, vf, c)
            err = cases.out_err(got[i], ref)
            worst = max(worst, err)
        return worst

    def check_plain(self, q16, got, T, layer=0):
        """check()'s comparison with the plain max-abs |got - ref| (no fp16-spacing allowance)."""
        worst = 0.0
        for i, (s, c) in enumerate(zip(self.slots, self.ctxs)):
            kf, vf = self.dec[(s, layer)]
            ref = O.attn_f64(q16[i].view(np.uint16), kf, vf, c)
            worst = max(worst, cases.plain_err(got[i], ref))
        return worst


def test_config0_single_sequence_decode():
    # 16 Q heads, 2 KV heads, d 256, context 4,096, T = 1
    st = Setup([4096], seed=1)
    q16 = cases.queries(1, (1, 1, HQ, 256))
    got = st.run(q16, 1)
    assert st.check(q16, got, 1) <= TOL
    assert st.check_plain(q16, got, 1) <= TOL  # BASELINE's distribution: the plain max-abs holds the bar too
    # and against the ggml-semantics CPU path
    kf, vf = st.dec[(0, 0)]
    k16, v16 = cases.kv_rows(100, 4096, HKV, 0)
    (kq, kd, _), (vq, vd, _) = cases.decoded(O, k16, v16)
    kb = O.to_block_q8_0(kq, kd)
    vb = O.to_block_q8_0(vq, vd)
    g = O.attn_ggml(q16[0].view(np.uint16), kb, vb, 4096, threads=4).view(np.float16)
    assert np.abs(got[0].astype(np.float32) - g.astype(np.float32)).max() <= 2 * TOL


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6])
def test_verify_depths_ragged_contexts(T):
    # contexts that end mid-tile, mid-page, at a page edge, and barely above T
    ctxs = [T, 33, 255, 256, 257, 1000, 3 * 256 + 31]
    st = Setup(ctxs, seed=10 + T, churn=0.3)
    q16 = cases.queries(20 + T, (len(ctxs), T, HQ, 256))
    got = st.run(q16, T)
    assert st.check(q16, got, T) <= TOL


def test_bitwise_reruns_and_page_placement_invariance():
    ctxs = [5000, 777, 12000]
    a = Setup(ctxs, seed=3, order_seed=1)
    b = Setup(ctxs, seed=3, order_seed=2, churn=0.5)
    assert a.pool.table(0) != b.pool.table(0)
    q16 = cases.queries(3, (3, 3, HQ, 256))
    r1 = a.run(q16, 3)
    r2 = a.run(q16, 3)
    r3 = b.run(q16, 3)
    assert np.array_equal(r1.view(np.uint16), r2.view(np.uint16))
    assert np.array_equal(r1.view(np.uint16), r3.view(np.uint16))
    assert a.check(q16, r1, 3) <= TOL


def test_fold_fallback_and_reused_workspace_bitwise():
    """The split-K fold inside the launch (stream.hip: row r of a (sequence, KV head) folded by its split r mod n after
    every split has arrived) against the merge launch: both within the tolerance, each bitwise on reruns. With the wait
    bound at zero the owners give their rows up to the last split to arrive, which folds them: bitwise the fold's
    outputs again. One workspace serves every launch (its fold counters stay consistent)."""
    ctxs = [30000, 9000, 65536]
    st = Setup(ctxs, seed=5)
    q16 = cases.queries(5, (3, 3, HQ, 256))
    q = torch.from_numpy(q16).cuda()
    ws = torch.zeros(st.pool.decode_ws_bytes(ctxs, 3, HQ), dtype=torch.uint8, device="cuda")
    outs = []
    L = fnkv.lib()
    for mode, spin in ((0, -1), (1, -1), (1, 0), (1, 0), (1, -1), (0, -1)):
        L.fnkv_test_decode_fold(mode, spin)
        try:
            out = torch.empty_like(q)
            st.pool.decode(st.slots, ctxs, 3, 0, q, out, ws)
            torch.cuda.synchronize()
        finally:
            L.fnkv_test_decode_fold(-1, -1)
        outs.append(out.cpu().numpy())
    same = lambda x, y: np.array_equal(x.view(np.uint16), y.view(np.uint16))
    # the merge launch twice, and the fold (default bound, zero bound twice, default again): each bitwise itself
    assert same(outs[0], outs[5])
    assert all(same(outs[1], o) for o in outs[2:5])
    # the two fold the same partials in different orders: equal to within an fp16 rounding
    assert float(np.abs(outs[0].astype(np.float32) - outs[1].astype(np.float32)).max()) <= 1e-3
    assert st.check(q16, outs[0], 3) <= TOL and st.check(q16, outs[1], 3) <= TOL
    # the fold region (the workspace's first bytes): each pair's arrival counter at a whole number of launches
    words = ws[: 16 * HKV * 50 * 4].view(torch.int32).cpu().numpy().reshape(16 * HKV, 50)
    assert np.all(words[:, 0] % 1024 == 0) and words[:, 0].max() > 0


def test_layers_are_separate():
    st = Setup([1500, 600], seed=4, layers=3)
    q16 = cases.queries(4, (2, 1, HQ, 256))
    for layer in range(3):
        got = st.run(q16, 1, layer=layer)
        assert st.check(q16, got, 1, layer=layer) <= TOL


def test_config1_shapes_one_layer():
    # BASELINE config 1's sequences (8K / 16K / 32K / 64K) at T = 3, one layer, pages interleaved
    ctxs = [8192, 16384, 32768, 65536]
    st = Setup(ctxs, seed=5, churn=0.2)
    q16 = cases.queries(5, (4, 3, HQ, 256))
    got = st.run(q16, 3)
    assert st.check(q16, got, 3) <= TOL
    assert st.check_plain(q16, got, 3) <= TOL


def test_config1_all_twelve_layers():
    # BASELINE config 1 in full: 4 sequences at 8K / 16K / 32K / 64K, T = 3, all 12 layers of one pool, K and V in
    # BASELINE's distribution (N(0, 1), 4 channels of each KV head x8), each layer's new cells appended by its launch
    # (as the bench's step); every layer's outputs checked against the fp64 attention over that layer's cells as the
    # pool holds them (exported as ggml block_q8_0 and decoded by the oracle), by out_err and by the plain max-abs
    ctxs, T, layers = [8192, 16384, 32768, 65536], 3, 12
    n_pages = sum(-(-c // 256) for c in ctxs) + 8
    pool = fnkv.Pool(len(ctxs) + 1, n_pages, layers, HKV)
    slots = list(range(len(ctxs)))
    cases.scatter_ensure(pool, slots, ctxs, 12, churn=0.2)
    kn = np.empty((layers, len(ctxs), T, HKV, 256), np.float16)
    vn = np.empty_like(kn)
    for layer in range(layers):
        for i, (s_, c) in enumerate(zip(slots, ctxs)):
            k16, v16 = cases.kv_rows(1200 + 10 * i, c, HKV, layer)
            pool.append(s_, layer, 0, torch.from_numpy(k16[: c - T]).cuda(), torch.from_numpy(v16[: c - T]).cuda())
            kn[layer, i], vn[layer, i] = k16[c - T:], v16[c - T:]
    q16 = cases.queries(13, (layers, len(ctxs), T, HQ, 256))
    q, k_new, v_new = (torch.from_numpy(x).cuda() for x in (q16, kn, vn))
    out = torch.empty_like(q)
    ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    for layer in range(layers):
        pool.decode(slots, ctxs, T, layer, q[layer], out[layer], ws, k_new=k_new[layer], v_new=v_new[layer])
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    worst = plain = 0.0
    for layer in range(layers):
        for i, (s_, c) in enumerate(zip(slots, ctxs)):
            kf = np.empty((c, HKV, 256), np.float32)
            vf = np.empty((c, HKV, 256), np.float32)
            for h in range(HKV):
                for kv, dst in ((0, kf), (1, vf)):
                    qs, d = O.from_block_q8_0(pool.export(s_, layer, h, kv, 0, c).cpu().numpy())
                    dst[:, h, :] = O.q8_0_dequantize(qs.reshape(c, 256), d.reshape(c, 8))
            ref = O.attn_f64(q16[layer, i].view(np.uint16), kf, vf, c)
            worst = max(worst, cases.out_err(got[layer, i], ref))
            plain = max(plain, cases.plain_err(got[layer, i], ref))
    assert worst <= TOL and plain <= TOL, (worst, plain)


@pytest.mark.parametrize("T", [1, 5])
def test_config2_deep_context(T):
    # 262,144 cells in scattered pages, decode (T = 1) and a depth-4 verify (T = 5)
    st = Setup([262144], seed=6, churn=0.3)
    q16 = cases.queries(6 + T, (1, T, HQ, 256))
    got = st.run(q16, T)
    assert st.check(q16, got, T) <= TOL
    assert st.check_plain(q16, got, T) <= TOL


def test_refusals_enqueue_nothing():
    st = Setup([300], seed=7)
    q = torch.zeros((1, 1, HQ, 256), dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(fnkv.FnkvError):
        st.pool.decode([0], [600], 1, 0, q, out, ws)  # past the mapped cells
    q7 = torch.zeros((1, 7, HQ, 256), dtype=torch.float16, device="cuda")
    with pytest.raises(fnkv.FnkvError):
        st.pool.decode([0], [300], 7, 0, q7, torch.zeros_like(q7), ws)  # 8 x 7 rows > 48
    with pytest.raises(fnkv.FnkvError):
        st.pool.decode([0], [300], 1, 0, q, out, ws[:16])  # workspace too small
    torch.cuda.synchronize()
    assert not out.any()


def test_fused_append_matches_separate_append():
    # the launch that appends its step's new cells (k_new / v_new) gives the same pool bytes and the same outputs,
    # bitwise, as a separate fnkv_q8_append followed by a launch without them; contexts put the new cells across a
    # tile edge, a page edge and a split edge
    T = 5
    ctxs = [1026, 4098, 300]
    a = Setup(ctxs, seed=8, order_seed=3)
    b = Setup(ctxs, seed=8, order_seed=3)
    q16 = cases.queries(8, (3, T, HQ, 256))
    kn = torch.from_numpy(cases.queries(9, (3, T, HKV, 256))).cuda()
    vn = torch.from_numpy(cases.queries(10, (3, T, HKV, 256))).cuda()
    q = torch.from_numpy(q16).cuda()
    oa, ob = torch.empty_like(q), torch.empty_like(q)
    ws = torch.zeros(a.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    a.pool.decode(a.slots, ctxs, T, 0, q, oa, ws, k_new=kn, v_new=vn)
    for i, (s, c) in enumerate(zip(b.slots, ctxs)):
        b.pool.append(s, 0, c - T, kn[i].contiguous(), vn[i].contiguous())
    b.pool.decode(b.slots, ctxs, T, 0, q, ob, ws)
    torch.cuda.synchronize()
    assert np.array_equal(oa.cpu().numpy().view(np.uint16), ob.cpu().numpy().view(np.uint16))
    for s, c in zip(a.slots, ctxs):
        for kv in (0, 1):
            for h in range(HKV):
                ea = a.pool.export(s, 0, h, kv, 0, c)
                eb = b.pool.export(s, 0, h, kv, 0, c)
                torch.cuda.synchronize()
                assert torch.equal(ea, eb)
    # and the outputs against the oracle over the cache with the new cells in place
    for i, (s, c) in enumerate(zip(a.slots, ctxs)):
        k16, v16 = cases.kv_rows(8 * 100 + s, c, HKV, 0)
        k16[c - T:] = kn[i].cpu().numpy()
        v16[c - T:] = vn[i].cpu().numpy()
        (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
        ref = O.attn_f64(q16[i].view(np.uint16), kf, vf, c)
        assert cases.out_err(oa.cpu().numpy()[i], ref) <= TOL


@pytest.mark.parametrize("T", [1, 2, 3, 5])
def test_first_launch_matches_reruns(T):
    # A launch on a freshly filled pool (cold TLB and caches, the slowest copies) gives the same bits as warm reruns:
    # the kernels' load-count waits must cover every copy whatever its latency. Deep contexts, so each workgroup runs
    # many iterations of its copy ring.
    for ctx in (112927, 262144):
        pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, HKV)
        try:
            cases.scatter_ensure(pool, [0], [ctx], 3, 0.3)
            g = torch.Generator(device="cuda")
            g.manual_seed(ctx + T)
            x = torch.randn((2, ctx, HKV, 256), generator=g, device="cuda").half()
            pool.append(0, 0, 0, x[0].contiguous(), x[1].contiguous())
            q = torch.randn((1, T, HQ, 256), generator=g, device="cuda").half()
            ws = torch.zeros(pool.decode_ws_bytes([ctx], T, HQ), dtype=torch.uint8, device="cuda")
            outs = []
            for _ in range(6):
                out = torch.full_like(q, float("nan"))
                pool.decode([0], [ctx], T, 0, q, out, ws)
                torch.cuda.synchronize()
                outs.append(out.cpu().numpy().view(np.uint16))
            assert all(np.array_equal(outs[0], o) for o in outs[1:]), (ctx, T)
            assert np.isfinite(outs[0].view(np.float16).astype(np.float32)).all()
        finally:
            pool.close()


@pytest.mark.parametrize("split", ["512", "992", "288"])
@pytest.mark.parametrize("strided", ["0", "1"])
@pytest.mark.parametrize("T", [1, 3, 5])
def test_split_walks_contiguous_and_strided(T, strided, split, monkeypatch):
    # a sequence's splits take either their own cell ranges or every n-th tile (the launch's choice, forced here):
    # both partitions give the same attention within the tolerance, the fused append of the new cells included; the
    # split sizes are tile multiples, 992 and 288 not page multiples (split edges inside a page; 2,016 = 7 x 288 is
    # the edge the second sequence's new cells straddle at T > 1)
    monkeypatch.setenv("FNKV_STRIDED", strided)
    monkeypatch.setenv("FNKV_SPLIT_TOKENS", split)
    ctxs = [40, 2016 + T // 2, 9000 + 17, 20000 + 5]
    st = Setup(ctxs, seed=70 + T, churn=0.3)
    q16 = cases.queries(71 + T, (len(ctxs), T, HQ, 256))
    got = st.run(q16, T)
    assert st.check(q16, got, T) <= TOL
    rng = np.random.default_rng([T, 72])
    kn = rng.standard_normal((len(ctxs), T, HKV, 256), dtype=np.float32).astype(np.float16)
    vn = rng.standard_normal((len(ctxs), T, HKV, 256), dtype=np.float32).astype(np.float16)
    q = torch.from_numpy(q16).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(st.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    st.pool.decode(st.slots, ctxs, T, 0, q, out, ws, k_new=torch.from_numpy(kn).cuda(),
                   v_new=torch.from_numpy(vn).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, (s, c) in enumerate(zip(st.slots, ctxs)):
        k16, v16 = cases.kv_rows((70 + T) * 100 + s, c, HKV, 0)  # the rows Setup appended
        k16, v16 = k16.copy(), v16.copy()
        k16[c - T:], v16[c - T:] = kn[i], vn[i]
        (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
        assert cases.out_err(got[i], O.attn_f64(q16[i].view(np.uint16), kf, vf, c)) <= TOL



@pytest.mark.parametrize("T", [1, 3, 5])
def test_eight_sequences_at_split_edges(T):
    # eight sequences, their contexts at and around the split sizes the planner
    # picks (1,024 / 2,048 cells) and the 32-cell tile and 256-cell page edges
    ctxs = [1024, 2048, 2049, 4096, 6143, 10240, 20481, 40000]
    st = Setup(ctxs, seed=30 + T, churn=0.25)
    q16 = cases.queries(40 + T, (len(ctxs), T, HQ, 256))
    got = st.run(q16, T)
    assert st.check(q16, got, T) <= TOL


@pytest.mark.parametrize("T", [1, 3])
def test_sixteen_sequences_the_launch_maximum(T):
    # FNKV_MAX_SEQS = 16 sequences in one launch (the split table's last entries, the merge's sequence index past 8),
    # contexts ragged around tile, page and split edges, pages interleaved with churn
    ctxs = [33, 255, 257, 1000, 1024, 1025, 2047, 2048, 3000, 4096, 5121, 6143, 7777, 8192, 9000, 12289]
    st = Setup(ctxs, seed=60 + T, churn=0.25)
    q16 = cases.queries(70 + T, (len(ctxs), T, HQ, 256))
    got = st.run(q16, T)
    assert st.check(q16, got, T) <= TOL


def test_seventeen_sequences_refused():
    st = Setup([64] * 17, seed=5)
    q = torch.zeros((17, 1, HQ, 256), dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    with pytest.raises(fnkv.FnkvError):
        st.pool.decode(st.slots, st.ctxs, 1, 0, q, out, ws)


@pytest.mark.parametrize("case", range(8))
def test_seeded_random_launches(case):
    # seeded launch shapes: 1-8 sequences, T 1-6, contexts log-uniform in [T, 40,000] (so split, page and tile edges
    # fall anywhere under the planner's tile-granular splits), pages interleaved with churn; every other case passes
    # the step's new cells to the launch, which writes them before reading
    rng = np.random.default_rng([case, 4242])
    n_seq = int(rng.integers(1, 9))
    T = int(rng.integers(1, 7))
    ctxs = [int(max(T, round(np.exp(rng.uniform(np.log(T + 1), np.log(40000)))))) for _ in range(n_seq)]
    seed = 300 + case
    st = Setup(ctxs, seed=seed, churn=0.25)
    q16 = cases.queries(seed, (n_seq, T, HQ, 256))
    print(f"case {case}: n_seq {n_seq} T {T} ctxs {ctxs}", flush=True)
    if case % 2 == 0:
        got = st.run(q16, T)
        assert st.check(q16, got, T) <= TOL
        return
    kn = rng.standard_normal((n_seq, T, HKV, 256), dtype=np.float32).astype(np.float16)
    vn = rng.standard_normal((n_seq, T, HKV, 256), dtype=np.float32).astype(np.float16)
    q = torch.from_numpy(q16).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(st.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    st.pool.decode(st.slots, ctxs, T, 0, q, out, ws, k_new=torch.from_numpy(kn).cuda(),
                   v_new=torch.from_numpy(vn).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, (s, c) in enumerate(zip(st.slots, ctxs)):
        k16, v16 = cases.kv_rows(seed * 100 + s, c, HKV, 0)  # the rows Setup appended
        k16, v16 = k16.copy(), v16.copy()
        k16[c - T:], v16[c - T:] = kn[i], vn[i]
        (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
        assert cases.out_err(got[i], O.attn_f64(q16[i].view(np.uint16), kf, vf, c)) <= TOL, (case, i)

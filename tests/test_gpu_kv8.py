"""FNFL's KV8 format (a scale a 64-value group, divide and round to even; fn/quant/kv_q8_ref.cpp:72-87, device
kv8::quantize8 fn/kernels/qsa/kv_q8.cuh:29-52) as a pool format: the append and the decode launch's fused append
bit-exact against the reference's own outputs (golden vectors from kv_q8_ref.cpp compiled in oracle/_ref) and the
oracle, and decode / verify / prefill attention over a KV8 pool against the fp64 attention over the KV8-decoded cache
(value = code x scale, exact, as the reference's kv8::decode4, kv_q8.cuh:58-68), max-abs 2e-3."""
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


def _export(pool, slot, layer, head, kv, tok0, n):
    c, s = pool.export_kv8(slot, layer, head, kv, tok0, n)
    torch.cuda.synchronize()
    return c.cpu().numpy(), s.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("name", ["stress", "rows", "nonfinite"])
def test_kv8_append_matches_reference_golden(golden, name):
    g = golden("kv8_golden.npz")
    x0 = g[f"{name}_x"].reshape(-1, 256)
    rows = x0.shape[0]
    p = fnkv.Pool(2, 4 + rows // 256, 1, 1, fmt=fnkv.FMT_KV8)
    assert p.fmt == fnkv.FMT_KV8 and fnkv.lib().fnkv_pool_format(p.h) == fnkv.FMT_KV8
    assert p.ensure(1, 256)[0] == 0
    assert p.ensure(0, rows + 45)[0] == 0
    x = np.ascontiguousarray(x0[:, None, :])
    kt = torch.from_numpy(x).cuda()
    vt = torch.from_numpy(np.ascontiguousarray(x[::-1])).cuda()
    p.append(0, 0, 45, kt, vt)
    kc, ks = _export(p, 0, 0, 0, 0, 45, rows)
    vc, vs = _export(p, 0, 0, 0, 1, 45, rows)
    # K in input order against the reference's own outputs, V (rows reversed) against the oracle
    assert np.array_equal(kc.reshape(-1), g[f"{name}_codes"])
    assert np.array_equal(ks.reshape(-1), g[f"{name}_scales"])
    rc, rs = O.kv8_quantize(np.ascontiguousarray(x0[::-1]))
    assert np.array_equal(vc, rc) and np.array_equal(vs, rs)
    # the stored cells read back as ggml blocks carry the group scale on both of its 32-value blocks
    blocks = p.export(0, 0, 0, 0, 45, rows)
    torch.cuda.synchronize()
    qs, d = O.from_block_q8_0(blocks.cpu().numpy().reshape(-1, 34))
    assert np.array_equal(qs.reshape(rows, 256), kc)
    assert np.array_equal(d.reshape(rows, 8), np.repeat(ks, 2, axis=1))
    p.close()


def test_kv8_fp16_rows_and_refusals():
    # BASELINE-distribution fp16 rows through the fp16 entry, two heads, against the oracle
    n = 700
    k16, v16 = cases.kv_rows(8, n, HKV)
    p = fnkv.Pool(2, 4, 2, HKV, fmt=fnkv.FMT_KV8)
    assert p.ensure(0, n)[0] == 0
    p.append(0, 1, 0, torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda())
    (kc, ks, _), (vc, vs, _) = cases.decoded_kv8(O, k16, v16)
    for h in range(HKV):
        c, s = _export(p, 0, 1, h, 0, 0, n)
        assert np.array_equal(c, kc[:, h]) and np.array_equal(s, ks[:, h])
        c, s = _export(p, 0, 1, h, 1, 0, n)
        assert np.array_equal(c, vc[:, h]) and np.array_equal(s, vs[:, h])
    q8 = fnkv.Pool(2, 4, 1, HKV)
    assert q8.ensure(0, 256)[0] == 0
    with pytest.raises(fnkv.FnkvError):  # a Q8_0 pool has no KV8 form
        q8.export_kv8(0, 0, 0, 0, 0, 4)
    with pytest.raises(fnkv.FnkvError):  # unmapped cells
        p.export_kv8(0, 0, 0, 0, n, 300)
    with pytest.raises(fnkv.FnkvError):
        fnkv.Pool(2, 4, 1, HKV, fmt=7)
    p.close()
    q8.close()


class KV8Setup:
    def __init__(self, ctxs, seed, churn=0.2):
        self.pool = fnkv.Pool(len(ctxs) + 1, sum(-(-c // 256) for c in ctxs) + 8, 1, HKV, fmt=fnkv.FMT_KV8)
        self.ctxs = list(ctxs)
        self.slots = list(range(len(ctxs)))
        cases.scatter_ensure(self.pool, self.slots, self.ctxs, seed, churn)
        self.rows = {}
        for s, c in zip(self.slots, self.ctxs):
            k16, v16 = cases.kv_rows(seed * 100 + s, c, HKV)
            self.rows[s] = (k16, v16)
        torch.cuda.synchronize()

    def append_all(self, upto=None):
        for s, c in zip(self.slots, self.ctxs):
            k16, v16 = self.rows[s]
            n = c if upto is None else upto[s]
            self.pool.append(s, 0, 0, torch.from_numpy(k16[:n]).cuda(), torch.from_numpy(v16[:n]).cuda())

    def ref(self, s, q16, rows=None):
        k16, v16 = self.rows[s]
        (_, _, kf), (_, _, vf) = cases.decoded_kv8(O, k16, v16)
        return O.attn_f64(q16.view(np.uint16), kf, vf, self.ctxs[s], rows=rows)


@pytest.mark.parametrize("T", [1, 3, 5])
def test_kv8_decode_and_verify(T):
    ctxs = [T + 2, 300, 4097, 20000]
    st = KV8Setup(ctxs, seed=30 + T)
    st.append_all()
    q16 = cases.queries(40 + T, (len(ctxs), T, HQ, 256))
    q = torch.from_numpy(q16).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(st.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    st.pool.decode(st.slots, ctxs, T, 0, q, out, ws)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    worst = max(cases.out_err(got[i], st.ref(s, q16[i])) for i, s in enumerate(st.slots))
    assert np.isfinite(got).all() and worst <= TOL


def test_kv8_fused_append_bit_exact_and_attention():
    T = 5
    ctxs = [1000, 9000]
    st = KV8Setup(ctxs, seed=51)
    st.append_all(upto={0: ctxs[0] - T, 1: ctxs[1] - T})
    kn = np.stack([st.rows[s][0][c - T:] for s, c in zip(st.slots, ctxs)])
    vn = np.stack([st.rows[s][1][c - T:] for s, c in zip(st.slots, ctxs)])
    q16 = cases.queries(52, (2, T, HQ, 256))
    q = torch.from_numpy(q16).cuda()
    out = torch.empty_like(q)
    ws = torch.zeros(st.pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    st.pool.decode(st.slots, ctxs, T, 0, q, out, ws, k_new=torch.from_numpy(kn).cuda(),
                   v_new=torch.from_numpy(vn).cuda())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    for i, (s, c) in enumerate(zip(st.slots, ctxs)):
        (kc, ks, _), (vc, vs, _) = cases.decoded_kv8(O, kn[i], vn[i])
        for h in range(HKV):
            ec, es = _export(st.pool, s, 0, h, 0, c - T, T)
            assert np.array_equal(ec, kc[:, h]) and np.array_equal(es, ks[:, h])
            ec, es = _export(st.pool, s, 0, h, 1, c - T, T)
            assert np.array_equal(ec, vc[:, h]) and np.array_equal(es, vs[:, h])
        assert cases.out_err(got[i], st.ref(s, q16[i])) <= TOL


@pytest.mark.parametrize("depth,rows", [(0, 130), (6000, 512)])
def test_kv8_prefill(depth, rows):
    ctx = depth + rows
    st = KV8Setup([ctx], seed=60 + rows)
    st.append_all()
    q16 = cases.queries(61, (rows, HQ, 256))
    q = torch.from_numpy(q16).cuda()
    out = torch.empty_like(q)
    st.pool.prefill(0, 0, ctx, q, out)
    torch.cuda.synchronize()
    check = sorted({0, 1, rows // 3, rows // 2, rows - 2, rows - 1})
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert cases.out_err(got[check], st.ref(0, q16, rows=check)) <= TOL

"""The CPU oracle, pinned (CPU only).

What pins each oracle function (oracle/fnkv_oracle.c):
  or_f32_to_f16        the reference's ggml_compute_fp32_to_fp16 on 40,000 seeded bit patterns + edges (golden), and
                       numpy's independent fp16 rounding on every non-NaN input
  or_f16_to_f32        the reference's ggml_compute_fp16_to_fp32 on all 65,536 halves (golden), and numpy's widening
  or_q8_0_quantize     quantize_row_q8_0_ref outputs (golden: stress rows, every finite fp16 value, exact ties, seeded
                       BASELINE rows), plus closed forms (|code| <= 127, the amax element at +-127, a zero block)
  or_q8_0_dequantize   dequantize_row_q8_0 outputs (golden)
  or_kv8_quantize      FNFL's kv_q8_quantize outputs (golden)
  or_pages_*           the reference's own known answers, fn/runtime/slots_test.cpp:26-84, 1:1
  or_reclaim_victim    the same file's reclaim answers
  or_attn_f64          closed forms (one visible key returns its V row; q = 0 returns the visible rows' mean; equal
                       keys give the mean), brute force by numpy on tiny inputs, and key-order invariance
  or_attn_ggml         closed forms (one visible cell returns its V row; q = 0 the visible rows' mean; a dominant
                       key its V row; the head mapping; causality as a shorter context) and the fp64 form within 2e-3
                       (fp32 Q) on a seeded BASELINE-shaped case
DA-TC (oracle.py):
  act_quantize         the reference's act_quantize_ref (fn/quant/act_ref.cpp) outputs, bitwise (golden: seeded rows,
                       exact ties, zero / subnormal / huge / NaN / inf runs)
  imrope_plane         the sector table written out by hand from imrope.cuh's sections (11, 11, 10, 0)
  theta_f32            the closed form pos * ts^i in fp64 (the F32 chain within i + 1 ulps)
  norm_rope_f64        closed forms: at position 0 the rotation is the identity and the row's mean square is
                       1 / (1 + eps / ms(x)) against w = 1; each pair's norm is preserved; each pair equals the complex
                       product (y_i + i y_{i+32}) e^(i theta) computed from the position-0 row; distinct planes pick
                       the sector's position
  datc_cells           hand-written dense and SP2 lists (the body's blocks' cells, then the tail and the chain)
  datc_attn_f64        closed forms (one dominant key returns its V row times sigmoid(gate); q = 0 the listed rows'
                       mean; gate 0 halves the output) and numpy brute force over a tiny case
"""
import numpy as np
import pytest

import oracle as O


def test_f32_to_f16_matches_ggml(golden):
    g = golden("f16_golden.npz")
    got = O.f32_to_f16(g["f32"])
    assert np.array_equal(got, g["f16"])
    x = g["f32"]
    ok = ~np.isnan(x)
    with np.errstate(over="ignore"):
        assert np.array_equal(got[ok], x[ok].astype(np.float16).view(np.uint16))


def test_f16_to_f32_matches_ggml(golden):
    g = golden("f16_golden.npz")
    h = np.arange(65536, dtype=np.uint16)
    got = O.f16_to_f32(h).view(np.uint32)
    assert np.array_equal(got, g["halves_f32_bits"])
    w = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(w)
    assert np.array_equal(got[ok], w[ok].view(np.uint32))


@pytest.mark.parametrize("name", ["stress", "allf16", "ties", "rows", "nonfinite"])
def test_q8_0_matches_reference(golden, name):
    g = golden("q8_0_golden.npz")
    x = g[f"{name}_x"]
    qs, d = O.q8_0_quantize(x)
    assert np.array_equal(qs, g[f"{name}_qs"])
    assert np.array_equal(d, g[f"{name}_d"])
    y = O.q8_0_dequantize(qs, d)
    assert np.array_equal(y.view(np.uint32), g[f"{name}_y"].view(np.uint32))


def test_q8_0_closed_forms():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((512, 32)) * rng.uniform(0.01, 100, (512, 1))).astype(np.float16).astype(np.float32)
    x[5] = 0.0
    qs, d = O.q8_0_quantize(x)
    assert np.abs(qs.astype(np.int32)).max() <= 127
    am = np.argmax(np.abs(x), axis=1)
    peak = qs[np.arange(512), am]
    nz = np.abs(x).max(axis=1) > 0
    assert np.all(np.abs(peak[nz]) == 127)
    assert np.all(np.sign(peak[nz]) == np.sign(x[np.arange(512), am][nz]))
    assert np.all(qs[5] == 0) and d[5] == 0
    # d is fp16(amax / 127)
    amax = np.abs(x).max(axis=1)
    assert np.array_equal(d.reshape(-1), O.f32_to_f16((amax / np.float32(127.0)).astype(np.float32)))


def test_q8_0_ties_round_away_from_zero(golden):
    g = golden("q8_0_golden.npz")
    x, qs = g["ties_x"][:64], g["ties_qs"][:64]  # amax 127: d = 1, x = k + 0.5 exactly
    want = (np.sign(x) * np.floor(np.abs(x) + 0.5)).astype(np.int8)
    assert np.array_equal(qs, want)
    assert np.array_equal(O.q8_0_quantize(x)[0], want)


@pytest.mark.parametrize("name", ["stress", "rows", "nonfinite"])
def test_kv8_rule_matches_reference(golden, name):
    g = golden("kv8_golden.npz")
    c, s = O.kv8_quantize(g[f"{name}_x"])
    assert np.array_equal(c, g[f"{name}_codes"])
    assert np.array_equal(s, g[f"{name}_scales"])


def test_pages_known_answers():
    # fn/runtime/slots_test.cpp:26-84, with its page of 16,384 cells and 262,144 cells (16 pages)
    pc, n = 16384, 16
    pf = O.Pages.pages_for
    assert pf(0, pc, n) == 0 and pf(1, pc, n) == 1 and pf(pc, pc, n) == 1 and pf(pc + 1, pc, n) == 2
    assert pf(262144, pc, n) == 16 and pf(262144 + 5, pc, n) == 16
    r5, r4 = pf(32768 + 128 + 69, pc, n), pf(131072 + 32 + 69, pc, n)
    assert r5 == 3 and 4 * r5 <= n and r4 == 9 and 2 * r4 > n
    p = O.Pages(4, n)
    ok, t = p.take(0, 9)
    assert ok and len(t) == 9 and t[0] == 0 and p.free_pages() == 7
    ok, t = p.take(1, 9)
    assert not ok and t == [] and p.mapped(1) == 0 and p.free_pages() == 7
    ok, t = p.take(1, 7)
    assert ok and t[0] == 9 and p.free_pages() == 0
    ok, _ = p.take(2, 1)
    assert not ok
    out = p.give(0, 3)
    assert len(out) == 6 and out[0] == 8 and p.mapped(0) == 3 and p.free_pages() == 6
    ok, t = p.take(2, 2)
    assert ok and t == [3, 4] and p.physical(2, 1) == 4
    p.give(0, 0)
    p.give(1, 0)
    p.give(2, 0)
    ok, _ = p.take(3, n)
    assert ok and p.free_pages() == 0 and p.mapped(3) == n and p.physical(3, n - 1) == n - 1
    ok, _ = p.take(3, n + 1)
    assert not ok and p.mapped(3) == n


def test_reclaim_known_answers():
    v = [[False, 3, 7], [False, 2, 4], [True, 5, 1], [False, 0, 2]]
    a = O.reclaim_victim(v, 0)
    b = O.reclaim_victim(v, 1)
    v[1][0] = True
    c = O.reclaim_victim(v, 0)
    v[0][2] = 0
    d = O.reclaim_victim(v, 3)
    assert (a, b, c, d) == (1, 0, -1, 0)


def _rand_case(rng, n_ctx, T, hq=4, hkv=2, d=64):
    q16 = (rng.standard_normal((T, hq, d))).astype(np.float16).view(np.uint16)
    k = rng.standard_normal((n_ctx, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n_ctx, hkv, d)).astype(np.float32)
    return q16, k, v


def test_attn_f64_closed_forms():
    rng = np.random.default_rng(11)
    q16, k, v = _rand_case(rng, 9, 1)
    # one visible key: the query at position 0 of a 1-cell context returns that cell's V row
    out = O.attn_f64(q16, k, v, 1)
    for h in range(4):
        assert np.array_equal(out[0, h], v[0, h // 2].astype(np.float64))
    # q = 0: the mean of the visible V rows
    z = np.zeros_like(q16)
    out = O.attn_f64(z, k, v, 9)
    for h in range(4):
        assert np.allclose(out[0, h], v[:9, h // 2].astype(np.float64).mean(axis=0), rtol=0, atol=1e-12)
    # equal keys: the mean whatever q is
    ke = np.repeat(k[:1], 9, axis=0)
    out = O.attn_f64(q16, ke, v, 9)
    assert np.allclose(out[0, 0], v[:9, 0].astype(np.float64).mean(axis=0), atol=1e-12)


def test_attn_f64_brute_force_and_causality():
    rng = np.random.default_rng(12)
    n, T, hq, hkv, d = 23, 3, 4, 2, 64
    q16, k, v = _rand_case(rng, n, T, hq, hkv, d)
    out = O.attn_f64(q16, k, v, n, scale=0.125)
    q = q16.view(np.float16).astype(np.float64)
    for t in range(T):
        last = n - T + t
        for h in range(hq):
            s = (k[: last + 1, h // 2].astype(np.float64) @ q[t, h]) * 0.125
            p = np.exp(s - s.max())
            ref = (p[:, None] * v[: last + 1, h // 2]).sum(0) / p.sum()
            assert np.allclose(out[t, h], ref, rtol=1e-12, atol=1e-12)
    # rows subset gives the same rows
    sub = O.attn_f64(q16, k, v, n, scale=0.125, rows=[2, 0])
    assert np.array_equal(sub[0], out[2]) and np.array_equal(sub[1], out[0])


def test_attn_f64_key_order_invariance():
    rng = np.random.default_rng(13)
    n = 40
    q16, k, v = _rand_case(rng, n, 1)
    perm = rng.permutation(n - 1)
    kp = np.concatenate([k[perm], k[n - 1:]])
    vp = np.concatenate([v[perm], v[n - 1:]])
    a = O.attn_f64(q16, k, v, n)
    b = O.attn_f64(q16, kp, vp, n)
    assert np.allclose(a, b, rtol=1e-12, atol=1e-13)


def test_attn_ggml_path_within_tolerance():
    rng = np.random.default_rng(14)
    n, T, hq, hkv, d = 700, 3, 16, 2, 256
    x = rng.standard_normal((2, n, hkv, d)).astype(np.float32)
    x[:, :, :, rng.choice(d, 4, replace=False)] *= 8
    x = x.astype(np.float16).astype(np.float32)
    kq, kd = O.q8_0_quantize(x[0])
    vq, vd = O.q8_0_quantize(x[1])
    kb = O.to_block_q8_0(kq, kd).reshape(n, hkv, 8, 34)
    vb = O.to_block_q8_0(vq, vd).reshape(n, hkv, 8, 34)
    q16 = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    ref = O.attn_f64(q16, O.q8_0_dequantize(kq, kd), O.q8_0_dequantize(vq, vd), n)
    got = O.attn_ggml(q16, kb, vb, n, threads=4).view(np.float16).astype(np.float64)
    assert np.abs(got - ref).max() <= 2e-3
    got8 = O.attn_ggml(q16, kb, vb, n, q_as_q8=True, threads=4).view(np.float16).astype(np.float64)
    # Q itself quantized to Q8_0 (ggml's vec_dot operand): a documented divergence of ~2.6e-2 here, bounded loosely
    assert np.abs(got8 - ref).max() <= 5e-2


def _ggml_case(rng, n, T, hq=4, hkv=2, d=64):
    x = rng.standard_normal((2, n, hkv, d)).astype(np.float16).astype(np.float32)
    kq, kd = O.q8_0_quantize(x[0])
    vq, vd = O.q8_0_quantize(x[1])
    kb = O.to_block_q8_0(kq, kd).reshape(n, hkv, d // 32, 34)
    vb = O.to_block_q8_0(vq, vd).reshape(n, hkv, d // 32, 34)
    return kb, vb, O.q8_0_dequantize(kq, kd), O.q8_0_dequantize(vq, vd)


def test_attn_ggml_closed_forms():
    # the ggml-semantics path pinned where the mathematics fixes the answer (its source is not in the checkout):
    # one visible cell returns that cell's decoded V row (rounded to fp16); q = 0 weighs the visible rows equally
    # (their mean); a key far above the others returns its V row; heads map to KV heads by h // (hq / hkv); query t of
    # T sees cells 0 .. n - T + t (causal)
    rng = np.random.default_rng(15)
    hq, hkv, d = 4, 2, 64
    kb, vb, kdec, vdec = _ggml_case(rng, 9, 1, hq, hkv, d)
    q16 = rng.standard_normal((1, hq, d)).astype(np.float16).view(np.uint16)
    got = O.attn_ggml(q16, kb, vb, 1, hkv=hkv).view(np.float16)
    for h in range(hq):
        assert np.array_equal(got[0, h], vdec[0, h // 2].astype(np.float16))
    z = np.zeros_like(q16)
    got = O.attn_ggml(z, kb, vb, 9, hkv=hkv).view(np.float16).astype(np.float64)
    for h in range(hq):
        mean = vdec[:9, h // 2].astype(np.float64).mean(axis=0)
        assert np.abs(got[0, h] - mean).max() <= np.abs(mean).max() * 2.0 ** -10 + 1e-6
    # a dominant key: q along key 5 of KV head 0, scaled so its score leads the others by > 30 (weights below e^-30)
    kd0 = kdec[5, 0].astype(np.float64)
    qd = (kd0 / np.linalg.norm(kd0) * 200.0).astype(np.float16)
    qh = np.zeros((1, hq, d), np.float16)
    qh[0, 0] = qd
    s = (kdec[:9, 0].astype(np.float64) @ qd.astype(np.float64)) / 16.0
    assert s[5] - np.delete(s, 5).max() > 30.0
    got = O.attn_ggml(qh.view(np.uint16), kb, vb, 9, hkv=hkv).view(np.float16)
    assert np.abs(got[0, 0].astype(np.float64) - vdec[5, 0]).max() <= np.abs(vdec[5, 0]).max() * 2.0 ** -10
    # causality: with T = 3 queries the first sees 7 of 9 cells, the same as a 7-cell context with one query
    q3 = rng.standard_normal((3, hq, d)).astype(np.float16).view(np.uint16)
    a = O.attn_ggml(q3, kb, vb, 9, hkv=hkv).view(np.uint16)
    b = O.attn_ggml(q3[:1], kb, vb, 7, hkv=hkv).view(np.uint16)
    assert np.array_equal(a[0], b[0])


def test_attn_f64_cells_pinned_by_the_dense_form():
    # over every causal cell of each row the per-row-cells form is the dense form (itself pinned above by closed
    # forms and brute force); one selected cell returns its V row; the order of a row's cells does not matter
    rng = np.random.default_rng(5)
    n, T, hq, hkv, d = 70, 3, 4, 2, 32
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    q16 = rng.standard_normal((T, hq, d)).astype(np.float16).view(np.uint16)
    cells = [np.arange(n - T + t + 1) for t in range(T)]
    np.testing.assert_allclose(O.attn_f64_cells(q16, k, v, cells), O.attn_f64(q16, k, v, n), rtol=0, atol=1e-12)
    one = O.attn_f64_cells(q16, k, v, [np.array([7])] * T)
    assert np.allclose(one[:, 0], v[7, 0][None, :]) and np.allclose(one[:, 3], v[7, 1][None, :])
    perm = [rng.permutation(c) for c in cells]
    np.testing.assert_allclose(O.attn_f64_cells(q16, k, v, perm), O.attn_f64(q16, k, v, n), rtol=0, atol=1e-12)
    # a float query is taken as its values: the fp16 bits' values give the same result
    q64 = q16.view(np.float16).astype(np.float64)
    np.testing.assert_array_equal(O.attn_f64_cells(q64, k, v, cells), O.attn_f64_cells(q16, k, v, cells))


def test_qsa_body_layout():
    # qsa.h:77-81: 2 + K + tail words a row, K = min((q + 1) / 4, 512), blocks ascending and whole, tail 4 n_vis .. q
    for depth, T in ((0, 1), (2, 5), (2045, 3), (9000, 5)):
        words, offs, cells = O.qsa_body(depth, T, seed=depth)
        assert offs[0] == 0 and offs[-1] == 4 * words.size
        for t in range(T):
            q = depth + t
            row = words[offs[t] // 4: offs[t + 1] // 4]
            K, tail = int(row[0]), int(row[1])
            assert K == min((q + 1) // 4, 512) and tail == (q + 1) % 4 and row.size == 2 + K + tail
            blocks = row[2:2 + K].astype(np.int64)
            assert np.all(np.diff(blocks) > 0) and (K == 0 or 4 * blocks[-1] + 3 <= q)
            assert list(row[2 + K:]) == list(range(4 * ((q + 1) // 4), q + 1))
            assert cells[t].size == 4 * K + tail and cells[t].max() <= q


# ---- DA-TC ----

def test_act_quantize_matches_reference(golden):
    g = golden("act_golden.npz")
    codes, scales = O.act_quantize(g["x"])
    assert np.array_equal(codes, g["codes"])
    assert np.array_equal(scales.reshape(-1).view(np.uint32), g["scales_bits"])


def test_imrope_plane_table():
    # sections (t 11, h 11, w 10, e 0), interleaved by sector % 3; n_rot 64 has sectors 0..31 only
    want = [0, 1, 2] * 10 + [0, 1]
    assert [O.imrope_plane(i) for i in range(32)] == want
    assert O.imrope_plane(33) == 3 and O.imrope_plane(30) == 0 and O.imrope_plane(32) == 3 and O.imrope_plane(31) == 1


def test_theta_f32_chain_closed_form():
    ts = np.float32(10000000.0) ** np.float32(-2.0 / 64.0)
    for p in (1, 7, 4095, 196607):
        for i in range(32):
            exact = p * float(ts) ** i
            got = O.theta_f32([p, p, p, p], i, float(ts))
            assert abs(got - exact) <= (i + 1) * 2.0**-23 * abs(exact) + 1e-300


def test_norm_rope_f64_closed_forms():
    rng = np.random.default_rng(3)
    ts = float(np.float32(10000000.0) ** np.float32(-2.0 / 64.0))
    x = rng.uniform(-2, 2, 256).astype(np.float32)
    w = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    y0 = O.norm_rope_f64(x, np.ones(256, np.float32), [0, 0, 0, 0], ts)
    ms = np.mean(x.astype(np.float64) ** 2)
    assert abs(np.mean(y0**2) - 1.0 / (1.0 + 1e-6 / ms)) < 1e-12
    assert np.allclose(y0 / x, y0[0] / x[0])  # the identity rotation: a common factor
    base = O.norm_rope_f64(x, w, [0, 0, 0, 0], ts)
    pos4 = [5000, 5017, 5034, 1250]
    y = O.norm_rope_f64(x, w, pos4, ts)
    a = base[:32] + 1j * base[32:64]
    b = y[:32] + 1j * y[32:64]
    th = np.array([O.theta_f32(pos4, i, ts) for i in range(32)])
    assert np.allclose(np.abs(a), np.abs(b), rtol=1e-13)
    assert np.allclose(a * np.exp(1j * th), b, rtol=0, atol=1e-12)
    assert np.array_equal(y[64:], base[64:])
    # pair i turns by its own plane's position: pair 1 (h) at 5017 * ts (an F32 angle near 3,000: within 1e-3; the
    # other planes' positions are 10 radians or more away)
    for i, p in ((1, 5017), (2, 5034), (3, 5000)):
        d = np.angle(b[i] / a[i]) - np.angle(np.exp(1j * p * float(ts) ** i))
        assert abs((d + np.pi) % (2 * np.pi) - np.pi) < 1e-3


def test_datc_cells_lists():
    assert O.datc_cells(5, 2).tolist() == list(range(8))
    # N = 14: n_vis 3 whole blocks, K = 3, tail cells 12, 13 and the chain's row0 + 1 = 2 cells 14, 15
    body = [3, 2, 0, 1, 2]
    assert O.datc_cells(14, 1, body).tolist() == list(range(12)) + [12, 13, 14, 15]
    body = [2, 0, 1, 5, 99]  # K 2 of N / 4 = 6 blocks (a test of the list, not of K's rule)
    assert O.datc_cells(24, 0, body).tolist() == [4, 5, 6, 7, 20, 21, 22, 23, 24]


def test_datc_attn_f64_closed_forms():
    rng = np.random.default_rng(5)
    n = 40
    kc = rng.uniform(-1, 1, (n, 256)).astype(np.float16)
    vc = rng.uniform(-1.5, 1.5, (n, 256)).astype(np.float16)
    gate = rng.uniform(-3, 3, (12, 256)).astype(np.float32)
    cells = np.arange(n)
    # q = 0: the mean of the listed V rows, times sigmoid(gate)
    q0 = np.zeros((12, 256), np.float16)
    o = O.datc_attn_f64(q0.view(np.uint16), gate, kc.view(np.uint16), vc.view(np.uint16), cells)
    sig = 1.0 / (1.0 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(o, vc.astype(np.float64).mean(0)[None] * sig, rtol=0, atol=1e-14)
    # one dominant key: its V row; gate 0 halves it
    kd = kc.copy()
    kd[17] = np.float16(4.0)
    q = np.full((12, 256), 4.0, np.float16)
    o = O.datc_attn_f64(q.view(np.uint16), np.zeros((12, 256), np.float32), kd.view(np.uint16),
                        vc.view(np.uint16), cells)
    assert np.allclose(o, 0.5 * vc[17].astype(np.float64)[None], rtol=0, atol=1e-12)
    # brute force on a tiny list (a subset, out of order)
    sub = np.array([3, 9, 1, 30])
    qr = rng.uniform(-1, 1, (12, 256)).astype(np.float16)
    o = O.datc_attn_f64(qr.view(np.uint16), gate, kc.view(np.uint16), vc.view(np.uint16), sub)
    for h in range(12):
        s = [sum(float(qr[h, d]) * 16.0 * float(kc[c, d]) for d in range(256)) / 16.0 for c in sub]
        m = max(s)
        p = [np.exp(v - m) for v in s]
        ref = sum(pi * vc[c].astype(np.float64) for pi, c in zip(p, sub)) / sum(p) * sig[h]
        assert np.allclose(o[h], ref, rtol=1e-12, atol=1e-14)

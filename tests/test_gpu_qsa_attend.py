"""The reference's decode attention with its prepare and gate over the 8-bit pool (fnkv_qsa_attend; attn::attend,
fn/kernels/qsa/attend.h:57-141) on the GPU against the oracle:
  prepare   the F32 q and k within 1e-6 (max |error| / max |ref|) of the FP64 RMS norm + IMROPE (attend.cu:151-198,
            the checker form of fn/kernels/draft/draft_test.cpp:474-489); the new cells in the pool bitwise the pool's
            quantizer (Q8_0 or KV8) of the launch's own F32 k and of v
  attend    every (row, head) within 1e-5 normalized (max |error| / max |ref|, the reference checker's bound,
            fn/kernels/qsa/qa2_test.cpp:58 and :556-572) and 2e-3 max-abs of FP64 attention over the row's selected
            cells of the decoded cache with the FP64 q (the RMS norm + IMROPE above), times sigmoid(gate); the codes
            and scales bitwise the activation rule (fn/quant/act_ref.cpp) of the F32 output; bitwise reruns
Shapes: the reference's card (12 query heads on one KV head) and BASELINE's (16 on 2), rows 1..5, shallow and deep
selections, distinct rope planes, both pool formats; refusals enqueue nothing."""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2e-3
NORM_TOL = 1e-5  # qa2_test.cpp:58


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def positions(depth, T, planes):
    pos = np.zeros((4, T), np.int32)
    for t in range(T):
        p = depth + t
        for pl in range(4):
            pos[pl, t] = p + 17 * pl - (3 * p // 4 if pl == 3 else 0) if planes else p
    return pos


def quant(fmt, x):
    """(codes, scales, decoded) of F32 rows by the pool's rule"""
    x = np.ascontiguousarray(x, np.float32)
    if fmt == fnkv.FMT_KV8:
        c, s = O.kv8_quantize(x)
        return c, s, c.astype(np.float32) * np.repeat(s.view(np.float16).astype(np.float32), 64, axis=-1)
    c, d = O.q8_0_quantize(x)
    return c, d, O.q8_0_dequantize(c, d)


def run_case(depth, T, hq, h_kv, seed, fmt=fnkv.FMT_Q8_0, clustered=False, planes=False):
    rng = np.random.default_rng([seed, 11])
    ctx = depth + T
    pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, h_kv, fmt=fmt)
    cases.scatter_ensure(pool, [0], [ctx], seed, churn=0.3)
    k16, v16 = cases.kv_rows(seed, ctx, h_kv)
    if depth:
        pool.append(0, 0, 0, torch.from_numpy(k16[:depth]).cuda(), torch.from_numpy(v16[:depth]).cuda())
    words, offs, cells = O.qsa_body(depth, T, seed, clustered)
    qfull = rng.uniform(-3.0, 3.0, (T, hq, 512)).astype(np.float32)
    kv_k = rng.uniform(-2.0, 2.0, (T, h_kv, 256)).astype(np.float32)
    kv_v = rng.uniform(-1.5, 1.5, (T, h_kv, 256)).astype(np.float32)
    q_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    k_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    pos = positions(depth, T, planes)
    d = {n: torch.from_numpy(x).cuda() for n, x in
         dict(qfull=qfull, kv_k=kv_k, kv_v=kv_v, q_norm=q_norm, k_norm=k_norm, pos=pos).items()}
    body = torch.from_numpy(words.view(np.int32)).cuda()
    offsets = torch.from_numpy(offs).cuda()
    out = torch.full((T, hq, 256), float("nan"), device="cuda")
    codes = torch.zeros((T, hq * 256), dtype=torch.int8, device="cuda")
    scales = torch.zeros((T, hq * 8, 2), device="cuda")
    q_f32 = torch.empty((T, hq, 256), device="cuda")
    k_f32 = torch.empty((T, h_kv, 256), device="cuda")

    def launch():
        pool.qsa_attend(0, depth, 0, d["qfull"], d["kv_k"], d["kv_v"], d["q_norm"], d["k_norm"], d["pos"], body,
                        offsets, out, codes, scales, q_f32=q_f32, k_f32=k_f32)
        torch.cuda.synchronize()
        return out.cpu().numpy().copy(), codes.cpu().numpy().copy(), scales.cpu().numpy().copy()

    got, got_codes, got_scales = launch()
    qf, kf = q_f32.cpu().numpy(), k_f32.cpu().numpy()
    ts = fnkv.rope_theta_scale()
    # prepare: F32 q and k against FP64
    q64 = np.zeros((T, hq, 256))
    for t in range(T):
        p4 = [int(pos[pl, t]) for pl in range(4)]
        for h in range(hq):
            q64[t, h] = O.norm_rope_f64(qfull[t, h, :256], q_norm, p4, ts)
            assert O.norm_err(q64[t, h], qf[t, h]) <= 1e-6
        for h in range(h_kv):
            assert O.norm_err(O.norm_rope_f64(kv_k[t, h], k_norm, p4, ts), kf[t, h]) <= 1e-6
    # the new cells: bitwise the pool's rule of the launch's own F32 k and of v
    kc_new, ks_new, kd_new = quant(fmt, kf)
    vc_new, vs_new, vd_new = quant(fmt, kv_v)
    for h in range(h_kv):
        for kv, (c, s) in enumerate(((kc_new, ks_new), (vc_new, vs_new))):
            if fmt == fnkv.FMT_KV8:
                gc, gs = pool.export_kv8(0, 0, h, kv, depth, T)
                torch.cuda.synchronize()
                assert np.array_equal(gc.cpu().numpy(), c[:, h])
                assert np.array_equal(gs.cpu().numpy().view(np.uint16), s[:, h])
            else:
                blocks = pool.export(0, 0, h, kv, depth, T)
                torch.cuda.synchronize()
                qs, dd = O.from_block_q8_0(blocks.cpu().numpy().reshape(-1, 34))
                assert np.array_equal(qs.reshape(T, 256), c[:, h]) and np.array_equal(dd.reshape(T, 8), s[:, h])
    # the attention over the decoded cache, with the FP64 q, gated
    if fmt == fnkv.FMT_KV8:
        (_, _, kdec), (_, _, vdec) = cases.decoded_kv8(O, k16, v16)
    else:
        (_, _, kdec), (_, _, vdec) = cases.decoded(O, k16, v16)
    kdec[depth:], vdec[depth:] = kd_new, vd_new
    ref = O.attn_f64_cells(q64, kdec, vdec, cells) / (1.0 + np.exp(-qfull[:, :, 256:].astype(np.float64)))
    err = float(np.abs(got.astype(np.float64) - ref).max())
    assert np.isfinite(got).all() and err <= TOL, err
    nerr = max(O.norm_err(ref[t, h], got[t, h]) for t in range(T) for h in range(hq))
    print(f"depth {depth} T {T} hq {hq} h_kv {h_kv}: max-abs {err:.3g}, normalized {nerr:.3g}")
    assert nerr <= NORM_TOL, nerr
    ac, asc = O.act_quantize(got.reshape(T, hq * 256))
    assert np.array_equal(ac, got_codes)
    assert np.array_equal(asc.reshape(T, hq * 8, 2).view(np.uint32), got_scales.view(np.uint32))
    again = launch()
    assert all(np.array_equal(a.view(np.uint8), b.view(np.uint8)) for a, b in zip(again, (got, got_codes, got_scales)))
    return nerr


@pytest.mark.parametrize("depth,T", [(0, 1), (37, 3), (2045, 5), (9000, 2)])
def test_reference_card_shape(depth, T):
    # 12 query heads on one KV head (attend.h:50-53)
    run_case(depth, T, 12, 1, seed=depth + T, planes=T == 3)


@pytest.mark.parametrize("T,fmt", [(3, fnkv.FMT_Q8_0), (1, fnkv.FMT_KV8)])
def test_reference_depth(T, fmt):
    # the reference checker's depth (qa2_test.cpp:56, 196,608 cells): 512 selected blocks and the tail a row
    run_case(196608 - T, T, 12, 1, seed=900 + T, fmt=fmt, planes=True)


@pytest.mark.parametrize("T", [1, 3, 5])
@pytest.mark.parametrize("clustered", [False, True])
def test_baseline_heads_deep(T, clustered):
    run_case(16003 - T, T, 16, 2, seed=50 + T + (7 if clustered else 0), clustered=clustered)


def test_kv8_pool():
    run_case(6000, 4, 12, 1, seed=77, fmt=fnkv.FMT_KV8, planes=True)


def test_refusals_enqueue_nothing():
    pool = fnkv.Pool(2, 8, 1, 1)
    assert pool.ensure(0, 1024)[0] == 0
    z = lambda *s: torch.zeros(s, device="cuda")  # noqa: E731
    qfull, kv, nrm = z(3, 12, 512), z(3, 1, 256), z(256)
    pos = torch.zeros((4, 3), dtype=torch.int32, device="cuda")
    body = torch.zeros(4096, dtype=torch.int32, device="cuda")
    offs = torch.zeros(8, dtype=torch.int32, device="cuda")
    out = z(3, 12, 256)
    codes = torch.zeros((3, 3072), dtype=torch.int8, device="cuda")
    scales = z(3, 96, 2)
    args = (0, 10, 0, qfull, kv, kv, nrm, nrm, pos, body, offs, out, codes, scales)
    with pytest.raises(fnkv.FnkvError):  # past the mapped cells
        pool.qsa_attend(0, 1022, *args[2:])
    with pytest.raises(fnkv.FnkvError):  # workspace too small
        pool.qsa_attend(*args, ws=torch.empty(64, dtype=torch.uint8, device="cuda"))
    shifted = z(3 * 12 * 512 + 4)[1:1 + 3 * 12 * 512].view(3, 12, 512)  # 4 bytes past a 16-byte boundary
    with pytest.raises(fnkv.FnkvError):  # misaligned q rows
        pool.qsa_attend(0, 10, 0, shifted, *args[4:])
    with pytest.raises(fnkv.FnkvError):  # six rows
        q6 = z(6, 12, 512)
        pool.qsa_attend(0, 10, 0, q6, z(6, 1, 256), z(6, 1, 256), nrm, nrm, torch.zeros((4, 6), dtype=torch.int32,
                        device="cuda"), body, offs, z(6, 12, 256), torch.zeros((6, 3072), dtype=torch.int8,
                        device="cuda"), z(6, 96, 2))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0 and torch.count_nonzero(kv).item() == 0


@pytest.mark.parametrize("depth,T,hq,h_kv,fmt", [(0, 1, 12, 1, fnkv.FMT_Q8_0), (5000, 1, 12, 1, fnkv.FMT_Q8_0),
                                                 (16002, 1, 16, 2, fnkv.FMT_Q8_0), (7001, 1, 12, 1, fnkv.FMT_KV8),
                                                 (0, 3, 12, 1, fnkv.FMT_Q8_0), (29, 5, 12, 1, fnkv.FMT_Q8_0),
                                                 (196605, 3, 12, 1, fnkv.FMT_Q8_0), (16000, 5, 16, 2, fnkv.FMT_Q8_0),
                                                 (7001, 4, 12, 1, fnkv.FMT_KV8)])
def test_rows_prepared_in_the_sparse_launch(depth, T, hq, h_kv, fmt, monkeypatch):
    # up to 16 query heads a KV head: the sparse launch forms each row's query heads and writes the new cells itself
    # (every workgroup that reads a new cell's tile writes it first); every output (F32 out, codes, scales, q_f32,
    # k_f32, the new cells in the pool) bitwise that of the separate prepare launch
    def once(two):
        if two:
            monkeypatch.setenv("FNKV_QSA_TWO_KERNELS", "1")
        else:
            monkeypatch.delenv("FNKV_QSA_TWO_KERNELS", raising=False)
        rng = np.random.default_rng([depth, T, 23])
        ctx = depth + T
        pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, h_kv, fmt=fmt)
        cases.scatter_ensure(pool, [0], [ctx], depth + 3, churn=0.3)
        k16, v16 = cases.kv_rows(depth + 3, ctx, h_kv)
        if depth:
            pool.append(0, 0, 0, torch.from_numpy(k16[:depth]).cuda(), torch.from_numpy(v16[:depth]).cuda())
        words, offs, _ = O.qsa_body(depth, T, depth + 5)
        d = {n: torch.from_numpy(x).cuda() for n, x in dict(
            qfull=rng.uniform(-3.0, 3.0, (T, hq, 512)).astype(np.float32),
            kv_k=rng.uniform(-2.0, 2.0, (T, h_kv, 256)).astype(np.float32),
            kv_v=rng.uniform(-1.5, 1.5, (T, h_kv, 256)).astype(np.float32),
            q_norm=rng.uniform(0.3, 1.8, 256).astype(np.float32),
            k_norm=rng.uniform(0.3, 1.8, 256).astype(np.float32),
            pos=positions(depth, T, True)).items()}
        out = torch.full((T, hq, 256), float("nan"), device="cuda")
        codes = torch.zeros((T, hq * 256), dtype=torch.int8, device="cuda")
        scales = torch.zeros((T, hq * 8, 2), device="cuda")
        q_f32 = torch.empty((T, hq, 256), device="cuda")
        k_f32 = torch.empty((T, h_kv, 256), device="cuda")
        pool.qsa_attend(0, depth, 0, d["qfull"], d["kv_k"], d["kv_v"], d["q_norm"], d["k_norm"], d["pos"],
                        torch.from_numpy(words.view(np.int32)).cuda(), torch.from_numpy(offs).cuda(), out, codes,
                        scales, q_f32=q_f32, k_f32=k_f32)
        cells = []
        for h in range(h_kv):
            for kv in range(2):
                if fmt == fnkv.FMT_KV8:
                    c, sc = pool.export_kv8(0, 0, h, kv, depth, T)
                    cells += [c.cpu().numpy(), sc.cpu().numpy()]
                else:
                    cells.append(pool.export(0, 0, h, kv, depth, T).cpu().numpy())
        torch.cuda.synchronize()
        res = [out.cpu().numpy(), codes.cpu().numpy(), scales.cpu().numpy(), q_f32.cpu().numpy(),
               k_f32.cpu().numpy()] + cells
        pool.close()
        return res

    two, one = once(True), once(False)
    for a, b in zip(two, one):
        assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8))


@pytest.mark.parametrize("T,hq", [(1, 32), (3, 32), (2, 48)])
def test_many_heads_a_kv_head(T, hq):
    # 32 and 48 query heads on one KV head: the row kernels' sparse instantiations (two and three row tiles), and at
    # T = 1 the separate prepare launch (the sparse launch prepares its own row only up to 16 heads a KV head)
    run_case(4000 - T, T, hq, 1, seed=300 + T, planes=True)

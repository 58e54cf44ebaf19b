"""The prompt path's own contract over the pool (fnkv_qsp_kv, fnkv_qsp_attend; fn::qsa::qsp_kv / qsp_attend,
fn/kernels/qsa/qsa_prompt.h:90-124) on the GPU against the oracle:
  qsp_kv      each row's k is the FP64 RMS norm + IMROPE (norm_rope_f64) at its rope position (text positions, or
              supplied planes); the written codes and scales bitwise the pool quantizer (Q8_0 / KV8) of that k rounded
              to F32, except where the rounding itself is ambiguous (the reference's check: "within its rounding",
              qsa_prompt.h:57-60); v's cells bitwise the quantizer of kv_v
  qsp_attend  every (row, head) within 2e-3 max-abs (F32 out) of FP64 attention over the row's selected cells of the
              decoded cache with q = fp16(F32(norm_rope_f64)), times sigmoid(gate); the fp16 out is the F32 out rounded
              to nearest even; bit 0 of err only for an output fp16 cannot hold
Rows cross slab (128) and launch-chunk (512) boundaries, up to the 4,096-row limit (eight full chunks) and up to the
deepest cell the selection layout addresses (a short last chunk there); 12 heads on 1 KV head (the reference's card)
and 16 on 2. qsp_kv's K and V cells are also bitwise those fnkv_qsa_attend's prepare step writes for the same rows."""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2e-3


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def quant(fmt, x):
    x = np.ascontiguousarray(x, np.float32)
    if fmt == fnkv.FMT_KV8:
        c, s = O.kv8_quantize(x)
        return c, s, c.astype(np.float32) * np.repeat(s.view(np.float16).astype(np.float32), 64, axis=-1)
    c, d = O.q8_0_quantize(x)
    return c, d, O.q8_0_dequantize(c, d)


def stored(pool, fmt, slot, head, kv, tok0, n):
    """the pool's codes and scales of cells tok0 .. + n - 1 in the quantizer's own form"""
    if fmt == fnkv.FMT_KV8:
        c, s = pool.export_kv8(slot, 0, head, kv, tok0, n)
        torch.cuda.synchronize()
        return c.cpu().numpy(), s.cpu().numpy().view(np.uint16)
    b = pool.export(slot, 0, head, kv, tok0, n)
    torch.cuda.synchronize()
    qs, d = O.from_block_q8_0(b.cpu().numpy().reshape(-1, 34))
    return qs.reshape(n, 256), d.reshape(n, 8)


def planes_of(pos0, rows, use_planes):
    if not use_planes:
        return None
    p = np.zeros((rows, 4), np.int32)
    for t in range(rows):
        q = pos0 + t
        p[t] = [q, q + 17, q - 3 if q >= 3 else q, q // 2]
    return p


def rope4(pos0, rope_off, t, planes):
    return [int(x) for x in planes[t]] if planes is not None else [pos0 + rope_off + t] * 4


def slab_bodies(pos0, rows, seed, clustered=False):
    """the rows' selection bodies in the reference's slab layout (qsa_prompt.h:44-53): slab k's words at
    k * 128 * 517, row i's body at byte offsets[129 k + i] of its slab; -> words, offsets, each row's cell list"""
    n_slabs = -(-rows // fnkv.SLAB_ROWS)
    words = np.zeros(n_slabs * fnkv.SLAB_ROWS * fnkv.ROW_WORDS, np.uint32)
    offsets = np.zeros(n_slabs * (fnkv.SLAB_ROWS + 1), np.int32)
    cells = []
    for k in range(n_slabs):
        off = 0
        for i in range(fnkv.SLAB_ROWS):
            t = k * fnkv.SLAB_ROWS + i
            offsets[k * (fnkv.SLAB_ROWS + 1) + i] = off
            if t >= rows:
                continue
            w, _, c = O.qsa_body(pos0 + t, 1, seed + 7 * t, clustered and t % 2 == 0)
            base = k * fnkv.SLAB_ROWS * fnkv.ROW_WORDS + off // 4
            words[base:base + w.size] = w
            off += 4 * w.size
            cells.append(c[0])
        offsets[k * (fnkv.SLAB_ROWS + 1) + fnkv.SLAB_ROWS] = off
    return words, offsets, cells


@pytest.mark.parametrize("fmt", [fnkv.FMT_Q8_0, fnkv.FMT_KV8])
@pytest.mark.parametrize("h_kv,use_planes", [(1, False), (2, True)])
def test_qsp_kv_norm_rope_quantize(fmt, h_kv, use_planes):
    rows, pos0, rope_off = 300, 777, 5
    rng = np.random.default_rng([rows, h_kv, fmt])
    pool = fnkv.Pool(2, -(-(pos0 + rows) // 256) + 4, 1, h_kv, fmt=fmt)
    cases.scatter_ensure(pool, [0], [pos0 + rows], 3, churn=0.3)
    kv_k = rng.uniform(-2.0, 2.0, (rows, h_kv, 256)).astype(np.float32)
    kv_v = rng.uniform(-1.5, 1.5, (rows, h_kv, 256)).astype(np.float32)
    k_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    planes = planes_of(pos0, rows, use_planes)
    pool.qsp_kv(0, 0, pos0, torch.from_numpy(kv_k).cuda(), torch.from_numpy(kv_v).cuda(),
                torch.from_numpy(k_norm).cuda(), planes=None if planes is None else torch.from_numpy(planes).cuda(),
                rope_off=rope_off)
    ts = fnkv.rope_theta_scale()
    k64 = np.stack([[O.norm_rope_f64(kv_k[t, h], k_norm, rope4(pos0, rope_off, t, planes), ts) for h in range(h_kv)]
                    for t in range(rows)])
    k32 = k64.astype(np.float32)
    kc, ks, _ = quant(fmt, k32)
    vc, vs, _ = quant(fmt, kv_v)
    group = 64 if fmt == fnkv.FMT_KV8 else 32
    for h in range(h_kv):
        gc, gs = stored(pool, fmt, 0, h, 0, pos0, rows)
        # V: the quantizer of kv_v exactly
        vgc, vgs = stored(pool, fmt, 0, h, 1, pos0, rows)
        assert np.array_equal(vgc, vc[:, h]) and np.array_equal(vgs.view(np.uint16), vs[:, h].view(np.uint16))
        # K: bitwise except where the F32 k's last bit decides (a scale whose amax sits at an fp16 rounding edge, a
        # code at a rounding tie); such blocks are rare and decode within one step of the reference
        sc_ok = gs.view(np.uint16) == ks[:, h].view(np.uint16)
        code_ok = (gc == kc[:, h]).reshape(rows, -1, group).all(-1)
        nblk = sc_ok.size
        bad = ~(sc_ok & code_ok)
        assert bad.sum() <= max(2, nblk // 500), (bad.sum(), nblk)
        if bad.any():
            sf = gs.view(np.float16).astype(np.float64)
            dec = gc.astype(np.float64) * np.repeat(sf, group, axis=-1)
            step = np.repeat(np.abs(sf), group, axis=-1)
            assert (np.abs(dec - k64[:, h]) <= step * 0.5 + 1e-6 * np.abs(k64[:, h]).max()).all()


@pytest.mark.parametrize("fmt", [fnkv.FMT_Q8_0, fnkv.FMT_KV8])
def test_qsp_kv_bitwise_the_decode_prepare(fmt):
    # the same F32 rows, norm and rope positions written once through fnkv_qsa_attend (its prepare step, T rows at a
    # time) and once through fnkv_qsp_kv (all rows in one launch): the stored cells are identical, byte for byte
    h_kv, hq, T, depth0, windows = 2, 16, 5, 3001, 12
    rows = T * windows
    ctx = depth0 + rows
    rng = np.random.default_rng([fmt, 41])
    kv_k = rng.uniform(-2.0, 2.0, (rows, h_kv, 256)).astype(np.float32)
    kv_v = rng.uniform(-1.5, 1.5, (rows, h_kv, 256)).astype(np.float32)
    kv_k[7, 0, :32] *= 1e-3  # a near-silent block and an outlier block
    kv_k[11, 1, 64:96] *= 300.0
    k_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    q_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    planes = planes_of(depth0, rows, True)
    pools = [fnkv.Pool(2, -(-ctx // 256) + 8, 1, h_kv, fmt=fmt) for _ in range(2)]
    for p in pools:
        cases.scatter_ensure(p, [0], [ctx], 8, churn=0.3)
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).cuda()  # noqa: E731
    kn = dev(k_norm)
    for w in range(windows):
        t0, depth = w * T, depth0 + w * T
        words, offs, _ = O.qsa_body(depth, T, w)
        out = torch.empty((T, hq, 256), device="cuda")
        codes = torch.empty((T, hq * 256), dtype=torch.int8, device="cuda")
        scales = torch.empty((T, hq * 8, 2), device="cuda")
        pools[0].qsa_attend(0, depth, 0, dev(rng.uniform(-3, 3, (T, hq, 512)).astype(np.float32)),
                            dev(kv_k[t0:t0 + T]), dev(kv_v[t0:t0 + T]), dev(q_norm), kn,
                            dev(planes[t0:t0 + T].T), dev(words.view(np.int32)), dev(offs), out, codes, scales)
    pools[1].qsp_kv(0, 0, depth0, dev(kv_k), dev(kv_v), kn, planes=dev(planes))
    torch.cuda.synchronize()
    for h in range(h_kv):
        for kv in range(2):
            a = stored(pools[0], fmt, 0, h, kv, depth0, rows)
            b = stored(pools[1], fmt, 0, h, kv, depth0, rows)
            assert np.array_equal(a[0], b[0]), (h, kv)
            assert np.array_equal(a[1].view(np.uint16), b[1].view(np.uint16)), (h, kv)
    for p in pools:
        p.close()


def run_attend(pos0, rows, hq, h_kv, seed, fmt=fnkv.FMT_Q8_0, use_planes=False, with_f32=True, big_v=False):
    rng = np.random.default_rng([seed, 3])
    ctx = pos0 + rows
    pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, h_kv, fmt=fmt)
    cases.scatter_ensure(pool, [0], [ctx], seed, churn=0.3)
    k16, v16 = cases.kv_rows(seed, ctx, h_kv)
    k32, v32 = k16.astype(np.float32), v16.astype(np.float32)
    if big_v:  # channel 0 of every V row beyond fp16's range (the Q8_0 scale, amax / 127, still holds it): every
        v32[:, :, 0] = 1.0e5  # row's mean of it is 1e5, and with gates above -0.42 the output passes 65,504
    pool.append(0, 0, 0, torch.from_numpy(k32).cuda(), torch.from_numpy(v32).cuda())
    _, _, kdec = quant(fmt, k32)
    _, _, vdec = quant(fmt, v32)
    words, offsets, cells = slab_bodies(pos0, rows, seed)
    qfull = rng.uniform(-3.0, 3.0, (rows, hq, 512)).astype(np.float32)
    q_norm = rng.uniform(0.3, 1.8, 256).astype(np.float32)
    planes = planes_of(pos0, rows, use_planes)
    out16 = torch.zeros((rows, hq, 256), dtype=torch.float16, device="cuda")
    out = torch.full((rows, hq, 256), float("nan"), device="cuda") if with_f32 else None
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pool.qsp_attend(0, 0, pos0, torch.from_numpy(qfull).cuda(), torch.from_numpy(q_norm).cuda(),
                    torch.from_numpy(words.view(np.int32)).cuda(), torch.from_numpy(offsets).cuda(), out16, out=out,
                    err=err, planes=None if planes is None else torch.from_numpy(planes).cuda())
    torch.cuda.synchronize()
    ts = fnkv.rope_theta_scale()
    q64 = np.stack([[O.norm_rope_f64(qfull[t, h, :256], q_norm, rope4(pos0, 0, t, planes), ts) for h in range(hq)]
                    for t in range(rows)])
    q16 = q64.astype(np.float32).astype(np.float16).view(np.uint16)
    ref = O.attn_f64_cells(q16, kdec, vdec, cells) / (1.0 + np.exp(-qfull[:, :, 256:].astype(np.float64)))
    return out16.cpu().numpy(), None if out is None else out.cpu().numpy(), int(err.item()), ref


@pytest.mark.parametrize("pos0,rows,hq,h_kv", [(0, 1, 12, 1), (5000, 300, 12, 1), (2000, 600, 16, 2)])
def test_qsp_attend_against_fp64(pos0, rows, hq, h_kv):
    o16, o32, err, ref = run_attend(pos0, rows, hq, h_kv, seed=rows + hq)
    assert err == 0 and np.isfinite(o32).all()
    e = float(np.abs(o32.astype(np.float64) - ref).max())
    assert e <= TOL, e
    assert np.array_equal(o16.view(np.uint16), o32.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("pos0,rows", [(100, 4096), (262144 + 32 - 576, 576)])
def test_qsp_attend_chunks_at_the_limits(pos0, rows):
    # eight full 512-row chunks (the workspace sized for the deepest one and reused by all); and a full chunk then a
    # 64-row one whose last row is the deepest cell the selection layout addresses
    o16, o32, err, ref = run_attend(pos0, rows, 12, 1, seed=rows)
    assert err == 0 and np.isfinite(o32).all()
    e = float(np.abs(o32.astype(np.float64) - ref).max())
    print(f"pos0 {pos0} rows {rows}: max-abs {e:.3g}", flush=True)
    assert e <= TOL, e
    assert np.array_equal(o16.view(np.uint16), o32.astype(np.float16).view(np.uint16))


def test_qsp_attend_deep_clustered_planes_kv8():
    o16, o32, err, ref = run_attend(20000, 140, 12, 1, seed=9, fmt=fnkv.FMT_KV8, use_planes=True)
    assert err == 0
    assert float(np.abs(o32.astype(np.float64) - ref).max()) <= TOL


def test_qsp_attend_fp16_only_and_overflow_bit():
    # without the F32 output; then V values beyond fp16's range after the gate set bit 0 of err (and the fp16 is inf)
    o16, _, err, ref = run_attend(300, 40, 12, 1, seed=4, with_f32=False)
    assert err == 0
    assert cases.out_err(o16, ref) <= TOL
    o16, o32, err, ref = run_attend(300, 40, 12, 1, seed=5, big_v=True)
    big = np.abs(o32) > 65504.0
    assert big.any() and err == 1
    assert np.isinf(o16[big].astype(np.float32)).all()


def test_qsp_refusals_enqueue_nothing():
    pool = fnkv.Pool(2, 8, 1, 1)
    assert pool.ensure(0, 1024)[0] == 0
    z = lambda *s: torch.zeros(s, device="cuda")  # noqa: E731
    kv = z(4, 1, 256)
    with pytest.raises(fnkv.FnkvError):  # past the mapped cells
        pool.qsp_kv(0, 0, 1022, kv, kv, z(256))
    with pytest.raises(fnkv.FnkvError):  # rows beyond 4,096
        pool.qsp_kv(0, 0, 0, z(4097, 1, 256), z(4097, 1, 256), z(256))
    out16 = torch.zeros((4, 12, 256), dtype=torch.float16, device="cuda")
    body = torch.zeros(4096, dtype=torch.int32, device="cuda")
    offs = torch.zeros(129, dtype=torch.int32, device="cuda")
    with pytest.raises(fnkv.FnkvError):  # workspace too small
        pool.qsp_attend(0, 0, 10, z(4, 12, 512), z(256), body, offs, out16,
                        ws=torch.empty(64, dtype=torch.uint8, device="cuda"))
    with pytest.raises(fnkv.FnkvError):  # heads not a multiple of the KV heads' ... (13 on 1 is fine; 0 is not)
        pool.qsp_attend(0, 0, 10, z(4, 0, 512), z(256), body, offs, out16)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out16).item() == 0

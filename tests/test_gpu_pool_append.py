"""The pool and the Q8_0 append on the GPU, through the C-ABI (libfnkv.so).

Bit-exact bars:
  * ensure / trim / the page table against the oracle's page book (kv_pool.cpp:85-144) and the reference's known
    answers (slots_test.cpp:26-84), the capacity refusal and a failure injected mid-transaction
    (slots_gpu_test.cpp:192-304: the slot's pages unchanged afterwards);
  * appended blocks against the reference's quantize_row_q8_0_ref outputs (golden fixtures) and the oracle, read
    back through the page table (fnkv_export_q8_0) and, for placement, straight out of the physical pages.
"""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    print("gpu tests: pool and append", flush=True)


def test_book_known_answers_on_the_pool():
    # slots_test.cpp:26-84 at pages of 256 cells: 16 pages
    p = fnkv.Pool(4, 16, 1, 2)
    ref = O.Pages(4, 16)
    pc = 256

    def ens(slot, pages):
        code, cap = p.ensure(slot, pages * pc)
        ok, _ = ref.take(slot, pages)
        assert (code == 0) == ok
        return code, cap

    assert ens(0, 9)[0] == 0 and p.table(0) == list(range(9)) and p.free_pages() == 7
    code, cap = ens(1, 9)
    assert code == fnkv.ERR_CAPACITY and cap and p.mapped_pages(1) == 0 and p.free_pages() == 7
    assert ens(1, 7)[0] == 0 and p.table(1)[0] == 9 and p.free_pages() == 0
    assert ens(2, 1)[0] == fnkv.ERR_CAPACITY
    assert p.trim(0, 3 * pc) == 0
    ref.give(0, 3)
    assert p.mapped_pages(0) == 3 and p.free_pages() == 6
    assert ens(2, 2)[0] == 0 and p.table(2) == [3, 4] and p.physical(2, 1) == 4
    for s in range(3):
        assert p.trim(s, 0) == 0
        ref.give(s, 0)
    assert ens(3, 16)[0] == 0 and p.mapped_pages(3) == 16 and p.physical(3, 15) == 15
    for s in range(4):
        assert p.table(s) == ref.table(s)
    assert p.ensure(3, 17 * pc)[0] == 0 and p.mapped_pages(3) == 16  # capped at the slot range
    assert any("16 pages of 256 cells" in l for l in p.ledger())
    p.close()


def test_book_random_churn_across_free_set_words():
    # seeded ensure / trim churn over 300 pages (the free set spans five 64-page words, and takes and gives cross
    # word edges) on 6 slots; after every call each slot's page table and the free count equal the oracle book's
    # (kv_pool.cpp:85-144: take lowest-first and all-or-nothing, give last-first)
    n_pages, n_slots, pc = 300, 6, 256
    p = fnkv.Pool(n_slots, n_pages, 1, 2)
    ref = O.Pages(n_slots, n_pages)
    rng = np.random.default_rng(20260)
    fails = 0
    for op in range(400):
        slot = int(rng.integers(0, n_slots))
        if rng.random() < 0.6:
            want = int(rng.integers(0, 160))
            code, cap = p.ensure(slot, want * pc)
            ok, _ = ref.take(slot, want)
            assert (code == 0) == ok, (op, slot, want)
            fails += 0 if ok else 1
            if not ok:
                assert code == fnkv.ERR_CAPACITY and cap
        else:
            keep = int(rng.integers(0, max(1, ref.mapped(slot) + 1)))
            assert p.trim(slot, keep * pc) == 0
            ref.give(slot, keep)
        assert p.free_pages() == ref.free_pages(), op
        for sl in range(n_slots):
            assert p.table(sl) == ref.table(sl), (op, sl)
    assert fails > 10  # the pool ran full often enough to exercise the all-or-nothing rule
    p.close()


def test_injected_failure_leaves_the_slot_unchanged():
    p = fnkv.Pool(2, 8, 2, 2)
    assert p.ensure(0, 2 * 256)[0] == 0
    before, free = p.table(0), p.free_pages()
    p.test_fail(1)
    code, cap = p.ensure(0, 5 * 256)
    assert code != 0 and not cap and "injected" in fnkv.last_error()
    assert p.table(0) == before and p.free_pages() == free
    assert p.ensure(0, 5 * 256)[0] == 0 and p.table(0) == [0, 1, 2, 3, 4]
    p.close()


def _export_blocks(pool, slot, layer, head, kv, tok0, n):
    out = pool.export(slot, layer, head, kv, tok0, n)
    torch.cuda.synchronize()
    return O.from_block_q8_0(out.cpu().numpy().reshape(-1, 34))


@pytest.mark.parametrize("name", ["stress", "allf16", "ties", "rows", "nonfinite"])
def test_append_matches_reference_golden(golden, name):
    g = golden("q8_0_golden.npz")
    x0 = g[f"{name}_x"]
    h_kv = 2
    n = -(-x0.size // 512) * 512  # whole rows of both heads; zero padding quantizes to zero blocks
    xf = np.zeros(n, np.float32)
    xf[: x0.size] = x0
    rows = n // 512
    x = xf.reshape(rows, h_kv, 256)
    p = fnkv.Pool(2, 4 + rows // 256, 1, h_kv)
    assert p.ensure(1, 256)[0] == 0  # slot 1 takes page 0 first: slot 0's cells land on later pages
    assert p.ensure(0, rows + 37)[0] == 0
    kt = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    vt = torch.from_numpy(np.ascontiguousarray(x[::-1].copy())).cuda()
    if name in ("allf16", "rows", "nonfinite"):
        kt, vt = kt.half(), vt.half()  # exact: these inputs are fp16 values
    p.append(0, 0, 37, kt, vt)
    got_q = np.empty((2, rows, h_kv, 256), np.int8)
    got_d = np.empty((2, rows, h_kv, 8), np.uint16)
    for kv in (0, 1):
        for h in range(h_kv):
            qs, d = _export_blocks(p, 0, 0, h, kv, 37, rows)
            got_q[kv, :, h] = qs.reshape(rows, 256)
            got_d[kv, :, h] = d.reshape(rows, 8)
    # K in input order against the reference's own outputs (golden), V (rows reversed) against the oracle
    assert np.array_equal(got_q[0].reshape(-1)[: x0.size], g[f"{name}_qs"])
    assert np.array_equal(got_d[0].reshape(-1)[: x0.size // 32], g[f"{name}_d"])
    rq, rd = O.q8_0_quantize(np.ascontiguousarray(x[::-1]).reshape(-1))
    assert np.array_equal(got_q[1].reshape(-1), rq) and np.array_equal(got_d[1].reshape(-1), rd.reshape(-1))
    p.close()


def _raw_page(pool, layer, phys, head):
    """The bytes of one (layer, physical page, head) block, copied straight out of the pool's allocation."""
    import ctypes
    base = fnkv.lib().fnkv_pool_device_base(pool.h)
    blk = fnkv.lib().fnkv_page_block_bytes()
    page_stride = pool.h_kv * blk
    off = layer * pool.n_pages * page_stride + phys * page_stride + head * blk
    buf = torch.empty(blk, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(base + off), blk, 3) == 0
    return buf.cpu().numpy()


def _unswizzle(page):
    """The page block's codes and scales in token order (the layout the library documents in csrc/layout.h)."""
    kq = np.empty((256, 256), np.int8)
    vq = np.empty((256, 256), np.int8)
    kd = np.empty((256, 8), np.uint16)
    vd = np.empty((256, 8), np.uint16)
    d = np.arange(256)
    for tok in range(256):
        tile = page[(tok // 32) * 17408:(tok // 32 + 1) * 17408]
        tt = tok % 32
        h, j = tt >> 4, tt & 15
        b, q, i = d >> 5, (d >> 3) & 3, d & 7
        koff = h * 4096 + (b >> 1) * 1024 + (16 * q + j) * 16 + (b & 1) * 8 + i
        kq[tok] = (tile[koff] ^ 0x80).view(np.int8)
        m, dd = d >> 4, d & 15
        qq, s = (tt & 15) >> 2, (tt & 3) + ((tt >> 4) << 2)
        voff = 8192 + (m >> 1) * 1024 + (16 * qq + dd) * 16 + (m & 1) * 8 + s
        vq[tok] = (tile[voff] ^ 0x80).view(np.int8)
        bb = np.arange(8)
        kd[tok] = tile[16384 + tt * 16 + bb * 2].astype(np.uint16) | (tile[16384 + tt * 16 + bb * 2 + 1].astype(
            np.uint16) << 8)
        vo = 16896 + qq * 128 + bb * 16 + s * 2
        vd[tok] = tile[vo].astype(np.uint16) | (tile[vo + 1].astype(np.uint16) << 8)
    return kq, kd, vq, vd


def test_page_table_gathers_and_append_offsets():
    # 3 sequences grown page by page in a seeded random order (their tables interleave), 2 layers, appends at
    # positions that straddle tiles and pages; every physical page's bytes must hold exactly the oracle's blocks of
    # the logical cells the oracle's book maps there
    h_kv, layers = 2, 2
    p = fnkv.Pool(4, 24, layers, h_kv)
    slots, ctxs = [0, 1, 2], [1000, 2100, 700]
    cases.scatter_ensure(p, slots, ctxs, seed=5, churn=0.3)
    data = {}
    for s, c in zip(slots, ctxs):
        for layer in range(layers):
            k16, v16 = cases.kv_rows(100 + s, c, h_kv, layer)
            data[(s, layer)] = (k16, v16)
            kt, vt = torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda()
            # in three appends: 0 .. 300, 301 .. c - 2, c - 1 (a decode-sized one)
            for a, b in ((0, 301), (301, c - 1), (c - 1, c)):
                p.append(s, layer, a, kt[a:b].contiguous(), vt[a:b].contiguous())
    torch.cuda.synchronize()
    for s, c in zip(slots, ctxs):
        table = p.table(s)
        assert len(table) == -(-c // 256)
        for layer in range(layers):
            k16, v16 = data[(s, layer)]
            (kq, kd, _), (vq, vd, _) = cases.decoded(O, k16, v16)
            for lp, phys in enumerate(table):
                n = min(256, c - lp * 256)
                for h in range(h_kv):
                    rk, rkd, rv, rvd = _unswizzle(_raw_page(p, layer, phys, h))
                    sl = slice(lp * 256, lp * 256 + n)
                    for what, a, b in (("K codes", rk[:n], kq[sl, h]), ("K scales", rkd[:n], kd[sl, h]),
                                       ("V codes", rv[:n], vq[sl, h]), ("V scales", rvd[:n], vd[sl, h])):
                        bad = np.argwhere(a != b)
                        assert bad.size == 0, (f"{what}: slot {s} layer {layer} page {lp}->{phys} head {h}: "
                                               f"{len(bad)} mismatches, first at {bad[:4].tolist()}")
    p.close()


def test_trim_keeps_the_kept_pages_bytes():
    p = fnkv.Pool(2, 8, 1, 2)
    assert p.ensure(0, 5 * 256)[0] == 0
    k16, v16 = cases.kv_rows(9, 5 * 256, 2)
    p.append(0, 0, 0, torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda())
    before = _export_blocks(p, 0, 0, 1, 1, 0, 2 * 256)
    assert p.trim(0, 2 * 256 - 5) == 0 and p.mapped_pages(0) == 2 and p.free_pages() == 6
    after = _export_blocks(p, 0, 0, 1, 1, 0, 2 * 256)
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])
    # the freed pages come back zeroed to the next taker
    assert p.ensure(1, 3 * 256)[0] == 0 and p.table(1) == [2, 3, 4]
    z = _export_blocks(p, 1, 0, 0, 0, 0, 3 * 256)
    assert np.all(z[0] == -128) and np.all(z[1] == 0)  # zero bytes are excess-128 code -128 with scale 0
    p.close()


def test_append_refuses_unmapped_cells_and_enqueues_nothing():
    p = fnkv.Pool(1, 4, 1, 2)
    assert p.ensure(0, 256)[0] == 0
    k = torch.zeros((4, 2, 256), dtype=torch.float16, device="cuda")
    with pytest.raises(fnkv.FnkvError) as e:
        p.append(0, 0, 254, k, k)
    assert e.value.code == fnkv.ERR_ARG and "not all mapped" in str(e.value)
    with pytest.raises(fnkv.FnkvError):
        p.append(0, 1, 0, k, k)  # no layer 1
    p.close()


def test_append_bit_exact_at_scale():
    # 65,536 fp16 rows of BASELINE's distribution through the append, every code and scale against the oracle
    # (pinned to quantize_row_q8_0_ref): ~8.4 M values per K/V, where exact x * id = k + 0.5 ties occur by the
    # thousand (x = amax / 2 gives 63.5)
    n, h_kv = 65536, 2
    p = fnkv.Pool(1, n // 256, 1, h_kv)
    assert p.ensure(0, n)[0] == 0
    k16, v16 = cases.kv_rows(4242, n, h_kv)
    p.append(0, 0, 0, torch.from_numpy(k16).cuda(), torch.from_numpy(v16).cuda())
    for kv, src in ((0, k16), (1, v16)):
        rq, rd = O.q8_0_quantize(src.astype(np.float32))
        for h in range(h_kv):
            qs, d = _export_blocks(p, 0, 0, h, kv, 0, n)
            bad = np.nonzero(qs != rq[:, h].reshape(-1))[0]
            assert bad.size == 0, f"kv {kv} head {h}: {bad.size} code mismatches, first at {bad[:4].tolist()}"
            assert np.array_equal(d, rd[:, h].reshape(-1))
    p.close()

"""Sparse (QSA) attention over selection bodies (fn/kernels/qsa/attend.h:97-141 with qsa.h:77-81's body) on the GPU
against the oracle's fp64 attention over each row's selected cells of the decoded cache (max-abs 2e-3): rows B = 1..5,
shallow contexts (every whole block selected) and deep ones (512 of tens of thousands of blocks, random and clustered
selections), Q8_0 and KV8 pools, the rows' own cells written by the launch, bitwise reruns, the full selection
against the dense launch, and bodies with out-of-range entries (ignored, nothing read past the row's cells)."""
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


def _decoded(k16, v16, fmt):
    if fmt == fnkv.FMT_KV8:
        (_, _, kf), (_, _, vf) = cases.decoded_kv8(O, k16, v16)
    else:
        (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
    return kf, vf


def sparse_case(depth, T, seed, clustered=False, fmt=fnkv.FMT_Q8_0, body=None, new_cells=True, hq=None, hkv=None):
    hq = HQ if hq is None else hq
    hkv = HKV if hkv is None else hkv
    ctx = depth + T
    pool = fnkv.Pool(2, -(-ctx // 256) + 8, 1, hkv, fmt=fmt)
    cases.scatter_ensure(pool, [0], [ctx], seed, churn=0.3)
    k16, v16 = cases.kv_rows(seed, ctx, hkv)
    upto = depth if new_cells else ctx
    if upto:
        pool.append(0, 0, 0, torch.from_numpy(k16[:upto]).cuda(), torch.from_numpy(v16[:upto]).cuda())
    words, offs, cells = O.qsa_body(depth, T, seed, clustered) if body is None else body
    q16 = cases.queries(seed + 1, (T, hq, D))
    q = torch.from_numpy(q16).cuda()
    out = torch.full_like(q, float("nan"))
    kn = torch.from_numpy(k16[depth:]).cuda() if new_cells else None
    vn = torch.from_numpy(v16[depth:]).cuda() if new_cells else None
    bt = torch.from_numpy(words.view(np.int32)).cuda()
    ot = torch.from_numpy(offs).cuda()
    pool.sparse(0, depth, 0, q, bt, ot, out, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    kf, vf = _decoded(k16, v16, fmt)
    ref = O.attn_f64_cells(q16.view(np.uint16), kf, vf, cells)
    return pool, out.cpu().numpy(), ref, (q, bt, ot)


@pytest.mark.parametrize("depth,T", [(0, 1), (2, 5), (37, 3), (300, 2), (2045, 5), (2050, 1)])
def test_sparse_shallow_every_block(depth, T):
    # n_vis <= 512: every whole block is selected, the tail adds the rest: the row's whole causal context
    pool, got, ref, _ = sparse_case(depth, T, seed=depth + T)
    assert np.isfinite(got).all()
    assert cases.out_err(got, ref) <= TOL


@pytest.mark.parametrize("T", [1, 2, 3, 5])
@pytest.mark.parametrize("clustered", [False, True])
def test_sparse_deep_selection(T, clustered):
    # 512 of ~4,000 whole blocks a row: most tiles hold one selected block, the rows' selections differ
    depth = 16003 - T
    pool, got, ref, _ = sparse_case(depth, T, seed=40 + T + (10 if clustered else 0), clustered=clustered)
    assert np.isfinite(got).all()
    assert cases.out_err(got, ref) <= TOL


@pytest.mark.parametrize("hq,T", [(32, 1), (32, 3), (48, 2), (48, 5)])
def test_sparse_many_heads_a_kv_head(hq, T):
    # more than 16 query heads on one KV head: each row's heads take two or three 16-row tiles (the row kernels'
    # sparse instantiation); up to 48 (FNKV_MAX_ROWS)
    pool, got, ref, _ = sparse_case(3001 - T, T, seed=90 + hq + T, hq=hq, hkv=1)
    assert np.isfinite(got).all()
    assert cases.out_err(got, ref) <= TOL


def test_sparse_kv8_pool():
    pool, got, ref, _ = sparse_case(9000, 3, seed=71, fmt=fnkv.FMT_KV8)
    assert cases.out_err(got, ref) <= TOL


def test_sparse_bitwise_reruns_and_own_cells_written():
    depth, T = 12000, 5
    pool, got, ref, (q, bt, ot) = sparse_case(depth, T, seed=81, clustered=True)
    assert cases.out_err(got, ref) <= TOL
    for _ in range(3):
        again = torch.full_like(q, float("nan"))
        pool.sparse(0, depth, 0, q, bt, ot, again)
        torch.cuda.synchronize()
        assert np.array_equal(again.cpu().numpy().view(np.uint16), got.view(np.uint16))
    # the launch wrote the rows' own cells (bit-exact Q8_0 of the inputs)
    k16, v16 = cases.kv_rows(81, depth + T, HKV)
    (kq, kd, _), _ = cases.decoded(O, k16[depth:], v16[depth:])
    for h in range(HKV):
        blocks = pool.export(0, 0, h, 0, depth, T)
        torch.cuda.synchronize()
        qs, d = O.from_block_q8_0(blocks.cpu().numpy().reshape(-1, 34))
        assert np.array_equal(qs.reshape(T, 256), kq[:, h]) and np.array_equal(d.reshape(T, 8), kd[:, h])


def test_sparse_full_selection_agrees_with_dense():
    # at n_vis <= 512 the selection is the whole causal context: the dense launch over the same pool agrees
    depth, T = 1800, 3
    pool, got, ref, (q, bt, ot) = sparse_case(depth, T, seed=91, new_cells=False)
    ws = torch.zeros(pool.decode_ws_bytes([depth + T], T, HQ), dtype=torch.uint8, device="cuda")
    dense = torch.empty_like(q)
    pool.decode([0], [depth + T], T, 0, q[None].contiguous(), dense[None], ws)
    torch.cuda.synchronize()
    assert np.abs(dense.cpu().numpy().astype(np.float32) - got.astype(np.float32)).max() <= 2 * TOL


def test_sparse_body_entries_outside_the_rows_are_ignored():
    # K larger than the row's whole blocks, block IDs past the row or negative: ignored (the launch finds the rows
    # from the positions and reads no word past a row); the result is attention over the valid entries
    depth, T = 5000, 3
    words, offs, cells = O.qsa_body(depth, T, seed=5)
    w = words.view(np.int32).copy()
    new_cells = []
    for t in range(T):
        o = offs[t] // 4
        K = w[o]
        w[o] = K + 1000  # clamped to the row's K
        bad = [2 + 5, 2 + 9, 2 + K - 1]
        w[o + bad[0]] = 10**6
        w[o + bad[1]] = -3
        w[o + bad[2]] = (depth + t + 1) // 4  # the tail block: not a whole block
        keep = np.ones(K, bool)
        keep[[5, 9, K - 1]] = False
        blocks = w[o + 2:o + 2 + K][keep]
        n_vis = (depth + t + 1) // 4
        blocks = blocks[(blocks >= 0) & (blocks < n_vis)].astype(np.int64)
        tail = np.arange(4 * n_vis, depth + t + 1)
        # the tail block's cells still count through the tail itself
        new_cells.append(np.unique(np.concatenate([(4 * blocks[:, None] + np.arange(4)).reshape(-1), tail])))
    pool, got, ref, _ = sparse_case(depth, T, seed=5, body=(w.view(np.uint32), offs, new_cells))
    assert np.isfinite(got).all()
    assert cases.out_err(got, ref) <= TOL


def test_sparse_refusals_enqueue_nothing():
    pool = fnkv.Pool(2, 8, 1, HKV)
    assert pool.ensure(0, 1024)[0] == 0
    q = torch.zeros((3, HQ, D), dtype=torch.float16, device="cuda")
    out = torch.zeros_like(q)
    body = torch.zeros(4096, dtype=torch.int32, device="cuda")
    offs = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(fnkv.FnkvError):  # past the mapped cells
        pool.sparse(0, 1022, 0, q, body, offs, out)
    with pytest.raises(fnkv.FnkvError):  # six rows
        q6 = torch.zeros((6, HQ, D), dtype=torch.float16, device="cuda")
        pool.sparse(0, 10, 0, q6, body, offs, torch.zeros_like(q6))
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    with pytest.raises(fnkv.FnkvError):  # workspace too small
        pool.sparse(0, 10, 0, q, body, offs, out, ws=ws)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out).item() == 0

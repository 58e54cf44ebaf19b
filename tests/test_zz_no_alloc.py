"""fnkv_attn_decode_noalloc (the decode entry point that allocates nothing: its split partials live in the library's
fixed device scratch) against fnkv_attn_decode_dev, the entry point it varies, on the same inputs: bitwise equal
outputs and appended cells, on two calls in a row, the second with a smaller input (fewer sequences, shorter
contexts, fewer query tokens), so the second reads none of the first's partials; and a launch too large for the
scratch is refused with nothing enqueued."""
import numpy as np
import pytest

import cases
import fnkv

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

HQ, HKV, D = 16, 2, 256


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def make(ctxs, T, seed):
    pool = fnkv.Pool(len(ctxs) + 1, sum(-(-c // 256) for c in ctxs) + 8, 1, HKV)
    slots = list(range(len(ctxs)))
    cases.scatter_ensure(pool, slots, ctxs, seed, churn=0.3)
    kv = []
    for s, c in zip(slots, ctxs):
        k16, v16 = cases.kv_rows(seed + s, c, HKV)
        pool.append(s, 0, 0, torch.from_numpy(k16[:c - T]).cuda(), torch.from_numpy(v16[:c - T]).cuda())
        kv.append((k16[c - T:], v16[c - T:]))
    kn = torch.from_numpy(np.stack([k for k, _ in kv])).cuda()
    vn = torch.from_numpy(np.stack([v for _, v in kv])).cuda()
    q = torch.from_numpy(cases.queries(seed, (len(ctxs), T, HQ, D))).cuda()
    return pool, slots, kn, vn, q


def cells(pool, slots, ctxs, T):
    return [pool.export(s, 0, h, kv, c - T, T).cpu() for s, c in zip(slots, ctxs) for h in range(HKV)
            for kv in range(2)]


@pytest.mark.parametrize("first,second", [(([8192, 16384, 32768, 65536], 3), ([3000, 700], 1)),
                                          (([262144], 5), ([40000], 3))])
def test_noalloc_matches_decode_dev_twice(first, second):
    for ctxs, T in (first, second):
        pool, slots, kn, vn, q = make(ctxs, T, seed=len(ctxs) * 10 + T)
        ctx_dev = torch.tensor(ctxs, dtype=torch.int64, device="cuda")
        err = torch.zeros(2, dtype=torch.int32, device="cuda")
        ref = torch.full_like(q, float("nan"))
        got = torch.full_like(q, float("nan"))
        ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
        pool.decode_dev(slots, ctx_dev, ctxs, T, 0, q, ref, ws, err[0:1], k_new=kn, v_new=vn)
        ref_cells = cells(pool, slots, ctxs, T)
        # the same launch again through the scratch (it rewrites the same new cells with the same values)
        pool.decode_noalloc(slots, ctx_dev, ctxs, T, 0, q, got, err[1:2], k_new=kn, v_new=vn)
        got_cells = cells(pool, slots, ctxs, T)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
        assert all(torch.equal(a, b) for a, b in zip(ref_cells, got_cells))
        assert err.sum().item() == 0
        pool.close()


def test_noalloc_refuses_a_launch_beyond_its_scratch():
    # 16 sequences of 65,536 cells at T = 3: 25 MB of split partials, more than the 16 MiB scratch
    n, c = 16, 65536
    pool = fnkv.Pool(n + 1, n * (c // 256) + 8, 1, HKV)
    for s in range(n):
        assert pool.ensure(s, c)[0] == 0
    ctxs = [c] * n
    assert pool.decode_ws_bytes(ctxs, 3, HQ) > 16 << 20
    q = torch.zeros((n, 3, HQ, D), dtype=torch.float16, device="cuda")
    out = torch.full_like(q, 2.0)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(fnkv.FnkvError, match="scratch"):
        pool.decode_noalloc(list(range(n)), torch.tensor(ctxs, dtype=torch.int64, device="cuda"), ctxs, 3, 0, q, out,
                            err)
    torch.cuda.synchronize()
    assert bool((out == 2.0).all()) and err.item() == 0
    pool.close()

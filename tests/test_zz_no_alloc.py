"""fnkv_attn_decode_noalloc (the decode entry point that allocates nothing: its split partials live in the library's
fixed device scratch) against fnkv_attn_decode_dev, the entry point it varies, on the same inputs: bitwise equal
outputs and appended cells, on two calls in a row, the second with a smaller input (fewer sequences, shorter
contexts, fewer query tokens), so the second reads none of the first's partials; the call captured into a HIP graph
and replayed (every replay bitwise equal to the eager result, and no device memory taken by the capture beyond what a
one-kernel graph takes); the scratch bound to one pool and one stream, calls from another refused until that pool is
destroyed; and a launch too large for the scratch refused with nothing enqueued."""
import gc

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


def _fresh(ctxs, T, seed):
    """A pool with `ctxs` cells per sequence, its decode_dev result (reference) and the call's arguments."""
    pool, slots, kn, vn, q = make(ctxs, T, seed)
    ctx_dev = torch.tensor(ctxs, dtype=torch.int64, device="cuda")
    ref = torch.full_like(q, float("nan"))
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
    pool.decode_dev(slots, ctx_dev, ctxs, T, 0, q, ref, ws, err, k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    assert err.item() == 0
    args = dict(slots=slots, ctx_dev=ctx_dev, max_ctx=ctxs, T=T, layer=0, q=q, k_new=kn, v_new=vn)
    return pool, ref, args


def test_noalloc_binds_one_pool_and_one_stream():
    a, ref_a, args_a = _fresh([5000, 1200], 2, seed=5)
    b, ref_b, args_b = _fresh([7000], 1, seed=6)
    try:
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        got_a = torch.full_like(ref_a, float("nan"))
        a.decode_noalloc(out=got_a, err=err, **args_a)
        got_b = torch.full_like(ref_b, 2.0)
        with pytest.raises(fnkv.FnkvError, match="another pool"):
            b.decode_noalloc(out=got_b, err=err, **args_b)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        again = torch.full_like(ref_a, 2.0)
        with torch.cuda.stream(side), pytest.raises(fnkv.FnkvError, match="another stream"):
            a.decode_noalloc(out=again, err=err, **args_a)
        torch.cuda.synchronize()
        assert torch.equal(ref_a.view(torch.int16), got_a.view(torch.int16))
        assert bool((got_b == 2.0).all()) and bool((again == 2.0).all()) and err.item() == 0
        a.close()  # releases the binding: pool b may now use the scratch
        b.decode_noalloc(out=got_b, err=err, **args_b)
        torch.cuda.synchronize()
        assert torch.equal(ref_b.view(torch.int16), got_b.view(torch.int16)) and err.item() == 0
    finally:
        a.close()
        b.close()


def _free_bytes():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return torch.cuda.mem_get_info()[0]


def test_noalloc_captured_in_a_graph_allocates_nothing():
    pool, ref, args = _fresh([8192, 20000, 3000], 3, seed=21)
    try:
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        got = torch.full_like(ref, float("nan"))
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            pool.decode_noalloc(out=got, err=err, **args)  # eager, on the stream the graph is captured on
        torch.cuda.synchronize()
        assert torch.equal(ref.view(torch.int16), got.view(torch.int16))
        # a one-kernel graph first, so the runtime's own first-capture memory is not counted against the call
        ctl = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ctl, stream=side):
            got.mul_(1.0)
        ctl.replay()
        free0 = _free_bytes()
        ctl2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(ctl2, stream=side):
            got.mul_(1.0)
        ctl2.replay()
        free1 = _free_bytes()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            pool.decode_noalloc(out=got, err=err, **args)
        for i in range(3):
            got.fill_(float("nan"))
            err.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), f"replay {i}"
            assert err.item() == 0
        free2 = _free_bytes()
        print(f"free bytes: one-kernel graph takes {free0 - free1}, the noalloc graph {free1 - free2}", flush=True)
        assert free1 - free2 <= max(free0 - free1, 0)
    finally:
        pool.close()

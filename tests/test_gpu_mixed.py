"""a mixed 8-sequence pool step with page churn — three finished sequences free their pages first
(a fragmented free list), two sequences append and attend a 4,096-token prefill chunk, six verify T = 5 — all in one
shared pool, every layer. Parity against the oracle's fp64 attention over the decoded cache (max-abs 2e-3) at
contexts the oracle finishes in seconds; at BASELINE's full contexts (1K..196K) the same step is checked through
properties that do not need the oracle (finite outputs, the verify launch over six sequences against each sequence
launched alone, the prefill chunk's last rows against a T = 5 verify of the same cells) and, for every verify row and
a spread of prefill rows, against the fp64 attention over the cells as the pool holds them (exported as ggml
block_q8_0)."""
import numpy as np
import pytest

import cases
import fnkv
import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 2e-3
HQ, HKV, D = 16, 2, 256
CHUNK = 4096


@pytest.fixture(scope="module", autouse=True)
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def churned_pool(n_pages, layers, seed):
    """An 8-slot pool (plus a filler slot) whose free list has holes: three finished sequences take interleaved pages,
    then give them back."""
    pool = fnkv.Pool(9, n_pages, layers, HKV)
    rng = np.random.default_rng([seed, 4])
    finished = [5, 6, 7]
    sizes = {s: int(rng.integers(8, 40)) for s in finished}
    have = {s: 0 for s in finished}
    while any(have[s] < sizes[s] for s in finished):
        s = int(rng.choice([x for x in finished if have[x] < sizes[x]]))
        have[s] += 1
        assert pool.ensure(s, have[s] * 256)[0] == 0
    for s in finished:
        assert pool.trim(s, 0) == 0
    return pool


def verify_inputs(seed, n, T):
    q = cases.queries(seed, (n, T, HQ, D))
    rng = np.random.default_rng([seed, 5])
    kn = rng.standard_normal((n, T, HKV, D), dtype=np.float32).astype(np.float16)
    vn = rng.standard_normal((n, T, HKV, D), dtype=np.float32).astype(np.float16)
    return q, kn, vn


def test_config4_mixed_step_parity():
    seed, layers, T = 4, 2, 5
    rng = np.random.default_rng([seed, 1])
    pf_slots, vf_slots = [0, 1], [2, 3, 4, 5, 6, 7]
    pf_depth = [int(rng.integers(1000, 6000)) for _ in pf_slots]
    vf_ctx = [int(rng.integers(1024, 24 * 1024)) for _ in vf_slots]  # BASELINE draws 1K..196K; scaled for the oracle
    n_pages = sum(-(-(d + CHUNK) // 256) for d in pf_depth) + sum(-(-c // 256) for c in vf_ctx) + 120
    pool = churned_pool(n_pages, layers, seed)
    ctx_of = {}
    for s, d in zip(pf_slots, pf_depth):
        ctx_of[s] = d + CHUNK
    for s, c in zip(vf_slots, vf_ctx):
        ctx_of[s] = c
    cases.scatter_ensure(pool, pf_slots + vf_slots, [ctx_of[s] for s in pf_slots + vf_slots], seed)
    dec = {}
    for layer in range(layers):
        for s in pf_slots + vf_slots:
            c = ctx_of[s]
            k16, v16 = cases.kv_rows(seed * 100 + s, c, HKV, layer)
            if s in vf_slots:  # the verify step's T new cells arrive with the launch
                k16[c - T:], v16[c - T:] = 0, 0
            upto = c - CHUNK if s in pf_slots else c - T
            pool.append(s, layer, 0, torch.from_numpy(k16[:upto]).cuda(), torch.from_numpy(v16[:upto]).cuda())
            dec[(s, layer)] = (k16, v16)
    q_v, kn, vn = verify_inputs(seed, len(vf_slots), T)
    errs = {}
    for layer in range(layers):
        # the two prefill chunks: append, then attend
        for s in pf_slots:
            c = ctx_of[s]
            k16, v16 = dec[(s, layer)]
            pool.append(s, layer, c - CHUNK, torch.from_numpy(k16[c - CHUNK:]).cuda(),
                        torch.from_numpy(v16[c - CHUNK:]).cuda())
            q16 = cases.queries(seed * 10 + s + layer, (CHUNK, HQ, D))
            out = torch.empty((CHUNK, HQ, D), dtype=torch.float16, device="cuda")
            pool.prefill(s, layer, c, torch.from_numpy(q16).cuda(), out)
            torch.cuda.synchronize()
            rows = [0, 1, 777, 2048, CHUNK - 2, CHUNK - 1]
            (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
            ref = O.attn_f64(q16.view(np.uint16), kf, vf, c, rows=rows)
            errs[("prefill", layer, s)] = cases.out_err(out.cpu().numpy()[rows], ref)
        # the six verify steps in one launch, their new cells appended by it
        q = torch.from_numpy(q_v).cuda()
        out = torch.empty_like(q)
        ctxs = [ctx_of[s] for s in vf_slots]
        ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
        pool.decode(vf_slots, ctxs, T, layer, q, out, ws, k_new=torch.from_numpy(kn).cuda(),
                    v_new=torch.from_numpy(vn).cuda())
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        for i, s in enumerate(vf_slots):
            c = ctx_of[s]
            k16, v16 = dec[(s, layer)]
            k16 = k16.copy()
            v16 = v16.copy()
            k16[c - T:], v16[c - T:] = kn[i], vn[i]
            (_, _, kf), (_, _, vf) = cases.decoded(O, k16, v16)
            ref = O.attn_f64(q_v[i].view(np.uint16), kf, vf, c)
            errs[("verify", layer, s)] = cases.out_err(got[i], ref)
    worst = max(errs.values())
    assert np.isfinite(worst) and worst <= TOL, errs


def exported_cells(pool, slot, layer, c):
    """The slot's first c cells of `layer` as the pool holds them (exported as ggml block_q8_0), decoded by the
    oracle: float32 K, V [c][HKV][256]."""
    kf = np.empty((c, HKV, D), np.float32)
    vf = np.empty((c, HKV, D), np.float32)
    for h in range(HKV):
        for kv, dst in ((0, kf), (1, vf)):
            qs, d = O.from_block_q8_0(pool.export(slot, layer, h, kv, 0, c).cpu().numpy())
            dst[:, h, :] = O.q8_0_dequantize(qs.reshape(c, D), d.reshape(c, D // 32))
    return kf, vf


def test_config4_full_contexts_properties():
    """BASELINE config 4 at its full contexts on a churned pool, two of its layers, K/V in BASELINE's distribution: the
    two prefill chunks (finite, their last five rows against a T = 5 verify over the same cells, a spread of rows
    against fp64), and the six-sequence verify launch writing its own new cells, against each sequence launched alone
    and against fp64 (out_err and the plain max-abs)."""
    seed, layers, T = 41, 2, 5
    rng = np.random.default_rng([seed, 1])
    pf_slots, vf_slots = [0, 1], [2, 3, 4, 5, 6, 7]
    pf_depth = [int(rng.integers(1024, 196 * 1024)) for _ in pf_slots]
    vf_ctx = [int(rng.integers(1024, 196 * 1024)) for _ in vf_slots]
    ctx_of = dict(zip(pf_slots, [d + CHUNK for d in pf_depth]))
    ctx_of.update(zip(vf_slots, vf_ctx))
    n_pages = sum(-(-c // 256) for c in ctx_of.values()) + 120
    pool = churned_pool(n_pages, layers, seed)
    order = pf_slots + vf_slots
    cases.scatter_ensure(pool, order, [ctx_of[s] for s in order], seed)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    new_cells = {}
    for layer in range(layers):
        for s in order:
            x = torch.randn((2, ctx_of[s], HKV, D), generator=g, device="cuda")
            for h in range(HKV):  # 4 of a KV head's 256 channels x8 (BASELINE's outliers)
                for kv in range(2):
                    ch = torch.randperm(D, generator=g, device="cuda")[:4]
                    x[kv, :, h, ch] *= 8.0
            x = x.half()
            upto = ctx_of[s] - T if s in vf_slots else ctx_of[s]  # a verify launch appends its own T cells
            pool.append(s, layer, 0, x[0, :upto].contiguous(), x[1, :upto].contiguous())
            if s in vf_slots:
                new_cells[(s, layer)] = (x[0, upto:].contiguous(), x[1, upto:].contiguous())
            del x
    # the prefill chunks: finite; the chunk's last five rows agree with a T = 5 verify over the same cells; a spread
    # of rows against the fp64 attention over the cells as the pool holds them
    errs, plain = {}, {}
    for layer in range(layers):
        for s in pf_slots:
            c = ctx_of[s]
            q = torch.randn((CHUNK, HQ, D), generator=g, device="cuda").half()
            out = torch.empty_like(q)
            pool.prefill(s, layer, c, q, out)
            qv = q[None, -5:].contiguous()
            ov = torch.empty_like(qv)
            ws = torch.zeros(pool.decode_ws_bytes([c], 5, HQ), dtype=torch.uint8, device="cuda")
            pool.decode([s], [c], 5, layer, qv, ov, ws)
            torch.cuda.synchronize()
            assert torch.isfinite(out.float()).all().item()
            assert (ov[0].float() - out[-5:].float()).abs().max().item() <= 2 * TOL
            rows = [0, 1, 511, 2047, 3000, CHUNK - 1]
            kf, vf = exported_cells(pool, s, layer, c)
            ref = O.attn_f64(q.cpu().numpy().view(np.uint16), kf, vf, c, rows=rows)
            errs[("prefill", layer, s)] = cases.out_err(out.cpu().numpy()[rows], ref)
            plain[("prefill", layer, s)] = cases.plain_err(out.cpu().numpy()[rows], ref)
        # the six verify steps in one launch, their new cells written by the launch, against each launched alone
        # (over the same cells, already written) and against fp64
        q = torch.randn((len(vf_slots), T, HQ, D), generator=g, device="cuda").half()
        ctxs = [ctx_of[s] for s in vf_slots]
        kn = torch.stack([new_cells[(s, layer)][0] for s in vf_slots])
        vn = torch.stack([new_cells[(s, layer)][1] for s in vf_slots])
        out = torch.empty_like(q)
        ws = torch.zeros(pool.decode_ws_bytes(ctxs, T, HQ), dtype=torch.uint8, device="cuda")
        pool.decode(vf_slots, ctxs, T, layer, q, out, ws, k_new=kn, v_new=vn)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all().item()
        got = out.cpu().numpy()
        q16 = q.cpu().numpy()
        for i, s in enumerate(vf_slots):
            one = torch.empty_like(q[i:i + 1])
            ws1 = torch.zeros(pool.decode_ws_bytes([ctxs[i]], T, HQ), dtype=torch.uint8, device="cuda")
            pool.decode([s], [ctxs[i]], T, layer, q[i:i + 1].contiguous(), one, ws1)
            torch.cuda.synchronize()
            assert (one[0].float() - out[i].float()).abs().max().item() <= 2 * TOL
            kf, vf = exported_cells(pool, s, layer, ctxs[i])
            ref = O.attn_f64(q16[i].view(np.uint16), kf, vf, ctxs[i])
            errs[("verify", layer, s)] = cases.out_err(got[i], ref)
            plain[("verify", layer, s)] = cases.plain_err(got[i], ref)
    worst = max(errs.values())
    assert np.isfinite(worst) and worst <= TOL, errs
    assert max(plain.values()) <= TOL, plain

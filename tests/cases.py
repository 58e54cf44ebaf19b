"""Seeded inputs and the oracle-side model of a pool, shared by the GPU tests, smoke() and bench.py.

Inputs follow BASELINE's distribution: K and V fp16 ~ N(0, 1) with 4 of the 256 channels of each KV head scaled x8
(channels fixed by seed per head and layer), Q fp16 ~ N(0, 1)."""
import numpy as np

D = 256


def kv_rows(seed, n, h_kv, layer=0):
    """fp16 K and V [n][h_kv][256] as numpy float16."""
    rng = np.random.default_rng([seed, layer])
    out = []
    for _ in range(2):
        x = rng.standard_normal((n, h_kv, D), dtype=np.float32)
        for h in range(h_kv):
            ch = rng.choice(D, 4, replace=False)
            x[:, h, ch] *= 8.0
        out.append(x.astype(np.float16))
    return out[0], out[1]


def queries(seed, shape):
    rng = np.random.default_rng([seed, 99])
    return rng.standard_normal(shape, dtype=np.float32).astype(np.float16)


def scatter_ensure(pool, slots, ctxs, seed, churn=0):
    """Grows the slots to their contexts one page at a time in a seeded random order, so that each slot's page table
    is a random interleaving of the pool's pages; with churn > 0 a filler slot (the pool's last) grabs pages between
    the growths and releases them at the end, leaving holes in the free list. Returns nothing; the pool's book is
    the record."""
    rng = np.random.default_rng([seed, 7])
    need = {s: -(-c // 256) for s, c in zip(slots, ctxs)}
    have = {s: 0 for s in slots}
    filler = pool.n_slots - 1
    fill = 0
    while any(have[s] < need[s] for s in slots):
        live = [s for s in slots if have[s] < need[s]]
        s = live[rng.integers(len(live))]
        have[s] += 1
        code, _ = pool.ensure(s, have[s] * 256)
        assert code == 0, code
        remaining = sum(need[x] - have[x] for x in slots)
        if churn and rng.random() < churn and filler not in slots and pool.free_pages() > remaining:
            fill += 1
            code, _ = pool.ensure(filler, fill * 256)
            assert code == 0
    if churn and filler not in slots:
        assert pool.trim(filler, 0) == 0


def decoded(oracle, k16, v16):
    """The oracle's Q8_0 codes, scales and decoded fp32 values of fp16 K and V rows [n][h][256]."""
    kq, kd = oracle.q8_0_quantize(k16.astype(np.float32))
    vq, vd = oracle.q8_0_quantize(v16.astype(np.float32))
    return (kq, kd, oracle.q8_0_dequantize(kq, kd)), (vq, vd, oracle.q8_0_dequantize(vq, vd))


def half_ulp_f16(x):
    """Half an fp16 ulp at |x|: the rounding any fp16 output carries on top of the computation's own error."""
    a = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0**-14)))
    return 0.5 * 2.0 ** (e - 10)


def out_err(got, ref):
    """Max-abs error of fp16 outputs against the fp64 reference, the quantity held to the 2e-3 tolerance. Where the
    output is below 4 in magnitude it is the plain |got - ref|; at 4 and above an fp16 output's own spacing is 2^-8 or
    more, so half of it (the rounding any fp16 output of the exact value carries, up to 2^-9 = 1.95e-3 in [4, 8)) is
    taken off there: at such magnitudes no fp16 output could hold a plain 2e-3 bound."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    mag = np.maximum(np.abs(g), np.abs(r))
    allow = np.where(mag >= 4.0, half_ulp_f16(mag), 0.0)
    return float(np.max(np.abs(g - r) - allow))


def plain_err(got, ref):
    """Plain max-abs error |got - ref| over every output."""
    return float(np.max(np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))))


def decoded_kv8(oracle, k16, v16):
    """The oracle's KV8 codes, group scales and decoded fp32 values (code x scale, exact) of fp16 K and V rows."""
    out = []
    for x in (k16, v16):
        c, s = oracle.kv8_quantize(x.astype(np.float32))
        sf = s.view(np.float16).astype(np.float32)
        out.append((c, s, c.astype(np.float32) * np.repeat(sf, 64, axis=-1)))
    return out[0], out[1]

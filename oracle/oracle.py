"""ctypes view of the C oracle (oracle/fnkv_oracle.c) — TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker or the timed CPU
baseline; the product path (fnfl-v100_amd/) never imports it. Each wrapper names the reference lines its C function
restates (see the C file's header).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libfnkv_ref.so")

_lib = None
_ref = None

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64


def _ptr(a):
    return a.ctypes.data_as(P)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f32_to_f16.argtypes = [ctypes.c_float]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        for n in ("or_f32_to_f16_n", "or_f16_to_f32_n"):
            getattr(L, n).argtypes = [P, I64, P]
        L.or_q8_0_quantize.argtypes = [P, I64, P, P]
        L.or_q8_0_dequantize.argtypes = [P, P, I64, P]
        L.or_kv8_quantize.argtypes = [P, I64, P, P]
        L.or_pages_new.restype = P
        L.or_pages_new.argtypes = [I32, I32]
        L.or_pages_free.argtypes = [P]
        L.or_pages_free_count.restype = I32
        L.or_pages_free_count.argtypes = [P]
        L.or_pages_mapped.restype = I32
        L.or_pages_mapped.argtypes = [P, I32]
        L.or_pages_physical.restype = I32
        L.or_pages_physical.argtypes = [P, I32, I32]
        L.or_pages_for.restype = I32
        L.or_pages_for.argtypes = [I64, I32, I32]
        L.or_pages_take.restype = I32
        L.or_pages_take.argtypes = [P, I32, I32, P, P]
        L.or_pages_give.argtypes = [P, I32, I32, P, P]
        L.or_reclaim_victim.restype = I32
        L.or_reclaim_victim.argtypes = [P, P, P, I32, I32]
        L.or_attn_f64.argtypes = [P, P, P, I32, I32, I32, I32, I32, ctypes.c_double, P, I32, P]
        L.or_attn_f64_mt.argtypes = [P, P, P, I32, I32, I32, I32, I32, ctypes.c_double, P, I32, P, I32]
        L.or_attn_ggml.argtypes = [P, P, P, I32, I32, I32, I32, I32, ctypes.c_float, I32, I32, P]
        L.or_block_q8_0_size.restype = I32
        _lib = L
    return _lib


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own quantizer sources built into oracle/_ref (present only where the checkout was)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH, mode=os.RTLD_LAZY | getattr(os, "RTLD_LOCAL", 0))
        R.fnkv_ref_q8_0_quantize.argtypes = [P, P, I64]
        R.fnkv_ref_q8_0_dequantize.argtypes = [P, P, I64]
        R.fnkv_ref_f32_to_f16.argtypes = [P, I64, P]
        R.fnkv_ref_f16_to_f32.argtypes = [P, I64, P]
        R.fnkv_ref_kv8_quantize.argtypes = [P, I32, P, P]
        R.fnkv_ref_f16_bits_rn.argtypes = [P, I64, P]
        R.fnkv_ref_f16_value.argtypes = [P, I64, P]
        R.fnkv_ref_stress_rows.restype = I64
        R.fnkv_ref_stress_rows.argtypes = [ctypes.c_uint64, I32, P, I64]
        R.fnkv_ref_act_quantize.argtypes = [P, I32, I32, P, P]
        _ref = R
    return _ref


# ---- conversions and quantizers ----

def f32_to_f16(x):
    """ggml-impl.h:414-438 rounding (RNE), as fp16 bit patterns (uint16)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_n(_ptr(x), x.size, _ptr(y))
    return y


def f16_to_f32(h):
    """ggml-impl.h:391-412 widening."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().or_f16_to_f32_n(_ptr(h), h.size, _ptr(y))
    return y


def q8_0_quantize(x):
    """quantize_row_q8_0_ref (ggml-quants.c:274-297): rows of x (last axis a multiple of 32) -> (codes int8 like x,
    scales uint16 [..., n / 32])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.shape[-1] % 32 == 0
    qs = np.empty(x.shape, np.int8)
    d = np.empty(x.shape[:-1] + (x.shape[-1] // 32,), np.uint16)
    lib().or_q8_0_quantize(_ptr(x), x.size, _ptr(qs), _ptr(d))
    return qs, d


def q8_0_dequantize(qs, d):
    """dequantize_row_q8_0 (ggml-quants.c:551-565)."""
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    d = np.ascontiguousarray(d, dtype=np.uint16)
    y = np.empty(qs.shape, np.float32)
    lib().or_q8_0_dequantize(_ptr(qs), _ptr(d), qs.size, _ptr(y))
    return y


def kv8_quantize(x):
    """FNFL's group-64 rule (kv_q8_ref.cpp:72-93) -> (codes, scales)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    codes = np.empty(x.shape, np.int8)
    sc = np.empty(x.shape[:-1] + (x.shape[-1] // 64,), np.uint16)
    lib().or_kv8_quantize(_ptr(x), x.size, _ptr(codes), _ptr(sc))
    return codes, sc


def to_block_q8_0(qs, d):
    """(codes [..., n], scales [..., n/32]) -> ggml block_q8_0 bytes (34 B a block: fp16 d, then 32 codes)."""
    qs = np.ascontiguousarray(qs, dtype=np.int8)
    d = np.ascontiguousarray(d, dtype=np.uint16)
    nb = d.size
    out = np.empty((nb, 34), np.uint8)
    out[:, 0:2] = d.reshape(nb, 1).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = qs.reshape(nb, 32).view(np.uint8)
    return out


def from_block_q8_0(blocks):
    """ggml block_q8_0 bytes [nb, 34] -> (codes [nb*32], scales [nb])."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 34)
    d = b[:, 0:2].copy().view(np.uint16).reshape(-1)
    qs = b[:, 2:].copy().view(np.int8).reshape(-1)
    return qs, d


# ---- page book ----

class Pages:
    """kv_pages (kv_pool.cpp:85-144)."""

    def __init__(self, n_slots, n_pages):
        self.h = lib().or_pages_new(n_slots, n_pages)
        self.n_pages = n_pages

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_pages_free(self.h)
            self.h = None

    def free_pages(self):
        return lib().or_pages_free_count(self.h)

    def mapped(self, slot):
        return lib().or_pages_mapped(self.h, slot)

    def physical(self, slot, logical):
        return lib().or_pages_physical(self.h, slot, logical)

    @staticmethod
    def pages_for(cells, page_cells, n_pages):
        return lib().or_pages_for(cells, page_cells, n_pages)

    def take(self, slot, want):
        buf = np.zeros(max(1, self.n_pages), np.int32)
        n = np.zeros(1, np.int32)
        ok = lib().or_pages_take(self.h, slot, want, _ptr(buf), _ptr(n))
        return bool(ok), buf[: n[0]].tolist()

    def give(self, slot, keep):
        buf = np.zeros(max(1, self.n_pages), np.int32)
        n = np.zeros(1, np.int32)
        lib().or_pages_give(self.h, slot, keep, _ptr(buf), _ptr(n))
        return buf[: n[0]].tolist()

    def table(self, slot):
        return [self.physical(slot, i) for i in range(self.mapped(slot))]


def reclaim_victim(views, for_slot):
    """kv_reclaim_victim (kv_pool.cpp:146-158); views: list of (active, pages, released)."""
    n = len(views)
    act = np.array([1 if v[0] else 0 for v in views], np.uint8)
    pg = np.array([v[1] for v in views], np.int32)
    rel = np.array([v[2] for v in views], np.uint64)
    return lib().or_reclaim_victim(_ptr(act), _ptr(pg), _ptr(rel), n, for_slot)


# ---- attention ----

def attn_f64(q16, k, v, n_ctx, scale=1.0 / 16.0, rows=None, threads=1):
    """FP64 dense causal attention over the decoded cache (qa2_test.cpp:532-583 form).
    q16: uint16 [T][hq][d]; k, v: float32 [n_ctx][hkv][d]; -> float64 [len(rows)][hq][d]. threads > 1 spreads the
    (row, KV head) pairs over threads (the same bits)."""
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    T, hq, d = q16.shape
    hkv = k.shape[1]
    assert k.shape[0] >= n_ctx and v.shape == k.shape
    if rows is None:
        rows_a = None
        nr = T
    else:
        rows_a = np.ascontiguousarray(rows, dtype=np.int32)
        nr = rows_a.size
    out = np.empty((nr, hq, d), np.float64)
    lib().or_attn_f64_mt(_ptr(q16), _ptr(k), _ptr(v), n_ctx, T, hq, hkv, d, scale,
                         _ptr(rows_a) if rows_a is not None else None, nr, _ptr(out), max(1, int(threads)))
    return out


def attn_f64_cells(q16, k, v, cells, scale=1.0 / 16.0):
    """FP64 attention of each query row over its own list of cells (the QSA attention's math, attend.h:16-18:
    softmax_c(q . K[c] * scale) . V[c] over row t's selected cells). q16: uint16 [T][hq][d]; k, v: float32
    [n][hkv][d] (decoded cache); cells: T int arrays -> float64 [T][hq][d]. A float q16 is taken as the query's
    values themselves (an F32 or FP64 query)."""
    if np.asarray(q16).dtype.kind == "f":
        q = np.asarray(q16, np.float64)
    else:
        q = np.ascontiguousarray(q16, dtype=np.uint16).view(np.float16).astype(np.float64)
    T, hq, d = q.shape
    hkv = k.shape[1]
    G = hq // hkv
    out = np.empty((T, hq, d), np.float64)
    for t in range(T):
        c = np.asarray(cells[t], dtype=np.int64)
        kk = k[c].astype(np.float64)  # [n][hkv][d]
        vv = v[c].astype(np.float64)
        for g in range(hkv):  # the G query heads of KV head g at once: s [n][G]
            s = (kk[:, g, :] @ q[t, g * G:(g + 1) * G].T) * scale
            p = np.exp(s - s.max(axis=0))
            out[t, g * G:(g + 1) * G] = (p.T @ vv[:, g, :]) / p.sum(axis=0)[:, None]
    return out


def qsa_body(depth, T, seed, clustered=False):
    """A selection body in the reference's layout (qsa.h:77-81) for rows t at positions q = depth + t: K =
    min((q + 1) / 4, 512) distinct ascending 4-cell blocks among the row's whole blocks, then the tail cells
    4 ((q + 1) / 4) .. q. -> (uint32 words, int32 byte offsets [T + 1], the rows' cell lists)."""
    rng = np.random.default_rng([seed, 17])
    words, offsets, cells = [], [0], []
    for t in range(T):
        q = depth + t
        n_vis = (q + 1) // 4
        K = min(n_vis, 512)
        if clustered and n_vis > K:
            # a sink, a local window and a few runs, as selections tend to be
            runs = [np.arange(0, min(16, n_vis)), np.arange(max(0, n_vis - 64), n_vis)]
            while sum(r.size for r in runs) < 2 * K:
                s0 = int(rng.integers(0, n_vis))
                runs.append(np.arange(s0, min(n_vis, s0 + int(rng.integers(8, 64)))))
            pool = np.unique(np.concatenate(runs))
            blocks = np.sort(rng.choice(pool, size=min(K, pool.size), replace=False))
            if blocks.size < K:
                rest = np.setdiff1d(np.arange(n_vis), blocks)
                blocks = np.sort(np.concatenate([blocks, rng.choice(rest, K - blocks.size, replace=False)]))
        else:
            blocks = np.sort(rng.choice(n_vis, size=K, replace=False)) if K else np.zeros(0, np.int64)
        tail = np.arange(4 * n_vis, q + 1)
        row = [K, tail.size] + [int(b) for b in blocks] + [int(c) for c in tail]
        words += row
        offsets.append(offsets[-1] + 4 * len(row))
        cells.append(np.concatenate([(4 * blocks[:, None] + np.arange(4)[None, :]).reshape(-1), tail]))
    return np.array(words, np.uint32), np.array(offsets, np.int32), cells


def attn_ggml(q16, k_blocks, v_blocks, n_ctx, scale=1.0 / 16.0, q_as_q8=False, threads=1, hkv=2):
    """ggml-semantics CPU flash attention over contiguous block_q8_0 K/V [cells][hkv][d/32][34 B] (at least n_ctx
    cells) -> fp16 bits [T][hq][d]."""
    q16 = np.ascontiguousarray(q16, dtype=np.uint16)
    T, hq, d = q16.shape
    kb = np.ascontiguousarray(k_blocks, dtype=np.uint8)
    vb = np.ascontiguousarray(v_blocks, dtype=np.uint8)
    assert hkv > 0 and hq % hkv == 0 and kb.size >= n_ctx * hkv * (d // 32) * 34 and vb.size == kb.size
    out = np.empty((T, hq, d), np.uint16)
    lib().or_attn_ggml(_ptr(q16), _ptr(kb), _ptr(vb), n_ctx, T, hq, hkv, d, scale, 1 if q_as_q8 else 0,
                       threads, _ptr(out))
    return out


# ---- DA-TC: the draft block's dense F16 attention (fn/kernels/draft/draft.h:47-83) ----

N_ROT = 64
RMS_EPS = 1e-6


def imrope_plane(sector):
    """IMROPE's plane of rotation pair `sector` (fn/kernels/qsa/imrope.cuh:14-20: sections 11, 11, 10, 0
    interleaved): 1 (h) for sector % 3 == 1 below 33, 2 (w) for % 3 == 2 below 30, 0 (t) for % 3 == 0 below 33,
    else 3 (e)."""
    return (1 if sector % 3 == 1 and sector < 33 else 2 if sector % 3 == 2 and sector < 30
            else 0 if sector % 3 == 0 and sector < 33 else 3)


def theta_f32(pos4, i, ts):
    """Pair i's angle as the reference forms it (attend.cu:172-183; its checker draft_test.cpp:460-472): the plane's
    position times theta_scale, i times, as an F32 product chain."""
    th = np.float32(pos4[imrope_plane(i)])
    ts = np.float32(ts)
    for _ in range(i):
        th = np.float32(th * ts)
    return float(th)


def norm_rope_f64(x, w, pos4, ts):
    """FP64 of the pinned order (draft_test.cpp:474-489): rms_norm(x) * w over 256 values (eps 1e-6), then pair i
    (< 32) of dims (i, i + 32) rotated by theta_f32(pos4, i, ts)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    r = 1.0 / np.sqrt(np.dot(x, x) / x.size + RMS_EPS)
    y = x * r * w
    half = N_ROT // 2
    for i in range(half):
        th = theta_f32(pos4, i, ts)
        c, s = np.cos(th), np.sin(th)
        x0, x1 = y[i], y[i + half]
        y[i] = x0 * c - x1 * s
        y[i + half] = x0 * s + x1 * c
    return y


def act_quantize(x):
    """FNFL's int8 activation format (fn/quant/act_ref.cpp:8-29), in F32: per run of 32 values amax = max |x|,
    d = amax / 127, id = 127 / amax (0 when amax is 0), q = round-half-even(x id) clamped to [-127, 127] (NaN: 0),
    s = d * sum q. x: float32 [..., k] (k a multiple of 32) -> (codes int8 like x, scales float32 [..., k / 32, 2])."""
    x = np.ascontiguousarray(x, np.float32)
    runs = x.reshape(-1, 32)
    amax = np.fmax.reduce(np.abs(runs), axis=1, initial=np.float32(0.0)).astype(np.float32)  # NaN ignored, as fmax
    with np.errstate(divide="ignore", invalid="ignore"):
        d = (amax / np.float32(127.0)).astype(np.float32)
        idv = np.where(amax > 0, np.float32(127.0) / np.where(amax > 0, amax, np.float32(1.0)),
                       np.float32(0.0)).astype(np.float32)
        e = (runs * idv[:, None]).astype(np.float32)
    q = np.clip(np.rint(e), -127, 127)
    q = np.where(np.isnan(e), 0, q).astype(np.int32)
    s = (d * q.sum(axis=1).astype(np.float32)).astype(np.float32)
    codes = q.astype(np.int8).reshape(x.shape)
    scales = np.stack([d, s], axis=1).reshape(x.shape[:-1] + (x.shape[-1] // 32, 2))
    return codes, scales


def datc_cells(n_before, row0, body=None):
    """The cells DA-TC's row row0 attends, in the kernel's logical order (draft.h:228-233, datc.cu:268-283): dense,
    0 .. n_before + row0; SP2, the body's K blocks' cells (4 b .. 4 b + 3, in body order), then 4 (N / 4) .. N + row0
    (N = n_before)."""
    n = n_before + row0 + 1
    if body is None:
        return np.arange(n, dtype=np.int64)
    body = np.asarray(body, np.int64)
    K = int(body[0])
    n_vis = n_before // 4
    blocks = body[2:2 + K]
    return np.concatenate([(4 * blocks[:, None] + np.arange(4)[None, :]).reshape(-1),
                           np.arange(4 * n_vis, n, dtype=np.int64)])


def datc_attn_f64(q16, gate, k_cache, v_cache, cells, chunk=16384):
    """FP64 attention of one DA-TC row over the listed cells of the F16 caches, gated (draft_test.cpp:682-709 form):
    q = 16 * q16 (exact), s_c = q . K[c] / 16, o = softmax(s) V, out = o / (1 + exp(-gate)).
    q16: uint16 [12][256]; gate: float32 [12][256]; k_cache, v_cache: uint16 [cells][256] -> float64 [12][256].
    The cells are taken `chunk` at a time (scores first, then the weighted rows), bounding the fp64 copies."""
    q = np.ascontiguousarray(q16, np.uint16).view(np.float16).astype(np.float64) * 16.0
    c = np.asarray(cells, np.int64)
    kc = np.ascontiguousarray(k_cache, np.uint16)
    vc = np.ascontiguousarray(v_cache, np.uint16)
    s = np.concatenate([(q @ kc[c[i:i + chunk]].view(np.float16).astype(np.float64).T) / 16.0
                        for i in range(0, c.size, chunk)], axis=1)  # [12][n]
    p = np.exp(s - s.max(axis=1, keepdims=True))
    o = np.zeros((q.shape[0], kc.shape[1]), np.float64)
    for i in range(0, c.size, chunk):
        o += p[:, i:i + chunk] @ vc[c[i:i + chunk]].view(np.float16).astype(np.float64)
    o /= p.sum(axis=1, keepdims=True)
    return o / (1.0 + np.exp(-np.asarray(gate, np.float64)))


def norm_err(ref, got):
    """max |got - ref| / max |ref| (draft_test.cpp:143-151; NaN counts as infinite)."""
    ref = np.asarray(ref, np.float64)
    got = np.asarray(got, np.float64)
    e = np.abs(got - ref)
    if np.isnan(e).any():
        return float("inf")
    rmax = np.abs(ref).max()
    return float(e.max() / rmax) if rmax > 0 else float(e.max())

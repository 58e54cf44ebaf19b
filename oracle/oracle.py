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

def attn_f64(q16, k, v, n_ctx, scale=1.0 / 16.0, rows=None):
    """FP64 dense causal attention over the decoded cache (qa2_test.cpp:532-583 form).
    q16: uint16 [T][hq][d]; k, v: float32 [n_ctx][hkv][d]; -> float64 [len(rows)][hq][d]."""
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
    lib().or_attn_f64(_ptr(q16), _ptr(k), _ptr(v), n_ctx, T, hq, hkv, d, scale,
                      _ptr(rows_a) if rows_a is not None else None, nr, _ptr(out))
    return out


def attn_f64_cells(q16, k, v, cells, scale=1.0 / 16.0):
    """FP64 attention of each query row over its own list of cells (the QSA attention's math, attend.h:16-18:
    softmax_c(q . K[c] * scale) . V[c] over row t's selected cells). q16: uint16 [T][hq][d]; k, v: float32
    [n][hkv][d] (decoded cache); cells: T int arrays -> float64 [T][hq][d]."""
    q = np.ascontiguousarray(q16, dtype=np.uint16).view(np.float16).astype(np.float64)
    T, hq, d = q.shape
    hkv = k.shape[1]
    G = hq // hkv
    out = np.empty((T, hq, d), np.float64)
    for t in range(T):
        c = np.asarray(cells[t], dtype=np.int64)
        kk = k[c].astype(np.float64)  # [n][hkv][d]
        vv = v[c].astype(np.float64)
        for h in range(hq):
            s = (kk[:, h // G, :] @ q[t, h]) * scale
            p = np.exp(s - s.max())
            out[t, h] = (p @ vv[:, h // G, :]) / p.sum()
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

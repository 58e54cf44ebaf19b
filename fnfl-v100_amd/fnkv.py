"""Python view of libfnkv.so (include/fnkv.h) through ctypes.

This is plumbing for the tests and the bench: the product is the HIP library; device buffers are torch tensors on
the GPU, passed by their data pointers, and streams are torch's current stream. Loading fails loudly when the
library was not built; there is no CPU fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# FNKV_LIB_PATH: another build of the library (for side-by-side measurement)
LIB_PATH = os.environ.get("FNKV_LIB_PATH", os.path.join(HERE, "libfnkv.so"))

OK, ERR_ARG, ERR_CAPACITY, ERR_HIP = 0, 1, 2, 3
F16, F32 = 0, 1
FMT_Q8_0, FMT_KV8 = 0, 1
PAGE_TOKENS = 256
HEAD_DIM = 256
EXPORTS = [
    "fnkv_last_error", "fnkv_pages_for", "fnkv_reclaim_victim", "fnkv_pool_create", "fnkv_pool_destroy",
    "fnkv_pool_ensure", "fnkv_pool_trim", "fnkv_pool_mapped_cells", "fnkv_pool_free_pages", "fnkv_pool_n_pages",
    "fnkv_pool_mapped_pages", "fnkv_pool_physical", "fnkv_page_table", "fnkv_pool_ledger", "fnkv_pool_test_fail",
    "fnkv_page_block_bytes", "fnkv_pool_device_base", "fnkv_pool_device_bytes", "fnkv_q8_append",
    "fnkv_export_q8_0", "fnkv_decode_workspace_bytes", "fnkv_attn_decode", "fnkv_prefill_workspace_bytes",
    "fnkv_attn_prefill", "fnkv_pool_create_fmt", "fnkv_pool_format", "fnkv_export_kv8",
    "fnkv_sparse_workspace_bytes", "fnkv_attn_sparse", "fnkv_rope_theta_scale", "fnkv_datc_part_bytes",
    "fnkv_datc_prepare", "fnkv_datc_attend", "fnkv_datc_step", "fnkv_qsa_workspace_bytes", "fnkv_qsa_attend",
    "fnkv_attn_decode_dev", "fnkv_attn_sparse_dev", "fnkv_attend_workspace_bytes", "fnkv_attend",
    "fnkv_attend_lanes", "fnkv_attn_decode_noalloc", "fnkv_qsp_kv", "fnkv_qsp_workspace_bytes", "fnkv_qsp_attend",
    "fnkv_test_decode_fold",
]
QSP_MAX_ROWS = 4096
SLAB_ROWS, ROW_WORDS = 128, 517
DEV_ERR_DEPTH = 2
MAX_LANES = 4
DATC_HEADS = 12
DATC_QSTRIDE = 512
DEV_ERR_DRAFT_DEPTH = 1 << 24

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64

_lib = None


class SlotView(ctypes.Structure):
    _fields_ = [("active", I32), ("pages", I32), ("released", ctypes.c_uint64)]


class DatcPrepareArgs(ctypes.Structure):
    """fnkv_datc_prepare_args (include/fnkv.h)"""
    _fields_ = [("qfull", P), ("kv_k", P), ("kv_v", P), ("q_norm", P), ("k_norm", P), ("n_before", P), ("pos", P),
                ("stride", P), ("row0", I32), ("theta_scale", ctypes.c_float), ("k_cache", P), ("v_cache", P),
                ("max_cells", I32), ("q16", P), ("q_f32", P), ("k_f32", P), ("err", P)]


class DatcAttendArgs(ctypes.Structure):
    """fnkv_datc_attend_args (include/fnkv.h)"""
    _fields_ = [("q16", P), ("qfull", P), ("k_cache", P), ("v_cache", P), ("n_before", P), ("row0", I32),
                ("max_cells", I32), ("part", P), ("out", P), ("codes", P), ("scales", P), ("err", P), ("body", P)]


class AttendArgs(ctypes.Structure):
    """fnkv_attend_args (include/fnkv.h)"""
    _fields_ = [("pool", P), ("slot", I32), ("layer", I32), ("hq", I32), ("qfull", P), ("kv_k", P), ("kv_v", P),
                ("q_norm", P), ("k_norm", P), ("body", P), ("offsets", P), ("pos", P), ("depth", P),
                ("max_cells", I32), ("theta_scale", ctypes.c_float), ("out", P), ("codes", P), ("scales", P),
                ("q_f32", P), ("k_f32", P), ("ws", P), ("ws_bytes", I64), ("err", P)]


class QspKvArgs(ctypes.Structure):
    """fnkv_qsp_kv_args (include/fnkv.h)"""
    _fields_ = [("pool", P), ("slot", I32), ("layer", I32), ("kv_k", P), ("kv_v", P), ("k_norm", P), ("rows", I32),
                ("pos0", I32), ("rope_off", I32), ("planes", P), ("theta_scale", ctypes.c_float)]


class QspAttendArgs(ctypes.Structure):
    """fnkv_qsp_attend_args (include/fnkv.h)"""
    _fields_ = [("pool", P), ("slot", I32), ("layer", I32), ("hq", I32), ("qfull", P), ("q_norm", P), ("body", P),
                ("offsets", P), ("rows", I32), ("pos0", I32), ("out", P), ("out16", P), ("err", P),
                ("rope_off", I32), ("planes", P), ("theta_scale", ctypes.c_float), ("ws", P), ("ws_bytes", I64)]


class FnkvError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"fnkv error {code}: {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() first")
        L = ctypes.CDLL(LIB_PATH)
        L.fnkv_last_error.restype = ctypes.c_char_p
        L.fnkv_pages_for.restype = I32
        L.fnkv_pages_for.argtypes = [I64, I32, I32]
        L.fnkv_reclaim_victim.restype = I32
        L.fnkv_reclaim_victim.argtypes = [P, I32, I32]
        L.fnkv_pool_create.restype = ctypes.c_int
        L.fnkv_pool_create.argtypes = [I32, I32, I32, I32, I32, I64, I32, ctypes.POINTER(P)]
        L.fnkv_pool_create_fmt.restype = ctypes.c_int
        L.fnkv_pool_create_fmt.argtypes = [I32, I32, I32, I32, I32, I64, I32, I32, ctypes.POINTER(P)]
        L.fnkv_pool_format.restype = I32
        L.fnkv_pool_format.argtypes = [P]
        L.fnkv_pool_destroy.argtypes = [P]
        L.fnkv_pool_ensure.restype = ctypes.c_int
        L.fnkv_pool_ensure.argtypes = [P, I32, I64, ctypes.POINTER(I32)]
        L.fnkv_pool_trim.restype = ctypes.c_int
        L.fnkv_pool_trim.argtypes = [P, I32, I64]
        L.fnkv_pool_mapped_cells.restype = I64
        L.fnkv_pool_mapped_cells.argtypes = [P, I32]
        for n in ("fnkv_pool_free_pages", "fnkv_pool_n_pages"):
            getattr(L, n).restype = I32
            getattr(L, n).argtypes = [P]
        L.fnkv_pool_mapped_pages.restype = I32
        L.fnkv_pool_mapped_pages.argtypes = [P, I32]
        L.fnkv_pool_physical.restype = I32
        L.fnkv_pool_physical.argtypes = [P, I32, I32]
        L.fnkv_page_table.restype = I32
        L.fnkv_page_table.argtypes = [P, I32, P, I32]
        L.fnkv_pool_ledger.restype = I32
        L.fnkv_pool_ledger.argtypes = [P, ctypes.c_char_p, I32]
        L.fnkv_pool_test_fail.argtypes = [P, I32]
        L.fnkv_page_block_bytes.restype = I64
        L.fnkv_pool_device_base.restype = P
        L.fnkv_pool_device_base.argtypes = [P]
        L.fnkv_pool_device_bytes.restype = I64
        L.fnkv_pool_device_bytes.argtypes = [P]
        L.fnkv_q8_append.restype = ctypes.c_int
        L.fnkv_q8_append.argtypes = [P, I32, I32, I64, I32, P, P, I32, P]
        L.fnkv_export_q8_0.restype = ctypes.c_int
        L.fnkv_export_q8_0.argtypes = [P, I32, I32, I32, I32, I64, I32, P, P]
        L.fnkv_export_kv8.restype = ctypes.c_int
        L.fnkv_export_kv8.argtypes = [P, I32, I32, I32, I32, I64, I32, P, P, P]
        if hasattr(L, "fnkv_test_decode_fold"):  # absent from builds of the library that predate it
            L.fnkv_test_decode_fold.restype = None
            L.fnkv_test_decode_fold.argtypes = [I32, I64]
        L.fnkv_decode_workspace_bytes.restype = I64
        L.fnkv_decode_workspace_bytes.argtypes = [P, I32, P, I32, I32]
        L.fnkv_attn_decode.restype = ctypes.c_int
        L.fnkv_attn_decode.argtypes = [P, I32, P, P, I32, I32, I32, ctypes.c_float, P, P, P, I32, P, P, I64, P]
        L.fnkv_sparse_workspace_bytes.restype = I64
        L.fnkv_sparse_workspace_bytes.argtypes = [P, I64, I32, I32]
        L.fnkv_attn_sparse.restype = ctypes.c_int
        L.fnkv_attn_sparse.argtypes = [P, I32, I64, I32, I32, I32, ctypes.c_float, P, P, P, P, P, I32, P, P, I64, P]
        L.fnkv_prefill_workspace_bytes.restype = I64
        L.fnkv_prefill_workspace_bytes.argtypes = [P, I64, I32, I32]
        L.fnkv_attn_prefill.restype = ctypes.c_int
        L.fnkv_attn_prefill.argtypes = [P, I32, I32, I64, I32, I32, ctypes.c_float, P, P, P, I64, P]
        L.fnkv_qsa_workspace_bytes.restype = I64
        L.fnkv_qsa_workspace_bytes.argtypes = [P, I64, I32, I32]
        L.fnkv_qsa_attend.restype = ctypes.c_int
        L.fnkv_qsa_attend.argtypes = [P, I32, I64, I32, I32, I32, P, P, P, P, P, P, ctypes.c_float, P, P, P, P, P, P,
                                      P, P, I64, P]
        L.fnkv_attn_decode_dev.restype = ctypes.c_int
        L.fnkv_attn_decode_dev.argtypes = [P, I32, P, P, P, I32, I32, I32, ctypes.c_float, P, P, P, I32, P, P, I64, P,
                                           P]
        L.fnkv_attn_decode_noalloc.restype = ctypes.c_int
        L.fnkv_attn_decode_noalloc.argtypes = [P, I32, P, P, P, I32, I32, I32, ctypes.c_float, P, P, P, I32, P, P, P]
        L.fnkv_attn_sparse_dev.restype = ctypes.c_int
        L.fnkv_attn_sparse_dev.argtypes = [P, I32, P, I64, I32, I32, I32, ctypes.c_float, P, P, P, P, P, I32, P, P,
                                           I64, P, P]
        L.fnkv_attend_workspace_bytes.restype = I64
        L.fnkv_attend_workspace_bytes.argtypes = [P, I32, I32, I32]
        L.fnkv_attend.restype = ctypes.c_int
        L.fnkv_attend.argtypes = [I32, ctypes.POINTER(AttendArgs), P]
        L.fnkv_attend_lanes.restype = ctypes.c_int
        L.fnkv_attend_lanes.argtypes = [I32, I32, ctypes.POINTER(AttendArgs), P]
        L.fnkv_qsp_kv.restype = ctypes.c_int
        L.fnkv_qsp_kv.argtypes = [ctypes.POINTER(QspKvArgs), P]
        L.fnkv_qsp_workspace_bytes.restype = I64
        L.fnkv_qsp_workspace_bytes.argtypes = [P, I32, I32, I32]
        L.fnkv_qsp_attend.restype = ctypes.c_int
        L.fnkv_qsp_attend.argtypes = [ctypes.POINTER(QspAttendArgs), P]
        L.fnkv_rope_theta_scale.restype = ctypes.c_float
        L.fnkv_rope_theta_scale.argtypes = []
        L.fnkv_datc_part_bytes.restype = I64
        L.fnkv_datc_part_bytes.argtypes = []
        L.fnkv_datc_prepare.restype = ctypes.c_int
        L.fnkv_datc_prepare.argtypes = [I32, ctypes.POINTER(DatcPrepareArgs), P]
        L.fnkv_datc_attend.restype = ctypes.c_int
        L.fnkv_datc_attend.argtypes = [ctypes.POINTER(DatcAttendArgs), P]
        L.fnkv_datc_step.restype = ctypes.c_int
        L.fnkv_datc_step.argtypes = [ctypes.POINTER(DatcPrepareArgs), ctypes.POINTER(DatcAttendArgs), P]
        _lib = L
    return _lib


def last_error():
    return lib().fnkv_last_error().decode()


def check(code):
    if code != OK:
        raise FnkvError(code, last_error())
    return code


def pages_for(cells, page_cells, n_pages):
    return lib().fnkv_pages_for(cells, page_cells, n_pages)


def reclaim_victim(views, for_slot):
    """views: list of (active, pages, released)"""
    arr = (SlotView * max(1, len(views)))()
    for i, (a, p, r) in enumerate(views):
        arr[i].active, arr[i].pages, arr[i].released = int(bool(a)), p, r
    return lib().fnkv_reclaim_victim(ctypes.cast(arr, P), len(views), for_slot)


def _stream(stream):
    if stream is not None:
        return P(stream)
    import torch
    return P(torch.cuda.current_stream().cuda_stream)


def _i32_array(xs):
    a = (I32 * len(xs))(*[int(x) for x in xs])
    return ctypes.cast(a, P), a


def _i64_array(xs):
    a = (I64 * len(xs))(*[int(x) for x in xs])
    return ctypes.cast(a, P), a


class Pool:
    """The page pool (kv_pool.h:63-138) and the kernels that read and write it."""

    def __init__(self, n_slots, n_pages, layers, h_kv, slot_tokens=0, device=0, page_tokens=PAGE_TOKENS,
                 fmt=FMT_Q8_0):
        h = P()
        check(lib().fnkv_pool_create_fmt(n_slots, n_pages, page_tokens, layers, h_kv, slot_tokens, fmt, device,
                                         ctypes.byref(h)))
        self.h = h
        self.fmt = fmt
        self.n_slots, self.n_pages, self.layers, self.h_kv = n_slots, n_pages, layers, h_kv

    def close(self):
        if getattr(self, "h", None):
            lib().fnkv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- book ----
    def ensure(self, slot, cells):
        cap = I32(0)
        code = lib().fnkv_pool_ensure(self.h, slot, cells, ctypes.byref(cap))
        return code, bool(cap.value)

    def trim(self, slot, keep_cells):
        return lib().fnkv_pool_trim(self.h, slot, keep_cells)

    def mapped_cells(self, slot):
        return lib().fnkv_pool_mapped_cells(self.h, slot)

    def free_pages(self):
        return lib().fnkv_pool_free_pages(self.h)

    def mapped_pages(self, slot):
        return lib().fnkv_pool_mapped_pages(self.h, slot)

    def physical(self, slot, logical):
        return lib().fnkv_pool_physical(self.h, slot, logical)

    def table(self, slot):
        n = lib().fnkv_page_table(self.h, slot, None, 0)
        ptr, arr = _i32_array([0] * max(1, n))
        lib().fnkv_page_table(self.h, slot, ptr, n)
        return list(arr[:n])

    def ledger(self):
        buf = ctypes.create_string_buffer(4096)
        lib().fnkv_pool_ledger(self.h, buf, 4096)
        return buf.value.decode().splitlines()

    def test_fail(self, after):
        lib().fnkv_pool_test_fail(self.h, after)

    def device_bytes(self):
        return lib().fnkv_pool_device_bytes(self.h)

    # ---- kernels (torch device tensors) ----
    def append(self, slot, layer, pos0, k, v, stream=None):
        """k, v: [rows][h_kv][256] fp16 or fp32 device tensors."""
        import torch
        assert k.shape == v.shape and k.dtype == v.dtype and k.is_contiguous() and v.is_contiguous()
        dt = F32 if k.dtype == torch.float32 else F16
        return check(lib().fnkv_q8_append(self.h, slot, layer, pos0, k.shape[0], P(k.data_ptr()),
                                          P(v.data_ptr()), dt, _stream(stream)))

    def export(self, slot, layer, head, kv, tok0, n_tok, out=None, stream=None):
        """-> uint8 device tensor [n_tok][8][34] of ggml block_q8_0."""
        import torch
        if out is None:
            out = torch.empty((n_tok, 8, 34), dtype=torch.uint8, device="cuda")
        check(lib().fnkv_export_q8_0(self.h, slot, layer, head, kv, tok0, n_tok, P(out.data_ptr()),
                                     _stream(stream)))
        return out

    def export_kv8(self, slot, layer, head, kv, tok0, n_tok, stream=None):
        """KV8 pool -> (int8 codes [n_tok][256], uint16 group scales [n_tok][4]) device tensors."""
        import torch
        codes = torch.empty((n_tok, HEAD_DIM), dtype=torch.int8, device="cuda")
        scales = torch.empty((n_tok, HEAD_DIM // 64), dtype=torch.int16, device="cuda")
        check(lib().fnkv_export_kv8(self.h, slot, layer, head, kv, tok0, n_tok, P(codes.data_ptr()),
                                    P(scales.data_ptr()), _stream(stream)))
        return codes, scales

    def decode_ws_bytes(self, ctx, T, hq):
        ptr, keep = _i64_array(ctx)
        return lib().fnkv_decode_workspace_bytes(self.h, len(ctx), ptr, T, hq)

    def decode(self, slots, ctx, T, layer, q, out, ws, scale=1.0 / 16.0, k_new=None, v_new=None, stream=None):
        """q, out: fp16 [n_seq][T][hq][256]; ws: a device tensor of at least decode_ws_bytes bytes; k_new, v_new
        (optional): the step's new cells [n_seq][T][h_kv][256], appended by the launch."""
        import torch
        sp, k1 = _i32_array(slots)
        cp, k2 = _i64_array(ctx)
        hq = q.shape[2]
        kp = P(k_new.data_ptr()) if k_new is not None else None
        vp = P(v_new.data_ptr()) if v_new is not None else None
        dt = F32 if (k_new is not None and k_new.dtype == torch.float32) else F16
        return check(lib().fnkv_attn_decode(self.h, len(slots), sp, cp, T, layer, hq, scale, P(q.data_ptr()), kp, vp,
                                            dt, P(out.data_ptr()), P(ws.data_ptr()), ws.numel() * ws.element_size(),
                                            _stream(stream)))

    def decode_dev(self, slots, ctx_dev, max_ctx, T, layer, q, out, ws, err, scale=1.0 / 16.0, k_new=None,
                   v_new=None, stream=None):
        """fnkv_attn_decode_dev: ctx_dev an int64 device tensor [n_seq] read by the launch, max_ctx the host bounds
        (the workspace: decode_ws_bytes(max_ctx, T, hq)), err an int32 device word (caller-cleared)."""
        import torch
        sp, k1 = _i32_array(slots)
        mp, k2 = _i64_array(max_ctx)
        kp = P(k_new.data_ptr()) if k_new is not None else None
        vp = P(v_new.data_ptr()) if v_new is not None else None
        dt = F32 if (k_new is not None and k_new.dtype == torch.float32) else F16
        return check(lib().fnkv_attn_decode_dev(self.h, len(slots), sp, _p(ctx_dev), mp, T, layer, q.shape[2], scale,
                                                P(q.data_ptr()), kp, vp, dt, P(out.data_ptr()), P(ws.data_ptr()),
                                                ws.numel() * ws.element_size(), _p(err), _stream(stream)))

    def decode_noalloc(self, slots, ctx_dev, max_ctx, T, layer, q, out, err, scale=1.0 / 16.0, k_new=None,
                       v_new=None, stream=None):
        """fnkv_attn_decode_noalloc: decode_dev without a workspace (the library's fixed device scratch)."""
        import torch
        sp, k1 = _i32_array(slots)
        mp, k2 = _i64_array(max_ctx)
        kp = P(k_new.data_ptr()) if k_new is not None else None
        vp = P(v_new.data_ptr()) if v_new is not None else None
        dt = F32 if (k_new is not None and k_new.dtype == torch.float32) else F16
        return check(lib().fnkv_attn_decode_noalloc(self.h, len(slots), sp, _p(ctx_dev), mp, T, layer, q.shape[2],
                                                    scale, P(q.data_ptr()), kp, vp, dt, P(out.data_ptr()), _p(err),
                                                    _stream(stream)))

    def sparse_dev(self, slot, depth_dev, max_cells, layer, q, body, offsets, out, ws, err, scale=1.0 / 16.0,
                   k_new=None, v_new=None, stream=None):
        """fnkv_attn_sparse_dev: depth_dev an int32 device word, max_cells the host bound on depth + T (the workspace:
        sparse_ws_bytes(max_cells - T, T, hq))."""
        import torch
        T, hq = q.shape[0], q.shape[1]
        kp = P(k_new.data_ptr()) if k_new is not None else None
        vp = P(v_new.data_ptr()) if v_new is not None else None
        dt = F32 if (k_new is not None and k_new.dtype == torch.float32) else F16
        return check(lib().fnkv_attn_sparse_dev(self.h, slot, _p(depth_dev), max_cells, T, layer, hq, scale,
                                                P(q.data_ptr()), P(body.data_ptr()), P(offsets.data_ptr()), kp, vp,
                                                dt, P(out.data_ptr()), P(ws.data_ptr()),
                                                ws.numel() * ws.element_size(), _p(err), _stream(stream)))

    def attend_ws_bytes(self, max_cells, rows, hq):
        return lib().fnkv_attend_workspace_bytes(self.h, max_cells, rows, hq)

    def attend_args(self, slot, layer, depth_dev, max_cells, qfull, kv_k, kv_v, q_norm, k_norm, pos, body, offsets,
                    out, codes, scales, ws, err, q_f32=None, k_f32=None, theta_scale=None):
        """fnkv_attend_args for this pool (device tensors; depth_dev an int32 device word)."""
        a = AttendArgs(self.h, slot, layer, qfull.shape[1], _p(qfull), _p(kv_k), _p(kv_v), _p(q_norm), _p(k_norm),
                       _p(body), _p(offsets), _p(pos), _p(depth_dev), max_cells,
                       rope_theta_scale() if theta_scale is None else theta_scale, _p(out), _p(codes), _p(scales),
                       _p(q_f32), _p(k_f32), _p(ws), ws.numel() * ws.element_size(), _p(err))
        a._keep = (qfull, kv_k, kv_v, q_norm, k_norm, pos, body, offsets, out, codes, scales, ws, err, q_f32, k_f32,
                   depth_dev)
        return a

    def qsp_kv(self, slot, layer, pos0, kv_k, kv_v, k_norm, planes=None, rope_off=0, stream=None):
        """qsp_kv: kv_k, kv_v F32 [rows][h_kv][256] device tensors, planes int32 [rows][4] or None."""
        a = QspKvArgs(self.h, slot, layer, _p(kv_k), _p(kv_v), _p(k_norm), kv_k.shape[0], pos0, rope_off,
                      _p(planes), rope_theta_scale())
        return check(lib().fnkv_qsp_kv(ctypes.byref(a), _stream(stream)))

    def qsp_ws_bytes(self, pos0, rows, hq):
        return lib().fnkv_qsp_workspace_bytes(self.h, pos0, rows, hq)

    def qsp_attend(self, slot, layer, pos0, qfull, q_norm, body, offsets, out16, out=None, err=None, planes=None,
                   rope_off=0, ws=None, stream=None):
        """qsp_attend: qfull F32 [rows][hq][512], body / offsets the slab layout (int32 device tensors), out16
        fp16 [rows][hq][256], out F32 (optional), err int32 [1] (optional)."""
        import torch
        rows, hq = qfull.shape[0], qfull.shape[1]
        if ws is None:
            ws = torch.empty(max(16, self.qsp_ws_bytes(pos0, rows, hq)), dtype=torch.uint8, device=qfull.device)
        a = QspAttendArgs(self.h, slot, layer, hq, _p(qfull), _p(q_norm), _p(body), _p(offsets), rows, pos0,
                          _p(out), _p(out16), _p(err), rope_off, _p(planes), rope_theta_scale(), _p(ws),
                          ws.numel() * ws.element_size())
        return check(lib().fnkv_qsp_attend(ctypes.byref(a), _stream(stream)))

    def sparse_ws_bytes(self, depth, T, hq):
        return lib().fnkv_sparse_workspace_bytes(self.h, depth, T, hq)

    def sparse(self, slot, depth, layer, q, body, offsets, out, ws=None, scale=1.0 / 16.0, k_new=None, v_new=None,
               stream=None):
        """QSA attention: q, out fp16 [T][hq][256]; body int32/uint32 device words, offsets int32 device [T + 1]
        (qsa.h layout); k_new, v_new (optional) [T][h_kv][256]: the rows' own cells."""
        import torch
        T, hq = q.shape[0], q.shape[1]
        if ws is None:
            ws = torch.empty(max(16, self.sparse_ws_bytes(depth, T, hq)), dtype=torch.uint8, device=q.device)
        kp = P(k_new.data_ptr()) if k_new is not None else None
        vp = P(v_new.data_ptr()) if v_new is not None else None
        dt = F32 if (k_new is not None and k_new.dtype == torch.float32) else F16
        return check(lib().fnkv_attn_sparse(self.h, slot, depth, T, layer, hq, scale, P(q.data_ptr()),
                                            P(body.data_ptr()), P(offsets.data_ptr()), kp, vp, dt,
                                            P(out.data_ptr()), P(ws.data_ptr()), ws.numel() * ws.element_size(),
                                            _stream(stream)))

    def qsa_ws_bytes(self, depth, T, hq):
        return lib().fnkv_qsa_workspace_bytes(self.h, depth, T, hq)

    def qsa_attend(self, slot, depth, layer, qfull, kv_k, kv_v, q_norm, k_norm, pos, body, offsets, out, codes,
                   scales, q_f32=None, k_f32=None, theta_scale=None, ws=None, stream=None):
        """attn::attend over the pool: qfull F32 [T][hq][512], kv_k / kv_v F32 [T][h_kv][256], pos int32 [4][T],
        body / offsets as for sparse(); out F32 [T][hq][256], codes int8 [T][hq * 256], scales F32 [T][hq * 8][2]."""
        import torch
        T, hq = qfull.shape[0], qfull.shape[1]
        if ws is None:
            ws = torch.empty(max(16, self.qsa_ws_bytes(depth, T, hq)), dtype=torch.uint8, device=qfull.device)
        ts = rope_theta_scale() if theta_scale is None else theta_scale
        return check(lib().fnkv_qsa_attend(self.h, slot, depth, T, layer, hq, _p(qfull), _p(kv_k), _p(kv_v),
                                           _p(q_norm), _p(k_norm), _p(pos), ts, _p(body), _p(offsets), _p(out),
                                           _p(codes), _p(scales), _p(q_f32), _p(k_f32), _p(ws),
                                           ws.numel() * ws.element_size(), _stream(stream)))

    def prefill_ws_bytes(self, ctx, rows, hq):
        return lib().fnkv_prefill_workspace_bytes(self.h, ctx, rows, hq)

    def prefill(self, slot, layer, ctx, q, out, scale=1.0 / 16.0, stream=None, ws=None):
        """q, out: fp16 [rows][hq][256]: the chunk's queries at positions ctx - rows .. ctx - 1. ws: a device tensor
        of at least prefill_ws_bytes bytes (None: allocated here; False: none, one key split)."""
        import torch
        rows, hq = q.shape[0], q.shape[1]
        if ws is None:
            n = self.prefill_ws_bytes(ctx, rows, hq)
            ws = torch.empty(max(n, 16), dtype=torch.uint8, device=q.device) if n > 0 else False
        wp, wn = (P(ws.data_ptr()), ws.numel() * ws.element_size()) if ws is not False else (None, 0)
        return check(lib().fnkv_attn_prefill(self.h, slot, layer, ctx, rows, hq, scale, P(q.data_ptr()),
                                             P(out.data_ptr()), wp, wn, _stream(stream)))


# ---- DA-TC: the draft block's dense F16 attention (fn/kernels/draft/draft.h:47-83) ----

def _p(t):
    return P(t.data_ptr()) if t is not None else None


def rope_theta_scale():
    return lib().fnkv_rope_theta_scale()


def datc_part_bytes():
    return lib().fnkv_datc_part_bytes()


def datc_prepare(rows, *, kv_k, kv_v, k_norm, n_before, pos, stride, k_cache, v_cache, err, row0=0, qfull=None,
                 q_norm=None, q16=None, q_f32=None, k_f32=None, theta_scale=None, stream=None):
    """datc_prepare (draft.h:243): device tensors; n_before, stride int32 [1], pos int32 [4][stride] on the device."""
    a = DatcPrepareArgs(_p(qfull), _p(kv_k), _p(kv_v), _p(q_norm), _p(k_norm), _p(n_before), _p(pos), _p(stride),
                        row0, rope_theta_scale() if theta_scale is None else theta_scale, _p(k_cache), _p(v_cache),
                        k_cache.shape[0], _p(q16), _p(q_f32), _p(k_f32), _p(err))
    return check(lib().fnkv_datc_prepare(rows, ctypes.byref(a), _stream(stream)))


def datc_attend(*, q16, qfull, k_cache, v_cache, n_before, part, out, codes, scales, err, row0=0, body=None,
                max_cells=None, stream=None):
    """datc_attend (draft.h:244): q16 the row's [12][256] fp16, qfull the row's [12][512] fp32, out fp32 [3072],
    codes int8 [3072], scales fp32 [96][2]; body (SP2) a uint32/int32 device tensor or None."""
    a = DatcAttendArgs(_p(q16), _p(qfull), _p(k_cache), _p(v_cache), _p(n_before), row0,
                       k_cache.shape[0] if max_cells is None else max_cells, _p(part), _p(out), _p(codes),
                       _p(scales), _p(err), _p(body))
    return check(lib().fnkv_datc_attend(ctypes.byref(a), _stream(stream)))


def datc_step(*, kv_k, kv_v, k_norm, q_norm, qfull, n_before, pos, stride, k_cache, v_cache, q16, part, out, codes,
              scales, err, row0=0, q_f32=None, k_f32=None, body=None, theta_scale=None, stream=None):
    """fnkv_datc_step: the prepare of row row0 (q from qfull's row [12][512]) and its attention in one call."""
    p = DatcPrepareArgs(_p(qfull), _p(kv_k), _p(kv_v), _p(q_norm), _p(k_norm), _p(n_before), _p(pos), _p(stride),
                        row0, rope_theta_scale() if theta_scale is None else theta_scale, _p(k_cache), _p(v_cache),
                        k_cache.shape[0], _p(q16), _p(q_f32), _p(k_f32), _p(err))
    a = DatcAttendArgs(None, _p(qfull), _p(k_cache), _p(v_cache), _p(n_before), row0, k_cache.shape[0], _p(part),
                       _p(out), _p(codes), _p(scales), _p(err), _p(body))
    return check(lib().fnkv_datc_step(ctypes.byref(p), ctypes.byref(a), _stream(stream)))


def attend(rows, args, stream=None):
    """fnkv_attend (attn::attend with the device depth)"""
    return check(lib().fnkv_attend(rows, ctypes.byref(args), _stream(stream)))


def attend_lanes(rows, args_list, stream=None):
    """fnkv_attend_lanes over a list of AttendArgs"""
    arr = (AttendArgs * len(args_list))(*args_list)
    return check(lib().fnkv_attend_lanes(len(args_list), rows, arr, _stream(stream)))

"""ctypes binding of libqk.so (include/qk.h) for tests, smoke() and bench.py.

The product is the C ABI; this module only marshals arguments.  Entry points mirror the
reference's host glue (qwen_cuda/qwen.cpp:150-247): `matmul` (T<16 -> GEMV else GEMM),
`gemv_group` (MmGroup launch with optional GLU), `dequant_rows` (the k_dq selftest vehicle) and
`upload` (whole-tensor HtoD + repack).  A non-zero status raises QkError (the reference prints and
_Exit(1)s instead, qwen_cuda/cu.h:21-27).

Device buffers are passed as integer addresses (e.g. torch tensor .data_ptr()); streams as
integer hipStream_t handles (torch.cuda.current_stream().cuda_stream), 0 = default stream.
The library is loaded from this directory; a missing libqk.so is an error, never a fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqk.so")

T_F32, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K = 0, 8, 12, 13, 14
LAYOUT_GGUF, LAYOUT_T16 = 0, 1
ACT_F32, ACT_F16, ACT_F16_XPERM = 0, 1, 2
OK, E_NULL, E_TYPE, E_SHAPE, E_LAYOUT, E_ALIGN, E_HIP, E_GROUP, E_RANGE = 0, -1, -2, -3, -4, -5, -6, -7, -8
# bytes of one row's run of 256 weights (Q8_0: eight 34-byte blocks)
BLOCK_BYTES = {T_Q8_0: 272, T_Q4_K: 144, T_Q5_K: 176, T_Q6_K: 210}


class QkError(RuntimeError):
    def __init__(self, status, where):
        self.status = status
        super().__init__(f"{where}: status {status}")


class Weight(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("type", ctypes.c_uint32), ("k", ctypes.c_int32),
                ("n", ctypes.c_int32), ("rb", ctypes.c_uint64), ("layout", ctypes.c_uint32)]

    def __repr__(self):
        return (f"Weight(data=0x{self.data or 0:x}, type={self.type}, k={self.k}, n={self.n}, "
                f"rb={self.rb}, layout={self.layout})")


class GemvPlanInfo(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int32), ("work_groups", ctypes.c_int32), ("waves_per_group", ctypes.c_int32),
                ("ring_depth", ctypes.c_int32), ("slices", ctypes.c_int32), ("token_slots", ctypes.c_int32),
                ("lds_bytes", ctypes.c_int32)]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


GEMV_INT8, GEMV_GENERAL, GEMV_F32 = 1, 2, 3

_P = ctypes.c_void_p
_SIGS = {
    "qk_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "qk_row_bytes": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint64)]),
    "qk_weight_view": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint32,
                                      ctypes.POINTER(Weight)]),
    "qk_init_stream": (ctypes.c_int, [_P]),
    "qk_upload": (ctypes.c_int, [_P, ctypes.c_uint32, ctypes.c_int32, ctypes.c_int32, ctypes.c_uint32, _P,
                                 ctypes.POINTER(Weight)]),
    "qk_free": (ctypes.c_int, [ctypes.POINTER(Weight)]),
    "qk_repack": (ctypes.c_int, [ctypes.POINTER(Weight), _P, ctypes.c_uint32, _P, ctypes.POINTER(Weight)]),
    "qk_dequant_rows": (ctypes.c_int, [ctypes.POINTER(Weight), _P, ctypes.c_int32, _P, _P]),
    "qk_matmul": (ctypes.c_int, [ctypes.POINTER(Weight), _P, ctypes.c_int32, _P, _P]),
    "qk_matmul_noalloc": (ctypes.c_int, [ctypes.POINTER(Weight), _P, ctypes.c_int32, _P, _P]),
    "qk_embed": (ctypes.c_int, [ctypes.POINTER(Weight), _P, _P, _P, ctypes.c_int32, _P, _P]),
    "qk_matmul_act": (ctypes.c_int, [ctypes.POINTER(Weight), _P, ctypes.c_uint32, ctypes.c_int32, _P, _P]),
    "qk_gemv_group_act": (ctypes.c_int, [ctypes.POINTER(ctypes.POINTER(Weight)), ctypes.POINTER(_P), ctypes.c_int32,
                                         ctypes.c_int32, _P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int32, _P]),
    "qk_gemv_group": (ctypes.c_int, [ctypes.POINTER(ctypes.POINTER(Weight)), ctypes.POINTER(_P), ctypes.c_int32,
                                     ctypes.c_int32, _P, ctypes.c_int32, _P]),
    "qk_gemv_plan": (ctypes.c_int, [ctypes.POINTER(ctypes.POINTER(Weight)), ctypes.c_int32, ctypes.c_int32,
                                    ctypes.c_int32, ctypes.POINTER(GemvPlanInfo)]),
    "qk_set_tuning": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int32]),
    "qk_synth_fill": (ctypes.c_int, [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, _P, _P]),
    "qk_gguf_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "qk_gguf_close": (None, [_P]),
    "qk_gguf_tensor_count": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int64)]),
    "qk_gguf_tensor_info": (ctypes.c_int, [_P, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p),
                                           ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32),
                                           ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint64),
                                           ctypes.POINTER(ctypes.c_uint64)]),
    "qk_gguf_find": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "qk_gguf_kv_num": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "qk_gguf_kv_str": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p)]),
    "qk_gguf_upload": (ctypes.c_int, [_P, _P]),
    "qk_gguf_weight": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(Weight)]),
}


class Lib:
    """Thin checked wrapper around libqk.so."""

    def __init__(self, path=LIB_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        self.path = path
        self.lib = ctypes.CDLL(path)
        for name, (res, args) in _SIGS.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args

    # -- helpers -------------------------------------------------------------------------------
    def _check(self, rc, where):
        if rc != OK:
            raise QkError(rc, f"{where} ({self.status_string(rc)})")

    def status_string(self, rc):
        return self.lib.qk_status_string(rc).decode()

    # -- ABI -----------------------------------------------------------------------------------
    def row_bytes(self, typ, k):
        rb = ctypes.c_uint64()
        self._check(self.lib.qk_row_bytes(typ, k, ctypes.byref(rb)), "qk_row_bytes")
        return rb.value

    def weight_view(self, data, typ, k, n, layout):
        w = Weight()
        self._check(self.lib.qk_weight_view(data, typ, k, n, layout, ctypes.byref(w)), "qk_weight_view")
        return w

    def init_stream(self, stream=0):
        self._check(self.lib.qk_init_stream(stream), "qk_init_stream")

    def upload(self, host_bytes, typ, k, n, layout=LAYOUT_T16, stream=0):
        """host_bytes: a C-contiguous numpy uint8 array holding the tensor's GGUF bytes."""
        w = Weight()
        self._check(self.lib.qk_upload(host_bytes.ctypes.data, typ, k, n, layout, stream, ctypes.byref(w)),
                    "qk_upload")
        return w

    def free(self, w):
        self._check(self.lib.qk_free(ctypes.byref(w)), "qk_free")

    def repack(self, w, dst, layout, stream=0):
        out = Weight()
        self._check(self.lib.qk_repack(ctypes.byref(w), dst, layout, stream, ctypes.byref(out)), "qk_repack")
        return out

    def dequant_rows(self, w, rows_dev, nrows, out_dev, stream=0):
        self._check(self.lib.qk_dequant_rows(ctypes.byref(w), rows_dev, nrows, out_dev, stream), "qk_dequant_rows")

    def matmul(self, w, x_dev, m, y_dev, stream=0):
        self._check(self.lib.qk_matmul(ctypes.byref(w), x_dev, m, y_dev, stream), "qk_matmul")

    def matmul_noalloc(self, w, x_dev, m, y_dev, stream=0):
        self._check(self.lib.qk_matmul_noalloc(ctypes.byref(w), x_dev, m, y_dev, stream), "qk_matmul_noalloc")

    def gemv_group(self, ws, ys, glu, x_dev, m, stream=0):
        cnt = len(ws)
        warr = (ctypes.POINTER(Weight) * max(cnt, 1))(*[ctypes.pointer(w) for w in ws])
        yarr = (_P * max(len(ys), 1))(*ys)
        self._check(self.lib.qk_gemv_group(warr, yarr, cnt, 1 if glu else 0, x_dev, m, stream), "qk_gemv_group")

    def embed(self, table, tokens_dev, mask_dev, embd_dev, m, x_dev, stream=0):
        self._check(self.lib.qk_embed(ctypes.byref(table), tokens_dev, mask_dev or None, embd_dev or None, m, x_dev,
                                      stream), "qk_embed")

    def matmul_act(self, w, x_dev, xfmt, m, y_dev, stream=0):
        self._check(self.lib.qk_matmul_act(ctypes.byref(w), x_dev, xfmt, m, y_dev, stream), "qk_matmul_act")

    def gemv_group_act(self, ws, ys, glu, x_dev, xfmt, m, glu_yfmt=ACT_F32, stream=0):
        cnt = len(ws)
        warr = (ctypes.POINTER(Weight) * max(cnt, 1))(*[ctypes.pointer(w) for w in ws])
        yarr = (_P * max(len(ys), 1))(*ys)
        self._check(self.lib.qk_gemv_group_act(warr, yarr, cnt, 1 if glu else 0, x_dev, xfmt, glu_yfmt, m, stream),
                    "qk_gemv_group_act")

    def gemv_plan(self, ws, glu, m):
        """What qk_gemv_group would launch first (a dict of qk_gemv_plan_info)."""
        cnt = len(ws)
        warr = (ctypes.POINTER(Weight) * max(cnt, 1))(*[ctypes.pointer(w) for w in ws])
        info = GemvPlanInfo()
        self._check(self.lib.qk_gemv_plan(warr, cnt, 1 if glu else 0, m, ctypes.byref(info)), "qk_gemv_plan")
        return info.as_dict()

    def set_tuning(self, name, value):
        self._check(self.lib.qk_set_tuning(name.encode(), value), "qk_set_tuning")

    def synth_fill(self, typ, seed, block0, nblocks, dst, stream=0):
        self._check(self.lib.qk_synth_fill(typ, seed, block0, nblocks, dst, stream), "qk_synth_fill")

    # GGUF files (include/qk_gguf.h)
    def gguf_open(self, path):
        h = ctypes.c_void_p()
        self._check(self.lib.qk_gguf_open(os.fsencode(path), ctypes.byref(h)), "qk_gguf_open")
        return h.value

    def gguf_close(self, h):
        self.lib.qk_gguf_close(h)

    def gguf_tensors(self, h):
        """[(name, type, dims, file_offset, nbytes)] in file order."""
        n = ctypes.c_int64()
        self._check(self.lib.qk_gguf_tensor_count(h, ctypes.byref(n)), "qk_gguf_tensor_count")
        out = []
        for i in range(n.value):
            name, typ, nd = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_int32()
            dims, off, nb = (ctypes.c_int64 * 4)(), ctypes.c_uint64(), ctypes.c_uint64()
            self._check(self.lib.qk_gguf_tensor_info(h, i, ctypes.byref(name), ctypes.byref(typ), ctypes.byref(nd),
                                                     dims, ctypes.byref(off), ctypes.byref(nb)), "qk_gguf_tensor_info")
            out.append((name.value.decode(), typ.value, list(dims[:nd.value]), off.value, nb.value))
        return out

    def gguf_kv_num(self, h, key):
        v = ctypes.c_double()
        self._check(self.lib.qk_gguf_kv_num(h, key.encode(), ctypes.byref(v)), "qk_gguf_kv_num")
        return v.value

    def gguf_kv_str(self, h, key):
        v = ctypes.c_char_p()
        self._check(self.lib.qk_gguf_kv_str(h, key.encode(), ctypes.byref(v)), "qk_gguf_kv_str")
        return v.value.decode()

    def gguf_upload(self, h, stream=0):
        self._check(self.lib.qk_gguf_upload(h, stream), "qk_gguf_upload")

    def gguf_weight(self, h, name):
        w = Weight()
        self._check(self.lib.qk_gguf_weight(h, name.encode(), ctypes.byref(w)), "qk_gguf_weight")
        return w


def exported_symbols(header_paths):
    """Function names declared in the given C headers (for the export check)."""
    import re
    names = []
    for p in header_paths:
        text = open(p).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(qk_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))

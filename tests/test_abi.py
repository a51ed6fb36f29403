"""CPU tests of the C ABI (include/qk.h): the library loads, exports every declared entry point, and
rejects bad arguments with the documented status codes before it touches the GPU (the reference's
get_w / gemv checks, qwen_cuda/qwen.cpp:152-173, 220-238, which there end in _Exit(1))."""
import ctypes
import glob
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))

OK, E_NULL, E_TYPE, E_SHAPE, E_LAYOUT, E_ALIGN, E_HIP, E_GROUP, E_RANGE = 0, -1, -2, -3, -4, -5, -6, -7, -8
T_F32, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K = 0, 8, 12, 13, 14
GGUF, T16 = 0, 1
FAKE = 0x7F0000000000  # a 16-byte aligned address that is never dereferenced by these checks


def test_exports_every_declared_symbol(qkmod, qk):
    names = qkmod.exported_symbols(HEADERS)
    assert "qk_matmul" in names and "qk_gemv_group" in names and "qk_synth_fill" in names
    missing = [n for n in names if not hasattr(qk.lib, n)]
    assert not missing, f"declared in include/*.h but not exported: {missing}"


def test_status_strings(qk):
    for rc in (OK, E_NULL, E_TYPE, E_SHAPE, E_LAYOUT, E_ALIGN, E_HIP, E_GROUP, E_RANGE):
        assert qk.status_string(rc) not in ("", "unknown status")
    assert qk.status_string(12345) == "unknown status"


@pytest.mark.parametrize("typ,k,rb", [(T_Q4_K, 5120, 2880), (T_Q6_K, 17408, 14280), (T_Q6_K, 5120, 4200),
                                      (T_Q8_0, 64, 68), (T_F32, 10, 40), (T_Q5_K, 256, 176)])
def test_row_bytes(qk, typ, k, rb):
    """qwen_cpu/quants.h:21-31; at the configs: Q4_K 5120 -> 2880 B, Q6_K 17408 -> 14280 B."""
    assert qk.row_bytes(typ, k) == rb


def test_row_bytes_errors(qk):
    rb = ctypes.c_uint64()
    assert qk.lib.qk_row_bytes(T_Q4_K, 300, ctypes.byref(rb)) == E_SHAPE
    assert qk.lib.qk_row_bytes(T_Q4_K, 0, ctypes.byref(rb)) == E_SHAPE
    assert qk.lib.qk_row_bytes(99, 256, ctypes.byref(rb)) == E_TYPE
    assert qk.lib.qk_row_bytes(T_Q4_K, 256, None) == E_NULL


def _view(qkmod, qk, data, typ, k, n, layout):
    w = qkmod.Weight()
    return qk.lib.qk_weight_view(data, typ, k, n, layout, ctypes.byref(w)), w


def test_weight_view_validation(qkmod, qk):
    rc, w = _view(qkmod, qk, FAKE, T_Q4_K, 5120, 17408, T16)
    assert rc == OK and (w.k, w.n, w.rb, w.layout, w.type) == (5120, 17408, 2880, T16, T_Q4_K)
    assert _view(qkmod, qk, None, T_Q4_K, 512, 16, T16)[0] == E_NULL
    assert _view(qkmod, qk, FAKE, T_F32, 512, 16, T16)[0] == E_LAYOUT  # F32 is used as stored
    rc, w = _view(qkmod, qk, FAKE, T_F32, 512, 48, GGUF)
    assert rc == OK and w.rb == 2048
    rc, w = _view(qkmod, qk, FAKE, T_Q8_0, 512, 16, T16)
    assert rc == OK and w.rb == 544
    rc, w = _view(qkmod, qk, FAKE, T_Q5_K, 512, 16, T16)
    assert rc == OK and w.rb == 352
    assert _view(qkmod, qk, FAKE, T_Q4_K, 500, 16, T16)[0] == E_SHAPE
    assert _view(qkmod, qk, FAKE, T_Q4_K, 512, 0, GGUF)[0] == E_SHAPE
    assert _view(qkmod, qk, FAKE, T_Q4_K, 512, 24, T16)[0] == E_SHAPE  # T16 tiles need n % 16 == 0
    assert _view(qkmod, qk, FAKE, T_Q4_K, 512, 24, GGUF)[0] == OK
    assert _view(qkmod, qk, FAKE, T_Q6_K, 512, 16, 7)[0] == E_LAYOUT
    assert _view(qkmod, qk, FAKE + 4, T_Q6_K, 512, 16, T16)[0] == E_ALIGN
    assert qk.lib.qk_weight_view(FAKE, T_Q4_K, 512, 16, T16, None) == E_NULL


def test_matmul_validation(qkmod, qk):
    _, w = _view(qkmod, qk, FAKE, T_Q4_K, 512, 16, T16)
    _, wg = _view(qkmod, qk, FAKE, T_Q4_K, 512, 16, GGUF)
    m = qk.lib.qk_matmul
    assert m(ctypes.byref(w), None, 1, FAKE, None) == E_NULL
    assert m(ctypes.byref(w), FAKE, 1, None, None) == E_NULL
    assert m(None, FAKE, 1, FAKE, None) == E_NULL
    assert m(ctypes.byref(wg), FAKE, 1, FAKE, None) == E_LAYOUT  # kernels read the T16 layout
    assert m(ctypes.byref(w), FAKE, 0, FAKE, None) == E_SHAPE
    assert m(ctypes.byref(w), FAKE + 8, 1, FAKE, None) == E_ALIGN
    bad = qkmod.Weight(FAKE, T_Q4_K, 512, 16, 999, T16)  # rb inconsistent with type and k
    assert m(ctypes.byref(bad), FAKE, 1, FAKE, None) == E_SHAPE


def test_gemv_group_validation(qkmod, qk):
    _, a = _view(qkmod, qk, FAKE, T_Q4_K, 512, 32, T16)
    _, b = _view(qkmod, qk, FAKE, T_Q4_K, 512, 32, T16)
    _, c = _view(qkmod, qk, FAKE, T_Q4_K, 1024, 32, T16)
    _, d = _view(qkmod, qk, FAKE, T_Q4_K, 512, 48, T16)
    P = ctypes.POINTER(qkmod.Weight)
    g = qk.lib.qk_gemv_group

    def call(ws, glu=0, m=1, x=FAKE, ys=None):
        warr = (P * max(len(ws), 1))(*[ctypes.pointer(w) for w in ws])
        ys = ys if ys is not None else [FAKE] * max(len(ws), 1)
        yarr = (ctypes.c_void_p * len(ys))(*ys)
        return g(warr, yarr, len(ws), glu, x, m, None)

    assert call([]) == E_GROUP
    assert call([a, b, a, b, a]) == E_GROUP  # at most four matrices share x (kernels.cu:403-408)
    assert call([a], glu=1) == E_GROUP
    assert call([a, c]) == E_GROUP  # k must match
    assert call([a, d], glu=1) == E_GROUP  # gate/up must have equal n
    assert call([a], m=16) == E_SHAPE  # m >= 16 is the GEMM's range (qwen.cpp:240-247)
    assert call([a], m=0) == E_SHAPE
    assert call([a], x=None) == E_NULL
    assert call([a], x=FAKE + 4) == E_ALIGN
    assert call([a], ys=[FAKE + 4]) == E_ALIGN
    assert call([a], ys=[None]) == E_NULL


def test_tuning_names(qk):
    assert qk.lib.qk_set_tuning(b"no_such_knob", 1) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_waves", -1) == E_RANGE
    assert qk.lib.qk_set_tuning(None, 1) == E_NULL
    assert qk.lib.qk_set_tuning(b"gemv_waves", 0) == OK
    assert qk.lib.qk_set_tuning(b"gemm_pairs", 7) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemm_pairs", 9) == OK
    assert qk.lib.qk_set_tuning(b"gemm_pairs", 0) == OK
    assert qk.lib.qk_set_tuning(b"gemv_fused", 2) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_fused", 1) == OK
    assert qk.lib.qk_set_tuning(b"gemv_wpg", 3) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_wpg", 17) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_wpg", 0) == OK
    assert qk.lib.qk_set_tuning(b"gemm_map", 2) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemm_map", 0) == OK
    assert qk.lib.qk_set_tuning(b"gemm_map", 1) == OK
    assert qk.lib.qk_set_tuning(b"gemv_dshift", -1) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_dshift", 32) == E_RANGE
    assert qk.lib.qk_set_tuning(b"gemv_dshift", 1) == OK


def test_binding_fails_loudly_without_library(qkmod, tmp_path):
    with pytest.raises(RuntimeError, match="not built"):
        qkmod.Lib(str(tmp_path / "libqk.so"))

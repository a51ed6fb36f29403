"""ctypes binding of the test oracle (oracle/liboracle.so) and, when built, of the reference's own
CPU path (oracle/_ref/libqkref.so).  Test infrastructure: imported only by tests/, smoke() and
bench.py's cpu_baseline leg, always as the checker, never as the thing measured on the GPU.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liboracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "libqkref.so")

T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K = 8, 12, 13, 14
# bytes of one row's run of 256 weights (Q8_0: eight 34-byte blocks)
BLOCK_BYTES = {T_Q8_0: 272, T_Q4_K: 144, T_Q5_K: 176, T_Q6_K: 210}
SEED_BASE = 0x5EED0000000000C0  # seed = SEED_BASE | config id
# qk_matmul (any activation format), grouped launches and gate/up pairs run m < GEMM_ROUTE_M on the
# GEMV (fp32-level results) and m >= GEMM_ROUTE_M on the GEMM (fp16 operands)
GEMM_ROUTE_M = 5
GLU_GEMM_M = GEMM_ROUTE_M

_P = ctypes.c_void_p


def _ptr(a):
    return a.ctypes.data_as(_P)


def cpu_has_avx512():
    try:
        flags = open("/proc/cpuinfo").read()
    except OSError:
        return False
    need = ("avx512f", "avx512bw", "avx512dq", "avx512vl", "f16c", "fma")
    for line in flags.splitlines():
        if line.startswith("flags"):
            have = set(line.split(":", 1)[1].split())
            return all(n in have for n in need)
    return False


def _time_seq(fn, mats, xs, T, reps):
    """Shared marshalling of the C timing loops: mats = [(type, weight bytes, k, n)], xs[i] = [T][k]
    fp32 input of matmul i.  Returns elapsed seconds for `reps` passes over the sequence."""
    cnt = len(mats)
    ws = [np.ascontiguousarray(w) for _, w, _, _ in mats]
    xs = [np.ascontiguousarray(x, dtype=np.float32) for x in xs]
    ys = [np.zeros((T, n), np.float32) for _, _, _, n in mats]
    P = ctypes.c_void_p * cnt
    ns = fn(cnt, P(*[w.ctypes.data for w in ws]), (ctypes.c_uint32 * cnt)(*[t for t, _, _, _ in mats]),
            (ctypes.c_int * cnt)(*[k for _, _, k, _ in mats]), (ctypes.c_int * cnt)(*[n for _, _, _, n in mats]),
            P(*[x.ctypes.data for x in xs]), T, P(*[y.ctypes.data for y in ys]), reps)
    assert ns >= 0, "timing loop rejected a shape"
    return ns * 1e-9


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: run `make -C oracle`")
        L = self.lib = ctypes.CDLL(path)
        L.qko_fp16_to_f32.restype = ctypes.c_float
        L.qko_fp16_to_f32.argtypes = [ctypes.c_uint16]
        L.qko_f32_to_fp16.restype = ctypes.c_uint16
        L.qko_f32_to_fp16.argtypes = [ctypes.c_float]
        L.qko_row_bytes.restype = ctypes.c_ulonglong
        L.qko_row_bytes.argtypes = [ctypes.c_uint32, ctypes.c_longlong]
        L.qko_scale_min_k4.argtypes = [ctypes.c_int, _P, _P, _P]
        for f in (L.qko_dequant_row, L.qko_dequant_row_fast):
            f.restype = ctypes.c_int
            f.argtypes = [ctypes.c_uint32, _P, _P, ctypes.c_longlong]
        L.qko_init.argtypes = [ctypes.c_int]
        L.qko_matmul.argtypes = [_P, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int, _P, ctypes.c_int]
        L.qko_matmul_f64.argtypes = [_P, ctypes.c_uint32, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int, _P, _P]
        for f in (L.qko_fill_q4k, L.qko_fill_q6k, L.qko_fill_q5k, L.qko_fill_q8_0):
            f.restype = None
            f.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, _P]
        L.qko_time_seq.restype = ctypes.c_longlong
        L.qko_time_seq.argtypes = [ctypes.c_int, _P, _P, _P, _P, _P, ctypes.c_int, _P, ctypes.c_int]
        L.qko_fill_normal.restype = None
        L.qko_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, _P]
        self.threads = 0

    def has_avx512(self):
        return bool(self.lib.qko_has_avx512())

    def init(self, threads):
        self.threads = self.lib.qko_init(int(threads))
        return self.threads

    def fp16_to_f32(self, h):
        return self.lib.qko_fp16_to_f32(int(h))

    def f32_to_fp16(self, f):
        return self.lib.qko_f32_to_fp16(float(f))

    def row_bytes(self, typ, k):
        return self.lib.qko_row_bytes(typ, k)

    def scale_min_k4(self, j, scales12):
        q = np.ascontiguousarray(scales12, dtype=np.uint8)
        sc = np.zeros(1, np.uint8)
        m = np.zeros(1, np.uint8)
        self.lib.qko_scale_min_k4(j, _ptr(q), _ptr(sc), _ptr(m))
        return int(sc[0]), int(m[0])

    def dequant(self, typ, row_bytes, k, fast=False):
        src = np.ascontiguousarray(row_bytes, dtype=np.uint8)
        y = np.zeros(k, np.float32)
        f = self.lib.qko_dequant_row_fast if fast else self.lib.qko_dequant_row
        assert f(typ, _ptr(src), _ptr(y), k) == 0
        return y

    def dequant_matrix(self, typ, w, k, n):
        rb = self.row_bytes(typ, k)
        w = np.ascontiguousarray(w, dtype=np.uint8).reshape(n, rb)
        return np.stack([self.dequant(typ, w[r], k) for r in range(n)])

    def matmul(self, typ, w, k, n, x, force_scalar=False):
        if not self.threads:
            self.init(os.cpu_count() or 1)
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        y = np.zeros((T, n), np.float32)
        rc = self.lib.qko_matmul(_ptr(np.ascontiguousarray(w)), typ, k, n, _ptr(x), T, _ptr(y), int(force_scalar))
        assert rc == 0, "oracle matmul rejected the shape"
        return y

    def time_seq(self, mats, xs, T, reps):
        if not self.threads:
            self.init(os.cpu_count() or 1)
        return _time_seq(self.lib.qko_time_seq, mats, xs, T, reps)

    def matmul_f64(self, typ, w, k, n, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        ref = np.zeros((T, n), np.float64)
        mag = np.zeros((T, n), np.float64)
        assert self.lib.qko_matmul_f64(_ptr(np.ascontiguousarray(w)), typ, k, n, _ptr(x), T, _ptr(ref), _ptr(mag)) == 0
        return ref, mag

    def fill(self, typ, seed, block0, nblocks):
        out = np.zeros(nblocks * BLOCK_BYTES[typ], np.uint8)
        f = {T_Q4_K: self.lib.qko_fill_q4k, T_Q6_K: self.lib.qko_fill_q6k, T_Q5_K: self.lib.qko_fill_q5k,
             T_Q8_0: self.lib.qko_fill_q8_0}[typ]
        f(seed, block0, nblocks, _ptr(out))
        return out

    def weights(self, typ, n, k, seed):
        """GGUF bytes of an n x k synthetic weight (rows of k/256 blocks)."""
        return self.fill(typ, seed, 0, n * (k // 256))

    def normal(self, seed, count):
        out = np.zeros(count, np.float32)
        self.lib.qko_fill_normal(seed, count, _ptr(out))
        return out


class RefLib:
    """The reference's own qwen_cpu quants.h/ops.h, compiled from /root/reference by oracle/Makefile.
    Needs an AVX-512 host (the reference's build flags)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing (make -C oracle ref, needs /root/reference)")
        if not cpu_has_avx512():
            raise RuntimeError("host lacks AVX-512: the reference CPU path cannot run here")
        L = self.lib = ctypes.CDLL(path)
        L.qkref_init.argtypes = [ctypes.c_int]
        L.qkref_row_bytes.restype = ctypes.c_ulonglong
        L.qkref_row_bytes.argtypes = [ctypes.c_uint, ctypes.c_longlong]
        L.qkref_scale_min_k4.argtypes = [ctypes.c_int, _P, _P, _P]
        for f in (L.qkref_dequant_scalar, L.qkref_dequant_avx):
            f.argtypes = [ctypes.c_uint, _P, _P, ctypes.c_longlong]
        L.qkref_matmul.argtypes = [_P, ctypes.c_uint, ctypes.c_int, ctypes.c_int, _P, ctypes.c_int, _P]
        L.qkref_time_seq.restype = ctypes.c_longlong
        L.qkref_time_seq.argtypes = [ctypes.c_int, _P, _P, _P, _P, _P, ctypes.c_int, _P, ctypes.c_int]
        self.threads = 0

    def init(self, threads):
        self.threads = self.lib.qkref_init(int(threads))
        return self.threads

    def scale_min_k4(self, j, scales12):
        q = np.ascontiguousarray(scales12, dtype=np.uint8)
        sc = np.zeros(1, np.uint8)
        m = np.zeros(1, np.uint8)
        self.lib.qkref_scale_min_k4(j, _ptr(q), _ptr(sc), _ptr(m))
        return int(sc[0]), int(m[0])

    def dequant(self, typ, row_bytes, k, avx=False):
        src = np.ascontiguousarray(row_bytes, dtype=np.uint8)
        y = np.zeros(k, np.float32)
        f = self.lib.qkref_dequant_avx if avx else self.lib.qkref_dequant_scalar
        assert f(typ, _ptr(src), _ptr(y), k) == 0
        return y

    def matmul(self, typ, w, k, n, x):
        if not self.threads:
            self.init(os.cpu_count() or 1)
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        y = np.zeros((T, n), np.float32)
        assert self.lib.qkref_matmul(_ptr(np.ascontiguousarray(w)), typ, k, n, _ptr(x), T, _ptr(y)) == 0
        return y


RefLib.time_seq = lambda self, mats, xs, T, reps: _time_seq(self.lib.qkref_time_seq, mats, xs, T, reps)


def ref_available():
    return os.path.exists(REF_SO) and cpu_has_avx512()


def rel_errors(y, ref, mag):
    """The two error metrics of the parity contract: max_{t,n} |y - ref| / sum_k |w x| (the
    reference selftest's normalisation, qwen_cpu/qwen.cpp:889-899) and normwise ||y-ref||/||ref||."""
    y = np.asarray(y, np.float64)
    e_max = float(np.max(np.abs(y - ref) / (mag + 1e-30)))
    e_norm = float(np.linalg.norm(y - ref) / (np.linalg.norm(ref) + 1e-30))
    return e_max, e_norm

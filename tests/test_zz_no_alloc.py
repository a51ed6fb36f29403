"""GPU check of qk_matmul_noalloc, the allocation-free form of qk_matmul (static device workspace
instead of per-stream buffers), through the C ABI.

Two calls in a row on each path, the second with a smaller input, each compared with qk_matmul on the
same inputs (the same kernels and plans: bitwise equal for the GEMV, within the GEMM's bar where its
K-split plan may differ) and with the f64 oracle at the path's bar.  The static workspace keeps the
last call's contents, so the second call also checks that a call leaves the combine slots and
counters in the state the next one needs.
"""
import os

import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q6_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu


def _run(qk, dev, W, x, noalloc):
    m = x.shape[0]
    xd = dev.put(x)
    yd = dev.empty(m * W.n * 4)
    yd.fill_nan()
    (qk.matmul_noalloc if noalloc else qk.matmul)(W, xd.ptr, m, yd.ptr, dev.stream())
    return yd.get(np.float32, (m, W.n))


# (type, k, n, m) of the first call; the second call uses a smaller n and m
CASES = [(T_Q4_K, 5120, 2048, 1), (T_Q6_K, 17408, 1024, 4), (T_Q8_0, 6144, 1024, 3), (T_Q4_K, 2048, 256, 2),
         (T_Q4_K, 5120, 1024, 160), (T_Q6_K, 2048, 512, 48)]


@pytest.mark.parametrize("typ,k,n,m", CASES, ids=[f"t{t}k{k}n{n}m{m}" for t, k, n, m in CASES])
def test_noalloc_matches_matmul(qk, oracle, dev, typ, k, n, m):
    for call, (nn, mm) in enumerate([(n, m), (max(16, n // 4), max(1, m // 2) if m < 16 else max(16, m // 2))]):
        seed = SEED_BASE | (0xD0 + 8 * call)
        w = oracle.weights(typ, nn, k, seed)
        x = oracle.normal(seed ^ 0x3C, mm * k).reshape(mm, k)
        W = qk.upload(w, typ, k, nn, 1)
        try:
            y_na = _run(qk, dev, W, x, True)
            y_ref = _run(qk, dev, W, x, False)
        finally:
            qk.free(W)
        assert np.isfinite(y_na).all()
        if mm < 16:
            assert np.array_equal(y_na.view(np.uint32), y_ref.view(np.uint32)), (call, nn, mm)
            ref, mag = oracle.matmul_f64(typ, w, k, nn, x)
            bar = 1e-5
        else:
            xr = x.astype(np.float16).astype(np.float32)
            ref, mag = oracle.matmul_f64(typ, w, k, nn, xr)
            bar = 5e-3
            e_max, e_norm = rel_errors(y_na, y_ref.astype(np.float64), mag)
            assert e_max <= bar and e_norm <= bar, ("vs qk_matmul", call, e_max, e_norm)
        e_max, e_norm = rel_errors(y_na, ref, mag)
        assert e_max <= bar and e_norm <= bar, (call, e_max, e_norm)


def test_noalloc_rejects_beyond_workspace(qk, dev):
    """A GEMM whose 128-token fp16 image exceeds the static array is refused with QK_E_RANGE before
    any launch (k = 131072: 32 MiB per chunk)."""
    k, n, m = 131072, 16, 16
    buf = dev.empty(n * (k // 256) * 144)
    xd = dev.empty(m * k * 4)
    yd = dev.empty(m * n * 4)
    try:
        W = qk.weight_view(buf.ptr, T_Q4_K, k, n, 1)
        with pytest.raises(Exception) as e:
            qk.matmul_noalloc(W, xd.ptr, m, yd.ptr, dev.stream())
        assert getattr(e.value, "status", None) == -8
    finally:
        buf.close()
        xd.close()
        yd.close()


def test_noalloc_first_call_under_capture():
    """The first qk_matmul_noalloc calls of a process (no qk_init_stream, nothing else touching the
    static workspace) come under graph capture; every replay equals qk_matmul bitwise.  Its own
    process (tests/noalloc_capture_check.py), since this one has used the workspace already."""
    import subprocess
    import sys

    script = os.path.join(os.path.dirname(os.path.abspath(__file__)), "noalloc_capture_check.py")
    res = subprocess.run([sys.executable, "-u", script], capture_output=True, text=True, timeout=110)
    print(res.stdout)
    assert res.returncode == 0, res.stdout[-3000:] + res.stderr[-3000:]
    assert res.stdout.strip().endswith("OK")

"""The reference-shaped C++ shim (include/qk_shim.h: upload / matmul / gemv with the reference's
fail-stop) driven by tests/_bin/shim_check, checked against the oracle."""
import os
import subprocess

import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q6_K, rel_errors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM = os.path.join(ROOT, "tests", "_bin", "shim_check")


def _run(tmp_path, w, typ, k, n, x, up=None):
    files = {"w": tmp_path / "w.bin", "x": tmp_path / "x.bin", "y": tmp_path / "y.bin"}
    w.tofile(files["w"])
    x.astype(np.float32).tofile(files["x"])
    args = [SHIM, str(files["w"]), str(typ), str(k), str(n), str(files["x"]), str(x.shape[0]), str(files["y"])]
    if up is not None:
        up.tofile(tmp_path / "u.bin")
        args.append(str(tmp_path / "u.bin"))
    res = subprocess.run(args, capture_output=True, text=True, timeout=120)
    return res, (np.fromfile(files["y"], np.float32).reshape(x.shape[0], n) if res.returncode == 0 else None)


@pytest.mark.gpu
@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("T", [1, 3, 20])
def test_shim_matmul(oracle, tmp_path, typ, T):
    k, n = 1024, 64
    w = oracle.weights(typ, n, k, SEED_BASE | 0x90)
    x = oracle.normal(SEED_BASE | 0x91, T * k).reshape(T, k)
    res, y = _run(tmp_path, w, typ, k, n, x)
    assert res.returncode == 0, res.stderr
    xin = x if T < 16 else x.astype(np.float16).astype(np.float32)  # the GEMM's fp16 operands
    ref, mag = oracle.matmul_f64(typ, w, k, n, xin)
    e_max, e_norm = rel_errors(y, ref, mag)
    tol = 1e-3 if T < 16 else 5e-3
    assert e_max <= tol and e_norm <= tol, (e_max, e_norm)


@pytest.mark.gpu
def test_shim_gemv_glu(oracle, tmp_path):
    k, n, T = 1024, 48, 2
    g = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x92)
    u = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x93)
    x = oracle.normal(SEED_BASE | 0x94, T * k).reshape(T, k)
    res, y = _run(tmp_path, g, T_Q4_K, k, n, x, up=u)
    assert res.returncode == 0, res.stderr
    gr, _ = oracle.matmul_f64(T_Q4_K, g, k, n, x)
    ur, _ = oracle.matmul_f64(T_Q4_K, u, k, n, x)
    want = gr / (1.0 + np.exp(-gr)) * ur
    # the int8 kernel's bar (T <= 4 per launch), normwise and against the largest output
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 2e-4
    assert np.abs(y - want).max() < 2e-4 * np.abs(want).max()


def test_shim_fail_stop(tmp_path):
    """A rejected call prints one line and ends the process with status 1 (qwen_cuda/cu.h:21-27).
    Runs anywhere: without a GPU the first call (use) fails, with one the upload's shape check."""
    if not os.path.exists(SHIM):
        pytest.skip("tests/_bin/shim_check not built (__graft_entry__.build())")
    w = np.zeros(144 * 16, np.uint8)
    x = np.zeros((1, 300), np.float32)
    res, _ = _run(tmp_path, w, T_Q4_K, 300, 16, x)
    assert res.returncode == 1
    assert res.stderr.startswith("qk: ") and "failed" in res.stderr

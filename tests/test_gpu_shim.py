"""The reference-shaped C++ shim (include/qk_shim.h) driven by tests/_bin/shim_check, checked against
the oracle.  The shim's gemv / matmul take fp16 activations as the reference's do (qwen_cuda/qwen.cpp:
220-247), in the xperm layout when the step runs it (set_xperm, the reference's G_xperm), and a GLU pair
writes fp16 silu(g) u at the xperm position of its row (qwen_cuda/kernels.cu:419-426); gemv_f32 /
matmul_f32 keep fp32.  load_weights + get_w give views into one device copy of a GGUF file
(qwen_cuda/qwen.cpp:152-173, 737-761) and embed is the k_embed_* launch (qwen.cpp:265)."""
import os
import subprocess

import numpy as np
import pytest

import gguf_writer as gw
from oracle_lib import GEMM_ROUTE_M, GLU_GEMM_M, SEED_BASE, T_Q4_K, T_Q6_K, rel_errors

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM = os.path.join(ROOT, "tests", "_bin", "shim_check")


def xperm_pos(i):
    """qwen_cuda/kernels.cu:27-28, restated: position of element i inside its row."""
    return (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7)


def to_xperm(a):
    """Rows of a [T][k] array placed in the xperm layout (out[:, xperm_pos(i)] = a[:, i])."""
    out = np.empty_like(a)
    out[:, xperm_pos(np.arange(a.shape[1]))] = a
    return out


def _run(tmp_path, mode, w, typ, k, n, x, up=None, out_dtype=np.float32):
    files = {"w": tmp_path / "w.bin", "x": tmp_path / "x.bin", "y": tmp_path / "y.bin"}
    w.tofile(files["w"])
    x.tofile(files["x"])
    args = [SHIM, mode, str(files["w"]), str(typ), str(k), str(n), str(files["x"]), str(x.shape[0]), str(files["y"])]
    if up is not None:
        up.tofile(tmp_path / "u.bin")
        args.append(str(tmp_path / "u.bin"))
    res = subprocess.run(args, capture_output=True, text=True, timeout=120)
    y = np.fromfile(files["y"], out_dtype).reshape(x.shape[0], n) if res.returncode == 0 else None
    return res, y


@pytest.mark.gpu
@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("T", [1, 3, 20])
def test_shim_matmul_f32(oracle, tmp_path, typ, T):
    k, n = 1024, 64
    w = oracle.weights(typ, n, k, SEED_BASE | 0x90)
    x = oracle.normal(SEED_BASE | 0x91, T * k).reshape(T, k)
    res, y = _run(tmp_path, "f32", w, typ, k, n, x)
    assert res.returncode == 0, res.stderr
    xin = x if T < GEMM_ROUTE_M else x.astype(np.float16).astype(np.float32)  # the GEMM's fp16 operands
    ref, mag = oracle.matmul_f64(typ, w, k, n, xin)
    e_max, e_norm = rel_errors(y, ref, mag)
    tol = 1e-5 if T < GEMM_ROUTE_M else 5e-3
    assert e_max <= tol and e_norm <= tol, (e_max, e_norm)


@pytest.mark.gpu
@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("T", [1, 4, 9, 13, 20])
@pytest.mark.parametrize("mode", ["f16", "f16x"])
def test_shim_matmul_f16(oracle, tmp_path, typ, T, mode):
    """fp16 x, plain or xperm (xperm applies for T < 16 only, as the reference's g.xp): the oracle
    is fed the same fp16 values, widened."""
    k, n = 2048, 64
    w = oracle.weights(typ, n, k, SEED_BASE | 0x95)
    xh = oracle.normal(SEED_BASE | 0x96, T * k).reshape(T, k).astype(np.float16)
    xin = to_xperm(xh) if (mode == "f16x" and T < 16) else xh
    res, y = _run(tmp_path, mode, w, typ, k, n, xin)
    assert res.returncode == 0, res.stderr
    ref, mag = oracle.matmul_f64(typ, w, k, n, xh.astype(np.float32))
    e_max, e_norm = rel_errors(y, ref, mag)
    tol = 1e-5 if T < GEMM_ROUTE_M else 5e-3  # the GEMM from nine tokens, plain or xperm x
    assert e_max <= tol and e_norm <= tol, (e_max, e_norm)


def _glu_ref(oracle, g, u, k, n, x):
    gr, _ = oracle.matmul_f64(T_Q4_K, g, k, n, x)
    ur, _ = oracle.matmul_f64(T_Q4_K, u, k, n, x)
    return gr / (1.0 + np.exp(-gr)) * ur


@pytest.mark.gpu
def test_shim_gemv_glu_f32(oracle, tmp_path):
    k, n, T = 1024, 48, 2
    g = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x92)
    u = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x93)
    x = oracle.normal(SEED_BASE | 0x94, T * k).reshape(T, k)
    res, y = _run(tmp_path, "f32", g, T_Q4_K, k, n, x, up=u)
    assert res.returncode == 0, res.stderr
    want = _glu_ref(oracle, g, u, k, n, x)
    assert np.linalg.norm(y - want) / np.linalg.norm(want) < 1e-5
    assert np.abs(y - want).max() < 1e-5 * np.abs(want).max()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["f16", "f16x"])
@pytest.mark.parametrize("T", [1, 3, 6, 13])
def test_shim_gemv_glu_f16(oracle, tmp_path, mode, T):
    """The reference's decode FFN launch: fp16 x (xperm in mode f16x), fp16 silu(g) u written at the
    xperm position of its row in mode f16x (n % 1024 == 0, so it is the down projection's input).
    Six and thirteen tokens take the GEMM (one weight pass), held to its bar."""
    k, n = 1024, 2048
    g = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x97)
    u = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x98)
    # x scaled so that silu(g) u stays inside the fp16 range (the reference's output type too)
    xh = (0.05 * oracle.normal(SEED_BASE | 0x99, T * k).reshape(T, k)).astype(np.float16)
    xin = to_xperm(xh) if mode == "f16x" else xh
    res, y = _run(tmp_path, mode, g, T_Q4_K, k, n, xin, up=u, out_dtype=np.float16)
    assert res.returncode == 0, res.stderr
    if mode == "f16x":
        y = y[:, xperm_pos(np.arange(n))]  # back to row order
    want = _glu_ref(oracle, g, u, k, n, xh.astype(np.float32))
    y = y.astype(np.float64)
    # fp16 output: within half an fp16 ulp of the exact value, plus the matmul bar (the GEMM's for a
    # gate/up pair from five tokens)
    bar = 1e-5 if T < GLU_GEMM_M else 5e-3
    assert np.all(np.abs(y - want) <= np.abs(want) * 2.0 ** -11 + bar * np.abs(want).max())


def _gguf_fixture(oracle, path):
    tensors = [
        ("blk.0.ffn_down.weight", T_Q4_K, [1024, 48], oracle.weights(T_Q4_K, 48, 1024, SEED_BASE | 0x9A)),
        ("token_embd.weight", T_Q6_K, [512, 64], oracle.weights(T_Q6_K, 64, 512, SEED_BASE | 0x9B)),
    ]
    gw.write(path, [("general.architecture", gw.STR, "qwen35")], tensors, 32)
    return {t[0]: t[3] for t in tensors}


@pytest.mark.gpu
def test_shim_get_w_views(oracle, tmp_path):
    """load_weights + get_w: a view into the one device copy of the file, used by matmul_f32."""
    path = tmp_path / "m.gguf"
    data = _gguf_fixture(oracle, str(path))
    k, n, T = 1024, 48, 2
    x = oracle.normal(SEED_BASE | 0x9C, T * k).reshape(T, k)
    x.tofile(tmp_path / "x.bin")
    res = subprocess.run([SHIM, "gguf", str(path), "blk.0.ffn_down.weight", str(k), str(n), str(tmp_path / "x.bin"),
                          str(T), str(tmp_path / "y.bin")], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    y = np.fromfile(tmp_path / "y.bin", np.float32).reshape(T, n)
    ref, mag = oracle.matmul_f64(T_Q4_K, data["blk.0.ffn_down.weight"], k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert e_max <= 1e-5 and e_norm <= 1e-5, (e_max, e_norm)
    # a wrong shape is fatal, as in the reference's get_w
    res = subprocess.run([SHIM, "gguf", str(path), "blk.0.ffn_down.weight", str(k), "32", str(tmp_path / "x.bin"),
                          str(T), str(tmp_path / "y.bin")], capture_output=True, text=True, timeout=120)
    assert res.returncode == 1 and "wrong shape" in res.stderr


@pytest.mark.gpu
def test_shim_embed(oracle, tmp_path):
    """embed: table rows bit-exact with the oracle's dequant, masked rows copied from embd."""
    path = tmp_path / "m.gguf"
    data = _gguf_fixture(oracle, str(path))
    k, n, T = 512, 64, 5
    tokens = np.array([3, 63, 0, 17, 40], np.int32)
    mask = np.array([0, 1, 0, 0, 1], np.uint8)
    embd = oracle.normal(SEED_BASE | 0x9D, T * k).reshape(T, k)
    for p, a in (("t.bin", tokens), ("m.bin", mask), ("e.bin", embd)):
        a.tofile(tmp_path / p)
    res = subprocess.run([SHIM, "embed", str(path), "token_embd.weight", str(k), str(n), str(tmp_path / "t.bin"),
                          str(T), str(tmp_path / "x.bin"), str(tmp_path / "m.bin"), str(tmp_path / "e.bin")],
                         capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    x = np.fromfile(tmp_path / "x.bin", np.float32).reshape(T, k)
    table = oracle.dequant_matrix(T_Q6_K, data["token_embd.weight"], k, n)
    want = np.where(mask[:, None] != 0, embd, table[tokens])
    assert np.array_equal(x.view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_shim_fail_stop(tmp_path):
    """A rejected call prints one line and ends the process with status 1 (qwen_cuda/cu.h:21-27).
    Runs anywhere: without a GPU the first call (use) fails, with one the upload's shape check."""
    if not os.path.exists(SHIM):
        pytest.skip("tests/_bin/shim_check not built (__graft_entry__.build())")
    w = np.zeros(144 * 16, np.uint8)
    x = np.zeros((1, 300), np.float32)
    res, _ = _run(tmp_path, "f32", w, T_Q4_K, 300, 16, x)
    assert res.returncode == 1
    assert res.stderr.startswith("qk: ") and "failed" in res.stderr

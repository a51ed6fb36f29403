"""GPU checks of the activation formats at the boundary (include/qk.h QK_ACT_*), through the C ABI.

fp16 activations are widened exactly to the fp32 the kernels work in, so each fp16 path must give
results bitwise equal to the fp32 entry points fed the widened values, on every kernel: the int8 GEMV
(one to eight tokens), the general Q4_K / Q6_K GEMV, the F32 weight kernel inside a group, and the GEMM
(whose conversion pass rounds fp32 to fp16, so fp16-exact fp32 input gives the same values; from nine
tokens it also reads xperm x, the reference's decode layout up to fifteen tokens).  The xperm layout
(qwen_cuda/kernels.cu:27-28) must give results bitwise equal to the plain layout, and a GLU pair's fp16
output must be the round-to-nearest-even fp16 of its fp32 output, placed at xperm(row) in the xperm
form (kernels.cu:419-426).  Together with the fp32 paths' oracle parity elsewhere, this pins the fp16
paths to the oracle.
"""
import numpy as np
import pytest

from oracle_lib import GEMM_ROUTE_M, SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu

F32, F16, F16X = 0, 1, 2
TYPES = [T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0]
IDS = ["q4k", "q5k", "q6k", "q8_0"]


def xperm_pos(i):
    return (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7)


def to_xperm(a):
    out = np.empty_like(a)
    out[:, xperm_pos(np.arange(a.shape[1]))] = a
    return out


def _same(a, b):
    return np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def test_xperm_is_a_permutation():
    """The restated layout maps each 1024-run onto itself one-to-one (CPU check of the test helper)."""
    p = xperm_pos(np.arange(4096))
    assert np.array_equal(np.sort(p), np.arange(4096))
    assert np.all(p // 1024 == np.arange(4096) // 1024)
    # any 4-aligned run of four stays contiguous (the kernels load four at a time)
    q = p.reshape(-1, 4)
    assert np.all(q[:, 1:] - q[:, :-1] == 1)


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 7, 8, 9, 13, 15, 20])
def test_matmul_f16_equals_f32(qk, oracle, dev, typ, m):
    k, n = 2048, 96
    w = oracle.weights(typ, n, k, SEED_BASE | 0xC0)
    xh = oracle.normal(SEED_BASE | 0xC1 + m, m * k).reshape(m, k).astype(np.float16)
    W = qk.upload(w, typ, k, n, 1)
    try:
        outs = {}
        for fmt, xa in ((F32, xh.astype(np.float32)), (F16, xh)) + (((F16X, to_xperm(xh)),) if m < 16 else ()):
            xd = dev.put(xa)
            yd = dev.empty(m * n * 4)
            yd.fill_nan()
            qk.matmul_act(W, xd.ptr, fmt, m, yd.ptr, dev.stream())
            outs[fmt] = yd.get(np.float32, (m, n))
    finally:
        qk.free(W)
    assert np.isfinite(outs[F32]).all()
    # every format takes the same kernel (the GEMV up to eight tokens, the GEMM from nine) and hands
    # it the same values in the same order (x is fp16-exact, xperm only moves it): bitwise equal
    ref, mag = oracle.matmul_f64(typ, w, k, n, xh.astype(np.float32))
    for fmt, y in outs.items():
        assert _same(y, outs[F32]), fmt
        e_max, e_norm = rel_errors(y, ref, mag)
        tol = 1e-5 if m < GEMM_ROUTE_M else 5e-3
        assert e_max <= tol and e_norm <= tol, (fmt, e_max, e_norm)


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("m", [1, 4])
def test_general_kernel_f16(qk, oracle, dev, typ, m):
    """The general kernel's prepass reads fp16 / xperm x too."""
    k, n = 1024, 64
    w = oracle.weights(typ, n, k, SEED_BASE | 0xC8)
    xh = oracle.normal(SEED_BASE | 0xC9, m * k).reshape(m, k).astype(np.float16)
    W = qk.upload(w, typ, k, n, 1)
    try:
        qk.set_tuning("gemv_fused", 0)
        outs = {}
        for fmt, xa in ((F32, xh.astype(np.float32)), (F16, xh), (F16X, to_xperm(xh))):
            xd = dev.put(xa)
            yd = dev.empty(m * n * 4)
            qk.matmul_act(W, xd.ptr, fmt, m, yd.ptr, dev.stream())
            outs[fmt] = yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemv_fused", 1)
        qk.free(W)
    assert _same(outs[F16], outs[F32]) and _same(outs[F16X], outs[F32])


def test_group_with_f32_weights_f16(qk, oracle, dev):
    """The {qkv, gate_z, alpha, beta} launch with F32 alpha/beta (docs/model.md:328) fed fp16 xperm x,
    as the reference's decode step feeds it."""
    k, m = 1024, 1
    rng = np.random.default_rng(7)
    wq = oracle.weights(T_Q4_K, 64, k, SEED_BASE | 0xCA)
    wa = rng.standard_normal((48, k)).astype(np.float32)
    xh = oracle.normal(SEED_BASE | 0xCB, m * k).reshape(m, k).astype(np.float16)
    Wq = qk.upload(wq, T_Q4_K, k, 64, 1)
    wad = dev.put(wa)
    try:
        Wa = qk.weight_view(wad.ptr, 0, k, 48, 0)
        outs = {}
        for fmt, xa in ((F32, xh.astype(np.float32)), (F16X, to_xperm(xh))):
            xd = dev.put(xa)
            y0, y1 = dev.empty(m * 64 * 4), dev.empty(m * 48 * 4)
            qk.gemv_group_act([Wq, Wa], [y0.ptr, y1.ptr], False, xd.ptr, fmt, m)
            outs[fmt] = (y0.get(np.float32, (m, 64)), y1.get(np.float32, (m, 48)))
    finally:
        qk.free(Wq)
    assert _same(outs[F16X][0], outs[F32][0]) and _same(outs[F16X][1], outs[F32][1])
    want = xh.astype(np.float64) @ wa.T.astype(np.float64)
    assert np.abs(outs[F32][1] - want).max() <= 1e-5 * np.abs(want).max()


# (type, fused): the general kernel (fused = 0) serves Q4_K and Q6_K only
GLU_F16_CASES = [(t, f) for t in TYPES for f in (1, 0) if f or t in (T_Q4_K, T_Q6_K)]


@pytest.mark.parametrize("typ,fused", GLU_F16_CASES, ids=[f"{IDS[TYPES.index(t)]}-fused{f}" for t, f in GLU_F16_CASES])
@pytest.mark.parametrize("m", [1, 2, 4, 6, 13])
def test_glu_f16_output(qk, oracle, dev, typ, m, fused):
    """GLU output in fp16: the RNE fp16 of the fp32 output, at the plain or xperm position (6 and 13
    tokens: the GEMM's k_glu_sum, from fp16 and xperm x alike)."""
    k, n = 1024, 2048
    wg = oracle.weights(typ, n, k, SEED_BASE | 0xCC)
    wu = oracle.weights(typ, n, k, SEED_BASE | 0xCD)
    xh = (0.05 * oracle.normal(SEED_BASE | 0xCE, m * k).reshape(m, k)).astype(np.float16)
    G = qk.upload(wg, typ, k, n, 1)
    U = qk.upload(wu, typ, k, n, 1)
    try:
        qk.set_tuning("gemv_fused", fused)
        xd = dev.put(xh)
        y32 = dev.empty(m * n * 4)
        qk.gemv_group_act([G, U], [y32.ptr], True, xd.ptr, F16, m, F32)
        base = y32.get(np.float32, (m, n))
        got = {}
        for yf, xf, xa in ((F16, F16, xh), (F16X, F16X, to_xperm(xh))):
            xd2 = dev.put(xa)
            yd = dev.empty(m * n * 2)
            qk.gemv_group_act([G, U], [yd.ptr], True, xd2.ptr, xf, m, yf)
            got[yf] = yd.get(np.float16, (m, n))
    finally:
        qk.set_tuning("gemv_fused", 1)
        qk.free(G)
        qk.free(U)
    assert np.isfinite(base).all()
    want = base.astype(np.float16)  # numpy rounds to nearest even
    assert np.array_equal(got[F16].view(np.uint16), want.view(np.uint16))
    assert np.array_equal(got[F16X][:, xperm_pos(np.arange(n))].view(np.uint16), want.view(np.uint16))


def test_act_argument_checks(qk, dev):
    """xperm needs k % 1024 == 0 and m < 16; an xperm GLU output n % 1024 == 0; unknown formats and a
    GLU format without glu are rejected, before any launch."""
    k, n = 512, 32
    buf = dev.empty(n * (k // 256) * 144)
    x = dev.empty(16 * 1024 * 4)
    y = dev.empty(16 * 2048 * 4)
    try:
        W = qk.weight_view(buf.ptr, T_Q4_K, k, n, 1)
        for args, code in (((W, x.ptr, F16X, 1, y.ptr), -3), ((W, x.ptr, 7, 1, y.ptr), -8)):
            with pytest.raises(Exception) as e:
                qk.matmul_act(*args)
            assert getattr(e.value, "status", None) == code
        with pytest.raises(Exception) as e:
            qk.gemv_group_act([W], [y.ptr], False, x.ptr, F16, 1, F16)
        assert e.value.status == -8
        with pytest.raises(Exception) as e:
            qk.gemv_group_act([W, W], [y.ptr], True, x.ptr, F16, 1, F16X)
        assert e.value.status == -3
    finally:
        buf.close()
        x.close()
        y.close()

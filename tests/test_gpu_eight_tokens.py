"""GPU parity of the GEMV at five to fifteen tokens (the reference's decode GEMV reads each weight once
per eight tokens: NT = 8 at qwen_cuda/kernels.cu:11, gemv_body's token loop at :412-436, used for
every T < 16 by qwen_cuda/qwen.cpp:232-245), through the C ABI.

The int8 kernel carries up to eight tokens per launch (eight token slots: 24 int8 activation parts,
six MFMAs per step), so m = 5..8 is one weight pass and m = 9..15 two; the outputs are held to the
int8 kernel's bar against the f64 oracle (1e-5 on both metrics, the reference's fp32 bar being
1e-3), at a moderate shape for all four types and at the C1 / C2 shapes of the BASELINE configs.
The plan query shows one launch of eight token slots per eight tokens.  By default qk_matmul (any
activation format), grouped launches and a gate/up pair send m >= 5 to the GEMM (one weight pass):
these tests keep the GEMV there with the gemm_min_m knob; test_default_route and test_glu_pair_gemm
check the default routes at the GEMM's bar."""
import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu

TOL_I8 = 1e-5
TYPES = [T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0]
IDS = ["q4k", "q5k", "q6k", "q8_0"]


def _matmul(qk, oracle, dev, typ, k, n, m, seed):
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0x5EED, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    try:
        qk.set_tuning("gemm_min_m", 16)  # the GEMV for every m < 16
        plan = qk.gemv_plan([W], False, m)
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemm_min_m", 0)
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert np.isfinite(y).all()
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm, plan)
    return plan


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [5, 6, 7, 8, 9, 13, 15])
def test_tokens_5_to_15(qk, oracle, dev, typ, m):
    plan = _matmul(qk, oracle, dev, typ, 3072, 512, m, SEED_BASE | 0xF0 | (m << 8) | (typ << 16))
    assert plan["kernel"] == 1 and plan["token_slots"] == 8, plan


@pytest.mark.parametrize("typ,k,n", [(T_Q4_K, 5120, 17408), (T_Q6_K, 17408, 5120)], ids=["c1", "c2"])
@pytest.mark.parametrize("m", [5, 8, 13, 15])
def test_config_shapes(qk, oracle, dev, typ, k, n, m):
    """C1 (Q4_K K=5120 N=17408) and C2 (Q6_K K=17408 N=5120) at 5, 8, 13 and 15 tokens."""
    plan = _matmul(qk, oracle, dev, typ, k, n, m, SEED_BASE | 0xF8 | (m << 8) | (typ << 16))
    assert plan["token_slots"] == 8, plan


def _glu(qk, oracle, dev, typ, k, n, m, tag):
    wg = oracle.weights(typ, n, k, SEED_BASE | 0xF5 | (typ << 8) | tag)
    wu = oracle.weights(typ, n, k, SEED_BASE | 0xF6 | (typ << 8) | tag)
    x = oracle.normal(SEED_BASE | 0xF7 | (m << 8) | tag, m * k).reshape(m, k)
    G = qk.upload(wg, typ, k, n, 1)
    U = qk.upload(wu, typ, k, n, 1)
    try:
        plan = qk.gemv_plan([G, U], True, m)
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    assert np.isfinite(y).all()
    return wg, wu, x, y, plan


def _glu_ref(oracle, typ, wg, wu, k, n, x):
    g, _ = oracle.matmul_f64(typ, wg, k, n, x)
    u, _ = oracle.matmul_f64(typ, wu, k, n, x)
    return g / (1.0 + np.exp(-g)) * u


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [6, 8, 13])
def test_glu_pair(qk, oracle, dev, typ, m):
    """The gate/up pair on the GEMV at 6, 8 and 13 tokens (through the gemm_min_m knob: by default the
    pair takes the GEMM from five tokens): silu(g) * u against the f64 oracle, with the matmul bar
    carried through the product (normwise)."""
    k, n = 5120, 2048
    qk.set_tuning("gemm_min_m", 16)
    try:
        wg, wu, x, y, plan = _glu(qk, oracle, dev, typ, k, n, m, 0)
    finally:
        qk.set_tuning("gemm_min_m", 0)
    ref = _glu_ref(oracle, typ, wg, wu, k, n, x)
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < TOL_I8, (err, plan)
    assert plan["kernel"] == 1 and plan["token_slots"] == 8, plan


GLU_GEMM = [(T_Q4_K, 5120, 17408, 13), (T_Q4_K, 5120, 2048, 5), (T_Q4_K, 5120, 2048, 9), (T_Q6_K, 5120, 2048, 8),
            (T_Q6_K, 5120, 2048, 15), (T_Q5_K, 3072, 2048, 13), (T_Q8_0, 3072, 2048, 6), (T_Q4_K, 1024, 80, 7),
            (T_Q6_K, 2048, 48, 11)]  # 80 / 48 rows: a half-empty last tile pair


@pytest.mark.parametrize("typ,k,n,m", GLU_GEMM, ids=[f"{IDS[TYPES.index(t)]}-k{k}n{n}m{m}" for t, k, n, m in GLU_GEMM])
def test_glu_pair_gemm(qk, oracle, dev, typ, k, n, m):
    """The gate/up pair from five tokens by default: both matrices in one GEMM launch, the K-parts
    added in order and silu(g) u applied by k_glu_sum (the C3a shape at 13 tokens included).  Held to
    the MFMA path's bar carried through the product, against the f64 oracle fed the fp16-rounded x
    the GEMM multiplies."""
    wg, wu, x, y, plan = _glu(qk, oracle, dev, typ, k, n, m, 0x1000)
    assert plan["kernel"] == 4, plan  # QK_GEMV_GEMM
    ref = _glu_ref(oracle, typ, wg, wu, k, n, x.astype(np.float16).astype(np.float32))
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < 5e-3, err
    assert np.abs(y - ref).max() <= 5e-3 * np.abs(ref).max()


@pytest.mark.parametrize("typ,k,n,m", [(T_Q4_K, 5120, 4096, 8), (T_Q6_K, 17408, 1024, 7), (T_Q5_K, 3072, 2048, 6)])
def test_eight_slot_splits_bitwise_equal(qk, oracle, dev, typ, k, n, m):
    """Which wave takes a unit never changes the eight-slot result: bitwise equal over the static /
    hand-out splits (gemv_dshift 0, 1, 31)."""
    w = oracle.weights(typ, n, k, SEED_BASE | 0xF9)
    x = oracle.normal(SEED_BASE | 0xFA, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    outs = []
    try:
        xd = dev.put(x)
        qk.set_tuning("gemm_min_m", 16)  # the eight-slot GEMV (qk_matmul takes the GEMM from five tokens)
        for sh in (0, 1, 31):
            qk.set_tuning("gemv_dshift", sh)
            yd = dev.empty(m * n * 4)
            yd.fill_nan()
            qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
            outs.append(yd.get(np.float32, (m, n)))
    finally:
        qk.set_tuning("gemv_dshift", 1)
        qk.set_tuning("gemm_min_m", 0)
        qk.free(W)
    for y in outs[1:]:
        assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32))
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    e_max, e_norm = rel_errors(outs[0], ref, mag)
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


@pytest.mark.parametrize("typ,k,n", [(T_Q4_K, 5120, 17408), (T_Q6_K, 17408, 5120), (T_Q5_K, 3072, 512),
                                     (T_Q8_0, 3072, 512)], ids=["c1", "c2", "q5k", "q8_0"])
@pytest.mark.parametrize("m", [5, 8, 9, 13, 15])
def test_default_route(qk, oracle, dev, typ, k, n, m):
    """qk_matmul's own route for five to fifteen tokens: the GEMM in one weight pass, held to the MFMA
    path's bar (5e-3 on both metrics) against the f64 oracle fed the fp16-rounded x the GEMM
    multiplies, and against the unrounded fp32 x.  The same x rounded to fp16 and laid out in the
    reference's xperm decode layout takes the same GEMM through qk_matmul_act: bitwise equal."""
    seed = SEED_BASE | 0xFB | (m << 8) | (typ << 16)
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0x5EED, m * k).reshape(m, k)
    i = np.arange(k)
    xcols = (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7)
    xp = np.empty((m, k), np.float16)
    xp[:, xcols] = x.astype(np.float16)
    W = qk.upload(w, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
        xpd = dev.put(xp)
        yd.fill_nan()
        qk.matmul_act(W, xpd.ptr, 2, m, yd.ptr, dev.stream())  # QK_ACT_F16_XPERM
        yx = yd.get(np.float32, (m, n))
    finally:
        qk.free(W)
    assert np.isfinite(y).all()
    assert np.array_equal(yx.view(np.uint32), y.view(np.uint32))
    rows = np.arange(0, n, max(1, n // 512))
    wsub = w.reshape(n, -1)[rows].reshape(-1)
    x16 = x.astype(np.float16).astype(np.float32)
    for xr in (x16, x):
        ref, mag = oracle.matmul_f64(typ, wsub, k, len(rows), xr)
        e_max, e_norm = rel_errors(y[:, rows], ref, mag)
        assert e_max <= 5e-3 and e_norm <= 5e-3, (e_max, e_norm)

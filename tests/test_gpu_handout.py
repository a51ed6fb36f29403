"""The int8 GEMV's split of a work-group's units between static positions and the LDS hand-out
counter ("gemv_dshift": about nu >> value units handed out dynamically) changes which wave computes
which unit, never the result: every unit's sums land in the unit's own LDS slot and each group adds
them in unit order.  So the output is bitwise the same for every split, all-static (31) and
all-dynamic (0) included, and matches the f64 oracle."""
import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu

TOL_I8 = 1e-5
SPLITS = (0, 1, 2, 31)


def _run(qk, dev, Ws, glu, x, m, n):
    xd = dev.put(x)
    yd = dev.empty(m * n * 4)
    yd.fill_nan()
    qk.gemv_group(Ws, [yd.ptr] * (1 if glu else len(Ws)), glu, xd.ptr, m, dev.stream())
    return yd.get(np.float32, (m, n))


@pytest.mark.parametrize("typ,k,n,m", [
    (T_Q6_K, 17408, 5120, 1),   # C2: two K-slices
    (T_Q4_K, 5120, 17408, 1),   # C1
    (T_Q4_K, 5120, 5120, 4),    # C3b: four tokens, four K-slices
    (T_Q8_0, 6144, 1024, 2),
    (T_Q5_K, 3072, 2048, 3),
])
def test_splits_bitwise_equal(qk, oracle, dev, typ, k, n, m):
    seed = SEED_BASE | 0xD5 | (typ << 8) | (m << 12)
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0x77, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    outs = []
    try:
        assert qk.gemv_plan([W], False, m)["kernel"] == 1
        for sh in SPLITS:
            qk.set_tuning("gemv_dshift", sh)
            outs.append(_run(qk, dev, [W], False, x, m, n))
    finally:
        qk.set_tuning("gemv_dshift", 1)
        qk.free(W)
    for sh, y in zip(SPLITS[1:], outs[1:]):
        assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32)), sh
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    e_max, e_norm = rel_errors(outs[0], ref, mag)
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


def test_splits_glu_pair_bitwise_equal(qk, oracle, dev):
    """The four-token gate/up pair (two-deep ring, addresses read from the LDS table)."""
    k, n, m = 5120, 4096, 4
    wg = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0xD51)
    wu = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0xD52)
    x = oracle.normal(SEED_BASE | 0xD53, m * k).reshape(m, k)
    G = qk.upload(wg, T_Q4_K, k, n, 1)
    U = qk.upload(wu, T_Q4_K, k, n, 1)
    outs = []
    try:
        assert qk.gemv_plan([G, U], True, m)["ring_depth"] == 2
        for sh in SPLITS:
            qk.set_tuning("gemv_dshift", sh)
            outs.append(_run(qk, dev, [G, U], True, x, m, n))
    finally:
        qk.set_tuning("gemv_dshift", 1)
        qk.free(G)
        qk.free(U)
    for sh, y in zip(SPLITS[1:], outs[1:]):
        assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32)), sh
    assert np.isfinite(outs[0]).all()

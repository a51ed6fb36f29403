"""GPU parity at the BASELINE workloads that are launched as something other than C1 / C2 / C4, through
the C ABI, against the f64 brute force of the oracle (tests/oracle_lib.py):

  * C3a: the Q4_K gate/up pair with the SiLU product, four tokens, K=5120, N=17408 x 2 (the int8
    kernel's four-token pair plan: two-deep ring, about 85 units per CU, 43 KB of unit sums);
  * C3b: Q4_K, four tokens, K=5120, N=5120;
  * the C5 decode step's launches not covered elsewhere: the gate/up pair at one token (5120 ->
    17408), Q4_K ffn_down at one token (17408 -> 5120), and the Q6_K output projection 248320 x 5120
    (1.04 GB; checked on a stride of rows, its weights synthesised on the GPU by the generator that is
    bitwise equal to the oracle's, so the host builds only the checked rows).

Bars: the reference's 1e-3 (both metrics: max |y - ref| / sum |w x| and normwise) and the int8
kernel's own TOL_I8.  The GLU product is held to the matmul bound carried through silu(g) u with
silu's Lipschitz constant (|silu'| < 1.1): |dy| <= 1.1 |u| dg + |silu(g)| du, dg and du the matmul
errors, each at most TOL times its sum |w x|.
"""
import numpy as np
import pytest

from oracle_lib import BLOCK_BYTES, SEED_BASE, T_Q4_K, T_Q6_K, rel_errors

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_I8 = 1e-5


def _silu(v):
    with np.errstate(over="ignore"):
        return v / (1.0 + np.exp(-v))


def glu_errors(y, g, gmag, u, umag):
    """(max, normwise) error of y = silu(g) u against the f64 g, u, the max normalised by the matmul
    metric's scale sum |w x| carried through silu(g) u (1.1 bounds |silu'|)."""
    with np.errstate(over="ignore"):
        ref = _silu(g) * u
        scale = 1.1 * np.abs(u) * gmag + np.abs(_silu(g)) * umag
    y = np.asarray(y, np.float64)
    e_max = float(np.max(np.abs(y - ref) / (scale + 1e-30)))
    e_norm = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    return e_max, e_norm


def _plan(qk, ws, glu, m):
    return qk.gemv_plan(ws, glu, m)


def test_config3a_glu_four_tokens(qk, oracle, dev):
    """C3a on the int8 kernel's four-token gate/up plan (two-deep ring, ten waves or more)."""
    k, n, m = 5120, 17408, 4
    wg = oracle.weights(T_Q4_K, n, k, SEED_BASE | 3)
    wu = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x303)
    x = oracle.normal(SEED_BASE | 0x313, m * k).reshape(m, k)
    G = qk.upload(wg, T_Q4_K, k, n, 1)
    U = qk.upload(wu, T_Q4_K, k, n, 1)
    try:
        plan = _plan(qk, [G, U], True, m)
        assert plan["kernel"] == 1 and plan["ring_depth"] == 2 and plan["token_slots"] == 4, plan
        assert plan["waves_per_group"] >= 10, plan
        assert 17408 // 16 * 20 / plan["work_groups"] > 2 * plan["waves_per_group"], plan  # the ring refills
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, gmag = oracle.matmul_f64(T_Q4_K, wg, k, n, x)
    u, umag = oracle.matmul_f64(T_Q4_K, wu, k, n, x)
    e_max, e_norm = glu_errors(y, g, gmag, u, umag)
    assert np.isfinite(y).all()
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


def _matmul_full(qk, oracle, dev, typ, k, n, m, seed, expect_kernel=None, expect_slots=None):
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0x5A5A, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    try:
        plan = _plan(qk, [W], False, m)
        if expect_kernel is not None:
            assert plan["kernel"] == expect_kernel, plan
        if expect_slots is not None:
            assert plan["token_slots"] == expect_slots, plan
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert np.isfinite(y).all()
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


def test_config3b_four_tokens(qk, oracle, dev):
    """C3b: Q4_K, four tokens, K=5120, N=5120 (one launch of the int8 kernel's four-token form)."""
    _matmul_full(qk, oracle, dev, T_Q4_K, 5120, 5120, 4, SEED_BASE | 0x3B, expect_kernel=1, expect_slots=4)


def test_c5_q4k_ffn_down_one_token(qk, oracle, dev):
    """C5's Q4_K ffn_down (odd layers): K=17408, N=5120, one token."""
    _matmul_full(qk, oracle, dev, T_Q4_K, 17408, 5120, 1, SEED_BASE | 0x5D, expect_kernel=1)


def test_c5_glu_one_token(qk, oracle, dev):
    """C5's ffn gate/up launch: the Q4_K pair 5120 -> 17408 at one token."""
    k, n, m = 5120, 17408, 1
    wg = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x5E)
    wu = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x5F)
    x = oracle.normal(SEED_BASE | 0x60A, m * k).reshape(m, k)
    G = qk.upload(wg, T_Q4_K, k, n, 1)
    U = qk.upload(wu, T_Q4_K, k, n, 1)
    try:
        assert _plan(qk, [G, U], True, m)["kernel"] == 1
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, gmag = oracle.matmul_f64(T_Q4_K, wg, k, n, x)
    u, umag = oracle.matmul_f64(T_Q4_K, wu, k, n, x)
    e_max, e_norm = glu_errors(y, g, gmag, u, umag)
    assert np.isfinite(y).all()
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


def test_c5_output_projection(qk, oracle, dev, hip):
    """C5's Q6_K output projection, 248320 x 5120 at one token (1.04 GB of weights): every 61st row
    and the first and last 16-row tiles against the f64 brute force of the same rows."""
    typ, k, n, m = T_Q6_K, 5120, 248320, 1
    seed = SEED_BASE | 11
    nsb = k // 256
    rb = nsb * BLOCK_BYTES[typ]
    tmp = dev.empty(n * rb)
    dst = dev.empty(n * rb)
    try:
        qk.synth_fill(typ, seed, 0, n * nsb, tmp.ptr)
        W = qk.repack(qk.weight_view(tmp.ptr, typ, k, n, 0), dst.ptr, 1)
        hip.sync()
        tmp.close()
        assert _plan(qk, [W], False, m)["kernel"] == 1
        x = oracle.normal(seed ^ 0x77, m * k).reshape(m, k)
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        tmp.close()
        dst.close()
    assert np.isfinite(y).all()
    rows = np.unique(np.concatenate([np.arange(0, n, 61), np.arange(16), np.arange(n - 16, n)]))
    w = np.concatenate([oracle.fill(typ, seed, int(r) * nsb, nsb) for r in rows])
    ref, mag = oracle.matmul_f64(typ, w, k, len(rows), x)
    e_max, e_norm = rel_errors(y[:, rows], ref, mag)
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm)


def test_glu_q6k_four_tokens_refill(qk, oracle, dev):
    """A Q6_K gate/up pair at four tokens with more units per work-group than its waves hold in their
    rings, on whichever kernel the plan picks (recorded in the assertion message)."""
    k, n, m = 5120, 8192, 4
    wg = oracle.weights(T_Q6_K, n, k, SEED_BASE | 0x6A)
    wu = oracle.weights(T_Q6_K, n, k, SEED_BASE | 0x6B)
    x = oracle.normal(SEED_BASE | 0x6C, m * k).reshape(m, k)
    G = qk.upload(wg, T_Q6_K, k, n, 1)
    U = qk.upload(wu, T_Q6_K, k, n, 1)
    try:
        plan = _plan(qk, [G, U], True, m)
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, gmag = oracle.matmul_f64(T_Q6_K, wg, k, n, x)
    u, umag = oracle.matmul_f64(T_Q6_K, wu, k, n, x)
    e_max, e_norm = glu_errors(y, g, gmag, u, umag)
    assert np.isfinite(y).all()
    assert e_max <= TOL_I8 and e_norm <= TOL_I8, (e_max, e_norm, plan)

"""GPU parity of the weight-placement path and the fused-dequant GEMV, through the C ABI.

Oracle: tests/oracle_lib.py (CPU restatement of qwen_cpu/quants.h + ops.h, pinned in
test_oracle.py).  Bars: dequant bit-exact; matmul max_{t,n}|y - ref|/sum|w x| <= 1e-3 and
normwise <= 1e-3 against the f64 brute force.  Tighter bars per path:
  * general kernel (gemv_fused = 0, or a forced wave count): x as an exact fp16 pair, fp32
    accumulation -> TOL_PAIR = 1e-5;
  * int8 kernel (the default for m <= 4 per launch): x as three int8 parts per super-block, each
    element within max|x| / 16387064 of its value, integer dot products -> TOL_I8 = 1e-5 (measured
    ~5e-7 normwise for N(0,1) x).
"""
import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q6_K, rel_errors

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL_PAIR = 1e-5
TOL_I8 = 1e-5


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("layout", [0, 1], ids=["gguf", "t16"])
def test_dequant_bitexact(qk, oracle, dev, typ, layout):
    k, n = 1024, 48
    w = oracle.weights(typ, n, k, SEED_BASE | 0x31)
    W = qk.upload(w, typ, k, n, layout)
    try:
        rows = np.array([0, 1, 15, 16, 17, 31, 47], np.int32)
        rows_d = dev.put(rows)
        out = dev.empty(len(rows) * k * 4)
        qk.dequant_rows(W, rows_d.ptr, len(rows), out.ptr, dev.stream())
        got = out.get(np.float32, (len(rows), k))
        ref = oracle.dequant_matrix(typ, w, k, n)[rows]
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    finally:
        qk.free(W)


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
def test_repack_roundtrip(qk, oracle, dev, typ):
    k, n = 2048, 32
    w = oracle.weights(typ, n, k, SEED_BASE | 0x32)
    W = qk.upload(w, typ, k, n, 1)
    try:
        t16 = dev.empty(w.size)
        back = dev.empty(w.size)
        # T16 bytes are a permutation of the GGUF bytes; T16 -> GGUF restores them exactly
        Wc = qk.repack(W, t16.ptr, 1)
        G = qk.repack(Wc, back.ptr, 0)
        perm = t16.get(np.uint8)
        assert np.array_equal(np.sort(perm), np.sort(w))
        assert not np.array_equal(perm, w)
        assert np.array_equal(back.get(np.uint8), w)
        assert G.layout == 0
    finally:
        qk.free(W)


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
def test_synth_matches_host(qk, oracle, dev, typ):
    seed, block0, nblocks = SEED_BASE | 0x33, 1234, 777
    bs = 144 if typ == T_Q4_K else 210
    out = dev.empty(nblocks * bs)
    qk.synth_fill(typ, seed, block0, nblocks, out.ptr, dev.stream())
    assert np.array_equal(out.get(np.uint8), oracle.fill(typ, seed, block0, nblocks))


def _check_matmul(qk, oracle, dev, typ, k, n, m, seed, waves=0, fused=1):
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0xABC, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        if waves:
            qk.set_tuning("gemv_waves", waves)
        qk.set_tuning("gemv_fused", fused)
        qk.set_tuning("gemm_min_m", 16)  # the GEMV at every m here (qk_matmul takes the GEMM from five)
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemv_waves", 0)
        qk.set_tuning("gemv_fused", 1)
        qk.set_tuning("gemm_min_m", 0)
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert np.isfinite(y).all()
    assert e_max <= TOL and e_norm <= TOL, (e_max, e_norm)
    return y, ref, e_max, e_norm


SHAPES = [(256, 16), (512, 48), (1024, 64), (5120, 256)]


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("k,n", SHAPES, ids=[f"k{k}n{n}" for k, n in SHAPES])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("fused", [1, 0])
def test_gemv_parity(qk, oracle, dev, typ, k, n, m, fused):
    """Both GEMV kernels (fused = 0 keeps Q4_K / Q6_K on the general kernel) at every token count of
    a launch (m = 3 leaves one of the int8 kernel's four token slots empty; m = 8 is two launches)."""
    _, _, e_max, e_norm = _check_matmul(qk, oracle, dev, typ, k, n, m, SEED_BASE | (0x40 + m), fused=fused)
    bar = TOL_I8 if fused else TOL_PAIR
    assert e_max < bar and e_norm < bar, (e_max, e_norm)


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("waves", [1, 3, 7, 20, 61, 140])
def test_gemv_stream_split(qk, oracle, dev, typ, waves):
    """Persistent grid with a forced wave count: whole tiles per wave (1, 7), tiles split in two
    (3, 20) and tiles shared by many waves (61, 140 > 7 tiles x 20 super-blocks / 2)."""
    _check_matmul(qk, oracle, dev, typ, 5120, 112, 3, SEED_BASE | 0x50, waves=waves)


# (13056, 2048): three K-slices (a slice-tree node without a sibling), ranges straddling slices and
# groups; (19200, 1600): five slices for Q6_K, three for Q4_K
FUSED_SHAPES = [(256, 16), (512, 48), (1024, 64), (5120, 256), (17408, 1024), (6144, 5120), (13056, 2048),
                (19200, 1600)]


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("k,n", FUSED_SHAPES, ids=[f"k{k}n{n}" for k, n in FUSED_SHAPES])
def test_gemv_single_token_kernels(qk, oracle, dev, typ, k, n):
    """m == 1 through the single-token kernel (x converted in LDS, units handed out inside a CU,
    tiles shared by several work-groups) and through the general kernel."""
    y1, _, e1, n1 = _check_matmul(qk, oracle, dev, typ, k, n, 1, SEED_BASE | 0x5A, fused=1)
    y0, _, e0, n0 = _check_matmul(qk, oracle, dev, typ, k, n, 1, SEED_BASE | 0x5A, fused=0)
    assert max(e1, n1) < TOL_I8 and max(e0, n0) < TOL_PAIR, (e1, n1, e0, n0)


@pytest.mark.parametrize("m", [11, 15])
def test_gemv_many_tokens(qk, oracle, dev, m):
    _check_matmul(qk, oracle, dev, T_Q4_K, 1024, 64, m, SEED_BASE | 0x51)


def test_config1_q4k_full(qk, oracle, dev):
    """Q4_K M=1 K=5120 N=17408."""
    _check_matmul(qk, oracle, dev, T_Q4_K, 5120, 17408, 1, SEED_BASE | 1)


def test_config2_q6k_full(qk, oracle, dev):
    """Q6_K M=1 K=17408 N=5120."""
    _check_matmul(qk, oracle, dev, T_Q6_K, 17408, 5120, 1, SEED_BASE | 2)


GLU_CASES = [(1, 1024, 128, 1), (1, 1024, 128, 0), (1, 5120, 1024, 1), (1, 13056, 2048, 1), (4, 1024, 128, 1),
             (4, 5120, 1024, 1), (4, 5120, 1024, 0), (2, 17408, 1024, 1), (3, 13056, 2048, 1)]


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q6_K], ids=["q4k", "q6k"])
@pytest.mark.parametrize("m,k,n,fused", GLU_CASES, ids=[f"m{m}k{k}n{n}f{f}" for m, k, n, f in GLU_CASES])
def test_gemv_glu(qk, oracle, dev, typ, m, k, n, fused):
    """Gate/up pair with the SiLU product, through the int8 kernel (fused=1) and the general kernel
    (fused=0)."""
    wg = oracle.weights(typ, n, k, SEED_BASE | 0x60)
    wu = oracle.weights(typ, n, k, SEED_BASE | 0x61)
    x = oracle.normal(SEED_BASE | 0x62, m * k).reshape(m, k)
    G = qk.upload(wg, typ, k, n, 1)
    U = qk.upload(wu, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.set_tuning("gemv_fused", fused)
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemv_fused", 1)
        qk.free(G)
        qk.free(U)
    g, _ = oracle.matmul_f64(typ, wg, k, n, x)
    u, _ = oracle.matmul_f64(typ, wu, k, n, x)
    ref = g / (1.0 + np.exp(-g)) * u
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < (TOL_I8 if fused else TOL_PAIR), err


@pytest.mark.parametrize("m", [1, 2])
def test_gemv_group_mixed(qk, oracle, dev, m):
    """MmGroup-style launch over matrices of different types and heights sharing x (m == 1: the
    single-token kernel, as the decode step's {qkv, gate_z, alpha, beta} launch uses it; small
    matrices may take either kernel, TOL_I8 bounds both)."""
    k = 2048
    tol = TOL_I8
    specs = [(T_Q4_K, 64), (T_Q4_K, 48), (T_Q6_K, 32), (T_Q4_K, 16)]
    x = oracle.normal(SEED_BASE | 0x70, m * k).reshape(m, k)
    ws, Ws, ys = [], [], []
    try:
        for i, (typ, n) in enumerate(specs):
            w = oracle.weights(typ, n, k, SEED_BASE | (0x71 + i))
            ws.append(w)
            Ws.append(qk.upload(w, typ, k, n, 1))
            ys.append(dev.empty(m * n * 4))
        xd = dev.put(x)
        qk.gemv_group(Ws, [y.ptr for y in ys], False, xd.ptr, m, dev.stream())
        for (typ, n), w, y in zip(specs, ws, ys):
            ref, mag = oracle.matmul_f64(typ, w, k, n, x)
            e_max, e_norm = rel_errors(y.get(np.float32, (m, n)), ref, mag)
            assert e_max < tol and e_norm < tol, (typ, n, e_max, e_norm)
    finally:
        for W in Ws:
            qk.free(W)


DECODE_GROUPS = {
    "linear_attn": [(T_Q4_K, 10240), (T_Q4_K, 6144), (T_Q4_K, 48), (T_Q4_K, 48)],
    "full_attn": [(T_Q4_K, 12288), (T_Q4_K, 1024), (T_Q6_K, 1024)],
}


@pytest.mark.parametrize("group", sorted(DECODE_GROUPS))
def test_gemv_group_decode_shapes(qk, oracle, dev, group):
    """The decode step's shared-x launches at their real shapes (qwen_cuda/qwen.cpp:262-290):
    {qkv, gate_z, alpha, beta} and {q, k, v} at K=5120, one token."""
    k, m = 5120, 1
    specs = DECODE_GROUPS[group]
    x = oracle.normal(SEED_BASE | 0x90, m * k).reshape(m, k)
    ws, Ws, ys = [], [], []
    try:
        for i, (typ, n) in enumerate(specs):
            w = oracle.weights(typ, n, k, SEED_BASE | (0x91 + i))
            ws.append(w)
            Ws.append(qk.upload(w, typ, k, n, 1))
            ys.append(dev.empty(m * n * 4))
        xd = dev.put(x)
        qk.gemv_group(Ws, [y.ptr for y in ys], False, xd.ptr, m, dev.stream())
        for (typ, n), w, y in zip(specs, ws, ys):
            ref, mag = oracle.matmul_f64(typ, w, k, n, x)
            e_max, e_norm = rel_errors(y.get(np.float32, (m, n)), ref, mag)
            assert e_max < TOL_I8 and e_norm < TOL_I8, (typ, n, e_max, e_norm)
    finally:
        for W in Ws:
            qk.free(W)


def test_repeat_launch_deterministic(qk, oracle, dev):
    """Split-K counters self-reset: repeated launches give bit-identical results."""
    k, n, m = 5120, 1024, 1
    w = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x80)
    x = oracle.normal(SEED_BASE | 0x81, m * k).reshape(m, k)
    W = qk.upload(w, T_Q4_K, k, n, 1)
    try:
        xd = dev.put(x)
        outs = []
        for _ in range(3):
            yd = dev.empty(m * n * 4)
            qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
            outs.append(yd.get(np.float32, (m, n)))
        assert all(np.array_equal(outs[0].view(np.uint32), o.view(np.uint32)) for o in outs[1:])
    finally:
        qk.free(W)

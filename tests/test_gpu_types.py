"""GPU parity of the Q8_0 and Q5_K paths (the other GGUF types of a Q4_K_M file; the reference's CUDA
backend instantiates its GEMV, GEMM and dequant for them: qwen_cuda/kernels.cu:74-125, 211-236,
397-401), through the C ABI.

Oracle: tests/oracle_lib.py (pinned for these types in test_oracle.py: closed forms and bitwise
against the reference's own quants.h/ops.h).  Bars: dequant bit-exact from both layouts; matmul
max_{t,n}|y - ref|/sum|w x| and normwise error against the f64 brute force: m < 16 runs the
int8 kernel (x as three int8 parts per super-block, each element within max|x| / 16387064 of its
value, integer dot products) -> TOL_I8 = 1e-5, under the 1e-3 bar of the reference's fp32 paths;
m >= 16 runs the fp16 MFMA GEMM ->
TOL_MFMA = 5e-3 against the unrounded x (test_gpu_gemm.py checks it against fp16-rounded x too).
"""
import numpy as np
import pytest

from oracle_lib import GEMM_ROUTE_M, SEED_BASE, T_Q4_K, T_Q5_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu

TOL_I8 = 1e-5
TOL_MFMA = 5e-3
TYPES = [T_Q8_0, T_Q5_K]
IDS = ["q8_0", "q5k"]
RUN_BYTES = {T_Q8_0: 272, T_Q5_K: 176}


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("layout", [0, 1], ids=["gguf", "t16"])
def test_dequant_bitexact(qk, oracle, dev, typ, layout):
    k, n = 1024, 48
    w = oracle.weights(typ, n, k, SEED_BASE | 0x131)
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


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
def test_repack_roundtrip(qk, oracle, dev, typ):
    k, n = 2048, 32
    w = oracle.weights(typ, n, k, SEED_BASE | 0x132)
    W = qk.upload(w, typ, k, n, 1)
    try:
        t16 = dev.empty(w.size)
        back = dev.empty(w.size)
        Wc = qk.repack(W, t16.ptr, 1)
        qk.repack(Wc, back.ptr, 0)
        perm = t16.get(np.uint8)
        assert np.array_equal(np.sort(perm), np.sort(w)) and not np.array_equal(perm, w)
        assert np.array_equal(back.get(np.uint8), w)
    finally:
        qk.free(W)


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
def test_synth_matches_host(qk, oracle, dev, typ):
    seed, block0, nblocks = SEED_BASE | 0x133, 1234, 777
    out = dev.empty(nblocks * RUN_BYTES[typ])
    qk.synth_fill(typ, seed, block0, nblocks, out.ptr, dev.stream())
    assert np.array_equal(out.get(np.uint8), oracle.fill(typ, seed, block0, nblocks))


def _matmul(qk, oracle, dev, typ, k, n, m, seed):
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0xABC, m * k).reshape(m, k)
    W = qk.upload(w, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    assert np.isfinite(y).all()
    e_max, e_norm = rel_errors(y, ref, mag)
    bar = TOL_I8 if m < GEMM_ROUTE_M else TOL_MFMA
    assert e_max < bar and e_norm < bar, (e_max, e_norm)
    return y


# small shapes, the model's shapes, several K-slices ((13056, 2048): three; (19200, 1600): more),
# and prefill-sized m (the GEMM)
CASES = [(256, 16, 1), (1024, 64, 2), (5120, 256, 4), (5120, 48, 1), (6144, 5120, 1), (5120, 1024, 1),
         (17408, 1024, 1), (13056, 2048, 1), (19200, 1600, 1), (5120, 1024, 3), (17408, 1024, 4),
         (13056, 2048, 2), (1024, 64, 7), (1024, 64, 16), (512, 48, 21)]


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("k,n,m", CASES, ids=[f"k{k}n{n}m{m}" for k, n, m in CASES])
def test_matmul_parity(qk, oracle, dev, typ, k, n, m):
    _matmul(qk, oracle, dev, typ, k, n, m, SEED_BASE | (0x140 + m))


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_glu(qk, oracle, dev, typ, m):
    k, n = 5120, 1024
    wg = oracle.weights(typ, n, k, SEED_BASE | 0x160)
    wu = oracle.weights(typ, n, k, SEED_BASE | 0x161)
    x = oracle.normal(SEED_BASE | 0x162, m * k).reshape(m, k)
    G = qk.upload(wg, typ, k, n, 1)
    U = qk.upload(wu, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, _ = oracle.matmul_f64(typ, wg, k, n, x)
    u, _ = oracle.matmul_f64(typ, wu, k, n, x)
    ref = g / (1.0 + np.exp(np.minimum(-g, 700.0))) * u
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < TOL_I8


def test_group_mixed_types(qk, oracle, dev):
    """A Q4_K_M-style attention group sharing x: q (Q4_K), k and v (Q8_0), o-shaped Q5_K, one token."""
    k = 5120
    mats = [(T_Q4_K, 1024), (T_Q8_0, 256), (T_Q8_0, 256), (T_Q5_K, 512)]
    x = oracle.normal(SEED_BASE | 0x170, k).reshape(1, k)
    ws, Ws, ys = [], [], []
    try:
        for i, (typ, n) in enumerate(mats):
            w = oracle.weights(typ, n, k, SEED_BASE | (0x171 + i))
            ws.append(w)
            Ws.append(qk.upload(w, typ, k, n, 1))
            y = dev.empty(n * 4)
            y.fill_nan()
            ys.append(y)
        xd = dev.put(x)
        qk.gemv_group(Ws, [y.ptr for y in ys], False, xd.ptr, 1, dev.stream())
        for (typ, n), w, y in zip(mats, ws, ys):
            ref, mag = oracle.matmul_f64(typ, w, k, n, x)
            e_max, e_norm = rel_errors(y.get(np.float32, (1, n)), ref, mag)
            assert e_max < TOL_I8 and e_norm < TOL_I8, (typ, e_max, e_norm)
    finally:
        for W in Ws:
            qk.free(W)


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
def test_repeat_launch_deterministic(qk, oracle, dev, typ):
    k, n = 17408, 1024  # several K-slices: the combine tree runs every launch
    w = oracle.weights(typ, n, k, SEED_BASE | 0x180)
    x = oracle.normal(SEED_BASE | 0x181, k).reshape(1, k)
    W = qk.upload(w, typ, k, n, 1)
    try:
        xd = dev.put(x)
        outs = []
        for _ in range(3):
            yd = dev.empty(n * 4)
            qk.matmul(W, xd.ptr, 1, yd.ptr, dev.stream())
            outs.append(yd.get(np.uint32, (1, n)))
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
    finally:
        qk.free(W)


# ------------------------------------------------------------------------------------------------
# F32 weights, used as stored (GGUF layout): fp32 FMA accumulation -> TOL_F32 = 1e-5
TOL_F32 = 1e-5
T_F32 = 0


def _f32_weights(n, k, seed):
    return np.random.default_rng(seed).standard_normal((n, k)).astype(np.float32).view(np.uint8).reshape(-1)


@pytest.mark.parametrize("k,n,m", [(5120, 48, 1), (5120, 48, 4), (1024, 100, 16), (2048, 37, 40)],
                         ids=["alpha_m1", "alpha_m4", "n100_m16", "n37_m40"])
def test_f32_matmul(qk, oracle, dev, k, n, m):
    w = _f32_weights(n, k, SEED_BASE | 0x190 | m)
    x = oracle.normal(SEED_BASE | 0x191, m * k).reshape(m, k)
    W = qk.upload(w, T_F32, k, n, 0)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
        rows = np.array([0, n // 2, n - 1], np.int32)
        rd = dev.put(rows)
        out = dev.empty(len(rows) * k * 4)
        qk.dequant_rows(W, rd.ptr, len(rows), out.ptr, dev.stream())
        assert np.array_equal(out.get(np.uint32, (len(rows), k)), w.view(np.uint32).reshape(n, k)[rows])
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(T_F32, w, k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert e_max < TOL_F32 and e_norm < TOL_F32, (e_max, e_norm)


def test_f32_in_decode_group(qk, oracle, dev):
    """The DeltaNet input group {qkv, gate_z, alpha, beta} with alpha/beta kept in F32, as the real
    file stores them (docs/model.md:328), one token."""
    k = 5120
    specs = [(T_Q4_K, 1024), (T_Q4_K, 512), (T_F32, 48), (T_F32, 48)]
    x = oracle.normal(SEED_BASE | 0x1A0, k).reshape(1, k)
    ws, Ws, ys = [], [], []
    try:
        for i, (typ, n) in enumerate(specs):
            w = _f32_weights(n, k, SEED_BASE | (0x1A1 + i)) if typ == T_F32 else oracle.weights(typ, n, k, SEED_BASE | (0x1A1 + i))
            ws.append(w)
            Ws.append(qk.upload(w, typ, k, n, 0 if typ == T_F32 else 1))
            y = dev.empty(n * 4)
            y.fill_nan()
            ys.append(y)
        xd = dev.put(x)
        qk.gemv_group(Ws, [y.ptr for y in ys], False, xd.ptr, 1, dev.stream())
        for (typ, n), w, y in zip(specs, ws, ys):
            ref, mag = oracle.matmul_f64(typ, w, k, n, x)
            e_max, e_norm = rel_errors(y.get(np.float32, (1, n)), ref, mag)
            bar = TOL_F32 if typ == T_F32 else TOL_I8
            assert e_max < bar and e_norm < bar, (typ, e_max, e_norm)
    finally:
        for W in Ws:
            qk.free(W)


def test_f32_rejects_t16(qk, qkmod, dev):
    w = _f32_weights(16, 256, 1)
    with pytest.raises(qkmod.QkError):
        qk.upload(w, T_F32, 256, 16, 1)


# Irregular shapes through the default plans of every type: super-block counts with few divisors
# (9, 18, 31, 44, 14, 38), odd tile counts, every token count of a launch, and prefill sizes that
# take the split-K GEMM.
IRREGULAR = [(2304, 80, 1), (4608, 144, 3), (7936, 400, 2), (11264, 208, 4), (3584, 2000, 1), (9728, 96, 1),
             (7936, 400, 24), (9728, 336, 130)]


@pytest.mark.parametrize("typ", [T_Q8_0, T_Q4_K, T_Q5_K, 14], ids=["q8_0", "q4k", "q5k", "q6k"])
@pytest.mark.parametrize("k,n,m", IRREGULAR, ids=[f"k{k}n{n}m{m}" for k, n, m in IRREGULAR])
def test_irregular_shapes(qk, oracle, dev, typ, k, n, m):
    _matmul(qk, oracle, dev, typ, k, n, m, SEED_BASE | (0x1D0 + m + n))


GLU_IRREGULAR = [(2304, 80, 1), (4608, 144, 3), (11264, 208, 4), (9728, 336, 2)]


@pytest.mark.parametrize("typ", [T_Q8_0, T_Q4_K, T_Q5_K, 14], ids=["q8_0", "q4k", "q5k", "q6k"])
@pytest.mark.parametrize("k,n,m", GLU_IRREGULAR, ids=[f"k{k}n{n}m{m}" for k, n, m in GLU_IRREGULAR])
def test_glu_irregular(qk, oracle, dev, typ, k, n, m):
    wg = oracle.weights(typ, n, k, SEED_BASE | 0x1E0)
    wu = oracle.weights(typ, n, k, SEED_BASE | 0x1E1)
    x = oracle.normal(SEED_BASE | (0x1E2 + m), m * k).reshape(m, k)
    G = qk.upload(wg, typ, k, n, 1)
    U = qk.upload(wu, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, _ = oracle.matmul_f64(typ, wg, k, n, x)
    u, _ = oracle.matmul_f64(typ, wu, k, n, x)
    ref = g / (1.0 + np.exp(np.minimum(-g, 700.0))) * u
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < TOL_I8


def _random_cases(count, seed):
    """Seeded shapes off the model's grid: super-block counts 1..72, tile counts 1..320 (odd ones
    included), every token count of a GEMV launch and a few prefill sizes."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        typ = [T_Q8_0, T_Q4_K, T_Q5_K, 14][i % 4]
        k = 256 * int(rng.integers(1, 73))
        n = 16 * int(rng.integers(1, 41 if i % 2 else 321))
        m = int(rng.choice([1, 1, 2, 3, 4, 17, 70]))
        out.append((typ, k, n, m))
    return out


RANDOM = _random_cases(28, 0x5EED)


@pytest.mark.parametrize("typ,k,n,m", RANDOM, ids=[f"t{t}k{k}n{n}m{m}" for t, k, n, m in RANDOM])
def test_random_shapes(qk, oracle, dev, typ, k, n, m):
    _matmul(qk, oracle, dev, typ, k, n, m, SEED_BASE | (0x2A0 + k // 256 + n + m))


RANDOM_GLU = [(t, k, n, m) for t, k, n, m in _random_cases(12, 0x61A) if m <= 4]


@pytest.mark.parametrize("typ,k,n,m", RANDOM_GLU, ids=[f"t{t}k{k}n{n}m{m}" for t, k, n, m in RANDOM_GLU])
def test_random_glu_shapes(qk, oracle, dev, typ, k, n, m):
    """The gate/up pair with its SiLU product at seeded shapes (the GLU launch runs m <= 4)."""
    seed = SEED_BASE | (0x2C0 + k // 256 + n + m)
    wg, wu = oracle.weights(typ, n, k, seed), oracle.weights(typ, n, k, seed + 1)
    x = oracle.normal(seed ^ 0x5A, m * k).reshape(m, k)
    G, U = qk.upload(wg, typ, k, n, 1), qk.upload(wu, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.gemv_group([G, U], [yd.ptr], True, xd.ptr, m, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(G)
        qk.free(U)
    g, _ = oracle.matmul_f64(typ, wg, k, n, x)
    u, _ = oracle.matmul_f64(typ, wu, k, n, x)
    ref = g / (1.0 + np.exp(np.minimum(-g, 700.0))) * u
    assert np.isfinite(y).all()
    assert np.linalg.norm(y - ref) / np.linalg.norm(ref) < TOL_I8

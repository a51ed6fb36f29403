"""GPU parity of the prefill GEMM (m >= 9 through qk_matmul, LDS-dequant MFMA, fp16 operands, fp32
accumulate), on fp32 x, fp16 x and the reference's xperm fp16 layout.

The bar of the MFMA path (5e-3, both metrics) is taken against the f64 brute force fed the same
fp16-rounded activations the kernel uses (as the reference's GPU selftest does with fp16-exact
inputs, qwen_cuda/qwen.cpp:1335-1356); the error against the unrounded fp32 x is checked too.
"""
import numpy as np
import pytest

from oracle_lib import BLOCK_BYTES, SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

TYPES = [T_Q4_K, T_Q6_K, T_Q5_K, T_Q8_0]
IDS = ["q4k", "q6k", "q5k", "q8_0"]

pytestmark = pytest.mark.gpu

TOL_MFMA = 5e-3


def _run_gemm(qk, dev, w, typ, k, n, x, pairs=0, gmap=1, ks=0):
    m = x.shape[0]
    W = qk.upload(w, typ, k, n, 1)
    try:
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        if pairs:
            qk.set_tuning("gemm_pairs", pairs)
        qk.set_tuning("gemm_ksplit", ks)
        qk.set_tuning("gemm_map", gmap)
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        return yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemm_pairs", 0)
        qk.set_tuning("gemm_ksplit", 0)
        qk.set_tuning("gemm_map", 1)
        qk.free(W)


def _check(qk, oracle, dev, typ, k, n, m, seed, pairs=0, rows=None, toks=None, gmap=1, ks=0):
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed ^ 0x5A5A, m * k).reshape(m, k)
    y = _run_gemm(qk, dev, w, typ, k, n, x, pairs, gmap, ks)
    assert np.isfinite(y).all()
    rows = np.arange(n) if rows is None else rows
    toks = np.arange(m) if toks is None else toks
    rb = len(w) // n
    wsub = w.reshape(n, rb)[rows].reshape(-1)
    x16 = x[toks].astype(np.float16).astype(np.float32)  # the kernel's operand rounding (RNE)
    ref, mag = oracle.matmul_f64(typ, wsub, k, len(rows), x16)
    ysub = y[np.ix_(toks, rows)]
    e_max, e_norm = rel_errors(ysub, ref, mag)
    assert e_max <= TOL_MFMA and e_norm <= TOL_MFMA, (e_max, e_norm)
    ref32, mag32 = oracle.matmul_f64(typ, wsub, k, len(rows), x[toks])
    e32 = rel_errors(ysub, ref32, mag32)
    assert e32[0] <= TOL_MFMA and e32[1] <= TOL_MFMA, e32
    return e_max, e_norm


SHAPES = [(256, 16, 16), (512, 48, 37), (1024, 80, 128), (2048, 272, 129), (5120, 160, 300)]


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("k,n,m", SHAPES, ids=[f"k{k}n{n}m{m}" for k, n, m in SHAPES])
def test_gemm_parity(qk, oracle, dev, typ, k, n, m):
    e_max, e_norm = _check(qk, oracle, dev, typ, k, n, m, SEED_BASE | (0x70 + m))
    # fp16 weights (scales rounded as in the reference's GEMM) and fp16 x: ~1e-4 typical
    assert e_max < 2e-3 and e_norm < 2e-3, (e_max, e_norm)


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("pairs", [2, 3, 4, 5, 8, 9])
def test_gemm_pair_counts(qk, oracle, dev, typ, pairs):
    """Every compiled tile-pairs-per-work-group width, with a partial last work-group and an odd
    tile count (23 tiles: the last pair has one tile)."""
    _check(qk, oracle, dev, typ, 1024, 23 * 16, 40, SEED_BASE | 0x7F, pairs=pairs)


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("ks", [2, 3, 5])
def test_gemm_split_k(qk, oracle, dev, typ, ks):
    """K cut into ks parts (uneven for 3 and 5 over 12 super-blocks), partials added in part order
    by the second kernel; 23 tiles and 40 tokens leave partial pair groups and token blocks."""
    _check(qk, oracle, dev, typ, 3072, 23 * 16, 40, SEED_BASE | 0x7D, pairs=3, ks=ks)


def test_gemm_split_k_deterministic(qk, oracle, dev):
    k, n, m = 4096, 256, 130
    w = oracle.weights(T_Q5_K, n, k, SEED_BASE | 0x85)
    x = oracle.normal(SEED_BASE | 0x86, m * k).reshape(m, k)
    y1 = _run_gemm(qk, dev, w, T_Q5_K, k, n, x, ks=4)
    y2 = _run_gemm(qk, dev, w, T_Q5_K, k, n, x, ks=4)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


MAP_CASES = [(128, 0, 0), (128, 1, 0), (200, 1, 0), (500, 0, 0), (500, 1, 0), (1000, 1, 0), (500, 0, 3),
             (500, 1, 3), (200, 0, 4), (200, 1, 4), (1000, 0, 2), (1000, 1, 3), (1100, 1, 2)]


@pytest.mark.parametrize("m,gmap,ks", MAP_CASES, ids=[f"m{m}map{g}ks{ks}" for m, g, ks in MAP_CASES])
def test_gemm_xcd_maps(qk, oracle, dev, m, gmap, ks):
    """Both work-group -> (pair group, token block, K-part) maps, each dealing the (K-part, pair group)
    units densely: over the XCDs of each token block (2, 4 and 8 token blocks: 4, 2 and 1 XCDs per
    block) or over all XCDs with a unit's token blocks side by side, with one K-part (planned) and with
    2, 3 and 4; 1100 tokens are nine token blocks, which take the second map whatever the knob says.
    23 tiles at 3 pairs per work-group leave a partial last pair group."""
    _check(qk, oracle, dev, T_Q4_K, 1024, 23 * 16, m, SEED_BASE | 0x7E, pairs=3, gmap=gmap, ks=ks)


@pytest.mark.parametrize("m,ks", [(500, 0), (500, 3), (1000, 2)])
def test_gemm_xcd_maps_bitwise_equal(qk, oracle, dev, m, ks):
    """Which work-group takes a (pair group, token block, K-part) never changes the result: both maps
    give the same bits (each part's sums in the same order, the parts added in part order)."""
    k, n = 2048, 23 * 16
    w = oracle.weights(T_Q6_K, n, k, SEED_BASE | 0x7F)
    x = oracle.normal(SEED_BASE | 0x80, m * k).reshape(m, k)
    y0 = _run_gemm(qk, dev, w, T_Q6_K, k, n, x, pairs=3, gmap=0, ks=ks)
    y1 = _run_gemm(qk, dev, w, T_Q6_K, k, n, x, pairs=3, gmap=1, ks=ks)
    assert np.isfinite(y0).all()
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


def test_gemm_deterministic(qk, oracle, dev):
    k, n, m = 2048, 128, 64
    w = oracle.weights(T_Q4_K, n, k, SEED_BASE | 0x81)
    x = oracle.normal(SEED_BASE | 0x82, m * k).reshape(m, k)
    y1 = _run_gemm(qk, dev, w, T_Q4_K, k, n, x)
    y2 = _run_gemm(qk, dev, w, T_Q4_K, k, n, x)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


@pytest.mark.parametrize("typ", [T_Q6_K, T_Q8_0], ids=["q6k", "q8_0"])
def test_gemm_single_activation(qk, oracle, dev, typ):
    """x with one nonzero element per token selects dequantized weight columns (types without a
    min term: each fp16 weight is the exact one rounded once)."""
    k, n, m = 1024, 64, 32
    w = oracle.weights(typ, n, k, SEED_BASE | 0x83)
    x = np.zeros((m, k), np.float32)
    cols = (np.arange(m) * 37) % k
    x[np.arange(m), cols] = 1.0
    y = _run_gemm(qk, dev, w, typ, k, n, x)
    deq = oracle.dequant_matrix(typ, w, k, n)
    want = deq[:, cols].T  # fp32 weights; the kernel holds them as fp16
    assert np.allclose(y, want, rtol=2 ** -10, atol=1e-7)


@pytest.mark.parametrize("typ,k,n", [(T_Q5_K, 17408, 5120), (T_Q8_0, 6144, 5120)], ids=["q5k_down", "q8_0_o"])
def test_gemm_model_shapes(qk, oracle, dev, typ, k, n):
    """The shapes these types take in a Q4_K_M file (ffn_down Q5_K, attn_output Q8_0), strided rows."""
    _check(qk, oracle, dev, typ, k, n, 160, SEED_BASE | 0x84, rows=np.arange(0, n, 37))


PLANNED = [(T_Q4_K, 100), (T_Q4_K, 200), (T_Q6_K, 100), (T_Q6_K, 200), (T_Q6_K, 300), (T_Q5_K, 200),
           (T_Q8_0, 300)]


@pytest.mark.parametrize("typ,m", PLANNED, ids=[f"t{t}m{m}" for t, m in PLANNED])
def test_gemm_planned_long_k(qk, oracle, dev, typ, m):
    """The ffn_down shape (K=17408 N=5120) at 100 to 300 tokens, where the planner splits K over two or
    more token blocks (the plans the (P, K-part) sweeps moved most): the default plan against the f64
    oracle on strided rows and tokens."""
    k, n = 17408, 5120
    _check(qk, oracle, dev, typ, k, n, m, SEED_BASE | 0x8A | (m << 8) | (typ << 16), rows=np.arange(0, n, 41),
           toks=np.arange(0, m, 7))


def test_config4_prefill_full(qk, oracle, dev):
    """Q4_K M=512 K=5120 N=17408, checked on strided rows and tokens
    (every 37th row as in the reference's selftest, qwen_cpu/qwen.cpp:889)."""
    rows = np.arange(0, 17408, 37)
    toks = np.arange(0, 512, 7)
    _check(qk, oracle, dev, T_Q4_K, 5120, 17408, 512, SEED_BASE | 4, rows=rows, toks=toks)


FEW_TOKENS = [(2, 3), (9, 9), (13, 5), (20, 2), (33, 4), (50, 8)]


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m,pairs", FEW_TOKENS, ids=[f"m{m}p{p}" for m, p in FEW_TOKENS])
def test_gemm_few_tokens(qk, oracle, dev, typ, m, pairs):
    """Token counts below one 128-token block run work-groups of one or two 32-token blocks (m = 2
    through the gemm_min_m knob, m >= 9 as qk_matmul routes them); every such width with shared pairs
    in the compute waves (2, 3 pairs), in the DMA waves (5, 9) or none (4, 8), 23 tiles."""
    qk.set_tuning("gemm_min_m", 2)
    try:
        _check(qk, oracle, dev, typ, 1024, 23 * 16, m, SEED_BASE | (0x90 + m), pairs=pairs)
    finally:
        qk.set_tuning("gemm_min_m", 0)


def _xperm_cols(k):
    """xperm position of each element of a row (qwen_cuda/kernels.cu:27-28), k % 1024 == 0."""
    i = np.arange(k)
    return (i & ~1023) | (((i >> 3) & 3) << 8) | (((i >> 8) & 3) << 6) | (((i >> 5) & 7) << 3) | (i & 7)


XPERM_CASES = [(9, 0), (13, 0), (15, 0), (13, 3), (13, 5)]


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m,ks", XPERM_CASES, ids=[f"m{m}ks{ks}" for m, ks in XPERM_CASES])
def test_gemm_xperm(qk, oracle, dev, typ, m, ks):
    """fp16 x in the xperm layout (the reference's decode activations for T < 16, which qk_matmul_act
    sends to the GEMM from nine tokens) gives the GEMM the same values in the same order as plain fp16
    x: bitwise equal outputs, also with K split into 3 or 5 uneven parts (parts starting inside a
    1024-element run), and parity with the oracle."""
    k, n = 3072, 23 * 16
    w = oracle.weights(typ, n, k, SEED_BASE | (0xA0 + m))
    xh = oracle.normal(SEED_BASE | (0xA1 + m), m * k).reshape(m, k).astype(np.float16)
    xp = np.empty_like(xh)
    xp[:, _xperm_cols(k)] = xh
    W = qk.upload(w, typ, k, n, 1)
    outs = {}
    try:
        qk.set_tuning("gemm_ksplit", ks)
        for name, fmt, xa in (("f16", 1, xh), ("xperm", 2, xp)):
            xd = dev.put(xa)
            yd = dev.empty(m * n * 4)
            yd.fill_nan()
            qk.matmul_act(W, xd.ptr, fmt, m, yd.ptr, dev.stream())
            outs[name] = yd.get(np.float32, (m, n))
    finally:
        qk.set_tuning("gemm_ksplit", 0)
        qk.free(W)
    assert np.array_equal(outs["xperm"].view(np.uint32), outs["f16"].view(np.uint32))
    ref, mag = oracle.matmul_f64(typ, w, k, n, xh.astype(np.float32))
    e = rel_errors(outs["xperm"], ref, mag)
    assert e[0] <= TOL_MFMA and e[1] <= TOL_MFMA, e


GROUPS = {
    "linear_attn": [(T_Q4_K, 10240), (T_Q4_K, 6144), (T_Q4_K, 48), (T_Q4_K, 48)],
    "full_attn": [(T_Q4_K, 12288), (T_Q4_K, 1024), (T_Q6_K, 1024)],
    "mixed": [(T_Q5_K, 80), (T_Q5_K, 368), (T_Q8_0, 48), (T_Q8_0, 32)],
}


@pytest.mark.parametrize("m", [9, 13, 15])
@pytest.mark.parametrize("group", sorted(GROUPS))
def test_gemm_group(qk, oracle, dev, group, m):
    """Shared-x launches (qk_gemv_group) from nine tokens: each run of one type in one GEMM launch, a
    matrix per grid z (the decode step's {qkv, gate_z, alpha, beta} and {q, k, v} at K=5120 and their
    real heights; runs split by type; 48- and 80-row matrices leave partial tile pairs).  Every output
    against the f64 oracle fed the fp16-rounded x, at the MFMA path's bar (strided rows of the large
    matrices)."""
    k = 5120 if group != "mixed" else 3072
    specs = GROUPS[group]
    x = oracle.normal(SEED_BASE | (0xB0 + m), m * k).reshape(m, k)
    x16 = x.astype(np.float16).astype(np.float32)
    ws, Ws, ys = [], [], []
    try:
        for i, (typ, n) in enumerate(specs):
            w = oracle.weights(typ, n, k, SEED_BASE | (0xB1 + i))
            ws.append(w)
            Ws.append(qk.upload(w, typ, k, n, 1))
            ys.append(dev.empty(m * n * 4))
            ys[-1].fill_nan()
        assert qk.gemv_plan(Ws, False, m)["kernel"] == 4  # QK_GEMV_GEMM
        xd = dev.put(x)
        qk.gemv_group(Ws, [y.ptr for y in ys], False, xd.ptr, m, dev.stream())
        for (typ, n), w, y in zip(specs, ws, ys):
            rows = np.arange(0, n, max(1, n // 256))
            wsub = w.reshape(n, -1)[rows].reshape(-1)
            yy = y.get(np.float32, (m, n))[:, rows]
            assert np.isfinite(yy).all()
            ref, mag = oracle.matmul_f64(typ, wsub, k, len(rows), x16)
            e_max, e_norm = rel_errors(yy, ref, mag)
            assert e_max <= TOL_MFMA and e_norm <= TOL_MFMA, (typ, n, e_max, e_norm)
    finally:
        for W in Ws:
            qk.free(W)


def test_gemm_group_with_f32(qk, oracle, dev):
    """{qkv, gate_z, alpha, beta} with F32 alpha / beta (the GGUF's own types) at 13 tokens: the Q4_K
    run on the GEMM, the F32 matrices on their own kernel (fp32, exact products)."""
    k, m = 1024, 13
    rng = np.random.default_rng(11)
    wq = [oracle.weights(T_Q4_K, n, k, SEED_BASE | (0xBA + i)) for i, n in enumerate((320, 192))]
    wa = [rng.standard_normal((48, k)).astype(np.float32) for _ in range(2)]
    x = oracle.normal(SEED_BASE | 0xBC, m * k).reshape(m, k)
    Wq = [qk.upload(w, T_Q4_K, k, w.size // (144 * (k // 256)), 1) for w in wq]
    wad = [dev.put(a) for a in wa]
    try:
        Wa = [qk.weight_view(d.ptr, 0, k, 48, 0) for d in wad]
        ys = [dev.empty(m * n * 4) for n in (320, 192, 48, 48)]
        xd = dev.put(x)
        qk.gemv_group(Wq + Wa, [y.ptr for y in ys], False, xd.ptr, m, dev.stream())
        for w, n, y in zip(wq, (320, 192), ys[:2]):
            ref, mag = oracle.matmul_f64(T_Q4_K, w, k, n, x.astype(np.float16).astype(np.float32))
            e = rel_errors(y.get(np.float32, (m, n)), ref, mag)
            assert e[0] <= TOL_MFMA and e[1] <= TOL_MFMA, e
        for a, y in zip(wa, ys[2:]):
            want = x.astype(np.float64) @ a.T.astype(np.float64)
            assert np.abs(y.get(np.float32, (m, 48)) - want).max() <= 1e-5 * np.abs(want).max()
    finally:
        for W in Wq:
            qk.free(W)

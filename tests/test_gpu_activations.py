"""GPU parity of the GEMV under hard activations, through the C ABI, for all four quantized types and
one to four tokens per launch.

The int8 kernel carries each token's x per 256-element super-block as three int8 parts with fp32
scales (s0 = max|x| / 127, s1 = s0 / 254, s2 = s1 / 254), so an element's error is at most
max|x| / 16387064 of its super-block's largest magnitude.  A single huge element therefore coarsens
its neighbours; these cases put one (or three) elements 1e3..1e5 times the rest into super-blocks,
mix scales 1e4 apart inside super-blocks, and draw heavy-tailed Student-t x (df 1 and 2), and hold
the result to the reference's 1e-3 bar on both metrics (max |y - ref| / sum |w x| and normwise)
and to the representation's own bound, per output:
    |y - ref| <= sum over super-blocks b of max_{k in b} |x_k| / 16387064 * sum_{k in b} |c_k|
                 + 1e-6 sum |w x|   (fp32 scaling and accumulation),
where c_k is the part of the weight that multiplies the int8 activation: d sc q for Q4_K / Q5_K (the
min term dmin m multiplies exact fp32 sums of x), d sc q for Q6_K (the -32 offset multiplies exact
fp32 sums of x), d q for Q8_0.  c is the dequantized weight minus the dequantized weight of the same
blocks with their quants zeroed (qwen_cpu/quants.h:45-121).  The reference's own GPU path rounds x to fp16 instead
(qwen_cuda/kernels.cu:27-28); the reason activation outliers matter is its own note on activation
quantization (notes/parallel_decode_experiments.md:92).

Non-finite activations: a NaN or an inf anywhere in a token's x makes every output of that token
non-finite in the reference's fp32 CPU path (each output sums over all of x); the GPU paths must
give non-finite outputs for that token too (the int8 kernel by NaN scales, the general kernel and the
GEMM by fp16 NaN / inf operands), and leave the other tokens untouched.
"""
import numpy as np
import pytest

from oracle_lib import SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

pytestmark = pytest.mark.gpu

TOL = 1e-3
TYPES = [T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0]
IDS = ["q4k", "q5k", "q6k", "q8_0"]
K, N = 2048, 256


def activations(case, m, k, seed):
    """m tokens of x for one of the hard cases (test-side inputs, seeded)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    if case.startswith("single"):
        ratio = float(case[6:])
        for t in range(m):  # one element per token, in a different super-block each
            x[t, 300 + 256 * t] = ratio * (1 if t % 2 == 0 else -1)
    elif case.startswith("three"):
        ratio = float(case[5:])
        for t in range(m):
            x[t, [301, 302, 640 + t]] = [ratio, -0.61 * ratio, 0.37 * ratio]
    elif case == "each1e4":  # one outlier in every super-block
        x[:, ::256] *= 1e4
    elif case == "mixed":  # halves of every super-block 1e4 apart
        x[:, ::2] *= 1e-4
    elif case == "t1":
        x = rng.standard_t(1, (m, k)).astype(np.float32)
    elif case == "t2":
        x = rng.standard_t(2, (m, k)).astype(np.float32)
    else:
        raise ValueError(case)
    return x


CASES = ["single1e3", "single1e4", "single1e5", "three1e4", "each1e4", "mixed", "t1", "t2"]
# bytes of the quants inside one block run of each type (zeroed to isolate d sc q from the offsets)
QUANT_SPANS = {T_Q4_K: (144, [(16, 144)]), T_Q5_K: (176, [(16, 176)]), T_Q6_K: (210, [(0, 192)]),
               T_Q8_0: (34, [(2, 34)])}


def quant_part(oracle, typ, w, k, n):
    """|c| = |dequant(w) - dequant(w with its quants zeroed)|, n x k."""
    blk, spans = QUANT_SPANS[typ]
    z = w.copy().reshape(-1, blk)
    for a, b in spans:
        z[:, a:b] = 0
    return np.abs(oracle.dequant_matrix(typ, w, k, n).astype(np.float64) -
                  oracle.dequant_matrix(typ, z.reshape(-1), k, n).astype(np.float64))


def representation_bound(oracle, typ, w, x, mag):
    """Per-output bound of the three-part int8 activation (see the module docstring)."""
    m, k = x.shape
    n = mag.shape[1]
    c = quant_part(oracle, typ, w, k, n).reshape(n, k // 256, 256).sum(axis=2)     # n x nsb
    smax = np.abs(x.astype(np.float64)).reshape(m, k // 256, 256).max(axis=2)      # m x nsb
    return 1.001 * smax / 16387064.0 @ c.T + 1e-6 * mag


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [1, 2, 3, 4])
@pytest.mark.parametrize("case", CASES)
def test_outlier_activations(qk, oracle, dev, typ, m, case):
    w = oracle.weights(typ, N, K, SEED_BASE | 0xA0)
    x = activations(case, m, K, 0xA1 + m)
    W = qk.upload(w, typ, K, N, 1)
    try:
        assert qk.gemv_plan([W], False, m)["kernel"] == 1
        xd = dev.put(x)
        yd = dev.empty(m * N * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, N))
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, K, N, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert np.isfinite(y).all()
    assert e_max <= TOL and e_norm <= TOL, (e_max, e_norm)
    excess = np.abs(y - ref) / representation_bound(oracle, typ, w, x, mag)
    assert excess.max() <= 1.0, (float(excess.max()), e_max, e_norm)


# (type, m, path): the general kernel serves Q4_K and Q6_K only
NONFINITE_CASES = [(t, m, path) for t in TYPES for m, path in
                   [(1, "int8"), (4, "int8"), (1, "general"), (4, "general"), (16, "gemm")]
                   if path != "general" or t in (T_Q4_K, T_Q6_K)]


@pytest.mark.parametrize("typ,m,path", NONFINITE_CASES,
                         ids=[f"{IDS[TYPES.index(t)]}-{m}-{p}" for t, m, p in NONFINITE_CASES])
@pytest.mark.parametrize("bad", ["nan", "inf"])
def test_nonfinite_activation(qk, oracle, dev, typ, m, path, bad):
    """One NaN or inf in the last token's x: that token's outputs are all non-finite, the others
    finite and within the bar of their path."""
    w = oracle.weights(typ, N, K, SEED_BASE | 0xB0)
    x = oracle.normal(SEED_BASE | 0xB1, m * K).reshape(m, K)
    x[m - 1, 777] = np.nan if bad == "nan" else -np.inf
    W = qk.upload(w, typ, K, N, 1)
    try:
        if path == "general":
            qk.set_tuning("gemv_fused", 0)
        xd = dev.put(x)
        yd = dev.empty(m * N * 4)
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, N))
    finally:
        qk.set_tuning("gemv_fused", 1)
        qk.free(W)
    assert not np.isfinite(y[m - 1]).any()
    if m > 1:
        good = x[: m - 1]
        if path == "gemm":  # the GEMM multiplies fp16-rounded activations
            good = good.astype(np.float16).astype(np.float32)
        ref, mag = oracle.matmul_f64(typ, w, K, N, good)
        e_max, e_norm = rel_errors(y[: m - 1], ref, mag)
        bar = 5e-3 if path == "gemm" else TOL
        assert np.isfinite(y[: m - 1]).all()
        assert e_max <= bar and e_norm <= bar, (e_max, e_norm)


def scaled_activations(case, m, k, seed):
    """N(0,1) x scaled per case (test-side inputs): whole tokens far below or far above 1, and one
    with super-blocks of very different magnitudes side by side (zero included)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k))
    if case == "x1e-35":  # products w x still normal fp32
        x *= 1e-35
    elif case == "x1e-40":  # fp32 subnormal activations
        x *= 1e-40
    elif case == "sb_mix":  # per super-block: 1, 1e-33, 0, 1e-38, 1e-20, 1e5, ...
        scales = [1.0, 1e-33, 0.0, 1e-38, 1e-20, 1e5, 1e-36, 3e-30]
        for b in range(k // 256):
            x[:, 256 * b: 256 * (b + 1)] *= scales[b % len(scales)]
    elif case == "x1e5":
        x *= 1e5
    elif case == "x1e30":
        x *= 1e30
    else:
        raise ValueError(case)
    return x.astype(np.float32)


SCALED_CASES = ["x1e-35", "x1e-40", "sb_mix", "x1e5", "x1e30"]


@pytest.mark.parametrize("typ", TYPES, ids=IDS)
@pytest.mark.parametrize("m", [1, 3])
@pytest.mark.parametrize("case", SCALED_CASES)
def test_scaled_activations_int8(qk, oracle, dev, typ, m, case):
    """The int8 kernel over activations of any finite fp32 magnitude (qwen_cpu/ops.h:54-76 accepts
    them all): super-blocks below 2^-100 are converted from x * 2^100 and scaled back, so they keep
    their three parts instead of reading as zero.  Bar: 1e-5 on both metrics and the representation
    bound where the products stay normal fp32; 1e-3 for subnormal activations, whose fp32 products
    and sums carry absolute errors of the order of 2^-149 in any fp32 path."""
    w = oracle.weights(typ, N, K, SEED_BASE | 0xC0)
    x = scaled_activations(case, m, K, 0xC1 + m)
    W = qk.upload(w, typ, K, N, 1)
    try:
        assert qk.gemv_plan([W], False, m)["kernel"] == 1
        xd = dev.put(x)
        yd = dev.empty(m * N * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, N))
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(typ, w, K, N, x)
    assert np.isfinite(y).all()
    assert np.abs(y).max() > 0.0
    # rel_errors' absolute floor (1e-30) would swamp outputs of 1e-35; these ratios have none
    d = np.abs(y.astype(np.float64) - ref)
    e_max = float(np.max(d / np.maximum(mag, 1e-300)))
    e_norm = float(np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-300))
    if case == "x1e-40":
        assert e_max <= TOL and e_norm <= TOL, (e_max, e_norm)
        return
    assert e_max <= 1e-5 and e_norm <= 1e-5, (e_max, e_norm)
    excess = np.abs(y - ref) / representation_bound(oracle, typ, w, x, mag)
    assert excess.max() <= 1.0, (float(excess.max()), e_max, e_norm)


def test_large_activations_ffn_down_three_tokens(qk, oracle, dev):
    """K=17408 N=5120 Q6_K at three tokens, the shape whose plan leaves the int8 kernel six waves per
    work-group (it used to go to the general kernel, whose fp16 pair overflows past 65504): x of
    magnitude 1e5 is within 1e-5 of the f64 reference, as for N(0,1) x."""
    k, n, m = 17408, 5120, 3
    w = oracle.weights(T_Q6_K, n, k, SEED_BASE | 0xC8)
    x = (oracle.normal(SEED_BASE | 0xC9, m * k).reshape(m, k) * np.float32(1e5)).astype(np.float32)
    W = qk.upload(w, T_Q6_K, k, n, 1)
    try:
        assert qk.gemv_plan([W], False, m)["kernel"] == 1
        xd = dev.put(x)
        yd = dev.empty(m * n * 4)
        yd.fill_nan()
        qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
        y = yd.get(np.float32, (m, n))
    finally:
        qk.free(W)
    ref, mag = oracle.matmul_f64(T_Q6_K, w, k, n, x)
    e_max, e_norm = rel_errors(y, ref, mag)
    assert np.isfinite(y).all()
    assert e_max <= 1e-5 and e_norm <= 1e-5, (e_max, e_norm)

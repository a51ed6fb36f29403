"""CPU tests that pin the parity oracle (oracle/qk_oracle.cpp) before it is trusted as the checker.

Each test fixes one function of the oracle against something other than its own formula: an exact
closed form (fp16 widening, the Q8_0/Q4_K/Q5_K/Q6_K dequant values in exact rational arithmetic),
an inverse map written here from the GGUF packing rule (6-bit scale/min bijection), brute force in
float64 (matmul), special inputs with known answers, and, where oracle/_ref is built, the
reference's own quants.h/ops.h compiled from /root/reference (bitwise).  The committed golden
fixtures under tests/golden/ were written by that reference build and are checked here too.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle_lib
from oracle_lib import BLOCK_BYTES, SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0

ALL_TYPES = [T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K]

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ------------------------------------------------------------------------------------------------
# fp16 <-> fp32 (qwen_cpu/quants.h:19, qwen_cuda/quants_ref.h:19-37)
def test_fp16_widening_exhaustive(oracle):
    codes = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.fp16_to_f32(int(h)) for h in codes], np.float32)
    want = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_fp16_narrowing_rne(oracle):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(0.01),
        rng.uniform(0, 0.01, 2000).astype(np.float32),
        # exact ties between neighbouring fp16 values (round half to even)
        (np.arange(1, 500, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
        np.array([6.0e-8, 2.0 ** -25, 3 * 2.0 ** -26, 65504.0, 65519.0, 1e-9, 0.0], np.float32),
    ])
    got = np.array([oracle.f32_to_fp16(float(v)) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------------------------------------
# 6-bit scale/min unpack (qwen_cpu/quants.h:33-41): the 12 bytes are a bijection of 16 fields
def pack_scale_min(sc, m):
    """GGUF Q4_K packing of eight 6-bit scales and mins into 12 bytes (inverse of the unpack)."""
    b = np.zeros(12, np.uint8)
    for i in range(4):
        b[i] = sc[i] | ((sc[i + 4] >> 4) << 6)
        b[i + 4] = m[i] | ((m[i + 4] >> 4) << 6)
        b[i + 8] = (sc[i + 4] & 15) | ((m[i + 4] & 15) << 4)
    return b


def test_scale_min_bijection(oracle):
    rng = np.random.default_rng(11)
    for _ in range(300):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        b = pack_scale_min(sc, m)
        for j in range(8):
            assert oracle.scale_min_k4(j, b) == (sc[j], m[j])
    for _ in range(300):  # and every 12-byte pattern is reached: unpack then repack is the identity
        b = rng.integers(0, 256, 12).astype(np.uint8)
        fields = [oracle.scale_min_k4(j, b) for j in range(8)]
        assert np.array_equal(pack_scale_min([f[0] for f in fields], [f[1] for f in fields]), b)


def test_scale_min_matches_reference(oracle, reflib):
    rng = np.random.default_rng(12)
    for _ in range(500):
        b = rng.integers(0, 256, 12).astype(np.uint8)
        for j in range(8):
            assert oracle.scale_min_k4(j, b) == reflib.scale_min_k4(j, b)


# ------------------------------------------------------------------------------------------------
# Dequant closed forms (a5/a6): exact rational value, rounded once to fp32
def _f16(b0, b1):
    return Fraction(float(np.frombuffer(bytes([b0, b1]), np.float16)[0]))


def _round_f32(fr):
    """Correctly rounded float32 of an exact rational (round half to even)."""
    if fr == 0:
        return np.float32(0.0)
    f = np.float32(float(fr))  # within an ulp; fix by comparing against the neighbours
    best = f
    for cand in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        d_c, d_b = abs(Fraction(float(cand)) - fr), abs(Fraction(float(best)) - fr)
        if d_c < d_b or (d_c == d_b and (int(np.float32(cand).view(np.uint32)) & 1) == 0):
            best = cand
    return np.float32(best)


def _signed_zero(negative):
    return np.float32(-0.0) if negative else np.float32(0.0)


def q8_0_closed_form(run):
    """Eight Q8_0 blocks: w = q*d, exact; a zero result carries the sign of the product."""
    out = np.zeros(256, np.float32)
    for j in range(8):
        blk = run[34 * j:34 * j + 34]
        d, d_neg = _f16(blk[0], blk[1]), bool(blk[1] & 0x80)
        for i, q in enumerate(blk[2:34].view(np.int8)):
            v = d * int(q)
            out[32 * j + i] = _round_f32(v) if v != 0 else _signed_zero(d_neg ^ (q < 0))
    return out


def q4k_closed_form(block, five_bit=False):
    """w = (d*sc)*q - dmin*m rounded once; a zero result carries the IEEE sign of a - b.  Q5_K
    (five_bit): q gains bit 2g + h of qh[l] as its fifth bit, qs start at byte 48."""
    d, dmin = _f16(block[0], block[1]), _f16(block[2], block[3])
    d_neg, dmin_neg = bool(block[1] & 0x80), bool(block[3] & 0x80)
    sc_b = block[4:16]
    qh, qs = (block[16:48], block[48:176]) if five_bit else (None, block[16:144])
    out = np.zeros(256, np.float32)
    for g in range(4):
        for h in range(2):
            j = 2 * g + h
            if j < 4:
                sc, m = sc_b[j] & 63, sc_b[j + 4] & 63
            else:
                sc = (sc_b[j + 4] & 0xF) | ((sc_b[j - 4] >> 6) << 4)
                m = (sc_b[j + 4] >> 4) | ((sc_b[j] >> 6) << 4)
            for l in range(32):
                q = (int(qs[32 * g + l]) >> (4 * h)) & 0xF
                if five_bit:
                    q |= ((int(qh[l]) >> (2 * g + h)) & 1) << 4
                a, b = d * int(sc) * int(q), dmin * int(m)
                if a == b:  # x - x = +0, and -0 - (+0) = -0
                    out[64 * g + 32 * h + l] = _signed_zero(a == 0 and d_neg and not dmin_neg)
                else:
                    out[64 * g + 32 * h + l] = _round_f32(a - b)
    return out


def q6k_closed_form(block):
    """w = (d*sc)*(q-32), exact; a zero result carries the sign of the product of its factors."""
    ql, qh, scales = block[0:128], block[128:192], block[192:208].view(np.int8)
    d = _f16(block[208], block[209])
    d_neg = bool(block[209] & 0x80)
    out = np.zeros(256, np.float32)
    for n in range(2):
        for s in range(4):
            for l in range(32):
                byte = int(ql[64 * n + 32 * (s & 1) + l])
                q = ((byte >> 4) if s >= 2 else (byte & 0xF)) | (((int(qh[32 * n + l]) >> (2 * s)) & 3) << 4)
                sc = int(scales[8 * n + 2 * s + l // 16])
                v = d * sc * (q - 32)
                out[128 * n + 32 * s + l] = _round_f32(v) if v != 0 else _signed_zero(d_neg ^ (sc < 0) ^ (q < 32))
    return out


CLOSED = {T_Q8_0: q8_0_closed_form, T_Q4_K: q4k_closed_form, T_Q5_K: lambda b: q4k_closed_form(b, True),
          T_Q6_K: q6k_closed_form}
FP16_FIELDS = {T_Q8_0: tuple(range(0, 272, 34)), T_Q4_K: (0, 2), T_Q5_K: (0, 2), T_Q6_K: (208,)}


def _random_blocks(typ, count, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (count, BLOCK_BYTES[typ])).astype(np.uint8)
    # keep the fp16 fields finite (the reference does not define inf/nan blocks)
    for off in FP16_FIELDS[typ]:
        hi = b[:, off + 1]
        b[:, off + 1] = np.where((hi & 0x7C) == 0x7C, hi & 0xBB, hi)
    return b


@pytest.mark.parametrize("typ", ALL_TYPES)
def test_dequant_closed_form(oracle, typ):
    closed = CLOSED[typ]
    blocks = list(_random_blocks(typ, 24, 21 + typ)) + list(oracle.fill(typ, SEED_BASE | 9, 0, 8).reshape(8, -1))
    for blk in blocks:
        want = closed(blk)
        for fast in (False, True):
            got = oracle.dequant(typ, blk, 256, fast=fast)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"fast={fast}"


@pytest.mark.parametrize("typ", ALL_TYPES)
def test_dequant_matches_reference(oracle, reflib, typ):
    k = 2048
    w = _random_blocks(typ, 64 * (k // 256), 31 + typ).reshape(64, -1)
    for row in w:
        want = reflib.dequant(typ, row, k, avx=False)
        assert np.array_equal(reflib.dequant(typ, row, k, avx=True).view(np.uint32), want.view(np.uint32))
        for fast in (False, True):
            assert np.array_equal(oracle.dequant(typ, row, k, fast=fast).view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------------------------------------
# Matmul (qwen_cpu/ops.h:54-76)
@pytest.mark.parametrize("typ", ALL_TYPES)
@pytest.mark.parametrize("k,n,T", [(256, 4, 1), (1024, 12, 3), (2560, 16, 5), (5120, 8, 1)])
def test_matmul_vs_f64(oracle, typ, k, n, T):
    seed = SEED_BASE | (0x100 + k + n + T)
    w = oracle.weights(typ, n, k, seed)
    x = oracle.normal(seed + 1, T * k).reshape(T, k)
    ref, mag = oracle.matmul_f64(typ, w, k, n, x)
    for force_scalar in (False, True):
        y = oracle.matmul(typ, w, k, n, x, force_scalar=force_scalar)
        e_max, e_norm = oracle_lib.rel_errors(y, ref, mag)
        assert e_max < 1e-6 and e_norm < 1e-6


def test_matmul_f64_is_brute_force(oracle):
    """matmul_f64 equals an independent numpy float64 dot of the dequantized rows."""
    k, n, T = 1024, 8, 2
    for typ in ALL_TYPES:
        w = oracle.weights(typ, n, k, SEED_BASE | 0x77)
        x = oracle.normal(SEED_BASE | 0x78, T * k).reshape(T, k)
        deq = oracle.dequant_matrix(typ, w, k, n).astype(np.float64)
        ref, mag = oracle.matmul_f64(typ, w, k, n, x)
        assert np.allclose(ref, x.astype(np.float64) @ deq.T, rtol=1e-12, atol=1e-12)
        assert np.allclose(mag, np.abs(x.astype(np.float64)) @ np.abs(deq).T, rtol=1e-12)


@pytest.mark.parametrize("typ", ALL_TYPES)
def test_matmul_bitwise_reference(oracle, reflib, typ):
    for k, n, T in ((1024, 8, 1), (2048, 16, 4), (5120, 12, 6)):
        seed = SEED_BASE | (0x200 + T)
        w = oracle.weights(typ, n, k, seed)
        x = oracle.normal(seed + 5, T * k).reshape(T, k)
        y_ref = reflib.matmul(typ, w, k, n, x)
        y = oracle.matmul(typ, w, k, n, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))


def test_matmul_special_inputs(oracle):
    k, n = 512, 4
    # all-zero nibbles with m = 0: every output is exactly 0
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[4:16] = pack_scale_min([5] * 8, [0] * 8)
    w = np.tile(blk, n * (k // 256))
    x = oracle.normal(3, k).reshape(1, k)
    assert np.all(oracle.matmul(T_Q4_K, w, k, n, x) == 0.0)
    # a single nonzero activation picks one dequantized column, rounded once
    w = oracle.weights(T_Q6_K, n, k, SEED_BASE | 0x33)
    deq = oracle.dequant_matrix(T_Q6_K, w, k, n)
    x = np.zeros((1, k), np.float32)
    x[0, 300] = np.float32(1.7)
    want = (deq[:, 300].astype(np.float64) * np.float64(np.float32(1.7))).astype(np.float32)
    assert np.array_equal(oracle.matmul(T_Q6_K, w, k, n, x)[0], want)


# ------------------------------------------------------------------------------------------------
# Synthetic input generator (splitmix64, BASELINE config distributions)
def test_generator_offsets_and_ranges(oracle):
    for typ in ALL_TYPES:
        bb = BLOCK_BYTES[typ]
        whole = oracle.fill(typ, SEED_BASE | 1, 0, 40)
        part = oracle.fill(typ, SEED_BASE | 1, 13, 27)
        assert np.array_equal(whole[13 * bb:], part)  # counter-based: any window reproduces
        assert not np.array_equal(whole, oracle.fill(typ, SEED_BASE | 2, 0, 40))
        blocks = oracle.fill(typ, SEED_BASE | 3, 0, 2000).reshape(2000, bb)
        if typ in (T_Q4_K, T_Q5_K, T_Q8_0):
            if typ == T_Q8_0:
                d = np.stack([blocks[:, o:o + 2] for o in FP16_FIELDS[T_Q8_0]], 1).copy().view(np.float16)
            else:
                d = blocks[:, 0:4].copy().view(np.float16)
            d = d.astype(np.float32)
            assert d.min() >= 0.0 and d.max() <= float(np.float16(0.01))  # U(0, 0.01) rounded to fp16
            assert abs(float(d.mean()) - 0.005) < 3e-4
        else:
            d = blocks[:, 208:210].copy().view(np.float16).astype(np.float32)
            assert d.min() >= 0.0 and d.max() <= float(np.float16(0.005))
            sc = blocks[:, 192:208].view(np.int8)
            assert sc.min() == -32 and sc.max() == 31
    x = oracle.normal(5, 200000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    assert np.array_equal(oracle.normal(5, 1000), x[:1000])


# ------------------------------------------------------------------------------------------------
# Golden fixtures written by the reference's own code (tests/golden/make_golden.py)
def _golden_files():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")) if os.path.isdir(GOLDEN) else []


def test_golden_present():
    assert _golden_files(), "tests/golden/*.npz missing (python tests/golden/make_golden.py)"


@pytest.mark.parametrize("name", _golden_files())
def test_oracle_matches_golden(oracle, name):
    g = np.load(os.path.join(GOLDEN, name))
    typ, k, n = int(g["type"]), int(g["k"]), int(g["n"])
    w = g["w"]
    for r in range(n):
        row = w.reshape(n, -1)[r]
        assert np.array_equal(oracle.dequant(typ, row, k).view(np.uint32), g["deq"][r].view(np.uint32))
    y = oracle.matmul(typ, w, k, n, g["x"])
    assert np.array_equal(y.view(np.uint32), g["y"].view(np.uint32))

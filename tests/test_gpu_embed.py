"""GPU checks of the token embedding (qk_embed, the reference's k_embed_*, qwen_cuda/kernels.cu:375-389,
launched at qwen_cuda/qwen.cpp:265) through the C ABI: rows of a real-shape table (248320 x 5120, the
model's vocabulary by its hidden size) on sampled token ids, bit-exact against the oracle's dequant of
the same rows, from both layouts and all four quantized types; masked tokens copy the caller's
embedding row; ids outside the table give NaN rows instead of out-of-bounds reads.  The table is
synthesised on the GPU by the generator that is bitwise equal to the oracle's, so the host builds only
the sampled rows."""
import numpy as np
import pytest

from oracle_lib import BLOCK_BYTES, SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 248320, 5120


def _table(qk, dev, hip, typ, n, k, seed, layout):
    nsb = k // 256
    rb = nsb * BLOCK_BYTES[typ]
    raw = dev.empty(n * rb)
    qk.synth_fill(typ, seed, 0, n * nsb, raw.ptr)
    if layout == 0:
        return qk.weight_view(raw.ptr, typ, k, n, 0), [raw]
    t16 = dev.empty(n * rb)
    W = qk.repack(qk.weight_view(raw.ptr, typ, k, n, 0), t16.ptr, 1)
    hip.sync()
    raw.close()
    return W, [t16]


def _rows(oracle, typ, k, seed, ids):
    nsb = k // 256
    w = np.concatenate([oracle.fill(typ, seed, int(r) * nsb, nsb) for r in ids])
    return oracle.dequant_matrix(typ, w, k, len(ids))


@pytest.mark.parametrize("typ,layout", [(T_Q6_K, 1), (T_Q6_K, 0), (T_Q4_K, 1)], ids=["q6k-t16", "q6k-gguf", "q4k-t16"])
def test_embed_real_table(qk, oracle, dev, hip, typ, layout):
    seed = SEED_BASE | 0xE0
    W, bufs = _table(qk, dev, hip, typ, VOCAB, HIDDEN, seed, layout)
    try:
        rng = np.random.default_rng(3)
        ids = np.concatenate([[0, 1, 15, 16, VOCAB - 1], rng.integers(0, VOCAB, 59)]).astype(np.int32)
        m = len(ids)
        td = dev.put(ids)
        xd = dev.empty(m * HIDDEN * 4)
        xd.fill_nan()
        qk.embed(W, td.ptr, None, None, m, xd.ptr, dev.stream())
        x = xd.get(np.float32, (m, HIDDEN))
    finally:
        for b in bufs:
            b.close()
    want = _rows(oracle, typ, HIDDEN, seed, ids)
    assert np.array_equal(x.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("typ", [T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0], ids=["q4k", "q5k", "q6k", "q8_0"])
def test_embed_mask_and_range(qk, oracle, dev, hip, typ):
    k, n = 1024, 64
    seed = SEED_BASE | 0xE1
    W, bufs = _table(qk, dev, hip, typ, n, k, seed, 1)
    try:
        ids = np.array([5, 63, 0, -1, 64, 7], np.int32)
        mask = np.array([0, 1, 0, 0, 0, 1], np.uint8)
        embd = oracle.normal(SEED_BASE | 0xE2, len(ids) * k).reshape(len(ids), k)
        td, md, ed = dev.put(ids), dev.put(mask), dev.put(embd)
        xd = dev.empty(len(ids) * k * 4)
        qk.embed(W, td.ptr, md.ptr, ed.ptr, len(ids), xd.ptr, dev.stream())
        x = xd.get(np.float32, (len(ids), k))
    finally:
        for b in bufs:
            b.close()
    table_rows = _rows(oracle, typ, k, seed, [5, 0])
    assert np.array_equal(x[0].view(np.uint32), table_rows[0].view(np.uint32))
    assert np.array_equal(x[2].view(np.uint32), table_rows[1].view(np.uint32))
    assert np.array_equal(x[[1, 5]].view(np.uint32), embd[[1, 5]].view(np.uint32))  # masked: copied
    assert np.isnan(x[3]).all() and np.isnan(x[4]).all()  # ids -1 and n: NaN rows


def test_embed_f32_table(qk, oracle, dev, hip):
    """F32 tables (rows used as stored, GGUF layout): each token's row is copied exactly; one run per
    wave, so a row longer than one 256-column run covers every run."""
    k, n = 1024, 40
    table = oracle.normal(SEED_BASE | 0xE3, n * k).reshape(n, k)
    ids = np.array([3, 0, 39, 17, 3], np.int32)
    tb, td = dev.put(table), dev.put(ids)
    xd = dev.empty(len(ids) * k * 4)
    xd.fill_nan()
    try:
        W = qk.weight_view(tb.ptr, 0, k, n, 0)
        qk.embed(W, td.ptr, None, None, len(ids), xd.ptr, dev.stream())
        x = xd.get(np.float32, (len(ids), k))
    finally:
        tb.close()
    assert np.array_equal(x.view(np.uint32), table[ids].view(np.uint32))

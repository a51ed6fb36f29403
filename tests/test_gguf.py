"""The GGUF file path (include/qk_gguf.h): parsing and error handling on the CPU, upload with the
in-place T16 repack and matmuls through the uploaded views on the GPU (oracle: oracle_lib)."""
import ctypes

import numpy as np
import pytest

import gguf_writer as gw
from oracle_lib import GEMM_ROUTE_M, SEED_BASE, T_Q4_K, T_Q5_K, T_Q6_K, T_Q8_0, rel_errors

T_F32 = 0
E_FORMAT, E_NOTFOUND, E_IO, E_RANGE = -9, -10, -11, -8


def _fixture(oracle, path, alignment=64):
    """A small model-shaped file: quantized matrices of the four types, an F32 projection, a 1-D
    norm, and key-values of every kind including arrays (skipped by the reader)."""
    rng = np.random.default_rng(5)
    tensors = [
        ("blk.0.attn_q.weight", T_Q4_K, [1024, 48], oracle.weights(T_Q4_K, 48, 1024, SEED_BASE | 0x1B0)),
        ("blk.0.ffn_down.weight", T_Q6_K, [512, 32], oracle.weights(T_Q6_K, 32, 512, SEED_BASE | 0x1B1)),
        ("blk.0.attn_k.weight", T_Q8_0, [512, 16], oracle.weights(T_Q8_0, 16, 512, SEED_BASE | 0x1B2)),
        ("blk.1.ffn_down.weight", T_Q5_K, [768, 32], oracle.weights(T_Q5_K, 32, 768, SEED_BASE | 0x1B3)),
        ("blk.0.ssm_alpha.weight", T_F32, [512, 48], rng.standard_normal((48, 512)).astype(np.float32).tobytes()),
        ("blk.0.attn_norm.weight", T_F32, [512], rng.standard_normal(512).astype(np.float32).tobytes()),
        ("token_embd.weight", T_Q6_K, [256, 40], oracle.weights(T_Q6_K, 40, 256, SEED_BASE | 0x1B4)),
    ]
    kvs = [("general.architecture", gw.STR, "qwen35"), ("general.alignment", gw.U32, alignment),
           ("qwen35.embedding_length", gw.U32, 5120), ("qwen35.rope.freq_base", gw.F32, 1e7),
           ("tokenizer.ggml.tokens", gw.ARR, (gw.STR, ["a", "bb", "ccc"])),
           ("tokenizer.ggml.scores", gw.ARR, (gw.F32, [0.5, 1.5])), ("qwen35.block_count", gw.U64, 64)]
    offs = gw.write(path, kvs, tensors, alignment)
    return tensors, offs


def test_gguf_parse(qk, oracle, tmp_path):
    path = tmp_path / "m.gguf"
    tensors, offs = _fixture(oracle, str(path))
    h = qk.gguf_open(path)
    try:
        got = qk.gguf_tensors(h)
        assert [g[0] for g in got] == [t[0] for t in tensors]
        for (name, typ, dims, off, nb), (tn, tt, td, data) in zip(got, tensors):
            assert (typ, dims, off, nb) == (tt, td, offs[tn], len(data))
            assert off % 64 == 0
        assert qk.gguf_kv_str(h, "general.architecture") == "qwen35"
        assert qk.gguf_kv_num(h, "qwen35.embedding_length") == 5120
        assert qk.gguf_kv_num(h, "qwen35.block_count") == 64
        assert abs(qk.gguf_kv_num(h, "qwen35.rope.freq_base") - 1e7) < 1
        with pytest.raises(Exception):
            qk.gguf_kv_num(h, "tokenizer.ggml.tokens")  # arrays are skipped
        idx = ctypes.c_int64()
        assert qk.lib.qk_gguf_find(h, b"blk.0.ffn_down.weight", ctypes.byref(idx)) == 0 and idx.value == 1
        assert qk.lib.qk_gguf_find(h, b"nope", ctypes.byref(idx)) == E_NOTFOUND
        assert qk.lib.qk_gguf_weight(h, b"blk.0.attn_q.weight", None) == -1  # null out-pointer
    finally:
        qk.gguf_close(h)


def test_gguf_errors(qk, qkmod, oracle, tmp_path):
    good = tmp_path / "g.gguf"
    _fixture(oracle, str(good))
    data = good.read_bytes()
    h = ctypes.c_void_p()
    assert qk.lib.qk_gguf_open(str(tmp_path / "missing.gguf").encode(), ctypes.byref(h)) == E_IO
    cases = {"magic": b"GGUX" + data[4:], "version": data[:4] + (2).to_bytes(4, "little") + data[8:],
             "header": data[:40], "data": data[:-100]}
    for what, blob in cases.items():
        p = tmp_path / f"{what}.gguf"
        p.write_bytes(blob)
        assert qk.lib.qk_gguf_open(str(p).encode(), ctypes.byref(h)) == E_FORMAT, what
    h = qk.gguf_open(good)
    try:
        w = qkmod.Weight()
        assert qk.lib.qk_gguf_weight(h, b"blk.0.attn_q.weight", ctypes.byref(w)) == E_RANGE  # not uploaded
    finally:
        qk.gguf_close(h)


@pytest.mark.gpu
def test_gguf_upload_and_matmul(qk, oracle, dev, tmp_path):
    path = tmp_path / "m.gguf"
    tensors, _ = _fixture(oracle, str(path))
    h = qk.gguf_open(path)
    try:
        qk.gguf_upload(h, dev.stream())
        for name, typ, dims, data in tensors:
            if len(dims) != 2:
                continue
            k, n = dims
            W = qk.gguf_weight(h, name)
            assert (W.type, W.k, W.n) == (typ, k, n)
            # quantized matrices with n % 16 == 0 are repacked to T16 in place; the rest stay as stored
            t16 = typ != T_F32 and n % 16 == 0
            assert W.layout == (1 if t16 else 0)
            if typ != T_F32 and not t16:  # n = 40: no T16, so no matmul (row lookups still work)
                assert qk.lib.qk_matmul(ctypes.byref(W), None, 1, None, dev.stream()) == -1  # null x first
                continue
            w = np.frombuffer(data, np.uint8)
            for m in (1, 3, 20):
                x = oracle.normal(SEED_BASE | (0x1C0 + m), m * k).reshape(m, k)
                xd = dev.put(x)
                yd = dev.empty(m * n * 4)
                yd.fill_nan()
                qk.matmul(W, xd.ptr, m, yd.ptr, dev.stream())
                y = yd.get(np.float32, (m, n))
                xin = x if m < GEMM_ROUTE_M or typ == T_F32 else x.astype(np.float16).astype(np.float32)
                ref, mag = oracle.matmul_f64(typ, w, k, n, xin)
                e_max, e_norm = rel_errors(y, ref, mag)
                bar = 1e-5 if typ == T_F32 else 2e-4 if m < GEMM_ROUTE_M else 5e-3
                assert e_max < bar and e_norm < bar, (name, m, e_max, e_norm)
        # token embedding lookup: rows of the uploaded (repacked) table, bit-exact
        E = qk.gguf_weight(h, "token_embd.weight")
        ids = np.array([0, 7, 39, 7], np.int32)
        idd = dev.put(ids)
        out = dev.empty(len(ids) * 256 * 4)
        qk.dequant_rows(E, idd.ptr, len(ids), out.ptr, dev.stream())
        emb = [t for t in tensors if t[0] == "token_embd.weight"][0][3]
        ref = oracle.dequant_matrix(T_Q6_K, np.frombuffer(emb, np.uint8), 256, 40)[ids]
        assert np.array_equal(out.get(np.uint32, (len(ids), 256)), ref.view(np.uint32))
    finally:
        qk.gguf_close(h)

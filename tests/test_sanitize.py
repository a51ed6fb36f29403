"""The host-side C ABI under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU: the GGUF reader
(replacing qwen_cpu/gguf.h:106-175) walks valid, truncated and crafted files, and the entry points'
argument checks run (tests/sanitize_check.cpp, built by build.py with g++ -fsanitize=address,undefined).
A sanitizer report makes the driver exit non-zero with the report on stderr."""
import os
import struct
import subprocess

import numpy as np
import pytest

import gguf_writer as gw
from oracle_lib import SEED_BASE, T_Q4_K, T_Q6_K

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "_bin", "sanitize_check")
E_FORMAT = -9

pytestmark = pytest.mark.skipif(not os.path.exists(BIN), reason="tests/_bin/sanitize_check not built (build())")


def _run(args):
    env = dict(os.environ, ASAN_OPTIONS="abort_on_error=0:exitcode=99", UBSAN_OPTIONS="print_stacktrace=1")
    return subprocess.run([BIN] + args, capture_output=True, text=True, timeout=300, env=env)


def test_abi_argument_checks():
    res = _run(["abi"])
    assert res.returncode == 0 and "abi ok" in res.stdout, res.stderr[-3000:]


def _header(n_tensors, kvs=b"", n_kv=0, version=3, magic=b"GGUF"):
    return magic + struct.pack("<IQQ", version, n_tensors, n_kv) + kvs


def _tensor_info(name, dims, typ, off):
    b = name.encode()
    return struct.pack("<Q", len(b)) + b + struct.pack("<I", len(dims)) + b"".join(
        struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", typ, off)


def _crafted(tmp_path, oracle):
    """(path, expected status) for valid, truncated and malformed files."""
    cases = []
    valid = tmp_path / "valid.gguf"
    tensors = [("a", T_Q4_K, [512, 32], oracle.weights(T_Q4_K, 32, 512, SEED_BASE | 0xF0)),
               ("b", T_Q6_K, [256, 16], oracle.weights(T_Q6_K, 16, 256, SEED_BASE | 0xF1)),
               ("norm", 0, [512], np.zeros(512, np.float32).tobytes())]
    kvs = [("general.architecture", gw.STR, "qwen35"), ("general.alignment", gw.U32, 64),
           ("arr", gw.ARR, (gw.ARR, [(gw.U8, [1, 2]), (gw.STR, ["x"])]))]
    gw.write(str(valid), kvs, tensors, 64)
    cases.append((valid, 0))
    blob = valid.read_bytes()
    # every prefix up to the end of the tensor infos, then a spread of prefixes into the data
    head_end = blob.index(b"norm") + 4 + 4 + 8 + 4 + 8
    cuts = list(range(0, head_end + 1)) + list(range(head_end + 1, len(blob), 997))
    for c in cuts:
        p = tmp_path / f"cut{c}.gguf"
        p.write_bytes(blob[:c])
        cases.append((p, E_FORMAT))
    bad = {
        "magic": _header(0, magic=b"GGUX"),
        "version2": _header(0, version=2),
        "dim0": _header(1) + _tensor_info("t", [256, 0], T_Q4_K, 0),
        "dimhuge": _header(1) + _tensor_info("t", [256, 1 << 31], T_Q4_K, 0),
        "numel_overflow": _header(1) + _tensor_info("t", [256, (1 << 31) - 1, (1 << 31) - 1, (1 << 31) - 1], T_Q4_K, 0),
        "ndims5": _header(1) + _tensor_info("t", [256, 1, 1, 1, 1], T_Q4_K, 0),
        "offset_past_end": _header(1) + _tensor_info("t", [256, 16], T_Q4_K, 1 << 40),
        "offset_wrap": _header(1) + _tensor_info("t", [256, 16], T_Q4_K, (1 << 64) - 64),
        "many_tensors": _header(1 << 40),
        "many_kv": _header(0, n_kv=1 << 40),
        "key_len_huge": _header(0, struct.pack("<Q", 1 << 62) + b"k", 1),
        "str_len_huge": _header(0, struct.pack("<Q", 1) + b"k" + struct.pack("<IQ", 8, (1 << 63) + 5), 1),
        "arr_count_huge": _header(0, struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 4, 1 << 60), 1),
        "arr_nested_deep": _header(0, struct.pack("<Q", 1) + b"k" + struct.pack("<I", 9)
                                   + struct.pack("<IQ", 9, 1) * 40 + struct.pack("<IQ", 4, 0), 1),
        "bad_kv_type": _header(0, struct.pack("<Q", 1) + b"k" + struct.pack("<I", 77), 1),
        "align_zero": _header(0, struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<II", 4, 0), 1),
    }
    for name, data in bad.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data + b"\0" * 64)
        cases.append((p, E_FORMAT))
    # alignment 0 falls back to 32: a valid (empty) file
    cases[-1] = (cases[-1][0], 0)
    return cases


def test_gguf_reader_crafted_files(oracle, tmp_path):
    cases = _crafted(tmp_path, oracle)
    res = _run([str(p) for p, _ in cases])
    assert res.returncode == 0, res.stderr[-3000:]
    got = {}
    for line in res.stdout.splitlines():
        rc, n, path = line.split(" ", 2)
        got[path] = (int(rc), int(n))
    for p, want in cases:
        assert got[str(p)][0] == want, (p.name, got[str(p)])
    assert got[str(cases[0][0])] == (0, 3)

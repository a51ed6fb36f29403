"""CPU test of the T16 group layouts (qk_device.h): the byte maps are bijections and inverse to each
other for every type, checked by the host build of the same header (tests/_bin/t16_check)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "_bin", "t16_check")


def test_t16_maps_are_inverse_bijections():
    if not os.path.exists(BIN):
        pytest.skip("tests/_bin/t16_check not built (__graft_entry__.build())")
    res = subprocess.run([BIN], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    got = {int(t): int(g) for _, t, g in (l.split() for l in res.stdout.split("\n") if l.startswith("ok"))}
    assert got == {8: 4352, 12: 2304, 13: 2816, 14: 3360}

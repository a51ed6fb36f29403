"""Machine-code check of the built library (CPU only): no kernel names the destination registers
of a global load before the s_waitcnt that covers it (see isa_scan.py for why the hand-waited
loads need this)."""
import os

import pytest

import isa_scan

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "qwen3.8_27b_reference_amd", "libqk.so")


@pytest.mark.skipif(not os.path.exists(LIB), reason="libqk.so not built")
@pytest.mark.skipif(not isa_scan.tools_present(), reason="ROCm LLVM tools not found")
def test_no_register_use_before_load_wait():
    text = isa_scan.disassemble(LIB)
    nloads, bad = isa_scan.early_uses(text)
    assert nloads > 1000  # the GEMV, GEMM, layout and F32 kernels' loads were all seen
    assert "k_gemv1" in text and "k_gemm" in text
    assert not bad, bad[:10]


def test_scan_flags_early_copy():
    """A load whose registers are copied before its wait is reported; after the wait it is not."""
    text = "\n".join([
        "0000000000001000 <kern>:",
        "\tglobal_load_dwordx4 v[4:7], v[2:3], off // 1000: x",
        "\tglobal_load_lds_dwordx4 v[8:9], off // 1008: x",
        "\tv_mov_b32_e32 v20, v5 // 1010: x",
        "\ts_waitcnt vmcnt(1) // 1014: x",
        "\tv_mov_b32_e32 v21, v6 // 1018: x",
        "\ts_endpgm // 101c: x",
    ])
    nloads, bad = isa_scan.early_uses(text)
    assert nloads == 1 and bad == [("kern", "v_mov_b32_e32 v20, v5")]
    # vmcnt(2) would still allow the load in flight: its use after that wait is reported too
    nloads, bad = isa_scan.early_uses(text.replace("vmcnt(1)", "vmcnt(2)"))
    assert len(bad) == 2

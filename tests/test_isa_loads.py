"""Machine-code check of the built library (CPU only): no kernel names the destination registers
of a global load, on any path through its control flow, before an s_waitcnt that covers the load
(see isa_scan.py for why the hand-waited loads need this)."""
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


def _kern(lines, base=0x1000):
    """Synthetic disassembly: (size in bytes, instruction) pairs laid out from base, in the
    llvm-objdump form (address after the comment marker; branches annotated <kern+0xoff>)."""
    out, addr = [f"{base:016x} <kern>:"], base
    for size, ins in lines:
        ins, sep, note = ins.partition(" <")
        out.append(f"\t{ins} // {addr:012X}: 00000000" + (f" <{note}" if sep else ""))
        addr += size
    return "\n".join(out)


def _br(op, at, to, base=0x1000):
    """A branch instruction at byte offset `at` to byte offset `to` (both from base)."""
    simm = ((to - at - 4) // 4) & 0xFFFF
    return f"{op} {simm} <kern+0x{to:x}>" if to is not None else f"{op} {simm}"


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


def test_scan_follows_a_branch_around_the_wait():
    """The wait lies between the load and the use in address order, but a branch skips it: the path
    without the wait is reported (an address-order scan would miss it)."""
    lines = [(8, "global_load_dwordx4 v[4:7], v[2:3], off"), (4, "s_cmp_eq_u32 s0, 0"),
             (4, _br("s_cbranch_scc1", 0xC, 0x14)), (4, "s_waitcnt vmcnt(0)"), (4, "v_mov_b32_e32 v20, v5"),
             (4, "s_endpgm")]
    assert isa_scan.early_uses(_kern(lines)) == (1, [("kern", "v_mov_b32_e32 v20, v5")])
    # the same branch encoded without the symbolic annotation (target from the word offset)
    lines_raw = list(lines)
    lines_raw[2] = (4, "s_cbranch_scc1 1")
    assert isa_scan.early_uses(_kern(lines_raw)) == (1, [("kern", "v_mov_b32_e32 v20, v5")])
    # with the wait before the branch both paths are covered
    fixed = [lines[0], (4, "s_waitcnt vmcnt(0)"), (4, "s_cmp_eq_u32 s0, 0"), (4, _br("s_cbranch_scc1", 0x10, 0x14)),
             (4, "v_mov_b32_e32 v21, v6"), (4, "v_mov_b32_e32 v20, v5"), (4, "s_endpgm")]
    assert isa_scan.early_uses(_kern(fixed)) == (1, [])


def test_scan_merges_the_arms_of_a_branch():
    """A wait on one arm of an if/else covers only that arm: the use after the merge is reported;
    with a wait on both arms it is not."""
    one = [(8, "global_load_dwordx4 v[4:7], v[2:3], off"), (4, _br("s_cbranch_scc1", 0x8, 0x14)),
           (4, "s_waitcnt vmcnt(0)"), (4, _br("s_branch", 0x10, 0x18)), (4, "s_nop 0"),
           (4, "v_mov_b32_e32 v20, v5"), (4, "s_endpgm")]
    assert isa_scan.early_uses(_kern(one))[1] == [("kern", "v_mov_b32_e32 v20, v5")]
    both = list(one)
    both[4] = (4, "s_waitcnt vmcnt(0)")
    assert isa_scan.early_uses(_kern(both))[1] == []
    # a count-based wait: one arm issues another memory operation after the load, so vmcnt(1)
    # covers the load there, but not on the arm that issued nothing
    counted = [(8, "global_load_dwordx4 v[4:7], v[2:3], off"), (4, _br("s_cbranch_scc1", 0x8, 0x18)),
               (8, "global_store_dword v[2:3], v9, off"), (4, _br("s_branch", 0x14, 0x1C)), (4, "s_nop 0"),
               (4, "s_waitcnt vmcnt(1)"), (4, "v_mov_b32_e32 v20, v5"), (4, "s_endpgm")]
    assert isa_scan.early_uses(_kern(counted))[1] == [("kern", "v_mov_b32_e32 v20, v5")]
    counted[4] = (4, "global_load_lds_dwordx4 v[8:9], off")
    counted[3] = (4, _br("s_branch", 0x14, 0x1C))
    assert isa_scan.early_uses(_kern(counted))[1] == []


def test_scan_follows_a_loop_back_edge():
    """A load issued at the end of a loop body and used at the top of the next iteration before the
    wait is reported (it comes after the use in address order); waiting first at the top is not."""
    loop = [(4, "s_mov_b32 s0, 4"), (4, "v_mov_b32_e32 v20, v5"), (4, "s_waitcnt vmcnt(0)"),
            (8, "global_load_dwordx4 v[4:7], v[2:3], off"), (4, "s_sub_u32 s0, s0, 1"),
            (4, _br("s_cbranch_scc0", 0x18, 0x4)), (4, "s_waitcnt vmcnt(0)"), (4, "s_endpgm")]
    assert isa_scan.early_uses(_kern(loop)) == (1, [("kern", "v_mov_b32_e32 v20, v5")])
    fixed = list(loop)
    fixed[1], fixed[2] = loop[2], loop[1]
    assert isa_scan.early_uses(_kern(fixed)) == (1, [])
    # a later load's address operands naming the pending registers are a use; a reissue of the same
    # load into the same registers (in-order returns) is not
    addr_use = list(fixed)
    addr_use[4] = (8, "global_load_dword v9, v[4:5], off")
    addr_use[5] = (4, _br("s_cbranch_scc0", 0x1C, 0x4))
    assert isa_scan.early_uses(_kern(addr_use))[1] == [("kern", "global_load_dword v9, v[4:5], off")]

"""Reads the gfx950 machine code of this repository's own libqk.so (built here) and checks the
vector-memory loads whose completion the kernels wait out by hand.

The kernels issue some global loads from inline assembly (so that the compiler's own waits do not
fall back to vmcnt(0) while LDS-DMAs are in flight) and wait for them with an explicit
`s_waitcnt vmcnt(N)` tied to the destination registers.  The compiler sees such a load as complete
when the asm statement ends: if it ever copied the destination registers, or gave them to another
value, before the wait, the data landing later would be lost or would overwrite that value.  The
scan walks each kernel's instructions in address order, counts the vector-memory operations issued
after every load, and reports any instruction that names a load's destination registers before a
wait that covers the load.  (Loads the compiler waits for itself are covered by its own waits, so
they never show up.)"""
import os
import re
import subprocess
import tempfile

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def tools_present():
    return all(os.path.exists(f"{LLVM}/{t}") for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"))


def disassemble(so):
    """Disassembly of every gfx950 code object in so's .hip_fatbin section (one bundle per
    translation unit, concatenated)."""
    with tempfile.TemporaryDirectory() as d:
        fb = os.path.join(d, "fatbin")
        subprocess.run([f"{LLVM}/llvm-objcopy", "--dump-section", f".hip_fatbin={fb}", so, os.path.join(d, "rest")],
                       check=True, capture_output=True)
        data = open(fb, "rb").read()
        starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
        out = []
        for i, s0 in enumerate(starts):
            b, co = os.path.join(d, f"b{i}"), os.path.join(d, f"co{i}")
            with open(b, "wb") as f:
                f.write(data[s0:starts[i + 1] if i + 1 < len(starts) else len(data)])
            subprocess.run([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--targets={TARGET}",
                            f"--input={b}", f"--output={co}"], check=True, capture_output=True)
            out.append(subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", co], check=True,
                                      capture_output=True, text=True).stdout)
        return "\n".join(out)


def _vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def early_uses(text):
    """(loads seen, [(kernel, instruction)] naming a pending load's registers before its wait)."""
    kernel, pending, bad, nloads = None, [], [], 0
    for line in text.split("\n"):
        m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
        if m:
            kernel, pending = m.group(1), []
            continue
        ins = line.split("//")[0].strip()
        if not ins or kernel is None:
            continue
        parts = ins.split(None, 1)
        op = parts[0]
        ops = [t.strip() for t in parts[1].split(",")] if len(parts) > 1 else []
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", ins)
            if m:  # a load is covered once at most n operations were issued after it
                n = int(m.group(1))
                pending = [p for p in pending if p[1] < n]
            continue
        if op == "s_endpgm":
            pending = []
            continue
        named = set()
        for t in ops:
            named |= _vregs(t)
        bad += [(kernel, ins) for p in pending if p[0] & named]
        if op.startswith(("global_", "buffer_", "flat_")):
            for p in pending:
                p[1] += 1
            if op.startswith("global_load") and "lds" not in op:
                nloads += 1
                pending.append([_vregs(ops[0]), 0])
    return nloads, bad

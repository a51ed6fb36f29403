"""Reads the gfx950 machine code of this repository's own libqk.so (built here) and checks the
vector-memory loads whose completion the kernels wait out by hand.

The kernels issue some global loads from inline assembly (so that the compiler's own waits do not
fall back to vmcnt(0) while LDS-DMAs are in flight) and wait for them with an explicit
`s_waitcnt vmcnt(N)` tied to the destination registers.  The compiler sees such a load as complete
when the asm statement ends: if it ever copied the destination registers, or gave them to another
value, before the wait, the data landing later would be lost or would overwrite that value.

The scan follows each kernel's control flow.  It cuts the instructions into basic blocks (a block
starts at a branch target and after a branch or s_endpgm), links them by their branches (taken and
fall-through edges, loop back-edges included) and runs a forward dataflow analysis to a fixed
point.  The state at a point is the set of loads that may still be in flight there, each with the
fewest vector-memory operations issued after it along any path reaching the point.  s_waitcnt
vmcnt(n) retires a load once at least n operations were issued after it (returns come back in
order), so a load counts as covered only when every path from it to the point passes a covering
wait.  Any instruction that names a still-pending load's registers (a later load's address
operands included; a later load writing the same registers is not a hazard, returns being in
order) is reported.  Loads the compiler waits for itself are covered by its own waits on every
path, so they never show up."""
import os
import re
import subprocess
import tempfile

LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
VMEM = ("global_", "buffer_load", "buffer_store", "buffer_atomic", "flat_", "scratch_")
MAXCNT = 64  # vmcnt is six bits: counts at or above 63 all cover every wait


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


class Ins:
    __slots__ = ("addr", "op", "ops", "text", "target")

    def __init__(self, addr, op, ops, text, target):
        self.addr, self.op, self.ops, self.text, self.target = addr, op, ops, text, target


def _is_branch(op):
    return op == "s_branch" or op.startswith("s_cbranch")


def parse(text):
    """{kernel: [Ins]} from llvm-objdump output.  Branch targets come from the `<sym+0xoff>`
    annotation (or, without it, from the 16-bit word offset: pc + 4 + 4 * simm16)."""
    kernels, base, cur = {}, {}, None
    for line in text.split("\n"):
        m = re.match(r"^([0-9a-f]+) <(\S+)>:", line)
        if m:
            cur = m.group(2)
            base[cur] = int(m.group(1), 16)
            kernels[cur] = []
            continue
        if cur is None:
            continue
        body, _, comment = line.partition("//")
        ins = body.strip()
        if not ins:
            continue
        ma = re.match(r"\s*([0-9A-Fa-f]+):", comment)
        if not ma:
            continue
        addr = int(ma.group(1), 16)
        parts = ins.split(None, 1)
        op = parts[0]
        ops = [t.strip() for t in parts[1].split(",")] if len(parts) > 1 else []
        target = None
        if _is_branch(op):
            mt = re.search(r"<(\S+?)\+0x([0-9a-f]+)>", comment)
            if mt and mt.group(1) in base:
                target = base[mt.group(1)] + int(mt.group(2), 16)
            else:
                simm = int(ops[0]) & 0xFFFF
                simm -= 0x10000 if simm >= 0x8000 else 0
                target = addr + 4 + 4 * simm
        kernels[cur].append(Ins(addr, op, ops, ins, target))
    return kernels


def _cfg(ins):
    """Basic blocks [(first, last)] over ins and their successor lists."""
    index = {x.addr: i for i, x in enumerate(ins)}
    leaders = {0}
    for i, x in enumerate(ins):
        if _is_branch(x.op):
            if x.target not in index:
                raise ValueError(f"branch at {x.addr:#x} to {x.target:#x} outside the kernel")
            leaders.add(index[x.target])
            leaders.add(i + 1)
        elif x.op.startswith("s_endpgm") or x.op.startswith(("s_setpc", "s_swappc", "s_rfe")):
            leaders.add(i + 1)
    starts = sorted(s for s in leaders if s < len(ins))
    blocks = [(s, (starts[j + 1] if j + 1 < len(starts) else len(ins)) - 1) for j, s in enumerate(starts)]
    bidx = {s: j for j, (s, _) in enumerate(blocks)}
    succ = []
    for s, e in blocks:
        x = ins[e]
        if x.op == "s_branch":
            succ.append([bidx[index[x.target]]])
        elif x.op.startswith("s_cbranch"):
            nxt = [bidx[index[x.target]]]
            if e + 1 < len(ins):
                nxt.append(bidx[e + 1])
            succ.append(nxt)
        elif x.op.startswith("s_endpgm"):
            succ.append([])
        elif x.op.startswith(("s_setpc", "s_swappc", "s_rfe")):
            raise ValueError(f"indirect control flow at {x.addr:#x}: {x.text}")
        else:
            succ.append([bidx[e + 1]] if e + 1 < len(ins) else [])
    return blocks, succ


def _step(state, x, regs, report):
    """Applies instruction x to state {load address: fewest operations issued after it}."""
    if x.op == "s_waitcnt":
        m = re.search(r"vmcnt\((\d+)\)", x.text)
        if m:
            n = int(m.group(1))
            for a in [a for a, k in state.items() if k >= n]:
                del state[a]
        return
    if x.op.startswith("s_endpgm"):
        state.clear()
        return
    is_vmem = x.op.startswith(VMEM)
    is_load = x.op.startswith("global_load") and "lds" not in x.op
    named = set()
    for t in (x.ops[1:] if is_load else x.ops):
        named |= _vregs(t)
    if report is not None and named:
        for a in state:
            if regs[a] & named:
                report(x, a)
    if is_vmem:
        for a in state:
            state[a] = min(state[a] + 1, MAXCNT)
    if is_load:
        regs[x.addr] = _vregs(x.ops[0])
        state[x.addr] = 0


def kernel_hazards(ins):
    """(loads, [instruction text]) for one kernel: instructions reached, on some path, while a load
    whose registers they name may still be in flight."""
    if not ins:
        return 0, []
    blocks, succ = _cfg(ins)
    regs = {}
    entry = [None] * len(blocks)
    entry[0] = {}
    work = [0]
    while work:
        b = work.pop()
        st = dict(entry[b])
        s, e = blocks[b]
        for i in range(s, e + 1):
            _step(st, ins[i], regs, None)
        for nb in succ[b]:
            cur = entry[nb]
            if cur is None:
                entry[nb] = dict(st)
                work.append(nb)
                continue
            changed = False
            for a, k in st.items():
                if a not in cur or k < cur[a]:
                    cur[a] = k
                    changed = True
            if changed:
                work.append(nb)
    bad = []
    for b, (s, e) in enumerate(blocks):
        if entry[b] is None:
            continue  # unreachable
        st = dict(entry[b])
        for i in range(s, e + 1):
            _step(st, ins[i], regs, lambda x, a: bad.append(x.text))
    nloads = sum(1 for x in ins if x.op.startswith("global_load") and "lds" not in x.op)
    return nloads, sorted(set(bad), key=bad.index)


def early_uses(text):
    """(loads seen, [(kernel, instruction)] naming a pending load's registers before its wait, on
    some path through the kernel's control flow)."""
    nloads, bad = 0, []
    for name, ins in parse(text).items():
        n, b = kernel_hazards(ins)
        nloads += n
        bad += [(name, t) for t in b]
    return nloads, bad

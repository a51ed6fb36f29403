"""Minimal GGUF v3 writer for test fixtures (header, scalar / string / array key-values, tensor
infos, aligned tensor data), written from the GGUF v3 layout the reference reads
(qwen_cpu/gguf.h:106-175).  Test infrastructure only."""
import struct

# GGUF value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STR:
        return _str(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, i) for i in items)
    return struct.pack(_FMT[t], v)


def write(path, kvs, tensors, alignment=32, version=3):
    """kvs: [(key, type, value)]; tensors: [(name, ggml_type, dims (innermost first), bytes)].
    Returns {name: absolute file offset of its data}."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for key, t, v in kvs:
        head += _str(key) + struct.pack("<I", t) + _value(t, v)
    rel, off = [], 0
    for _, _, _, data in tensors:
        rel.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, typ, dims, _), r in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", typ, r)
    start = (len(head) + alignment - 1) // alignment * alignment
    blob = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), r in zip(tensors, rel):
        blob += b"\0" * (start + r - len(blob)) + bytes(data)
    with open(path, "wb") as f:
        f.write(blob)
    return {name: start + r for (name, _, _, _), r in zip(tensors, rel)}

"""GGUF writer with the byte layout of gguf.rs's GgufWriter (gguf.rs:472-620): magic, version,
counts (u64 for v3, u32 for v2), metadata key/values, the tensor-info table, padding to the
alignment, then each tensor's bytes at an offset that is a multiple of it. The alignment is the
general.alignment value when the metadata has one (U32 or U64), else the argument.
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(kind: int, v) -> bytes:
    """Encoded value of `kind`; arrays are (element kind, [items])."""
    if kind == STR:
        return gstr(v)
    if kind == ARRAY:
        ek, items = v
        return struct.pack("<IQ", ek, len(items)) + b"".join(value(ek, x) for x in items)
    return struct.pack(_FMT[kind], v)


def header(kvs, tensors, version=3) -> bytes:
    """kvs: [(key, kind, value)]; tensors: [(name, dims, ggml_type, offset)]."""
    counts = struct.pack("<QQ", len(tensors), len(kvs)) if version >= 3 else struct.pack("<II", len(tensors),
                                                                                          len(kvs))
    b = b"GGUF" + struct.pack("<I", version) + counts
    for k, kind, v in kvs:
        b += gstr(k) + struct.pack("<I", kind) + value(kind, v)
    for name, dims, ty, off in tensors:
        b += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        b += struct.pack("<IQ", ty, off)
    return b


_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 6: (32, 22), 8: (32, 34), 12: (256, 144),
          13: (256, 176), 14: (256, 210)}


def write(kvs, tensors, alignment=32, version=3) -> bytes:
    """A whole file. tensors: [(name, dims, ggml_type, data bytes)]; a sized type's data must
    hold exactly its element count (gguf.rs:551-563)."""
    for k, kind, v in kvs:
        if k == "general.alignment" and kind in (U32, U64):
            alignment = v
            break
    alignment = max(int(alignment), 1)
    for name, dims, ty, data in tensors:
        if ty in _BLOCK:
            numel = 1
            for d in dims:
                numel *= d
            qk, bb = _BLOCK[ty]
            if numel % qk == 0 and numel // qk * bb != len(data):
                raise ValueError(f"tensor {name} byte size mismatch: expected {numel // qk * bb}, got {len(data)}")
    offs, off = [], 0
    for _, _, _, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    h = header(kvs, [(n, d, t, o) for (n, d, t, _), o in zip(tensors, offs)], version)
    start = (len(h) + alignment - 1) // alignment * alignment
    out = bytearray(h + bytes(start - len(h)))
    for (_, _, _, data), o in zip(tensors, offs):
        pos = start + o
        if len(out) < pos:
            out += bytes(pos - len(out))
        out += bytes(data)
    return bytes(out)

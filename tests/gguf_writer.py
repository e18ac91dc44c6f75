"""A minimal GGUF v2/v3 writer for the tests (test infrastructure; the library only reads).

Restated from the public GGUF specification: u32 magic "GGUF", u32 version, u64 tensor count,
u64 kv count; kv entries {string key, u32 type, value}; tensor infos {string name, u32 n_dims,
u64 ne[n_dims], u32 type, u64 offset}; padding to the alignment; the data section, each
tensor at its offset (a multiple of the alignment) from the section start. Strings are a u64
length and the bytes.
"""
import struct

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f", T_BOOL: "<B",
        T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


def gstr(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def gval(t, v):
    if t == T_STR:
        return gstr(v)
    if t == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(gval(et, it) for it in items)
    return struct.pack(_FMT[t], v)


def build_gguf(kvs, tensors, alignment=32, version=3, offsets=None):
    """kvs: [(key, type, value)]; tensors: [(name, ggml type, ne, data bytes)]. Returns the file
    bytes, the data section start and the tensors' offsets within the section."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += gstr(k) + struct.pack("<I", t) + gval(t, v)
    if offsets is None:
        offsets, off = [], 0
        for _, _, _, data in tensors:
            off = (off + alignment - 1) // alignment * alignment
            offsets.append(off)
            off += len(data)
    for (name, t, ne, _), o in zip(tensors, offsets):
        head += gstr(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", e) for e in ne)
        head += struct.pack("<IQ", t, o)
    start = (len(head) + alignment - 1) // alignment * alignment
    end = max([start + o + len(d) for (_, _, _, d), o in zip(tensors, offsets)] + [start])
    buf = bytearray(end)
    buf[:len(head)] = head
    for (_, _, _, data), o in zip(tensors, offsets):
        buf[start + o:start + o + len(data)] = data
    return bytes(buf), start, offsets


def write_gguf(path, kvs, tensors, alignment=32, version=3):
    blob, start, offsets = build_gguf(kvs, tensors, alignment, version)
    with open(path, "wb") as f:
        f.write(blob)
    return start, offsets

"""A small GGUF v3 writer for tests: the layout the reference's fixture writes
(Tests/IshizukiKitTests/GGUFFixture.swift:51-79) — header, metadata, tensor table with dims
innermost-first and offsets rounded up to 32, zero padding to 32, then the data section."""
import struct

from ishizuki_amd.gguf import GGML_TYPES, byte_count

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)


def string(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def u32(v):
    return struct.pack("<I", v)


def f32(v):
    return struct.pack("<f", v)


def int_array(vals):
    return u32(I32 if any(v < 0 for v in vals) else U32) + struct.pack("<Q", len(vals)) + b"".join(
        struct.pack("<i" if v < 0 else "<I", v) for v in vals)


def string_array(vals):
    return u32(STRING) + struct.pack("<Q", len(vals)) + b"".join(string(v) for v in vals)


def build(tensors, metadata=(), payloads=None, version=3, magic=MAGIC, fill=0xAB, alignment=32):
    """`tensors`: (name, dims row-major, ggml type); `payloads`: optional name -> bytes (else the
    tensor's byte count of `fill`). Returns the file bytes."""
    out = bytearray(struct.pack("<IIQQ", magic, version, len(tensors), len(metadata)))
    for key, typ, payload in metadata:
        out += string(key) + u32(typ) + payload
    payloads = payloads or {}
    cursor, data = 0, bytearray()
    for name, dims, typ in tensors:
        out += string(name) + u32(len(dims))
        for d in reversed(dims):
            out += struct.pack("<Q", d)
        n = 1
        for d in dims:
            n *= d
        cursor = (cursor + alignment - 1) // alignment * alignment
        out += u32(typ) + struct.pack("<Q", cursor)
        body = payloads.get(name)
        if body is None:
            known = typ in GGML_TYPES
            body = bytes([fill]) * (byte_count(typ, n) if known and n % _block(typ) == 0 else 64)
        data += bytes(cursor - len(data)) + body
        cursor += len(body)
    out += bytes((alignment - len(out) % alignment) % alignment)
    return bytes(out + data)


def _block(typ):
    from ishizuki_amd.gguf import geometry
    return geometry(typ)[0]


def write(path, *args, **kw):
    with open(path, "wb") as f:
        f.write(build(*args, **kw))
    return path

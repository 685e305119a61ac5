"""GGUF byte builder for the GGUF tests: the reference's test helpers (header, Val,
write_kv, build, f32_tensor in crates/gguf/src/tests.rs:90-264) restated in Python, so
the same files can be fed to libferrum_kv.so and to oracle.gguf_ref."""
from __future__ import annotations

import struct


def header(version, tensors, kvs):
    return b"GGUF" + struct.pack("<IQQ", version, tensors, kvs)


def s(text):
    b = text.encode() if isinstance(text, str) else bytes(text)
    return struct.pack("<Q", len(b)) + b


# Val(type_id, payload writer)
def U8(v): return (0, struct.pack("<B", v))
def I8(v): return (1, struct.pack("<b", v))
def U16(v): return (2, struct.pack("<H", v))
def I16(v): return (3, struct.pack("<h", v))
def U32(v): return (4, struct.pack("<I", v))
def I32(v): return (5, struct.pack("<i", v))
def F32(v): return (6, struct.pack("<f", v))
def Bool(v): return (7, struct.pack("<B", v))
def Str(v): return (8, s(v))
def Raw(b): return (8, struct.pack("<Q", len(b)) + bytes(b))
def U64(v): return (10, struct.pack("<Q", v))
def I64(v): return (11, struct.pack("<q", v))
def F64(v): return (12, struct.pack("<d", v))


def Arr(elem, values, count=None):
    body = b"".join(v[1] for v in values)
    return (9, struct.pack("<IQ", elem, len(values) if count is None else count) + body)


def kv(key, val):
    return s(key) + struct.pack("<I", val[0]) + val[1]


def align_up(off, a):
    return off + (a - off % a) % a


def build(version, kvs, tensors, pad_alignment=None):
    """tensors: (name, dims, ggml_type, offset, bytes). With pad_alignment the data section
    is laid out at that alignment and each tensor's bytes written at its offset."""
    out = bytearray(header(version, len(tensors), len(kvs)))
    for key, val in kvs:
        out += kv(key, val)
    for name, dims, gt, off, _ in tensors:
        out += s(name) + struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", gt, off)
    if pad_alignment is not None:
        ds = align_up(len(out), pad_alignment)
        out += b"\0" * (ds - len(out))
        for _, _, _, off, data in tensors:
            if not data or off + len(data) > 8 << 20:
                continue
            end = ds + off + len(data)
            if end > len(out):
                out += b"\0" * (end - len(out))
            out[ds + off:end] = data
    return bytes(out)


def f32_tensor(name, shape, offset, data):
    return (name, list(shape), 0, offset, bytes(data))

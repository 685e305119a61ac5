"""Pure-Python restatement of Ferrum's GGUF decoder (TEST INFRASTRUCTURE).

Only tests/ use this module, as the checker of libferrum_kv.so's fkv_gguf_* reader; the
product never imports it. It follows crates/gguf/src/parse.rs (parse_view :100-181,
read_metadata :183-205, read_tensor_directory/read_tensor_info :207-258, read_value
:285-304, read_array :306-323, min_value_bytes :325-338, alignment_of/validate_alignment/
align_offset :340-366, bound_count :368-379, Reader :381-471), crates/gguf/src/layout.rs
:12-72 (stored sizes), crates/core-types/src/dtype.rs:47-129 (type names, shape_elements,
tensor_nbytes) and source.rs:25-56,70-92 (TensorDesc::try_new, format_gguf_dump). Errors
are raised as GgufRefError with the reference's message text.

Pinned by the reference's own test expectations (crates/gguf/src/tests.rs), restated in
tests/test_cpu_gguf.py against both this module and the library.
"""
from __future__ import annotations

import struct

MAGIC = b"GGUF"
MIN_KV_BYTES = 13
MIN_TENSOR_INFO_BYTES = 24
MAX_ARRAY_DEPTH = 64

LAYOUTS = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
    9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
    14: (256, 210), 15: (256, 292), 16: (256, 66), 17: (256, 74), 18: (256, 98),
    19: (256, 50), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136), 24: (1, 1),
    25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 29: (256, 56), 30: (1, 2),
    34: (256, 54), 35: (256, 66), 39: (32, 17),
}

TYPE_NAMES = {
    0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 4: "q4_2", 5: "q4_3", 6: "q5_0", 7: "q5_1",
    8: "q8_0", 9: "q8_1", 10: "q2_K", 11: "q3_K", 12: "q4_K", 13: "q5_K", 14: "q6_K",
    15: "q8_K", 16: "iq2_xxs", 17: "iq2_xs", 18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl",
    21: "iq3_s", 22: "iq2_s", 23: "iq4_xs", 24: "i8", 25: "i16", 26: "i32", 27: "i64",
    28: "f64", 29: "iq1_m", 30: "bf16", 34: "tq1_0", 35: "tq2_0", 39: "mxfp4",
}

U64_MAX = (1 << 64) - 1


class GgufRefError(Exception):
    pass


def _bad(msg):
    raise GgufRefError(msg)


def bound_count(count, min_elem, remaining):
    if min_elem == 0:
        _bad("element size is zero")
    if count > remaining // min_elem:
        _bad("count exceeds remaining bytes")
    return count


def min_value_bytes(t):
    return {0: 1, 1: 1, 7: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 9: 12}.get(t, 8)


class _Reader:
    def __init__(self, data):
        self.data, self.pos = data, 0

    def remaining(self):
        return max(0, len(self.data) - self.pos)

    def exact(self, n):
        if n > len(self.data) - self.pos:
            _bad("unexpected end of gguf file")
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def le(self, fmt):
        return struct.unpack("<" + fmt, self.exact(struct.calcsize(fmt)))[0]

    def string(self):
        n = bound_count(self.le("Q"), 1, self.remaining())
        b = self.exact(n)
        try:
            return b.decode("utf-8", errors="strict")
        except UnicodeDecodeError:
            _bad("invalid utf-8")


_SCALARS = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 10: "Q", 11: "q", 12: "d"}


def _read_value(r, t, depth):
    if t in _SCALARS:
        return (t, r.le(_SCALARS[t]))
    if t == 7:
        b = r.le("B")
        if b > 1:
            _bad("invalid bool byte")
        return (t, b == 1)
    if t == 8:
        return (t, r.string())
    return _read_array(r, depth)


def _read_array(r, depth):
    if depth >= MAX_ARRAY_DEPTH:
        _bad("metadata array nested too deeply")
    elem = r.le("I")
    if elem > 12:
        _bad(f"unknown metadata type {elem}")
    n = bound_count(r.le("Q"), min_value_bytes(elem), r.remaining())
    return (9, (elem, [_read_value(r, elem, depth + 1) for _ in range(n)]))


def shape_elements(shape):
    if not shape or len(shape) > 4:
        _bad("tensor rank must be from 1 to 4 inclusive")
    n = 1
    for d in shape:
        if d == 0:
            _bad("tensor dimension is zero")
        n *= d
        if n > U64_MAX:
            _bad("tensor element count overflow")
    return n


def stored_nbytes(t, elements):
    if t not in LAYOUTS:
        _bad(f"ggml type {t} has no stored size")
    block, nbytes = LAYOUTS[t]
    if elements % block:
        _bad("tensor element count is not a multiple of the block size")
    n = elements // block * nbytes
    if n > U64_MAX:
        _bad("tensor size overflow")
    return n


def validate_alignment(a):
    if a == 0 or a % 8:
        _bad("alignment must be a non-zero multiple of 8")
    return a


def _try_new(t):
    name, shape, gt, _off, nbytes = t
    elements = shape_elements(shape)
    if gt in (0, 1, 8):
        if gt == 8:
            if elements % 32:
                _bad("q8_0 element count is not a multiple of 32")
            expected = elements // 32 * 34
        else:
            expected = elements * (4 if gt == 0 else 2)
        if expected > U64_MAX:
            _bad("tensor size overflow")
        if expected != nbytes:
            _bad(f"tensor {name} byte count {nbytes} does not match layout {expected}")
    elif nbytes == 0:
        _bad("unsupported tensor has zero bytes")


def parse(data: bytes):
    """Returns dict(version, alignment, metadata {key: (type, value)}, tensors [(name,
    shape, ggml_type, data_offset, nbytes)], data_start); raises GgufRefError."""
    r = _Reader(data)
    if r.exact(4) != MAGIC:
        _bad("bad gguf magic")
    version = r.le("I")
    if version not in (2, 3):
        _bad(f"unsupported gguf version {version}")
    tensor_count, kv_count = r.le("Q"), r.le("Q")
    meta = {}
    for _ in range(bound_count(kv_count, MIN_KV_BYTES, r.remaining())):
        key = r.string()
        t = r.le("I")
        if t > 12:
            _bad(f"unknown metadata type {t}")
        v = _read_value(r, t, 0)
        if key in meta:
            _bad(f"duplicate metadata key {key}")
        meta[key] = v
    al = meta.get("general.alignment")
    if al is None:
        alignment = 32
    elif al[0] in (4, 10):
        alignment = validate_alignment(al[1])
    else:
        _bad("general.alignment must be uint32 or uint64")
    tensors, seen = [], set()
    for _ in range(bound_count(tensor_count, MIN_TENSOR_INFO_BYTES, r.remaining())):
        name = r.string()
        if name in seen:
            _bad(f"duplicate tensor name {name}")
        seen.add(name)
        n_dims = r.le("I")
        if n_dims == 0 or n_dims > 4:
            _bad("tensor rank must be from 1 to 4 inclusive")
        bound_count(n_dims, 8, r.remaining())
        shape = [r.le("Q") for _ in range(n_dims)]
        gt, off = r.le("I"), r.le("Q")
        tensors.append((name, shape, gt, off, stored_nbytes(gt, shape_elements(shape))))
    info_end = r.pos
    a = validate_alignment(alignment)
    data_start = info_end + (a - info_end % a) % a
    if data_start > U64_MAX:
        _bad("aligned offset overflows")
    if data_start > len(data):
        _bad("alignment padding exceeds file")
    if any(data[info_end:data_start]):
        _bad("alignment padding is not zero")
    data_len = len(data) - data_start
    for t in tensors:
        name, _, _, off, nbytes = t
        if off % alignment:
            _bad(f"tensor {name} data_offset is not aligned")
        if off + nbytes > U64_MAX:
            _bad(f"tensor {name} data range overflows")
        if off + nbytes > data_len:
            _bad(f"tensor {name} extends past end of file")
        _try_new(t)
    return {"version": version, "alignment": alignment, "metadata": meta,
            "tensors": tensors, "data_start": data_start}


def dump(p) -> str:
    """format_gguf_dump (crates/core-types/src/source.rs:70-92)."""
    out = (f"ferrum-gguf version={p['version']} alignment={p['alignment']} "
           f"metadata={len(p['metadata'])} tensors={len(p['tensors'])}\n")
    for name, shape, gt, _, _ in p["tensors"]:
        out += f"{name} [{', '.join(str(d) for d in shape)}] {TYPE_NAMES.get(gt, 'unknown')}\n"
    return out

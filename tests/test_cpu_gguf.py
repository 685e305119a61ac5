"""CPU: the GGUF reader (fkv_gguf_*) against Ferrum's gguf::load.

Every case of crates/gguf/src/tests.rs is restated with the same bytes (tests/gguf_build.py
restates its builders). Each file is decoded by libferrum_kv.so (through a real file:
open, mmap, decode) and by oracle/gguf_ref.py (an independent restatement of parse.rs);
both must accept or reject it alike, with the same message, and every message must
contain what the reference's own test asserts. Accepted files are compared field by field
(version, alignment, metadata types and values bit for bit, tensor directory, dump text).
A seeded differential fuzz (truncations, byte flips, field overwrites of a rich file)
extends the comparison past the hand-written cases.
"""
import math
import os
import struct

import numpy as np
import pytest

import ferrum_amd as fa
from oracle import gguf_ref
from tests import gguf_build as gb
from tests.gguf_build import (Arr, Bool, F32, F64, I8, I16, I32, I64, Raw, Str, U8, U16, U32,
                              U64, build, f32_tensor, header)


@pytest.fixture
def path(tmp_path):
    return str(tmp_path / "model.gguf")


def _write(path, data):
    with open(path, "wb") as f:
        f.write(data)


def load_ok(path, data):
    _write(path, data)
    f = fa.GgufFile(path)
    ref = gguf_ref.parse(data)
    _same_file(f, ref)
    return f


def load_err(path, data):
    """The library's message (without "gguf: "), equal to the oracle's."""
    _write(path, data)
    with pytest.raises(fa.GgufError) as e:
        fa.GgufFile(path)
    msg = str(e.value)
    assert msg.startswith("gguf: "), msg
    with pytest.raises(gguf_ref.GgufRefError) as r:
        gguf_ref.parse(data)
    assert msg[len("gguf: "):] == str(r.value)
    return msg[len("gguf: "):]


def _same_value(f, key, want):
    t, v = want
    assert f.metadata_type(key) == t, key
    got = f.metadata(key)
    _same_scalar_or_array(f, key, t, v, got)


def _same_scalar_or_array(f, key, t, v, got):
    if t == 9:
        elem, vals = v
        assert isinstance(got, list) and len(got) == len(vals), key
        for g, (et, ev) in zip(got, vals):
            if et == 9:
                assert g == ("array", ev[0], len(ev[1])), key
            else:
                _same_scalar(et, ev, g, key)
    else:
        _same_scalar(t, v, got, key)


def _same_scalar(t, v, got, key):
    if t == 6:
        assert np.float32(got).view(np.uint32) == np.float32(v).view(np.uint32), key
    elif t == 12:
        assert struct.pack("<d", got) == struct.pack("<d", v), key
    else:
        assert got == v, key


def _same_file(f, ref):
    assert f.version == ref["version"]
    assert f.alignment == ref["alignment"]
    assert f.metadata_len == len(ref["metadata"])
    assert f.data_start == ref["data_start"]
    assert [(t.name, list(t.shape), t.ggml_type, t.data_offset, t.nbytes) for t in f.tensors] == \
        [(n, list(s), g, o, b) for n, s, g, o, b in ref["tensors"]]
    assert f.dump() == gguf_ref.dump(ref)
    assert f.dump().endswith("\n")
    for key, val in ref["metadata"].items():
        _same_value(f, key, val)


def tensor_bytes(path, f, name):
    t = f.tensor(name)
    with open(path, "rb") as h:
        h.seek(f.data_start + t.data_offset)
        return h.read(t.nbytes)


# ---------------------------------------------------------------------------
# crates/gguf/src/tests.rs, case by case
# ---------------------------------------------------------------------------

def test_loads_f32_tensor_relative_to_the_data_section(path):
    payload, second = bytes([1, 2, 3, 4]), bytes([5, 6, 7, 8])
    data = build(3, [("general.alignment", U32(32)), ("name", Str("x"))],
                 [f32_tensor("a", [1], 0, payload), f32_tensor("b", [1], 32, second)], 32)
    f = load_ok(path, data)
    assert (f.version, f.alignment, f.metadata_len) == (3, 32, 2)
    assert f.metadata("name") == "x"
    assert f.metadata("missing") is None
    assert tensor_bytes(path, f, "a") == payload and tensor_bytes(path, f, "b") == second
    assert f.tensor("a").ggml_type == 0 and f.tensor("a").nbytes == 4
    with pytest.raises(fa.GgufError, match="^gguf: missing tensor missing$"):
        f.tensor("missing")
    assert f.dump() == "ferrum-gguf version=3 alignment=32 metadata=2 tensors=2\na [1] f32\nb [1] f32\n"


def test_version_two_and_odd_f32_and_f16_lengths(path):
    data = build(2, [], [f32_tensor("f", [3], 0, range(1, 13)),
                         ("h", [3], 1, 32, bytes([9, 8, 7, 6, 5, 4]))], 32)
    f = load_ok(path, data)
    assert (f.version, f.alignment, f.metadata_len) == (2, 32, 0)
    assert f.tensor("f").nbytes == 12 and f.tensor("h").nbytes == 6
    assert tensor_bytes(path, f, "h") == bytes([9, 8, 7, 6, 5, 4])


def test_empty_directory_uses_default_alignment_and_zero_padding(path):
    data = header(3, 0, 0)
    assert len(data) == 24
    assert "padding" in load_err(path, data)
    padded = data + b"\0" * 8
    f = load_ok(path, padded)
    assert f.dump() == "ferrum-gguf version=3 alignment=32 metadata=0 tensors=0\n"
    dirty = bytearray(padded)
    dirty[24] = 1
    assert "not zero" in load_err(path, bytes(dirty))
    assert load_ok(path, header(2, 0, 0) + b"\0" * 8).version == 2


def test_alignment_key_accepts_u32_and_u64_multiples_of_eight(path):
    payload = bytes([9, 8, 7, 6])
    f = load_ok(path, build(3, [("general.alignment", U64(64))],
                            [f32_tensor("w", [1], 0, payload)], 64))
    assert f.alignment == 64 and tensor_bytes(path, f, "w") == payload
    assert load_ok(path, build(3, [("general.alignment", U32(8))],
                               [f32_tensor("w", [1], 0, payload)], 8)).alignment == 8
    for bad in (U32(0), U32(12), U64(0), U64(4), U16(32)):
        assert "alignment" in load_err(path, build(3, [("general.alignment", bad)], []))
    err = load_err(path, build(3, [("general.alignment", U64(1 << 33))], []))
    assert "padding" in err or "overflow" in err


def test_magic_version_and_short_buffers(path):
    assert "end of" in load_err(path, bytes([0x47, 0x47, 0x55]))
    assert "magic" in load_err(path, b"gguf")
    wrong = bytearray(header(3, 0, 0))
    wrong[0] = 0
    assert "magic" in load_err(path, bytes(wrong))
    for v in (1, 0, 4):
        assert "version" in load_err(path, header(v, 0, 0))
    big_endian = b"GGUF" + struct.pack(">I", 3)
    err = load_err(path, big_endian)
    assert "version" in err or "end of" in err
    assert "end of" in load_err(path, b"")   # an empty file


def test_missing_path_and_directory_are_errors(tmp_path):
    with pytest.raises(fa.GgufError, match=r"^gguf: failed to open .*No such file or directory \(os error 2\)$"):
        fa.GgufFile(str(tmp_path / "missing.gguf"))
    with pytest.raises(fa.GgufError, match=r"^gguf: failed to map "):
        fa.GgufFile(str(tmp_path))


def test_every_metadata_type_and_nested_arrays_round_trip(path):
    nested = Arr(9, [Arr(0, [U8(9), U8(8)])])
    words = Arr(8, [Str("a"), Str("bb"), Str("▁")])
    data = build(3, [("u8", U8(255)), ("i8", I8(-1)), ("u16", U16(65535)), ("i16", I16(-300)),
                     ("u32", U32(0x8000_0000)), ("i32", I32(-2)), ("f32", F32(-0.0)),
                     ("bf", Bool(0)), ("bt", Bool(1)), ("s", Str("héllo")),
                     ("arr", Arr(2, [U16(1), U16(2), U16(3)])), ("words", words),
                     ("u64", U64(2 ** 64 - 1)), ("i64", I64(-2 ** 63)), ("f64", F64(1.5)),
                     ("nest", nested)], [], 32)
    f = load_ok(path, data)
    assert f.metadata_len == 16
    assert f.metadata("u8") == 255 and f.metadata("i8") == -1 and f.metadata("i16") == -300
    assert f.metadata("u32") == 0x8000_0000 and f.metadata("u64") == 2 ** 64 - 1
    assert f.metadata("i64") == -2 ** 63
    assert math.copysign(1.0, f.metadata("f32")) == -1.0 and f.metadata("f32") == 0.0
    assert f.metadata("bf") is False and f.metadata("bt") is True
    assert f.metadata("s") == "héllo" and f.metadata("f64") == 1.5
    assert f.metadata("arr") == [1, 2, 3] and f.metadata("words") == ["a", "bb", "▁"]
    assert f.metadata("nest") == [("array", 0, 2)]


def test_invalid_bool_utf8_and_type_tag(path):
    assert "bool" in load_err(path, build(3, [("b", Bool(2))], []))
    assert "bool" in load_err(path, build(3, [("b", Bool(0xff))], []))
    assert "bool" in load_err(path, build(3, [("b", Arr(7, [Bool(0), Bool(1), Bool(2)]))], []))
    bad_key = header(3, 0, 1) + struct.pack("<Q", 2) + bytes([0xff, 0xfe]) + struct.pack("<I", 0) + b"\1"
    assert "utf-8" in load_err(path, bad_key)
    assert "utf-8" in load_err(path, build(3, [("a", Raw([0xff, 0xfe]))], []))
    assert "utf-8" in load_err(path, build(3, [("a", Arr(8, [Str("ok"), Raw([0xff])]))], []))
    # overlong and surrogate encodings are not UTF-8 either (Rust's str::from_utf8)
    for raw in ([0xc0, 0x80], [0xed, 0xa0, 0x80], [0xf4, 0x90, 0x80, 0x80], [0xe2, 0x82]):
        assert "utf-8" in load_err(path, build(3, [("a", Raw(raw))], []))
    unknown = header(3, 0, 1) + gb.s("a") + struct.pack("<I", 13)
    assert "unknown metadata type" in load_err(path, unknown)


def test_claimed_counts_are_rejected_without_panicking(path):
    assert "count" in load_err(path, header(3, 0, 2 ** 64 - 1))
    assert "count" in load_err(path, header(3, 2 ** 64 - 1, 0))
    err = load_err(path, header(3, 0, 1) + struct.pack("<Q", 2 ** 64 - 1))
    assert "count" in err or "end of" in err
    huge_array = header(3, 0, 1) + gb.s("a") + struct.pack("<IIQ", 9, 0, 2 ** 64 - 1)
    assert "count" in load_err(path, huge_array)
    just_over = header(3, 0, 1) + gb.s("a") + struct.pack("<IIQ", 9, 0, 11) + b"\1" * 10
    assert "count" in load_err(path, just_over)
    nested_huge = header(3, 0, 1) + gb.s("a") + struct.pack("<IIQIQ", 9, 9, 1, 0, 2 ** 64 - 1)
    assert "count" in load_err(path, nested_huge)
    rank = header(3, 1, 0) + gb.s("w") + struct.pack("<I", 2 ** 32 - 1) + b"\0" * 64
    assert "rank" in load_err(path, rank)


def nested_u8(depth):
    return Arr(0, [U8(7)]) if depth == 1 else Arr(9, [nested_u8(depth - 1)])


def test_nested_array_depth_is_bounded(path):
    f = load_ok(path, build(3, [("a", nested_u8(3))], [], 32))
    assert f.metadata("a") == [("array", 9, 1)]
    assert load_ok(path, build(3, [("a", nested_u8(64))], [], 32)).metadata_len == 1
    assert "nested" in load_err(path, build(3, [("a", nested_u8(65))], []))


def test_tensor_shape_offset_and_range_are_checked(path):
    assert "rank" in load_err(path, build(3, [], [("w", [], 0, 0, b"")]))
    assert "rank" in load_err(path, build(3, [], [("w", [1, 1, 1, 1, 1], 0, 0, b"")]))
    assert "zero" in load_err(path, build(3, [], [f32_tensor("w", [0], 0, b"")]))
    assert "zero" in load_err(path, build(3, [], [f32_tensor("w", [4, 0, 1], 0, b"")]))
    assert "overflow" in load_err(path, build(3, [], [f32_tensor("w", [1 << 62], 0, b"")]))
    assert "aligned" in load_err(path, build(3, [("general.alignment", U32(32))],
                                             [f32_tensor("w", [1], 8, [1, 2, 3, 4])], 32))
    exact = build(3, [], [f32_tensor("w", [1], 0, [1, 2, 3, 4])], 32)
    assert "past end" in load_err(path, exact[:-1])
    err = load_err(path, build(3, [("general.alignment", U32(8))],
                               [f32_tensor("w", [1], 2 ** 64 - 8, [1, 2, 3, 4])], 8))
    assert "overflow" in err or "past end" in err
    f = load_ok(path, build(3, [], [f32_tensor("w", [2, 3, 1, 1], 0, bytes(24))], 32))
    assert f.tensor("w").shape == (2, 3, 1, 1) and f.tensor("w").nbytes == 24


def test_q8_0_and_other_ggml_types_are_bounds_checked(path):
    f = load_ok(path, build(3, [], [("q", [32], 8, 0, b"\x11" * 34)], 32))
    assert f.tensor("q").ggml_type == 8 and f.tensor("q").nbytes == 34
    assert tensor_bytes(path, f, "q") == b"\x11" * 34 and "q8_0" in f.dump()
    assert "multiple" in load_err(path, build(3, [], [("q", [16], 8, 0, b"")]))
    f = load_ok(path, build(3, [], [("k", [256], 12, 0, b"\x22" * 144)], 32))
    assert f.tensor("k").nbytes == 144 and "q4_K" in f.dump()
    short = build(3, [], [("q", [32], 2, 0, b"\x33" * 18)], 32)
    assert load_ok(path, short).tensor("q").nbytes == 18
    assert "past end" in load_err(path, short[:-1])
    for gid in (4, 5, 31, 100):
        assert "no stored size" in load_err(path, build(3, [], [("w", [1], gid, 0, b"")]))


def test_every_sized_ggml_type_is_listed_and_bounded(path):
    tensors, cursor = [], 0
    for gid, (block, nbytes) in gguf_ref.LAYOUTS.items():
        off = gb.align_up(cursor, 32)
        tensors.append((f"t{gid}", [block], gid, off, b"\xab" * nbytes))
        cursor = off + nbytes
    data = build(3, [], tensors, 32)
    f = load_ok(path, data)
    assert len(f.tensors) == len(gguf_ref.LAYOUTS)
    for gid, (block, nbytes) in gguf_ref.LAYOUTS.items():
        t = f.tensor(f"t{gid}")
        assert t.shape == (block,) and t.nbytes == nbytes and t.ggml_type == gid
        assert tensor_bytes(path, f, t.name) == b"\xab" * nbytes
        assert f"] {fa.gguf.GGML_TYPE_NAMES[gid]}\n" in f.dump()
    assert "past end" in load_err(path, data[:-1])


def test_duplicate_metadata_key_and_tensor_name(path):
    assert "duplicate metadata" in load_err(path, build(3, [("a", U8(1)), ("a", U8(2))], []))
    assert "duplicate tensor" in load_err(path, build(3, [], [f32_tensor("w", [1], 0, [1, 2, 3, 4]),
                                                            f32_tensor("w", [1], 32, [5, 6, 7, 8])]))


def test_llama_metadata_is_readable(path):
    """tests.rs:891-930's file: the keys a Llama config is read from."""
    toks = Arr(8, [Str("<unk>"), Str("<s>"), Str("</s>"), Str("a")])
    data = build(3, [("general.architecture", Str("llama")), ("general.name", Str("tiny")),
                     ("llama.context_length", U64(32)), ("llama.embedding_length", U32(8)),
                     ("llama.block_count", U32(2)), ("llama.feed_forward_length", U32(16)),
                     ("llama.attention.head_count", U32(2)),
                     ("llama.attention.head_count_kv", U64(1)),
                     ("llama.attention.layer_norm_rms_epsilon", F32(1e-5)),
                     ("tokenizer.ggml.model", Str("llama")),
                     ("tokenizer.ggml.bos_token_id", U32(1)),
                     ("tokenizer.ggml.eos_token_id", U32(2)), ("tokenizer.ggml.tokens", toks)],
                 [], 32)
    f = load_ok(path, data)
    assert f.metadata("general.architecture") == "llama" and f.metadata("general.name") == "tiny"
    assert f.metadata("llama.block_count") == 2 and f.metadata("llama.attention.head_count_kv") == 1
    assert len(f.metadata("tokenizer.ggml.tokens")) == 4
    assert np.float32(f.metadata("llama.attention.layer_norm_rms_epsilon")) == np.float32(1e-5)


# ---------------------------------------------------------------------------
# Differential fuzz against the restatement
# ---------------------------------------------------------------------------

def _rich():
    tensors = [f32_tensor("a", [3, 2], 0, bytes(range(24))), ("q", [64], 8, 32, b"\x05" * 68),
               ("h", [5], 1, 128, bytes(10)), ("k", [256], 12, 160, b"\x07" * 144)]
    kvs = [("general.alignment", U32(32)), ("s", Str("héllo")), ("f", F32(2.5)),
           ("arr", Arr(4, [U32(1), U32(2)])), ("n", nested_u8(3)), ("b", Bool(1)),
           ("i", I64(-5)), ("d", F64(-0.25))]
    return build(3, kvs, tensors, 32)


def test_differential_fuzz(path):
    base = _rich()
    gguf_ref.parse(base)  # valid
    rng = np.random.default_rng(12345)
    outcomes = {"ok": 0, "err": 0}
    for case in range(600):
        data = bytearray(base)
        kind = case % 4
        if kind == 0:
            data = data[:int(rng.integers(0, len(data)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 4))):
                data[int(rng.integers(0, len(data)))] = int(rng.integers(0, 256))
        elif kind == 2:  # overwrite an 8-byte field with a small, large or random value
            at = int(rng.integers(0, len(data) - 8))
            picks = [0, 1, 3, 8, 2 ** 63, 2 ** 64 - 1, int(rng.integers(0, 2 ** 32))]
            val = picks[int(rng.integers(0, len(picks)))]
            data[at:at + 8] = struct.pack("<Q", val)
        else:
            at = int(rng.integers(0, len(data)))
            data = data[:at] + bytes(rng.integers(0, 256, int(rng.integers(1, 40)), dtype=np.uint8)) + data[at:]
        data = bytes(data)
        _write(path, data)
        try:
            want = gguf_ref.parse(data)
        except gguf_ref.GgufRefError as e:
            with pytest.raises(fa.GgufError) as got:
                fa.GgufFile(path)
            assert str(got.value) == "gguf: " + str(e), f"case {case}"
            outcomes["err"] += 1
            continue
        with fa.GgufFile(path) as f:
            _same_file(f, want)
        outcomes["ok"] += 1
    assert outcomes["ok"] >= 20 and outcomes["err"] >= 300, outcomes

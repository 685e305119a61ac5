"""ctypes wrapper of the CPU oracle (oracle/_build/libferrum_oracle.so).

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module, always as the checker. The product path
(ferrum_amd / libferrum_kv.so) never imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libferrum_oracle.so")

c_void_p, u32, u64, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32


class LayoutC(ctypes.Structure):
    _fields_ = [("n_layers", u32), ("n_kv_heads", u32), ("head_dim", u32),
                ("block_size", u32), ("num_blocks", u64), ("dtype", i32), ("rounding", i32)]


_SIGS = {
    "fo_tile_bytes": (u64, [c_void_p]),
    "fo_block_bytes": (u64, [c_void_p]),
    "fo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "fo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float, i32]),
    "fo_f32_to_f16_array": (None, [c_void_p, c_void_p, u64, i32]),
    "fo_f16_to_f32_array": (None, [c_void_p, c_void_p, u64]),
    "fo_q8_quantize_block": (None, [c_void_p, i32, c_void_p, c_void_p]),
    "fo_q8_quantize_row": (None, [c_void_p, u64, i32, c_void_p]),
    "fo_q8_dequant": (None, [c_void_p, u64, c_void_p]),
    "fo_q8_gemm": (None, [c_void_p, u64, u64, c_void_p, u64, c_void_p, i32]),
    "fo_dot": (ctypes.c_float, [c_void_p, c_void_p, u64]),
    "fo_softmax": (None, [c_void_p, u64]),
    "fo_rope": (None, [c_void_p, u64, u32, u32, u32, ctypes.c_float]),
    "fo_append": (u64, [c_void_p, c_void_p, u32, c_void_p, c_void_p, c_void_p, u64]),
    "fo_gather_slots": (None, [c_void_p, c_void_p, u32, c_void_p, u64, i32, c_void_p, c_void_p]),
    "fo_gather_tables": (None, [c_void_p, c_void_p, u32, c_void_p, u32, c_void_p, c_void_p, u32,
                                i32, c_void_p, c_void_p]),
    "fo_copy_blocks": (None, [c_void_p, c_void_p, c_void_p, u64]),
    "fo_attention": (None, [c_void_p, c_void_p, u32, u32, c_void_p, c_void_p, c_void_p, u32,
                            c_void_p, u32, ctypes.c_float]),
    "fo_prefill_attention": (None, [c_void_p, c_void_p, u32, u32, c_void_p, c_void_p, c_void_p,
                                    u32, c_void_p, c_void_p, c_void_p, u32, ctypes.c_float]),
    "fo_avx2_available": (i32, []),
    "fo_avx2_dot": (ctypes.c_float, [c_void_p, c_void_p, u64]),
    "fo_avx2_softmax": (None, [c_void_p, u64]),
    "fo_avx2_attention": (None, [c_void_p, c_void_p, u32, u32, c_void_p, c_void_p, c_void_p,
                                 u32, c_void_p, u32, ctypes.c_float, i32]),
    "fo_max_threads": (i32, []),
    "fo_dense_new": (i32, [u64, u64, u64, u64, u64, ctypes.POINTER(c_void_p),
                           ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_destroy": (None, [c_void_p]),
    "fo_dense_storage_len": (u64, [c_void_p]),
    "fo_dense_alloc": (i32, [c_void_p, ctypes.POINTER(u32), ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_free": (i32, [c_void_p, u32, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_seq_len": (i32, [c_void_p, u32, ctypes.POINTER(u64), ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_append_layer": (i32, [c_void_p, u32, u64, c_void_p, u64, c_void_p, u64,
                                    ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_commit_token": (i32, [c_void_p, u32, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_k": (i32, [c_void_p, u32, u64, u64, c_void_p, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_v": (i32, [c_void_p, u32, u64, u64, c_void_p, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_abandon_partial": (i32, [c_void_p, u32, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_dense_uncommit_token": (i32, [c_void_p, u32, ctypes.POINTER(ctypes.c_char_p)]),
    "fo_selftest_f16": (u64, [i32, u32, ctypes.POINTER(u32)]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


@dataclass(frozen=True)
class Layout:
    n_layers: int
    n_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    dtype: int = 1
    rounding: int = 0

    def c(self) -> LayoutC:
        return LayoutC(self.n_layers, self.n_kv_heads, self.head_dim, self.block_size,
                       self.num_blocks, self.dtype, self.rounding)

    @property
    def tile_bytes(self) -> int:
        return lib().fo_tile_bytes(ctypes.byref(self.c()))

    @property
    def block_bytes(self) -> int:
        return lib().fo_block_bytes(ctypes.byref(self.c()))

    @property
    def pool_bytes(self) -> int:
        return self.block_bytes * self.num_blocks

    def raw_head_bytes(self) -> int:
        d = self.head_dim
        return {0: d * 4, 1: d * 2, 8: d // 32 * 34}[self.dtype]


# -- codecs -------------------------------------------------------------------

def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().fo_f16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_f16(x: np.ndarray, rounding: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().fo_f32_to_f16_array(_p(a), _p(out), a.size, rounding)
    return out


def q8_quantize_block(x32: np.ndarray, rounding: int = 0):
    a = np.ascontiguousarray(x32, dtype=np.float32)
    assert a.size == 32
    s = np.zeros(1, dtype=np.uint16)
    q = np.zeros(32, dtype=np.int8)
    lib().fo_q8_quantize_block(_p(a), rounding, _p(s), _p(q))
    return int(s[0]), q


def q8_quantize_row(x: np.ndarray, rounding: int = 0) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(a.size // 32 * 34, dtype=np.uint8)
    lib().fo_q8_quantize_row(_p(a), a.size, rounding, _p(out))
    return out


def q8_dequant(blocks: np.ndarray, n: int) -> np.ndarray:
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    lib().fo_q8_dequant(_p(b), n, _p(out))
    return out


def q8_gemm(w: np.ndarray, rows: int, cols: int, x: np.ndarray, threads: int = 0) -> np.ndarray:
    """Kernels::gemm/gemv for Q8_0 weights (fo_q8_gemm): x [n_tokens, cols] (or
    [cols]) -> y [n_tokens, rows] float32, rows split over `threads` (0: default)."""
    wb = np.ascontiguousarray(w, dtype=np.uint8).ravel()
    xa = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    assert cols % 32 == 0 and wb.size == rows * (cols // 32) * 34
    y = np.empty((xa.shape[0], rows), dtype=np.float32)
    lib().fo_q8_gemm(_p(wb), rows, cols, _p(xa), xa.shape[0], _p(y), threads)
    return y


def dot(a, b) -> np.float32:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return np.float32(lib().fo_dot(_p(a), _p(b), a.size))


def softmax(x) -> np.ndarray:
    a = np.array(x, dtype=np.float32, copy=True)
    lib().fo_softmax(_p(a), a.size)
    return a


def rope(x, rope_dim: int, pos: int, theta: float) -> np.ndarray:
    """A copy of x (f32 [..., head_dim]) with every row rotated at position pos."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    d = a.shape[-1]
    lib().fo_rope(_p(a), a.size // d if d else 0, d, rope_dim, pos, theta)
    return a


def rope_step(q, k, ctx_lens, rope_dim: int, theta: float):
    """q [n_seqs][Hq][D] and k [n_seqs][Hkv][D] rotated per sequence at position
    ctx_lens[s] - 1 (0 for an empty context), as the RoPE decode step does."""
    q = np.array(q, dtype=np.float32, copy=True)
    k = np.array(k, dtype=np.float32, copy=True)
    for s, c in enumerate(np.asarray(ctx_lens)):
        pos = int(c) - 1 if int(c) > 0 else 0
        q[s] = rope(q[s], rope_dim, pos, theta)
        k[s] = rope(k[s], rope_dim, pos, theta)
    return q, k


def avx2_available() -> bool:
    return bool(lib().fo_avx2_available())


def avx2_dot(a, b) -> np.float32:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return np.float32(lib().fo_avx2_dot(_p(a), _p(b), a.size))


def avx2_softmax(x) -> np.ndarray:
    a = np.array(x, dtype=np.float32, copy=True)
    lib().fo_avx2_softmax(_p(a), a.size)
    return a


def selftest_f16(which: int, stride: int = 1):
    fb = u32(0)
    bad = lib().fo_selftest_f16(which, stride, ctypes.byref(fb))
    return int(bad), int(fb.value)


# -- paged pool image ------------------------------------------------------------

def new_pool(layout: Layout) -> np.ndarray:
    return np.zeros(layout.pool_bytes, dtype=np.uint8)


def append(layout: Layout, pool: np.ndarray, layer: int, k, v, slots) -> int:
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    s = np.ascontiguousarray(slots, dtype=np.int64)
    return int(lib().fo_append(ctypes.byref(layout.c()), _p(pool), layer, _p(k), _p(v), _p(s),
                               s.size))


def _out_rows(layout: Layout, n: int, fmt: int):
    if fmt == 0:
        shape = (n, layout.n_kv_heads, layout.head_dim)
        return np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    b = layout.n_kv_heads * layout.raw_head_bytes()
    return np.zeros((n, b), np.uint8), np.zeros((n, b), np.uint8)


def gather_slots(layout: Layout, pool: np.ndarray, layer: int, slots, fmt: int = 0):
    s = np.ascontiguousarray(slots, dtype=np.int64)
    ok, ov = _out_rows(layout, s.size, fmt)
    lib().fo_gather_slots(ctypes.byref(layout.c()), _p(pool), layer, _p(s), s.size, fmt, _p(ok),
                          _p(ov))
    return ok, ov


def gather_tables(layout: Layout, pool: np.ndarray, layer: int, tables, ctx_lens, fmt: int = 0):
    t = np.ascontiguousarray(tables, dtype=np.int32)
    c = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    offs = np.zeros(c.size, dtype=np.int64)
    offs[1:] = np.cumsum(c[:-1].astype(np.int64))
    total = int(c.astype(np.int64).sum())
    ok, ov = _out_rows(layout, total, fmt)
    lib().fo_gather_tables(ctypes.byref(layout.c()), _p(pool), layer, _p(t), t.shape[1], _p(c),
                           _p(offs), c.size, fmt, _p(ok), _p(ov))
    return ok, ov, offs


def copy_blocks(layout: Layout, pool: np.ndarray, pairs) -> None:
    p = np.ascontiguousarray(pairs, dtype=np.int64)
    lib().fo_copy_blocks(ctypes.byref(layout.c()), _p(pool), _p(p), p.shape[0])


def attention(layout: Layout, pool: np.ndarray, layer: int, q, tables, ctx_lens,
              scale: float) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    t = np.ascontiguousarray(tables, dtype=np.int32)
    c = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    out = np.zeros_like(q)
    lib().fo_attention(ctypes.byref(layout.c()), _p(pool), layer, q.shape[1], _p(q), _p(out),
                       _p(t), t.shape[1], _p(c), c.size, scale)
    return out


def prefill_attention(layout: Layout, pool: np.ndarray, layer: int, q, tables, ctx_lens, q_lens,
                      q_offsets, scale: float) -> np.ndarray:
    """q: [rows, n_heads, head_dim]; sequence s's q_lens[s] queries are rows q_offsets[s]..
    at the end of its ctx_lens[s]-token context, attending causally."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    t = np.ascontiguousarray(tables, dtype=np.int32)
    c = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    ql = np.ascontiguousarray(q_lens, dtype=np.int32)
    qo = np.ascontiguousarray(q_offsets, dtype=np.int64)
    out = np.zeros_like(q)
    lib().fo_prefill_attention(ctypes.byref(layout.c()), _p(pool), layer, q.shape[1], _p(q),
                               _p(out), _p(t), t.shape[1], _p(c), _p(ql), _p(qo), c.size, scale)
    return out


def avx2_attention(layout: Layout, pool: np.ndarray, layer: int, q, tables, ctx_lens,
                   scale: float, n_threads: int = 1) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    t = np.ascontiguousarray(tables, dtype=np.int32)
    c = np.ascontiguousarray(ctx_lens, dtype=np.int32)
    out = np.zeros_like(q)
    lib().fo_avx2_attention(ctypes.byref(layout.c()), _p(pool), layer, q.shape[1], _p(q),
                            _p(out), _p(t), t.shape[1], _p(c), c.size, scale, n_threads)
    return out


def max_threads() -> int:
    return int(lib().fo_max_threads())


# -- dense revision-1 pool (pool.rs) ---------------------------------------------

class DensePool:
    """The reference's dense pool restated (crates/kvcache/src/pool.rs). Methods
    return (code, message, value); code 0 ok, 1 cache, 2 unavailable."""

    def __init__(self, n_layers, n_kv_heads, head_dim, max_seq_len, max_slots):
        self._l = lib()
        h = c_void_p()
        m = ctypes.c_char_p()
        self.code = self._l.fo_dense_new(n_layers, n_kv_heads, head_dim, max_seq_len, max_slots,
                                         ctypes.byref(h), ctypes.byref(m))
        self.msg = m.value.decode() if m.value else ""
        self._h = h.value
        self.row = n_kv_heads * head_dim

    def __del__(self):
        if getattr(self, "_h", None):
            self._l.fo_dense_destroy(self._h)
            self._h = None

    def storage_len(self) -> int:
        return int(self._l.fo_dense_storage_len(self._h))

    def _call(self, fn, *args):
        m = ctypes.c_char_p()
        code = fn(self._h, *args, ctypes.byref(m))
        return code, (m.value.decode() if m.value else "")

    def alloc(self):
        s = u32()
        code, msg = self._call(self._l.fo_dense_alloc, ctypes.byref(s))
        return code, msg, s.value

    def free(self, slot):
        return self._call(self._l.fo_dense_free, slot) + (None,)

    def seq_len(self, slot):
        n = u64()
        code, msg = self._call(self._l.fo_dense_seq_len, slot, ctypes.byref(n))
        return code, msg, n.value

    def append_layer(self, slot, layer, k, v):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        return self._call(self._l.fo_dense_append_layer, slot, layer, _p(k), k.size, _p(v),
                          v.size) + (None,)

    def commit_token(self, slot):
        return self._call(self._l.fo_dense_commit_token, slot) + (None,)

    def k(self, slot, layer, pos):
        out = np.zeros(self.row, np.float32)
        code, msg = self._call(self._l.fo_dense_k, slot, layer, pos, _p(out))
        return code, msg, out

    def v(self, slot, layer, pos):
        out = np.zeros(self.row, np.float32)
        code, msg = self._call(self._l.fo_dense_v, slot, layer, pos, _p(out))
        return code, msg, out

    def abandon_partial(self, slot):
        return self._call(self._l.fo_dense_abandon_partial, slot) + (None,)

    def uncommit_token(self, slot):
        return self._call(self._l.fo_dense_uncommit_token, slot) + (None,)


# -- Llama::forward's KV sequence (crates/model/src/llama.rs:345-389) ----------------

# FerrumError::Model (crates/core-types/src/error.rs:38-39, Display "model: {0}"): raised
# by the model's own logic, never by a KV pool. Codes 0-6 are the pools' (FKV_* / fo_*).
MODEL = 7


def forward_kv(pool, slot, position0, tokens, fail=None):
    """The KV calls `Llama::forward` makes (llama.rs:345-381) and its rewind on error
    (`rewind_forward`, :383-389), with the model's arithmetic left out.

    tokens[t][layer] = (k, v): the rows `append_layer` receives for token t
    (post-RoPE K, llama.rs:207-218). fail = (t, layer, where) makes the model fail at
    token t: where "embed" (embed_token, :367-370), "before" (an error of layer
    `layer` before its append, e.g. a projection, :183-206) or "after" (after its
    append, e.g. attn_output, :249-255). pool follows DensePool's protocol: every
    method returns (code, message, value). Returns (code, message) of the call."""
    code, msg, seq = pool.seq_len(slot)                                   # :354
    if code:
        return code, msg
    if position0 != seq:                                                  # :355-360
        return MODEL, f"model: position0 {position0} does not match sequence length {seq}"
    for idx, layers in enumerate(tokens):                                 # :362
        if position0 + idx > 0xFFFFFFFF:                                  # :363-365, no rewind
            return MODEL, "model: position overflow"
        if fail is not None and fail[0] == idx and fail[2] == "embed":    # :367-370
            err = (MODEL, "model: injected failure")
        else:
            err = _forward_one_token_kv(pool, slot, idx, layers, fail)    # :371-376
        if err[0]:
            rw = rewind_forward(pool, slot, seq)
            return rw if rw[0] else err
    return 0, ""


def _forward_one_token_kv(pool, slot, idx, layers, fail):
    """forward_one_token's KV calls (llama.rs:150-293): abandon_partial (:166), one
    append_layer per layer in order (:218), commit_token after the last (:291)."""
    code, msg, _ = pool.abandon_partial(slot)
    if code:
        return code, msg
    for layer, (k, v) in enumerate(layers):
        if fail == (idx, layer, "before"):
            return MODEL, "model: injected failure"
        code, msg, _ = pool.append_layer(slot, layer, k, v)
        if code:
            return code, msg
        if fail == (idx, layer, "after"):
            return MODEL, "model: injected failure"
    code, msg, _ = pool.commit_token(slot)
    return code, msg


def rewind_forward(pool, slot, committed):
    """llama.rs:383-389: uncommit tokens until seq_len == committed, then drop the
    partial token's layers."""
    while True:
        code, msg, n = pool.seq_len(slot)
        if code:
            return code, msg
        if n <= committed:
            break
        code, msg, _ = pool.uncommit_token(slot)
        if code:
            return code, msg
    code, msg, _ = pool.abandon_partial(slot)
    return code, msg

"""Host-side mirror of Ferrum's KV-cache interface over libferrum_kv.so.

``PreallocatedKvPool`` keeps the revision-1 ``KvPool`` surface
(crates/core-types/src/kv.rs:21-46, crates/kvcache/src/pool.rs:20-231): same
method names, same argument meaning, same error variants and messages. K/V are
host f32 arrays at this surface, and storage is device memory.

``PagedKvPool`` is the paged surface: device-resident K/V addressed through
slot mappings and block tables, appended, gathered, copied, swapped and read by
paged decode attention with HIP kernels. Its device arguments are torch tensors
(used only for device memory and streams); every call goes through the C ABI.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import _lib
from .errors import check

__all__ = ["KvPoolConfig", "PreallocatedKvPool", "PagedConfig", "PagedKvPool",
           "default_scale"]


def default_scale(head_dim: int) -> float:
    """`1.0 / (head_dim as f32).sqrt()` in f32 (crates/model/src/llama.rs:169)."""
    return float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))


# ---------------------------------------------------------------------------
# Revision-1 compat surface
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class KvPoolConfig:
    """`KvPoolConfig` (crates/core-types/src/kv.rs:12-19)."""

    n_layers: int
    n_kv_heads: int
    head_dim: int
    max_seq_len: int
    max_slots: int


class PreallocatedKvPool:
    """`PreallocatedKvPool` over device storage (crates/kvcache/src/pool.rs)."""

    def __init__(self, handle: int, lib):
        self._h = handle
        self._lib = lib

    @classmethod
    def new(cls, config: KvPoolConfig, device: int = 0) -> "PreallocatedKvPool":
        """`PreallocatedKvPool::new` (pool.rs:21-46)."""
        lib = _lib.load()
        c = _lib.KvPoolConfigC(config.n_layers, config.n_kv_heads, config.head_dim,
                               config.max_seq_len, config.max_slots)
        h = ctypes.c_void_p()
        check(lib.fkv_kvpool_new(ctypes.byref(c), device, ctypes.byref(h)))
        return cls(h.value, lib)

    def close(self) -> None:
        if self._h:
            self._lib.fkv_kvpool_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def config(self) -> KvPoolConfig:
        c = _lib.KvPoolConfigC()
        check(self._lib.fkv_kvpool_get_config(self._h, ctypes.byref(c)))
        return KvPoolConfig(c.n_layers, c.n_kv_heads, c.head_dim, c.max_seq_len, c.max_slots)

    def storage_len(self) -> int:
        n = ctypes.c_uint64()
        check(self._lib.fkv_kvpool_storage_len(self._h, ctypes.byref(n)))
        return n.value

    def alloc(self) -> int:
        s = ctypes.c_uint32()
        check(self._lib.fkv_kvpool_alloc(self._h, ctypes.byref(s)))
        return s.value

    def free(self, slot: int) -> None:
        check(self._lib.fkv_kvpool_free(self._h, slot))

    def seq_len(self, slot: int) -> int:
        n = ctypes.c_uint64()
        check(self._lib.fkv_kvpool_seq_len(self._h, slot, ctypes.byref(n)))
        return n.value

    def append_layer(self, slot: int, layer: int, k, v) -> None:
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        check(self._lib.fkv_kvpool_append_layer(self._h, slot, layer, k.ctypes.data, k.size,
                                                v.ctypes.data, v.size))

    def commit_token(self, slot: int) -> None:
        check(self._lib.fkv_kvpool_commit_token(self._h, slot))

    def _read(self, fn, slot: int, layer: int, pos: int) -> np.ndarray:
        c = self.config()
        out = np.empty(c.n_kv_heads * c.head_dim, dtype=np.float32)
        check(fn(self._h, slot, layer, pos, out.ctypes.data, out.size))
        return out

    def k(self, slot: int, layer: int, pos: int) -> np.ndarray:
        return self._read(self._lib.fkv_kvpool_k, slot, layer, pos)

    def v(self, slot: int, layer: int, pos: int) -> np.ndarray:
        return self._read(self._lib.fkv_kvpool_v, slot, layer, pos)

    def abandon_partial(self, slot: int) -> None:
        check(self._lib.fkv_kvpool_abandon_partial(self._h, slot))

    def uncommit_token(self, slot: int) -> None:
        check(self._lib.fkv_kvpool_uncommit_token(self._h, slot))


# ---------------------------------------------------------------------------
# Paged surface
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class PagedConfig:
    n_layers: int
    n_kv_heads: int
    head_dim: int
    num_blocks: int
    block_size: int = 16
    num_host_blocks: int = 0
    kv_dtype: int = _lib.DTYPE_F16
    f16_rounding: int = _lib.ROUND_NEAREST_EVEN
    device: int = 0


def _stream_ptr(stream) -> int:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _dev(t, dtype, name):
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr()


class PagedKvPool:
    """Paged K/V block pool on one GPU (layout in include/ferrum_kv.h)."""

    def __init__(self, config: PagedConfig):
        self._lib = _lib.load()
        self.config = config
        c = _lib.PagedConfigC(config.n_layers, config.n_kv_heads, config.head_dim,
                              config.block_size, config.num_blocks, config.num_host_blocks,
                              config.kv_dtype, config.f16_rounding, config.device, 0)
        h = ctypes.c_void_p()
        check(self._lib.fkv_paged_create(ctypes.byref(c), ctypes.byref(h)))
        self._h = h.value
        info = self.info()
        self.tile_bytes = info.tile_bytes
        self.block_bytes = info.block_bytes
        self.pool_bytes = info.pool_bytes

    @property
    def handle(self) -> int:
        return self._h

    def close(self) -> None:
        if self._h:
            self._lib.fkv_paged_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> "_lib.PagedInfoC":
        i = _lib.PagedInfoC()
        check(self._lib.fkv_paged_get_info(self._h, ctypes.byref(i)))
        return i

    def free_block_count(self) -> int:
        return int(self.info().free_blocks)

    # -- block allocator ----------------------------------------------------
    def alloc_blocks(self, n: int) -> np.ndarray:
        ids = np.empty(n, dtype=np.int32)
        check(self._lib.fkv_block_alloc(self._h, n, ids.ctypes.data))
        return ids

    def free_blocks(self, ids: Sequence[int]) -> None:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        check(self._lib.fkv_block_free(self._h, a.size, a.ctypes.data))

    def ref_blocks(self, ids: Sequence[int]) -> None:
        a = np.ascontiguousarray(ids, dtype=np.int32)
        check(self._lib.fkv_block_ref(self._h, a.size, a.ctypes.data))

    def refcount(self, block: int) -> int:
        n = ctypes.c_uint32()
        check(self._lib.fkv_block_refcount(self._h, block, ctypes.byref(n)))
        return n.value

    # -- raw image ---------------------------------------------------------
    def read(self, offset: int = 0, nbytes: Optional[int] = None, stream=None) -> np.ndarray:
        """Bytes of the pool image, after the work enqueued on `stream` (default: the
        current stream)."""
        if nbytes is None:
            nbytes = self.pool_bytes - offset
        out = np.empty(nbytes, dtype=np.uint8)
        check(self._lib.fkv_paged_read(self._h, offset, nbytes, out.ctypes.data,
                                       _stream_ptr(stream)))
        return out

    def write(self, data: np.ndarray, offset: int = 0, stream=None) -> None:
        data = np.ascontiguousarray(data).view(np.uint8)
        check(self._lib.fkv_paged_write(self._h, offset, data.size, data.ctypes.data,
                                        _stream_ptr(stream)))

    def fill(self, byte: int, stream=None) -> None:
        check(self._lib.fkv_paged_fill(self._h, byte, _stream_ptr(stream)))

    def marked_blocks(self, stream=None) -> int:
        """Device blocks marked as holding a value the fast attention instances cannot
        take (a Q8_0 scale of 512 or more, an F16 Inf/NaN K or V), after the work
        enqueued on `stream`."""
        n = ctypes.c_uint64()
        check(self._lib.fkv_paged_marked_blocks(self._h, _stream_ptr(stream), ctypes.byref(n)))
        return n.value

    def take_fault_flags(self, stream=None) -> int:
        """FKV_FAULT_* bits raised by the work enqueued on `stream` (default: the current
        stream) and by work already finished elsewhere; clears them."""
        f = ctypes.c_uint32()
        check(self._lib.fkv_paged_take_fault_flags(self._h, _stream_ptr(stream), ctypes.byref(f)))
        return f.value

    # -- device operations --------------------------------------------------
    def append(self, layer: int, k, v, slot_mapping, stream=None) -> None:
        import torch
        n = slot_mapping.numel()
        row = self.config.n_kv_heads * self.config.head_dim
        if k.numel() != n * row or v.numel() != n * row:
            raise ValueError("k/v must be [n_tokens, n_kv_heads, head_dim]")
        check(self._lib.fkv_append(self._h, layer, _dev(k, torch.float32, "k"),
                                   _dev(v, torch.float32, "v"),
                                   _dev(slot_mapping, torch.int64, "slot_mapping"), n,
                                   _stream_ptr(stream)))

    def gather_slots(self, layer: int, slot_mapping, out_k, out_v,
                     fmt: int = _lib.GATHER_F32, stream=None) -> None:
        import torch
        check(self._lib.fkv_gather_slots(self._h, layer,
                                         _dev(slot_mapping, torch.int64, "slot_mapping"),
                                         slot_mapping.numel(), fmt,
                                         out_k.data_ptr(), out_v.data_ptr(), _stream_ptr(stream)))

    def gather_tables(self, layer: int, block_tables, ctx_lens, out_offsets, max_ctx_len: int,
                      out_k, out_v, fmt: int = _lib.GATHER_F32, stream=None) -> None:
        import torch
        n_seqs, max_blocks = block_tables.shape
        check(self._lib.fkv_gather_tables(self._h, layer,
                                          _dev(block_tables, torch.int32, "block_tables"),
                                          max_blocks, _dev(ctx_lens, torch.int32, "ctx_lens"),
                                          _dev(out_offsets, torch.int64, "out_offsets"), n_seqs,
                                          max_ctx_len, fmt, out_k.data_ptr(), out_v.data_ptr(),
                                          _stream_ptr(stream)))

    def copy_blocks(self, pairs, stream=None) -> None:
        import torch
        check(self._lib.fkv_copy_blocks(self._h, _dev(pairs, torch.int64, "pairs"),
                                        pairs.shape[0], _stream_ptr(stream)))

    def swap_out(self, pairs: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(pairs, dtype=np.int64)
        check(self._lib.fkv_swap_out(self._h, a.ctypes.data, a.shape[0], _stream_ptr(stream)))

    def swap_in(self, pairs: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(pairs, dtype=np.int64)
        check(self._lib.fkv_swap_in(self._h, a.ctypes.data, a.shape[0], _stream_ptr(stream)))

    def attention_workspace_bytes(self, n_heads: int, n_seqs: int, max_ctx_len: int) -> int:
        n = ctypes.c_uint64()
        check(self._lib.fkv_decode_attention_workspace_size(self._h, n_heads, n_seqs,
                                                            max_ctx_len, ctypes.byref(n)))
        return n.value

    def rope_attention_workspace_bytes(self, n_heads: int, n_seqs: int, max_ctx_len: int) -> int:
        """Bytes of the workspace of a rope_append_decode_attention call."""
        n = ctypes.c_uint64()
        check(self._lib.fkv_rope_append_decode_attention_workspace_size(
            self._h, n_heads, n_seqs, max_ctx_len, ctypes.byref(n)))
        return n.value

    def decode_attention(self, layer: int, q, out, block_tables, ctx_lens, max_ctx_len: int,
                         scale: Optional[float] = None, workspace=None, stream=None) -> None:
        """q, out: float32 [n_seqs, n_heads, head_dim]; block_tables int32 [n_seqs, max_blocks];
        ctx_lens int32 [n_seqs]."""
        import torch
        n_seqs, n_heads, d = q.shape
        if d != self.config.head_dim or tuple(out.shape) != tuple(q.shape):
            raise ValueError("q/out must be [n_seqs, n_heads, head_dim]")
        if block_tables.shape[0] != n_seqs or ctx_lens.numel() != n_seqs:
            raise ValueError("block_tables/ctx_lens must have one row per sequence")
        if scale is None:
            scale = default_scale(d)
        need = self.attention_workspace_bytes(n_heads, n_seqs, max_ctx_len)
        ws_ptr, ws_bytes = 0, 0
        if need:
            if workspace is None:
                workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.fkv_decode_attention(
            self._h, layer, n_heads, _dev(q, torch.float32, "q"), _dev(out, torch.float32, "out"),
            _dev(block_tables, torch.int32, "block_tables"), block_tables.shape[1],
            _dev(ctx_lens, torch.int32, "ctx_lens"), n_seqs, max_ctx_len, scale, ws_ptr,
            ws_bytes, _stream_ptr(stream)))


    def append_decode_attention(self, layer: int, k_new, v_new, q, out, block_tables, ctx_lens,
                                max_ctx_len: int, scale: Optional[float] = None, workspace=None,
                                stream=None) -> None:
        """One decode step of one layer (llama.rs:218-247): store k_new/v_new (float32
        [n_seqs, n_kv_heads, head_dim]) at position ctx_lens[s] - 1 through the block
        tables, then decode attention over ctx_lens[s] positions."""
        import torch
        n_seqs, n_heads, d = q.shape
        if d != self.config.head_dim or tuple(out.shape) != tuple(q.shape):
            raise ValueError("q/out must be [n_seqs, n_heads, head_dim]")
        kv_shape = (n_seqs, self.config.n_kv_heads, d)
        if tuple(k_new.shape) != kv_shape or tuple(v_new.shape) != kv_shape:
            raise ValueError("k_new/v_new must be [n_seqs, n_kv_heads, head_dim]")
        if block_tables.shape[0] != n_seqs or ctx_lens.numel() != n_seqs:
            raise ValueError("block_tables/ctx_lens must have one row per sequence")
        if scale is None:
            scale = default_scale(d)
        n = ctypes.c_uint64()
        check(self._lib.fkv_append_decode_attention_workspace_size(
            self._h, n_heads, n_seqs, max_ctx_len, ctypes.byref(n)))
        need = n.value
        ws_ptr, ws_bytes = 0, 0
        if need:
            if workspace is None:
                workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.fkv_append_decode_attention(
            self._h, layer, n_heads, _dev(k_new, torch.float32, "k_new"),
            _dev(v_new, torch.float32, "v_new"), _dev(q, torch.float32, "q"),
            _dev(out, torch.float32, "out"), _dev(block_tables, torch.int32, "block_tables"),
            block_tables.shape[1], _dev(ctx_lens, torch.int32, "ctx_lens"), n_seqs, max_ctx_len,
            scale, ws_ptr, ws_bytes, _stream_ptr(stream)))

    def append_decode_attention_noalloc(self, layer: int, k_new, v_new, q, out, block_tables,
                                        ctx_lens, max_ctx_len: int,
                                        scale: Optional[float] = None, stream=None) -> None:
        """append_decode_attention with no workspace and no allocation: the split
        partials go to the library's static per-GPU scratch (STATIC_SCRATCH_BYTES).
        Calls that overlap on one GPU race on it; a step needing more is InvalidRequest."""
        import torch
        n_seqs, n_heads, d = q.shape
        if d != self.config.head_dim or tuple(out.shape) != tuple(q.shape):
            raise ValueError("q/out must be [n_seqs, n_heads, head_dim]")
        kv_shape = (n_seqs, self.config.n_kv_heads, d)
        if tuple(k_new.shape) != kv_shape or tuple(v_new.shape) != kv_shape:
            raise ValueError("k_new/v_new must be [n_seqs, n_kv_heads, head_dim]")
        if block_tables.shape[0] != n_seqs or ctx_lens.numel() != n_seqs:
            raise ValueError("block_tables/ctx_lens must have one row per sequence")
        if scale is None:
            scale = default_scale(d)
        check(self._lib.fkv_append_decode_attention_noalloc(
            self._h, layer, n_heads, _dev(k_new, torch.float32, "k_new"),
            _dev(v_new, torch.float32, "v_new"), _dev(q, torch.float32, "q"),
            _dev(out, torch.float32, "out"), _dev(block_tables, torch.int32, "block_tables"),
            block_tables.shape[1], _dev(ctx_lens, torch.int32, "ctx_lens"), n_seqs, max_ctx_len,
            scale, _stream_ptr(stream)))

    def rope_append_decode_attention(self, layer: int, k_new, v_new, q, out, block_tables,
                                     ctx_lens, max_ctx_len: int, rope_dim: int, theta: float,
                                     scale: Optional[float] = None, workspace=None,
                                     stream=None) -> None:
        """append_decode_attention with q and k_new before RoPE (llama.rs:207-247):
        each sequence's q and k_new are rotated at position ctx_lens[s] - 1 (dims
        (2i, 2i+1) below rope_dim, angle pos / theta^(2i/rope_dim); scalar.rs:167-189)
        before the append and the attention. q is not written back."""
        import torch
        n_seqs, n_heads, d = q.shape
        if d != self.config.head_dim or tuple(out.shape) != tuple(q.shape):
            raise ValueError("q/out must be [n_seqs, n_heads, head_dim]")
        kv_shape = (n_seqs, self.config.n_kv_heads, d)
        if tuple(k_new.shape) != kv_shape or tuple(v_new.shape) != kv_shape:
            raise ValueError("k_new/v_new must be [n_seqs, n_kv_heads, head_dim]")
        if block_tables.shape[0] != n_seqs or ctx_lens.numel() != n_seqs:
            raise ValueError("block_tables/ctx_lens must have one row per sequence")
        if scale is None:
            scale = default_scale(d)
        n = ctypes.c_uint64()
        check(self._lib.fkv_rope_append_decode_attention_workspace_size(
            self._h, n_heads, n_seqs, max_ctx_len, ctypes.byref(n)))
        need = n.value
        ws_ptr, ws_bytes = 0, 0
        if need:
            if workspace is None:
                workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
            ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.fkv_rope_append_decode_attention(
            self._h, layer, n_heads, rope_dim, theta, _dev(k_new, torch.float32, "k_new"),
            _dev(v_new, torch.float32, "v_new"), _dev(q, torch.float32, "q"),
            _dev(out, torch.float32, "out"), _dev(block_tables, torch.int32, "block_tables"),
            block_tables.shape[1], _dev(ctx_lens, torch.int32, "ctx_lens"), n_seqs, max_ctx_len,
            scale, ws_ptr, ws_bytes, _stream_ptr(stream)))

    def prefill_workspace_bytes(self, n_heads: int, n_seqs: int, max_q_len: int,
                                max_ctx_len: int) -> int:
        """Bytes of the partials workspace of a prefill call (0: no workgroup splits)."""
        n = ctypes.c_uint64(0)
        check(self._lib.fkv_prefill_attention_workspace_size(self._h, n_heads, n_seqs, max_q_len,
                                                             max_ctx_len, ctypes.byref(n)))
        return n.value

    def prefill_attention(self, layer: int, q, out, block_tables, ctx_lens, q_lens, q_offsets,
                          max_q_len: int, max_ctx_len: int, scale: Optional[float] = None,
                          workspace=None, split: bool = True, stream=None) -> None:
        """Chunked prefill (F16 or Q8_0 KV): q, out float32 [rows, n_heads, head_dim];
        sequence s's q_lens[s] queries are rows q_offsets[s].. and sit at the end of its
        ctx_lens[s] context, each attending causally (crates/model/src/llama.rs:363-378).
        workspace: device scratch for the key-range pieces (allocated here when None);
        split=False passes none, so every workgroup reads its whole key range."""
        import torch
        rows, n_heads, d = q.shape
        if d != self.config.head_dim or tuple(out.shape) != tuple(q.shape):
            raise ValueError("q/out must be [rows, n_heads, head_dim]")
        n_seqs = block_tables.shape[0]
        if ctx_lens.numel() != n_seqs or q_lens.numel() != n_seqs or q_offsets.numel() != n_seqs:
            raise ValueError("ctx_lens/q_lens/q_offsets must have one entry per sequence")
        if scale is None:
            scale = default_scale(d)
        ws_ptr, ws_bytes = 0, 0
        if split:
            need = self.prefill_workspace_bytes(n_heads, n_seqs, max_q_len, max_ctx_len)
            if need:
                if workspace is None:
                    workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
                ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
        check(self._lib.fkv_prefill_attention(
            self._h, layer, n_heads, _dev(q, torch.float32, "q"), _dev(out, torch.float32, "out"),
            _dev(block_tables, torch.int32, "block_tables"), block_tables.shape[1],
            _dev(ctx_lens, torch.int32, "ctx_lens"), _dev(q_lens, torch.int32, "q_lens"),
            _dev(q_offsets, torch.int64, "q_offsets"), n_seqs, max_q_len, max_ctx_len, scale,
            ws_ptr, ws_bytes, _stream_ptr(stream)))


class SequenceManager:
    """Per-sequence block lists over one PagedKvPool (fkv_seqs_*): the scheduler's KV
    bookkeeping on paged storage (crates/scheduler/src/batcher.rs: admission :108-129,
    rollback :291-308, finish :329-338), with copy-on-write forks and swap preemption."""

    def __init__(self, pool: PagedKvPool):
        self._lib = pool._lib
        self.pool = pool
        h = ctypes.c_void_p()
        check(self._lib.fkv_seqs_create(pool.handle, ctypes.byref(h)))
        self._h = h.value

    def close(self) -> None:
        if self._h:
            self._lib.fkv_seqs_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def add(self, n_tokens: int) -> int:
        """Admission: a new sequence with blocks for n_tokens (Unavailable if none)."""
        sid = ctypes.c_uint32()
        check(self._lib.fkv_seqs_add(self._h, n_tokens, ctypes.byref(sid)))
        return sid.value

    def reserve(self, seq: int, n: int):
        """Blocks for n more tokens; returns the copy-on-write (src, dst) pair or None."""
        pair = np.full(2, -1, dtype=np.int64)
        check(self._lib.fkv_seqs_reserve(self._h, seq, n, pair.ctypes.data))
        return None if pair[0] < 0 else (int(pair[0]), int(pair[1]))

    def slots(self, seq: int, pos: int, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.int64)
        check(self._lib.fkv_seqs_slots(self._h, seq, pos, n, out.ctypes.data))
        return out

    def commit(self, seq: int, n: int) -> None:
        check(self._lib.fkv_seqs_commit(self._h, seq, n))

    def truncate(self, seq: int, n_tokens: int) -> None:
        check(self._lib.fkv_seqs_truncate(self._h, seq, n_tokens))

    def fork(self, parent: int) -> int:
        sid = ctypes.c_uint32()
        check(self._lib.fkv_seqs_fork(self._h, parent, ctypes.byref(sid)))
        return sid.value

    def free(self, seq: int) -> None:
        check(self._lib.fkv_seqs_free(self._h, seq))

    def length(self, seq: int):
        """(committed length, swapped out)."""
        n, sw = ctypes.c_uint64(), ctypes.c_int32()
        check(self._lib.fkv_seqs_len(self._h, seq, ctypes.byref(n), ctypes.byref(sw)))
        return n.value, bool(sw.value)

    def swap_out(self, seq: int, stream=None) -> None:
        check(self._lib.fkv_seqs_swap_out(self._h, seq, _stream_ptr(stream)))

    def swap_in(self, seq: int, stream=None) -> None:
        check(self._lib.fkv_seqs_swap_in(self._h, seq, _stream_ptr(stream)))

    def tables(self, seqs: Sequence[int], max_blocks: int):
        """Host block-table rows [n, max_blocks] (padded with block 0) and lengths [n]."""
        ids = np.ascontiguousarray(seqs, dtype=np.uint32)
        tab = np.empty((ids.size, max_blocks), dtype=np.int32)
        ctx = np.empty(ids.size, dtype=np.int32)
        check(self._lib.fkv_seqs_tables(self._h, ids.ctypes.data, ids.size, max_blocks,
                                        tab.ctypes.data, ctx.ctypes.data))
        return tab, ctx


def device_copy(dst, src, nbytes: int, stream=None) -> None:
    """16-byte vector device copy (the HBM calibration kernel)."""
    lib = _lib.load()
    check(lib.fkv_device_copy(dst.data_ptr(), src.data_ptr(), nbytes, _stream_ptr(stream)))

"""ctypes bindings of libferrum_kv.so (the C ABI declared in include/ferrum_kv.h).

The shared library is built in-tree by ``__graft_entry__.build()`` (``make`` in
``ferrum_amd/csrc``). Loading fails loudly when it is missing: there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libferrum_kv.so")

# FKV_ABI_VERSION of include/ferrum_kv.h that these signatures follow; a library built
# from another header revision is refused at load (C symbols carry no signature).
ABI_VERSION = 2

FKV_OK = 0
FKV_ERR_CACHE = 1
FKV_ERR_UNAVAILABLE = 2
FKV_ERR_KERNEL = 3
FKV_ERR_INVALID = 4
FKV_ERR_INTERNAL = 5
FKV_ERR_GGUF = 6

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_Q8_0 = 8

ROUND_NEAREST_EVEN = 0
ROUND_HALF_AWAY = 1

GATHER_F32 = 0
GATHER_RAW = 1

TUNE_ATTN_SPLIT_TOKENS = 0
TUNE_ATTN_STREAM = 1
TUNE_ATTN_ORDER = 2
TUNE_PREFILL_SPLIT_BLOCKS = 3
TUNE_ATTN_ENGINE = 4
TUNE_ATTN_WGS_PER_CU = 5

FAULT_SLOT_RANGE = 1
FAULT_BLOCK_RANGE = 2
FAULT_CTX_RANGE = 4
FAULT_VALUE_RANGE = 8

# FKV_STATIC_SCRATCH_BYTES: the per-GPU static scratch of fkv_append_decode_attention_noalloc.
STATIC_SCRATCH_BYTES = 32 << 20

c_void_p = ctypes.c_void_p
u32, u64, i32, i64 = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int32, ctypes.c_int64
f32 = ctypes.c_float
P = ctypes.POINTER


class KvPoolConfigC(ctypes.Structure):
    _fields_ = [("n_layers", u64), ("n_kv_heads", u64), ("head_dim", u64),
                ("max_seq_len", u64), ("max_slots", u64)]


class PagedConfigC(ctypes.Structure):
    _fields_ = [("n_layers", u32), ("n_kv_heads", u32), ("head_dim", u32),
                ("block_size", u32), ("num_blocks", u64), ("num_host_blocks", u64),
                ("kv_dtype", i32), ("f16_rounding", i32), ("device", i32),
                ("reserved", i32)]


class PagedInfoC(ctypes.Structure):
    _fields_ = [("tile_bytes", u64), ("block_bytes", u64), ("pool_bytes", u64),
                ("free_blocks", u64), ("device_base", c_void_p), ("host_base", c_void_p)]


class GgufTensorInfoC(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("name_len", u64), ("n_dims", u32),
                ("ggml_type", u32), ("shape", u64 * 4), ("data_offset", u64), ("nbytes", u64)]


class GgufValueC(ctypes.Structure):
    _fields_ = [("type", u32), ("elem_type", u32), ("count", u64), ("u", u64), ("i", i64),
                ("f", ctypes.c_double), ("str", ctypes.c_void_p), ("str_len", u64)]


# name -> (restype, argtypes). Must list every function include/*.h declares.
SIGNATURES = {
    "fkv_abi_version": (i32, []),
    "fkv_last_error": (ctypes.c_char_p, []),
    "fkv_device_count": (i32, []),
    "fkv_kvpool_new": (i32, [P(KvPoolConfigC), i32, P(c_void_p)]),
    "fkv_kvpool_destroy": (i32, [c_void_p]),
    "fkv_kvpool_get_config": (i32, [c_void_p, P(KvPoolConfigC)]),
    "fkv_kvpool_storage_len": (i32, [c_void_p, P(u64)]),
    "fkv_kvpool_alloc": (i32, [c_void_p, P(u32)]),
    "fkv_kvpool_free": (i32, [c_void_p, u32]),
    "fkv_kvpool_seq_len": (i32, [c_void_p, u32, P(u64)]),
    "fkv_kvpool_append_layer": (i32, [c_void_p, u32, u64, c_void_p, u64, c_void_p, u64]),
    "fkv_kvpool_commit_token": (i32, [c_void_p, u32]),
    "fkv_kvpool_k": (i32, [c_void_p, u32, u64, u64, c_void_p, u64]),
    "fkv_kvpool_v": (i32, [c_void_p, u32, u64, u64, c_void_p, u64]),
    "fkv_kvpool_abandon_partial": (i32, [c_void_p, u32]),
    "fkv_kvpool_uncommit_token": (i32, [c_void_p, u32]),
    "fkv_paged_create": (i32, [P(PagedConfigC), P(c_void_p)]),
    "fkv_paged_destroy": (i32, [c_void_p]),
    "fkv_paged_get_info": (i32, [c_void_p, P(PagedInfoC)]),
    "fkv_paged_take_fault_flags": (i32, [c_void_p, c_void_p, P(u32)]),
    "fkv_paged_marked_blocks": (i32, [c_void_p, c_void_p, P(u64)]),
    "fkv_set_tuning": (i32, [i32, i64]),
    "fkv_paged_fill": (i32, [c_void_p, ctypes.c_uint8, c_void_p]),
    "fkv_paged_read": (i32, [c_void_p, u64, u64, c_void_p, c_void_p]),
    "fkv_paged_write": (i32, [c_void_p, u64, u64, c_void_p, c_void_p]),
    "fkv_block_alloc": (i32, [c_void_p, u32, c_void_p]),
    "fkv_block_free": (i32, [c_void_p, u32, c_void_p]),
    "fkv_block_ref": (i32, [c_void_p, u32, c_void_p]),
    "fkv_block_refcount": (i32, [c_void_p, i32, P(u32)]),
    "fkv_append": (i32, [c_void_p, u32, c_void_p, c_void_p, c_void_p, u32, c_void_p]),
    "fkv_gather_slots": (i32, [c_void_p, u32, c_void_p, u32, i32, c_void_p, c_void_p, c_void_p]),
    "fkv_gather_tables": (i32, [c_void_p, u32, c_void_p, u32, c_void_p, c_void_p, u32, u32, i32,
                                c_void_p, c_void_p, c_void_p]),
    "fkv_copy_blocks": (i32, [c_void_p, c_void_p, u32, c_void_p]),
    "fkv_swap_out": (i32, [c_void_p, c_void_p, u32, c_void_p]),
    "fkv_swap_in": (i32, [c_void_p, c_void_p, u32, c_void_p]),
    "fkv_decode_attention_workspace_size": (i32, [c_void_p, u32, u32, u32, P(u64)]),
    "fkv_decode_attention": (i32, [c_void_p, u32, u32, c_void_p, c_void_p, c_void_p, u32,
                                   c_void_p, u32, u32, f32, c_void_p, u64, c_void_p]),
    "fkv_append_decode_attention_workspace_size": (i32, [c_void_p, u32, u32, u32, P(u64)]),
    "fkv_append_decode_attention": (i32, [c_void_p, u32, u32, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_void_p, u32, c_void_p, u32, u32, f32,
                                          c_void_p, u64, c_void_p]),
    "fkv_append_decode_attention_noalloc": (i32, [c_void_p, u32, u32, c_void_p, c_void_p,
                                                  c_void_p, c_void_p, c_void_p, u32, c_void_p,
                                                  u32, u32, f32, c_void_p]),
    "fkv_rope_append_decode_attention_workspace_size": (i32, [c_void_p, u32, u32, u32, P(u64)]),
    "fkv_rope_append_decode_attention": (i32, [c_void_p, u32, u32, u32, f32, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_void_p, u32, c_void_p, u32,
                                               u32, f32, c_void_p, u64, c_void_p]),
    "fkv_prefill_attention_workspace_size": (i32, [c_void_p, u32, u32, u32, u32, P(u64)]),
    "fkv_prefill_attention": (i32, [c_void_p, u32, u32, c_void_p, c_void_p, c_void_p, u32,
                                    c_void_p, c_void_p, c_void_p, u32, u32, u32, f32, c_void_p,
                                    u64, c_void_p]),
    "fkv_device_copy": (i32, [c_void_p, c_void_p, u64, c_void_p]),
    "fkv_seqs_create": (i32, [c_void_p, P(c_void_p)]),
    "fkv_seqs_destroy": (i32, [c_void_p]),
    "fkv_seqs_add": (i32, [c_void_p, u64, P(u32)]),
    "fkv_seqs_reserve": (i32, [c_void_p, u32, u64, c_void_p]),
    "fkv_seqs_slots": (i32, [c_void_p, u32, u64, u64, c_void_p]),
    "fkv_seqs_commit": (i32, [c_void_p, u32, u64]),
    "fkv_seqs_truncate": (i32, [c_void_p, u32, u64]),
    "fkv_seqs_fork": (i32, [c_void_p, u32, P(u32)]),
    "fkv_seqs_free": (i32, [c_void_p, u32]),
    "fkv_seqs_len": (i32, [c_void_p, u32, P(u64), P(i32)]),
    "fkv_seqs_swap_out": (i32, [c_void_p, u32, c_void_p]),
    "fkv_seqs_swap_in": (i32, [c_void_p, u32, c_void_p]),
    "fkv_seqs_tables": (i32, [c_void_p, c_void_p, u32, u32, c_void_p, c_void_p]),
    "fkv_gemv_q8_0": (i32, [c_void_p, u64, u64, u64, c_void_p, u64, c_void_p, u64, c_void_p]),
    "fkv_gemm_q8_0": (i32, [c_void_p, u64, u64, u64, c_void_p, u64, u64, c_void_p, u64,
                            c_void_p]),
    "fkv_gemm_q8_0_multi": (i32, [u32, c_void_p, c_void_p, c_void_p, u64, c_void_p, u64, u64,
                                  c_void_p, c_void_p, c_void_p]),
    "fkv_gemm_q8_0_batched_workspace_size": (i32, [u64, u64, P(u64)]),
    "fkv_gemm_q8_0_batched": (i32, [u32, c_void_p, c_void_p, c_void_p, u64, c_void_p, u64, u64,
                                    c_void_p, c_void_p, c_void_p, u64, c_void_p]),
    "fkv_gguf_open": (i32, [ctypes.c_char_p, P(c_void_p)]),
    "fkv_gguf_close": (i32, [c_void_p]),
    "fkv_gguf_info": (i32, [c_void_p, P(u32), P(u64), P(u64), P(u64), P(u64), P(u64)]),
    "fkv_gguf_tensor": (i32, [c_void_p, u64, P(GgufTensorInfoC)]),
    "fkv_gguf_find": (i32, [c_void_p, ctypes.c_char_p, u64, P(u64)]),
    "fkv_gguf_meta": (i32, [c_void_p, ctypes.c_char_p, u64, P(GgufValueC)]),
    "fkv_gguf_meta_array_elem": (i32, [c_void_p, ctypes.c_char_p, u64, u64, P(GgufValueC)]),
    "fkv_gguf_dump": (i32, [c_void_p, ctypes.c_char_p, u64, P(u64)]),
    "fkv_gguf_upload": (i32, [c_void_p, c_void_p, u64, u64, u32]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libferrum_kv.so and bind every signature; raises if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(there is no CPU fallback for the KV-cache path)")
        # PyTorch-ROCm ships its own libamdhip64.so.7 and its libc10_hip asks for it
        # by the unversioned name. Importing torch first makes that runtime the one
        # our NEEDED libamdhip64.so.7 binds to, so the process has a single HIP
        # runtime (and torch's device pointers and streams are valid for our kernels).
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        got = lib.fkv_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {got}, these bindings need "
                               f"{ABI_VERSION}: rebuild it with __graft_entry__.build()")
        _lib = lib
        return lib

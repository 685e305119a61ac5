"""ferrum_amd — MI355X (gfx950) paged KV-cache hot path of the Ferrum engine.

The product is ``libferrum_kv.so`` (HIP kernels + C ABI, include/ferrum_kv.h and
include/ferrum_q8.h); this package binds it and mirrors Ferrum's KvPool interface
and the Q8_0 Kernels::gemv/gemm on the host.
"""
from . import _lib
from ._lib import (DTYPE_F16, DTYPE_F32, DTYPE_Q8_0, FAULT_BLOCK_RANGE, FAULT_CTX_RANGE,
                   FAULT_SLOT_RANGE, FAULT_VALUE_RANGE, GATHER_F32, GATHER_RAW, ROUND_HALF_AWAY,
                   ROUND_NEAREST_EVEN, STATIC_SCRATCH_BYTES, TUNE_ATTN_ENGINE, TUNE_ATTN_ORDER,
                   TUNE_ATTN_SPLIT_TOKENS, TUNE_ATTN_STREAM, TUNE_ATTN_WGS_PER_CU,
                   TUNE_PREFILL_SPLIT_BLOCKS)
from .errors import (CacheError, FerrumError, GgufError, InternalError, InvalidRequest,
                     KernelError, Unavailable)
from .gguf import GgufFile
from .kvcache import (KvPoolConfig, PagedConfig, PagedKvPool, PreallocatedKvPool,
                      SequenceManager, default_scale, device_copy)
from .layer import DecodeAttentionLayer
from .q8 import (gemm_q8_0, gemm_q8_0_batched, gemm_q8_0_batched_workspace_bytes, gemm_q8_0_multi,
                 gemv_q8_0, q8_0_row_bytes)

__all__ = [
    "DTYPE_F16", "DTYPE_F32", "DTYPE_Q8_0", "FAULT_BLOCK_RANGE", "FAULT_CTX_RANGE",
    "FAULT_SLOT_RANGE", "FAULT_VALUE_RANGE", "GATHER_F32", "GATHER_RAW", "ROUND_HALF_AWAY",
    "ROUND_NEAREST_EVEN", "STATIC_SCRATCH_BYTES", "CacheError", "DecodeAttentionLayer", "FerrumError", "GgufError", "GgufFile", "InternalError",
    "InvalidRequest",
    "KernelError", "Unavailable", "KvPoolConfig", "PagedConfig", "PagedKvPool",
    "PreallocatedKvPool", "SequenceManager", "default_scale", "device_copy", "gemm_q8_0", "gemm_q8_0_batched",
    "gemm_q8_0_batched_workspace_bytes", "gemm_q8_0_multi",
    "gemv_q8_0", "load_library", "q8_0_row_bytes", "set_tuning", "TUNE_ATTN_ENGINE", "TUNE_ATTN_ORDER",
    "TUNE_ATTN_SPLIT_TOKENS", "TUNE_ATTN_STREAM", "TUNE_ATTN_WGS_PER_CU",
    "TUNE_PREFILL_SPLIT_BLOCKS",
]


def load_library():
    """Load libferrum_kv.so (raises if it has not been built)."""
    return _lib.load()


def set_tuning(knob: int, value: int) -> None:
    """fkv_set_tuning: a process-wide override of the launch planners (TUNE_* knobs), for
    measurements and tests; -1 (0 for the split length and stream mode) restores the
    planner's own rule."""
    from .errors import check
    check(_lib.load().fkv_set_tuning(knob, value))

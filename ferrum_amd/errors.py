"""FerrumError mirror for the C ABI's status codes.

The variants and their Display strings follow crates/core-types/src/error.rs:21-46:
Cache -> "cache: {msg}", Kernel -> "kernel: {msg}", Unavailable -> "{msg}" (HTTP 503,
error.rs:30-31,101), InvalidRequest -> "{msg}" (400), Internal -> "{msg}" (500).
The C library already formats the message; ``str(err)`` is that Display string.
"""
from __future__ import annotations

from . import _lib


class FerrumError(Exception):
    """Base of every error the KV-cache path returns."""

    http_status = 500

    def __init__(self, display: str):
        super().__init__(display)
        self.display = display

    def __str__(self) -> str:
        return self.display


class CacheError(FerrumError):
    """FerrumError::Cache."""


class Unavailable(FerrumError):
    """FerrumError::Unavailable; the scheduler stops admission on it."""

    http_status = 503


class KernelError(FerrumError):
    """FerrumError::Kernel."""


class InvalidRequest(FerrumError):
    """FerrumError::InvalidRequest (bad pointer, size or format at the boundary)."""

    http_status = 400


class InternalError(FerrumError):
    """FerrumError::Internal (a HIP runtime failure)."""


class GgufError(FerrumError):
    """FerrumError::Gguf ("gguf: {msg}", HTTP 500)."""


_BY_CODE = {
    _lib.FKV_ERR_CACHE: CacheError,
    _lib.FKV_ERR_UNAVAILABLE: Unavailable,
    _lib.FKV_ERR_KERNEL: KernelError,
    _lib.FKV_ERR_INVALID: InvalidRequest,
    _lib.FKV_ERR_INTERNAL: InternalError,
    _lib.FKV_ERR_GGUF: GgufError,
}


def check(code: int) -> None:
    """Raise the FerrumError subclass for a non-zero fkv status."""
    if code == _lib.FKV_OK:
        return
    msg = _lib.load().fkv_last_error()
    text = msg.decode() if msg else ""
    raise _BY_CODE.get(code, InternalError)(text)

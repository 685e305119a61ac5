"""Q8_0 weight GEMV/GEMM on the GPU: Kernels::gemv / Kernels::gemm for DType::Q8_0.

Mirrors the reference's trait methods (crates/kernels/src/scalar.rs:84-116) with the
same argument meaning (``rows``, ``cols``, weight bytes, ``x``, ``y``, and
``n_tokens`` for gemm) and the same error variants and messages
(crates/kernels/src/validate.rs:110-150); the result is the reference's
ggml q8_0 . q8_0 product bit for bit (include/ferrum_q8.h). Every call goes through
libferrum_kv.so's C ABI; there is no CPU fallback.

Device arguments are torch tensors (device memory and streams only): ``w`` a uint8
tensor holding the GGUF Q8_0 bytes (rows x cols/32 blocks of 34 bytes), ``x`` and
``y`` float32. Lengths passed to the library are element counts, as the
reference's slice lengths, so a wrongly sized tensor gets the reference's
"kernel: length mismatch".
"""
from __future__ import annotations

import ctypes

from . import _lib
from .errors import check
from .kvcache import _stream_ptr

__all__ = ["Q8_0_BLOCK", "Q8_0_BLOCK_BYTES", "gemv_q8_0", "gemm_q8_0", "gemm_q8_0_multi",
           "gemm_q8_0_batched", "gemm_q8_0_batched_workspace_bytes", "q8_0_row_bytes"]

Q8_0_BLOCK = 32        # crates/core-types/src/dtype.rs:19-21
Q8_0_BLOCK_BYTES = 34


def q8_0_row_bytes(cols: int) -> int:
    """Bytes of one Q8_0 weight row (pack.rs:37-44)."""
    return cols // Q8_0_BLOCK * Q8_0_BLOCK_BYTES


def _dev_any(t, dtype, name):
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t.data_ptr(), t.numel()


def gemv_q8_0(w, rows: int, cols: int, x, y, stream=None) -> None:
    """Kernels::gemv(DType::Q8_0, w, rows, cols, x, y): y[r] for one activation row."""
    import torch
    wp, wn = _dev_any(w, torch.uint8, "w")
    xp, xn = _dev_any(x, torch.float32, "x")
    yp, yn = _dev_any(y, torch.float32, "y")
    check(_lib.load().fkv_gemv_q8_0(wp, wn, rows, cols, xp, xn, yp, yn, _stream_ptr(stream)))


def gemm_q8_0(w, rows: int, cols: int, x, n_tokens: int, y, stream=None) -> None:
    """Kernels::gemm(GemmArgs { dtype: Q8_0, w, rows, cols, x, n_tokens, y }):
    y[t * rows + r], each token as gemv_q8_0 of x[t]."""
    import torch
    wp, wn = _dev_any(w, torch.uint8, "w")
    xp, xn = _dev_any(x, torch.float32, "x")
    yp, yn = _dev_any(y, torch.float32, "y")
    check(_lib.load().fkv_gemm_q8_0(wp, wn, rows, cols, xp, xn, n_tokens, yp, yn,
                                    _stream_ptr(stream)))


def gemm_q8_0_multi(ws, rows, cols: int, x, n_tokens: int, ys, stream=None) -> None:
    """gemm_q8_0 of up to 4 matrices that take the same x (q/k/v, gate/up) in one launch;
    ys[m] equals gemm_q8_0(ws[m], rows[m], cols, x, n_tokens, ys[m]) bit for bit."""
    import torch
    n = len(ws)
    if len(rows) != n or len(ys) != n:
        raise ValueError("ws, rows and ys must have one entry per matrix")
    wp = [_dev_any(w, torch.uint8, "w") for w in ws]
    yp = [_dev_any(y, torch.float32, "y") for y in ys]
    xp, xn = _dev_any(x, torch.float32, "x")
    arr_p = ctypes.c_void_p * max(n, 1)
    arr_u = ctypes.c_uint64 * max(n, 1)
    check(_lib.load().fkv_gemm_q8_0_multi(
        n, arr_p(*[p for p, _ in wp]), arr_u(*[k for _, k in wp]), arr_u(*rows), cols, xp, xn,
        n_tokens, arr_p(*[p for p, _ in yp]), arr_u(*[k for _, k in yp]), _stream_ptr(stream)))


def gemm_q8_0_batched_workspace_bytes(cols: int, n_tokens: int) -> int:
    """Workspace bytes of gemm_q8_0_batched (0 where the call runs the GEMV)."""
    n = ctypes.c_uint64()
    check(_lib.load().fkv_gemm_q8_0_batched_workspace_size(cols, n_tokens, ctypes.byref(n)))
    return n.value


def gemm_q8_0_batched(ws, rows, cols: int, x, n_tokens: int, ys, workspace=None,
                      stream=None) -> None:
    """gemm_q8_0_multi on the matrix cores for batches (n_tokens >= 8, cols a multiple of
    1024, 16-byte aligned weights; otherwise the GEMV), bit-identical. `workspace`: a
    device uint8 tensor of gemm_q8_0_batched_workspace_bytes (allocated here when None)."""
    import torch
    n = len(ws)
    if len(rows) != n or len(ys) != n:
        raise ValueError("ws, rows and ys must have one entry per matrix")
    wp = [_dev_any(w, torch.uint8, "w") for w in ws]
    yp = [_dev_any(y, torch.float32, "y") for y in ys]
    xp, xn = _dev_any(x, torch.float32, "x")
    need = gemm_q8_0_batched_workspace_bytes(cols, n_tokens)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    wsp, wsn = (workspace.data_ptr(), workspace.numel()) if workspace is not None else (0, 0)
    arr_p = ctypes.c_void_p * max(n, 1)
    arr_u = ctypes.c_uint64 * max(n, 1)
    check(_lib.load().fkv_gemm_q8_0_batched(
        n, arr_p(*[p for p, _ in wp]), arr_u(*[k for _, k in wp]), arr_u(*rows), cols, xp, xn,
        n_tokens, arr_p(*[p for p, _ in yp]), arr_u(*[k for _, k in yp]), wsp, wsn,
        _stream_ptr(stream)))

"""CPU: the Q8_0 GEMV/GEMM entry points validate before any device work, in the
reference's order and with its strings (crates/kernels/src/validate.rs:110-150;
the reference's own error cases, crates/kernels/src/tests.rs:425-460 and
tests/accept/tests/kernels_contract.rs:640-690). No kernel is launched here:
every call below fails (or, for rows == 0 / n_tokens == 0, succeeds) on the host."""
import ctypes

import pytest

import ferrum_amd as fa
from ferrum_amd import _lib
from ferrum_amd.errors import check

FAKE = 0x10000  # never dereferenced: each call returns before touching memory


def gemv(w_len, rows, cols, x_len, y_len, w=FAKE, x=FAKE, y=FAKE):
    return check(_lib.load().fkv_gemv_q8_0(w, w_len, rows, cols, x, x_len, y, y_len, None))


def gemm(w_len, rows, cols, x_len, n_tokens, y_len, w=FAKE, x=FAKE, y=FAKE):
    return check(_lib.load().fkv_gemm_q8_0(w, w_len, rows, cols, x, x_len, n_tokens, y, y_len,
                                           None))


def kernel_error(msg):
    return pytest.raises(fa.KernelError, match=f"^kernel: {msg}$")


def test_empty_dot_then_q8_k_then_lengths():
    with kernel_error("empty dot"):
        gemv(0, 1, 0, 0, 1)
    for cols in (1, 16, 17, 31, 33, 63):                 # kernels_contract.rs:640-650
        with kernel_error("q8_0 k is not a multiple of 32"):
            gemv(16, 2, cols, cols, 2)
    with kernel_error("length mismatch"):                # w one block short
        gemv(34, 2, 32, 32, 2)
    with kernel_error("length mismatch"):
        gemv(68, 2, 32, 31, 2)
    with kernel_error("length mismatch"):
        gemv(68, 2, 32, 32, 3)
    with kernel_error("shape overflow"):
        gemv(0, 2 ** 63, 2 ** 32, 0, 0)
    # the order: a bad cols wins over bad lengths
    with kernel_error("q8_0 k is not a multiple of 32"):
        gemv(1, 2, 48, 1, 1)


def test_gemm_lengths_and_zero_tokens():
    with kernel_error("length mismatch"):
        gemm(68, 2, 32, 32, 2, 4)                        # x holds one token of two
    with kernel_error("length mismatch"):
        gemm(68, 2, 32, 64, 2, 3)
    with kernel_error("shape overflow"):
        gemm(68, 2, 32, 0, 2 ** 62, 0)
    # n_tokens == 0 is Ok before any check (scalar.rs:99-101), even with bad shapes
    gemm(0, 5, 7, 0, 0, 0, w=0, x=0, y=0)


def test_rows_zero_succeeds_without_a_launch():
    gemv(0, 0, 64, 64, 0, w=0, y=0)
    gemm(0, 0, 64, 128, 2, 0, w=0, y=0)


def test_device_boundary_errors():
    with pytest.raises(fa.InvalidRequest, match="^null argument$"):
        gemv(68, 2, 32, 32, 2, w=0)
    with pytest.raises(fa.InvalidRequest, match="^w must be 2-byte aligned$"):
        gemv(68, 2, 32, 32, 2, w=FAKE + 1)
    with pytest.raises(fa.InvalidRequest, match="^x and y must be 4-byte aligned$"):
        gemv(68, 2, 32, 32, 2, x=FAKE + 2)
    cols = 65536 + 32                                    # one token's LDS beyond 160 KiB
    with pytest.raises(fa.InvalidRequest, match="^matrix too large for one launch$"):
        gemv(cols // 32 * 34, 1, cols, cols, 1)


def multi(n, w_len, rows, cols, x_len, n_tokens, y_len, w=None, y=None):
    arr_p = ctypes.c_void_p * max(n, 1)
    arr_u = ctypes.c_uint64 * max(n, 1)
    w = w if w is not None else [FAKE] * n
    y = y if y is not None else [FAKE] * n
    return check(_lib.load().fkv_gemm_q8_0_multi(
        n, arr_p(*w), arr_u(*w_len), arr_u(*rows), cols, FAKE, x_len, n_tokens, arr_p(*y),
        arr_u(*y_len), None))


def test_multi_checks_each_matrix_in_order():
    with pytest.raises(fa.InvalidRequest, match="^n_mats must be 1..4$"):
        multi(0, [], [], 64, 64, 1, [])
    with pytest.raises(fa.InvalidRequest, match="^n_mats must be 1..4$"):
        multi(5, [68] * 5, [2] * 5, 32, 32, 1, [2] * 5)
    # the second matrix's weight bytes are one block short: its length mismatch
    with pytest.raises(fa.KernelError, match="^kernel: length mismatch$"):
        multi(2, [68, 34], [2, 2], 32, 32, 1, [2, 2])
    # a bad cols fails on the first matrix already
    with pytest.raises(fa.KernelError, match="^kernel: q8_0 k is not a multiple of 32$"):
        multi(2, [68, 68], [2, 2], 48, 48, 1, [2, 2])
    with pytest.raises(fa.InvalidRequest, match="^null argument$"):
        multi(2, [68, 68], [2, 2], 32, 32, 1, [2, 2], w=[FAKE, 0])
    # n_tokens == 0 and all-empty matrices succeed without a launch
    multi(2, [0, 0], [0, 0], 32, 0, 0, [0, 0])
    multi(2, [0, 0], [0, 0], 32, 32, 1, [0, 0], w=[0, 0], y=[0, 0])

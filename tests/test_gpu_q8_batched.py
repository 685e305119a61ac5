"""GPU parity: fkv_gemm_q8_0_batched (Q8_0 GEMM of a token batch on the matrix cores).

The bar is the reference's own one between its backends, bit-identity
(crates/kernels/src/tests.rs:770-830, bits_eq on Q8_0 gemm): every output equals the
oracle's fo_q8_gemm (dot_q8_row_q8_act, q8_dot.rs:72-109, pinned in
test_cpu_oracle_q8_gemm.py) and fkv_gemm_q8_0's GEMV result, bit for bit, on:
- token counts on and off the 16-token MFMA tile and the 64-token workgroup, row counts
  off the 16-row tile, the Llama-3-8B projection shapes of a 64-sequence decode batch;
- several matrices sharing the activation in one launch;
- non-finite and extreme activations and weight scales;
- the calls the matrix-core path does not take (fewer than 8 tokens, columns off a
  multiple of 1024, weights not 16-byte aligned), which run the GEMV;
and a workspace that is too small is rejected before anything runs.
"""
import numpy as np
import pytest

from oracle import ref
from tests.test_gpu_q8_gemm import _dev, _same, _weights

pytestmark = pytest.mark.gpu


def _batched(ws, rows, cols, x, offset=0, workspace=None):
    """fkv_gemm_q8_0_batched through ferrum_amd; each weight placed `offset` bytes into
    its device buffer."""
    import torch
    import ferrum_amd as fa
    n_tokens = x.shape[0]
    wd = []
    for w in ws:
        buf = torch.zeros(w.size + offset + 16, dtype=torch.uint8, device="cuda")
        buf[offset:offset + w.size] = _dev(w)
        wd.append(buf[offset:offset + w.size])
    ys = [torch.full((n_tokens, r), 3.0, dtype=torch.float32, device="cuda") for r in rows]
    fa.gemm_q8_0_batched(wd, rows, cols, _dev(x.astype(np.float32)), n_tokens, ys,
                         workspace=workspace)
    torch.cuda.synchronize()
    return [y.cpu().numpy() for y in ys]


def _gemv(w, rows, cols, x):
    import torch
    import ferrum_amd as fa
    y = torch.full((x.shape[0], rows), 5.0, dtype=torch.float32, device="cuda")
    fa.gemm_q8_0(_dev(w), rows, cols, _dev(x), x.shape[0], y)
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("rows,cols,n_tokens", [
    (16, 1024, 8), (16, 1024, 16), (33, 1024, 17), (48, 2048, 63), (40, 1024, 64),
    (17, 3072, 65), (64, 2048, 200), (1, 1024, 8), (40, 4096, 37), (4100, 2048, 50),
    (16400, 2048, 40),
])
def test_matches_oracle_and_gemv(rows, cols, n_tokens):
    rng = np.random.default_rng(rows * 131 + cols + n_tokens)
    w = _weights(rng, rows, cols)
    x = (rng.standard_normal((n_tokens, cols)) *
         rng.choice([1e-4, 1.0, 300.0], (n_tokens, 1))).astype(np.float32)
    got, = _batched([w], [rows], cols, x)
    _same(got, ref.q8_gemm(w, rows, cols, x))
    _same(got, _gemv(w, rows, cols, x))


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (14336, 4096),
                                       (4096, 14336)])
def test_llama3_8b_shapes_decode_batch(rows, cols):
    """attn_q/attn_output, attn_k/attn_v, ffn_gate/up and ffn_down of a 64-sequence
    decode step (C2's batch), against the GEMV bit for bit."""
    rng = np.random.default_rng(rows ^ cols)
    w = _weights(rng, rows, cols)
    x = rng.standard_normal((64, cols)).astype(np.float32)
    got, = _batched([w], [rows], cols, x)
    _same(got, _gemv(w, rows, cols, x))
    sel = rng.choice(rows, 24, replace=False)  # and a sample of rows against the oracle
    wr = w.reshape(rows, -1)[sel].reshape(-1)
    _same(got[:, sel], ref.q8_gemm(wr, sel.size, cols, x))


def test_several_matrices_one_launch():
    """q/k/v of one activation: each output is its own call's, with an empty matrix in
    the middle of the batch."""
    rng = np.random.default_rng(77)
    cols, n_tokens = 2048, 40
    shapes = [64, 16, 0, 33]
    ws = [_weights(rng, r, cols) if r else np.zeros(0, np.uint8) for r in shapes]
    x = rng.standard_normal((n_tokens, cols)).astype(np.float32)
    ys = _batched(ws, shapes, cols, x)
    for r, w, y in zip(shapes, ws, ys):
        if r:
            _same(y, ref.q8_gemm(w, r, cols, x))


def test_non_finite_and_extreme_inputs():
    rng = np.random.default_rng(12)
    rows, cols = 40, 1024
    w = _weights(rng, rows, cols, special=True)
    x = rng.standard_normal((20, cols)).astype(np.float32)
    x[0, 3] = np.nan
    x[1, 70] = np.inf
    x[2, 64:96] = 0.0
    x[2, 100] = -np.inf
    x[3, :32] = np.float32(1e-40)
    x[3, 32:64] = np.float32(3e38)
    x[19, 1000] = np.nan
    want = ref.q8_gemm(w, rows, cols, x)
    assert np.isnan(want).any() and np.isfinite(want).any()
    got, = _batched([w], [rows], cols, x)
    _same(got, want)


@pytest.mark.parametrize("rows,cols,n_tokens,offset", [
    (20, 1024, 7, 0),    # too few tokens: GEMV
    (20, 544, 30, 0),    # columns off a multiple of 1024: GEMV
    (20, 1024, 30, 2),   # weights 2 mod 16: GEMV
    (20, 1024, 30, 8),   # 8 mod 16: GEMV
])
def test_calls_the_matrix_cores_do_not_take(rows, cols, n_tokens, offset):
    rng = np.random.default_rng(rows + cols + n_tokens + offset)
    w = _weights(rng, rows, cols)
    x = rng.standard_normal((n_tokens, cols)).astype(np.float32)
    got, = _batched([w], [rows], cols, x, offset=offset)
    _same(got, ref.q8_gemm(w, rows, cols, x))


def test_workspace_size_and_rejection():
    import torch
    import ferrum_amd as fa
    assert fa.gemm_q8_0_batched_workspace_bytes(4096, 7) == 0
    assert fa.gemm_q8_0_batched_workspace_bytes(544, 64) == 0
    need = fa.gemm_q8_0_batched_workspace_bytes(4096, 64)
    assert need == 4 * 128 * 16 * 32 + 4 * 128 * 16 * 4
    rng = np.random.default_rng(1)
    w = _dev(_weights(rng, 16, 4096))
    x = _dev(rng.standard_normal((64, 4096)).astype(np.float32))
    y = torch.full((64, 16), 5.0, dtype=torch.float32, device="cuda")
    small = torch.empty(need - 16, dtype=torch.uint8, device="cuda")
    with pytest.raises(fa.InvalidRequest, match="^gemm workspace too small$"):
        fa.gemm_q8_0_batched([w], [16], 4096, x, 64, [y], workspace=small)
    torch.cuda.synchronize()
    assert np.all(y.cpu().numpy() == 5.0)


@pytest.mark.parametrize("case", range(20))
def test_randomized_batches_against_oracle_and_gemv(case):
    """Seeded random launches: 1 to 4 matrices (an empty one possible) sharing an
    activation, row counts from 1 to ~5,000 (all three kernel instances: 16-block chunks,
    32-block chunks with and without the producer wave), columns 1,024 to 6,144, 8 to 150
    tokens with activation rows of widely different scales; every output against the GEMV
    bit for bit and a sample of rows against the oracle bit for bit."""
    rng = np.random.default_rng(4000 + case)
    cols = int(rng.choice([1024, 2048, 3072, 4096, 6144]))
    n_tokens = int(rng.integers(8, 151))
    nm = int(rng.integers(1, 5))
    rows = [int(rng.choice([0, 1, 15, 16, 17, int(rng.integers(1, 300)), int(rng.integers(300, 5000))]))
            for _ in range(nm)]
    if not any(rows):
        rows[0] = 33
    ws = [_weights(rng, r, cols) if r else np.zeros(0, np.uint8) for r in rows]
    x = (rng.standard_normal((n_tokens, cols)) *
         rng.choice([1e-3, 1.0, 50.0], (n_tokens, 1))).astype(np.float32)
    ys = _batched(ws, rows, cols, x)
    for r, w, y in zip(rows, ws, ys):
        if not r:
            continue
        _same(y, _gemv(w, r, cols, x))
        sel = np.unique(rng.integers(0, r, min(r, 24)))
        wr = w.reshape(r, -1)[sel].reshape(-1)
        _same(y[:, sel], ref.q8_gemm(wr, sel.size, cols, x))

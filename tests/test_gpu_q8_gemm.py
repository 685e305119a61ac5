"""GPU parity: fkv_gemv_q8_0 / fkv_gemm_q8_0 against the oracle, bit for bit.

The reference's own bar for this product is bit-identity between its backends
(crates/kernels/src/tests.rs:770-830, bits_eq on Q8_0 gemv and gemm); the GPU meets
it against fo_q8_gemm (pinned in test_cpu_oracle_q8_gemm.py) on:
- the reference's shapes (kernels_contract.rs:616-637: cols 32/64 x rows 1/3, 2 tokens;
  tests.rs:770-830: cols 32..4096, 4 tokens) and its known answer (tests.rs:291-309);
- row counts off the 16-row workgroup tile, block counts off the 16-block step, every
  token count 1..9 (token chunks of 4/2/1), 2-byte-misaligned weights;
- the full Llama-3-8B / 70B projection shapes (4096, 14336 and 28672 columns);
- non-finite and extreme inputs (NaN/Inf activations, Inf/NaN/subnormal weight scales,
  -128 quants, all-zero blocks).
NaN outputs are compared as NaN (payloads are not part of the contract).
"""
import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _weights(rng, rows, cols, special=False):
    nb = cols // 32
    e = rng.integers(-10, -2, size=(rows, nb))
    bits = ((e + 15) << 10).astype(np.uint16) | rng.integers(0, 1024, (rows, nb)).astype(np.uint16)
    bits |= (rng.random((rows, nb)) < 0.5).astype(np.uint16) << 15          # negative scales
    wq = rng.integers(-128, 128, size=(rows, nb, 32)).astype(np.int8)
    if special:
        flat = bits.reshape(-1)
        picks = rng.choice(flat.size, size=min(flat.size, 6), replace=False)
        for p, v in zip(picks, [0x7c00, 0xfc00, 0x7e01, 0x0001, 0x0000, 0x8000]):
            flat[p] = v
        wq.reshape(-1)[rng.choice(wq.size, size=wq.size // 10, replace=False)] = -128
    out = np.empty((rows, nb, 34), np.uint8)
    out[..., 0], out[..., 1] = bits & 0xff, bits >> 8
    out[..., 2:] = wq.view(np.uint8)
    return out.reshape(-1)


def _same(got, want):
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(g), nan), "NaN positions differ"
    bad = np.nonzero(g[~nan].view(np.uint32) != w[~nan].view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} outputs differ, first {g[~nan][bad[0]]} vs {w[~nan][bad[0]]}"


def _run(w, rows, cols, x, offset=0):
    """Through the C ABI (ferrum_amd.gemm_q8_0 / gemv_q8_0); w placed `offset` bytes
    into its device buffer."""
    import torch
    import ferrum_amd as fa
    n_tokens = x.shape[0]
    buf = torch.zeros(w.size + offset + 2, dtype=torch.uint8, device="cuda")
    buf[offset:offset + w.size] = _dev(w)
    wv = buf[offset:offset + w.size]
    xd = _dev(x.astype(np.float32))
    y = torch.full((n_tokens, rows), 3.0, dtype=torch.float32, device="cuda")
    if n_tokens == 1:
        fa.gemv_q8_0(wv, rows, cols, xd[0], y[0])
    else:
        fa.gemm_q8_0(wv, rows, cols, xd, n_tokens, y)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_reference_known_answer():
    qs = (np.arange(32) - 8).astype(np.int8)
    w = np.concatenate([np.array([0x00, 0x3c], np.uint8), qs.view(np.uint8)])
    y = _run(w, 1, 32, np.ones((1, 32), np.float32))
    scale_x = np.float32(np.float16(np.float32(1.0) / np.float32(127.0)))
    assert y[0, 0].view(np.uint32) == (np.float32(240 * 127) * scale_x).view(np.uint32)


@pytest.mark.parametrize("rows,cols,n_tokens", [
    (1, 32, 1), (3, 32, 2), (1, 64, 1), (3, 64, 2),          # kernels_contract.rs:616-637
    (2, 256, 4), (2, 4096, 4),                               # tests.rs:770-830
    (17, 96, 1), (33, 544, 3), (16, 512, 5), (100, 1056, 9), (1000, 4096, 1),
    (5, 8192, 7), (48, 2080, 8), (7, 57344, 2),
    (3, 65536, 2),   # the widest accepted: one token's activation copies fill 160 KB of LDS
    # one token past 4096 columns: 3 activation passes a thread, and 32 (more than the
    # 8 loaded up front, so the rest go through the loop)
    (33, 4128, 1), (600, 4128, 1), (3, 65536, 1), (520, 65536, 1),
])
def test_matches_oracle(rows, cols, n_tokens):
    rng = np.random.default_rng(rows * 7919 + cols + n_tokens)
    w = _weights(rng, rows, cols)
    x = (rng.standard_normal((n_tokens, cols)) *
         rng.choice([1e-4, 1.0, 300.0], (n_tokens, 1))).astype(np.float32)
    _same(_run(w, rows, cols, x), ref.q8_gemm(w, rows, cols, x))


@pytest.mark.parametrize("n_tokens", range(1, 10))
def test_every_token_count(n_tokens):
    rng = np.random.default_rng(n_tokens)
    rows, cols = 37, 1024
    w = _weights(rng, rows, cols)
    x = rng.standard_normal((n_tokens, cols)).astype(np.float32)
    y = _run(w, rows, cols, x)
    _same(y, ref.q8_gemm(w, rows, cols, x))
    # gemm rows equal gemv of each token (tests.rs:848-862)
    for t in range(n_tokens):
        _same(_run(w, rows, cols, x[t:t + 1])[0], y[t])


def test_misaligned_weights():
    """Blocks start 2 mod 4 and 0 mod 4 in turn; a buffer at +2 swaps every one."""
    rng = np.random.default_rng(5)
    rows, cols = 19, 96
    w = _weights(rng, rows, cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    want = ref.q8_gemm(w, rows, cols, x)
    for off in (0, 2, 6):
        _same(_run(w, rows, cols, x, offset=off), want)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1024, 4096), (14336, 4096),
                                       (4096, 14336), (1024, 8192), (8192, 28672)])
def test_full_model_shapes(rows, cols):
    """Llama-3-8B attn_q/attn_output, attn_k/attn_v, ffn_gate/up, ffn_down; Llama-3-70B
    attn_k/v and ffn_down. One token (the decode call) and four."""
    rng = np.random.default_rng(rows + cols)
    w = _weights(rng, rows, cols)
    for n_tokens in (1, 4):
        x = rng.standard_normal((n_tokens, cols)).astype(np.float32)
        _same(_run(w, rows, cols, x), ref.q8_gemm(w, rows, cols, x))


def test_non_finite_and_extreme_inputs():
    rng = np.random.default_rng(11)
    rows, cols = 40, 512
    w = _weights(rng, rows, cols, special=True)
    x = rng.standard_normal((4, cols)).astype(np.float32)
    x[0, 3] = np.nan                     # skipped by amax, quantizes to 0
    x[1, 70] = np.inf                    # block scale Inf: that block's products NaN
    x[2, 64:96] = 0.0                    # all-zero block
    x[2, 100] = -np.inf
    x[3, :32] = np.float32(1e-40)        # subnormal block: d subnormal, id huge
    x[3, 32:64] = np.float32(3e38)       # near f32 max
    want = ref.q8_gemm(w, rows, cols, x)
    assert np.isnan(want).any() and np.isfinite(want).any()
    _same(_run(w, rows, cols, x), want)


def test_errors_and_no_work_cases():
    import torch
    import ferrum_amd as fa
    w = torch.zeros(68, dtype=torch.uint8, device="cuda")
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    y = torch.full((2,), 5.0, dtype=torch.float32, device="cuda")
    with pytest.raises(fa.KernelError, match="^kernel: length mismatch$"):
        fa.gemv_q8_0(w, 2, 32, x, y)                  # x has 64 values for cols = 32
    with pytest.raises(fa.KernelError, match="^kernel: q8_0 k is not a multiple of 32$"):
        fa.gemv_q8_0(w, 2, 48, x, y)
    fa.gemm_q8_0(w, 2, 32, x, 0, y)                   # n_tokens == 0: nothing written
    torch.cuda.synchronize()
    assert y.cpu().tolist() == [5.0, 5.0]


@pytest.mark.parametrize("n_tokens", [1, 3, 4])
def test_multi_matrix_launch_equals_separate_calls(n_tokens):
    """q/k/v (and gate/up) in one launch: each output bit-identical to its own call and to
    the oracle, including a matrix with no rows in the middle of the batch."""
    import torch
    import ferrum_amd as fa
    rng = np.random.default_rng(40 + n_tokens)
    cols = 512
    shapes = [64, 16, 0, 17]
    ws = [_weights(rng, r, cols) if r else np.zeros(0, np.uint8) for r in shapes]
    x = rng.standard_normal((n_tokens, cols)).astype(np.float32)
    xd = _dev(x)
    wd = [_dev(w) if w.size else torch.zeros(0, dtype=torch.uint8, device="cuda") for w in ws]
    ys = [torch.full((n_tokens, r), 7.0, dtype=torch.float32, device="cuda") for r in shapes]
    fa.gemm_q8_0_multi(wd, shapes, cols, xd, n_tokens, ys)
    torch.cuda.synchronize()
    for r, w, y in zip(shapes, ws, ys):
        if not r:
            continue
        _same(y.cpu().numpy(), ref.q8_gemm(w, r, cols, x))
        _same(y.cpu().numpy(), _run(w, r, cols, x))


def test_multi_matrix_rejects_before_writing():
    import torch
    import ferrum_amd as fa
    w = torch.zeros(68, dtype=torch.uint8, device="cuda")
    short = torch.zeros(34, dtype=torch.uint8, device="cuda")
    x = torch.zeros(32, dtype=torch.float32, device="cuda")
    ys = [torch.full((1, 2), 5.0, device="cuda") for _ in range(2)]
    with pytest.raises(fa.KernelError, match="^kernel: length mismatch$"):
        fa.gemm_q8_0_multi([w, short], [2, 2], 32, x, 1, ys)
    torch.cuda.synchronize()
    assert all(y.cpu().tolist() == [[5.0, 5.0]] for y in ys)

"""Pins the oracle's Q8_0 GEMV/GEMM (fo_q8_gemm) before it checks the GPU's.

The reference: Kernels::gemv/gemm for DType::Q8_0 (crates/kernels/src/scalar.rs:84-116,
191-204) quantize the activation row (Q8Activation::quantize_into, q8_dot.rs:35-61)
and take dot_q8_row_q8_act of every weight row (q8_dot.rs:72-109). What pins it here:
- the reference's known answer (crates/kernels/src/tests.rs:291-309);
- exact closed forms: with power-of-two scales every product and partial sum is exact,
  so y is an integer matrix product times a power of two;
- the order of the f32 sum: a 4-block row whose left-to-right sum (the reference's
  loop) differs from pairwise and reversed orders;
- the activation scale's binary16 rounding at an exact tie: the reference's
  f32_to_f16_bits rounds half away from zero (q8_dot.rs:111-139), not to even;
- sign and power-of-two scaling symmetries, bit for bit;
- an f64 bound, and an independent numpy quantizer and block loop on small shapes.
"""
import numpy as np
import pytest

from oracle import ref


def _pack(scale_bits, quants):
    """Rows of Q8_0 blocks: scale_bits [rows, nb] uint16, quants [rows, nb*32] int8."""
    rows, nb = scale_bits.shape
    out = np.empty((rows, nb, 34), np.uint8)
    out[:, :, 0] = scale_bits & 0xff
    out[:, :, 1] = scale_bits >> 8
    out[:, :, 2:] = quants.reshape(rows, nb, 32).view(np.uint8)
    return out.reshape(-1)


def _pow2_bits(e):
    return np.uint16((e + 15) << 10)


def test_reference_known_answer():
    """tests.rs:291-309: qs = i - 8, scale 1.0, x = 1 -> sum(qs)*127 * (1 * f16(1/127))."""
    qs = (np.arange(32) - 8).astype(np.int8)
    w = _pack(np.array([[0x3c00]], np.uint16), qs[None, :])
    y = ref.q8_gemm(w, 1, 32, np.ones(32, np.float32))
    scale_x = np.float32(np.float16(np.float32(1.0) / np.float32(127.0)))  # not a tie
    assert np.float16(scale_x).view(np.uint16) == 0x2008
    want = np.float32(240 * 127) * (np.float32(1.0) * scale_x)
    assert y.shape == (1, 1) and y[0, 0].view(np.uint32) == want.view(np.uint32)


@pytest.mark.parametrize("nb,ks", [(8, (0, 1)), (32, (2,)), (1, (-5,))])
def test_power_of_two_scales_are_an_exact_integer_product(nb, ks):
    """x = u * 2^k with max|u| = 127 per block -> q = u, x_scale = 2^k exactly; weight
    scale 2^m. Every product and partial sum is then exact, so
    y = sum_b (Wq_b . u_b) * 2^(m + k_b) computed in integers."""
    rng = np.random.default_rng(nb)
    rows, cols, m = 7, nb * 32, -3
    wq = rng.integers(-128, 128, size=(rows, cols), dtype=np.int64).astype(np.int8)
    w = _pack(np.full((rows, nb), _pow2_bits(m), np.uint16), wq)
    for trial in range(3):
        u = rng.integers(-127, 128, size=(nb, 32))
        u[np.arange(nb), rng.integers(0, 32, nb)] = 127 * rng.choice([-1, 1], nb)
        k = rng.choice(ks, size=nb)
        x = (u * np.exp2(k)[:, None]).astype(np.float32).reshape(-1)
        y = ref.q8_gemm(w, rows, cols, x)[0]
        sumi = (wq.astype(np.int64).reshape(rows, nb, 32) * u[None]).sum(-1)   # [rows, nb]
        kmin = min(ks)
        total = (sumi * (2 ** (k - kmin))[None]).sum(-1)                       # integers
        want = (total.astype(np.float64) * 2.0 ** (m + kmin)).astype(np.float32)
        assert np.abs(total).max() < 2 ** 24
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32)), trial


def test_blocks_are_summed_left_to_right():
    """Products [A, s, -A, s] with A in [2^23, 2^24) and s < 1/2: left to right
    (A + s rounds to A) gives s; pairwise gives 0, reversed gives 0."""
    cols = 4 * 32
    x = np.zeros(cols, np.float32)
    x[0] = 127.0              # block 0: q = 127 at 0, scale 1
    x[32] = 127.0 / 1024.0    # block 1: q = 127, scale 2^-10
    x[64] = 127.0             # block 2
    x[96] = 127.0 / 1024.0    # block 3
    wq = np.zeros((1, cols), np.int8)
    wq[0, 0], wq[0, 32], wq[0, 64], wq[0, 96] = 127, 1, -127, 1
    scales = np.array([[_pow2_bits(10), 0x3c00, _pow2_bits(10), 0x3c00]], np.uint16)
    y = ref.q8_gemm(_pack(scales, wq), 1, cols, x)[0, 0]
    a, s = np.float32(127 * 127 * 1024), np.float32(127.0 / 1024.0)
    assert 2 ** 23 <= a < 2 ** 24 and s < 0.5
    assert (a + s) == a and (-a + s) == -a
    assert y == s, y


def test_activation_scale_tie_rounds_away_from_zero():
    """amax = 127 * (1 + 2^-11) -> d = 1 + 2^-11 exactly, halfway between two binary16
    values; the reference's f32_to_f16_bits takes 1 + 2^-10 (nearest-even would take 1)."""
    x = np.zeros(32, np.float32)
    x[0] = np.float32(127.0 * (1.0 + 2.0 ** -11))
    assert float(x[0]) == 127.0 * (1.0 + 2.0 ** -11)
    wq = np.zeros((1, 32), np.int8)
    wq[0, 0] = 1
    y = ref.q8_gemm(_pack(np.array([[0x3c00]], np.uint16), wq), 1, 32, x)[0, 0]
    assert y == np.float32(127.0 * (1.0 + 2.0 ** -10))
    assert np.float16(np.float32(1.0 + 2.0 ** -11)) == np.float16(1.0)   # RNE differs


def _random_weights(rng, rows, cols, lo=-9, hi=-3):
    nb = cols // 32
    bits = np.array([_pow2_bits(int(e)) for e in rng.integers(lo, hi, size=rows * nb)],
                    np.uint16).reshape(rows, nb)
    bits |= rng.integers(0, 1024, size=bits.shape).astype(np.uint16)  # random mantissas
    wq = rng.integers(-128, 128, size=(rows, cols), dtype=np.int64).astype(np.int8)
    return _pack(bits, wq), bits, wq


def test_sign_and_power_of_two_symmetries():
    rng = np.random.default_rng(7)
    rows, cols = 9, 256
    w, bits, wq = _random_weights(rng, rows, cols)
    x = rng.standard_normal((3, cols), dtype=np.float32)
    y = ref.q8_gemm(w, rows, cols, x)
    assert np.array_equal(ref.q8_gemm(w, rows, cols, -x).view(np.uint32), (-y).view(np.uint32))
    assert np.array_equal(ref.q8_gemm(w, rows, cols, 2 * x).view(np.uint32),
                          (2 * y).view(np.uint32))
    w2 = _pack(bits + np.uint16(0x0400), wq)        # every weight scale doubled
    assert np.array_equal(ref.q8_gemm(w2, rows, cols, x).view(np.uint32), (2 * y).view(np.uint32))


def _np_quantize(x):
    """Independent restatement of quantize_into for the check below (numpy f32 ops;
    half-away rounding from trunc; ties-away binary16 from the pinned ref encoder)."""
    blocks = x.reshape(-1, 32).astype(np.float32)
    amax = np.nanmax(np.abs(blocks), axis=1, initial=np.float32(0))
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (blocks * idv[:, None]).astype(np.float32)
    t = np.trunc(v)
    r = np.where(np.abs(v - t) >= 0.5, t + np.sign(v), t)
    q = np.clip(np.nan_to_num(r, nan=0), -128, 127).astype(np.int32)
    xs = ref.f16_to_f32(ref.f32_to_f16(d, rounding=1)).astype(np.float32)
    return q, xs


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 64), (5, 96), (4, 1024)])
def test_against_independent_block_loop_and_f64(rows, cols):
    rng = np.random.default_rng(rows * cols)
    w, bits, wq = _random_weights(rng, rows, cols)
    ws = ref.f16_to_f32(bits).astype(np.float32)                       # [rows, nb]
    x = (rng.standard_normal((2, cols)) * rng.choice([1e-3, 1, 50], (2, 1))).astype(np.float32)
    y = ref.q8_gemm(w, rows, cols, x)
    nb = cols // 32
    for t in range(2):
        q, xs = _np_quantize(x[t])
        sumi = (wq.astype(np.int64).reshape(rows, nb, 32) * q[None]).sum(-1)
        p = sumi.astype(np.float32) * (ws * xs[None])                  # f32, one rounding
        acc = np.zeros(rows, np.float32)
        for b in range(nb):
            acc = (acc + p[:, b]).astype(np.float32)
        assert np.array_equal(y[t].view(np.uint32), acc.view(np.uint32))
        exact = (sumi * ws.astype(np.float64) * xs.astype(np.float64)[None]).sum(-1)
        bound = nb * 2.0 ** -23 * np.abs(p.astype(np.float64)).sum(-1) + 1e-30
        assert np.all(np.abs(y[t] - exact) <= bound)


def test_non_finite_and_zero_activations():
    """NaN is skipped by amax (Rust f32::max) and quantizes to 0 (`as i32` of NaN);
    an Inf makes d = Inf, id = 0, every q 0 and the block's product 0 * Inf = NaN;
    an all-zero block has d = 0, q = 0 and contributes +0."""
    cols = 64
    wq = np.ones((1, cols), np.int8)
    w = _pack(np.array([[0x3c00, 0x3c00]], np.uint16), wq)
    x = np.zeros(cols, np.float32)
    assert ref.q8_gemm(w, 1, cols, x)[0, 0].view(np.uint32) == 0
    x[0], x[1] = np.nan, 127.0           # block 0: q = [0, 127, 0...]
    y = ref.q8_gemm(w, 1, cols, x)[0, 0]
    assert y == np.float32(127) * np.float32(1.0)
    x[40] = np.inf
    assert np.isnan(ref.q8_gemm(w, 1, cols, x)[0, 0])

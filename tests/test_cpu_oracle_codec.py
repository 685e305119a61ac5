"""CPU: the oracle's codecs and scalar kernels against the reference's known-answer
tests and against what IEEE 754 / the mathematics fixes (no GPU).

Pins (reference file:line -> check here):
  f16_to_f32   crates/core-types/src/dtype.rs:160-173 known values; :175-199 every
               code vs the closed-form f64 formula; numpy float16 decode
  f32_to_f16   RNE: all 2^32 inputs vs the x86 F16C instruction and vs an f64 nearest-
               even search; a boundary sweep vs numpy astype(float16).
               Ties-away: all 2^32 inputs vs an f64 nearest-away search; a sweep vs a
               numpy statement of Ferrum's f32_to_f16_bits (kernels/src/q8_dot.rs:113-139)
  Q8_0         quantize: KAT tests.rs:299-309 (x == 1 -> q == 127, scale f16(1/127)),
               ties, invariants; dequant: every code x every scale code
               (kernels_contract.rs:700-744, tests.rs:553-566)
  dot/softmax  tests.rs:178-195, kernels_contract.rs:437-467; AVX2 dot bit-identical
               to the scalar dot at tests.rs:616-621's lengths (LCG of tests.rs:21-33)
"""
import ctypes
import ctypes.util
import os
import sys

import numpy as np
import pytest

from oracle import ref

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
from make_golden import ferrum_f16_bits_away  # noqa: E402


def f16_sweep_bits(seed=0):
    """f32 bit patterns straddling every binary16 rounding case: every value of the
    top 19 bits with low-13-bit patterns (exact, just below/at/above half, max),
    plus random patterns."""
    hi = np.arange(1 << 19, dtype=np.uint32) << 13
    lows = np.array([0x0000, 0x0001, 0x0fff, 0x1000, 0x1001, 0x1fff], dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    rng = np.random.default_rng(seed)
    return np.concatenate([bits, rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32)])


# -- binary16 decode ----------------------------------------------------------------

def test_f16_known_values():
    # dtype.rs:160-173
    f = lambda b: np.float32(ref.lib().fo_f16_to_f32(b))
    assert f(0x0000).view(np.uint32) == 0
    assert f(0x8000).view(np.uint32) == 0x80000000
    assert f(0x3C00) == 1.0 and f(0x4000) == 2.0 and f(0x3800) == 0.5 and f(0xC000) == -2.0
    assert f(0x7C00) == np.inf and f(0xFC00) == -np.inf and np.isnan(f(0x7E00))
    assert f(0x0001) == np.float32(2.0 ** -24) and f(0x0400) == np.float32(2.0 ** -14)


def test_every_f16_code_matches_closed_form_and_numpy():
    # dtype.rs:175-199: (-1)^s * (frac * 2^-24 | (1 + frac/1024) * 2^(e-15)), NaN payload kept
    bits = np.arange(1 << 16, dtype=np.uint32)
    got = ref.f16_to_f32(bits.astype(np.uint16))
    e, fr, s = (bits >> 10) & 0x1F, bits & 0x3FF, np.where(bits >> 15, -1.0, 1.0)
    mag = np.where(e == 0, fr * 2.0 ** -24, (1.0 + fr / 1024.0) * 2.0 ** (e.astype(np.float64) - 15))
    finite = e != 31
    assert np.array_equal(got[finite].view(np.uint32), (s * mag)[finite].astype(np.float32).view(np.uint32))
    assert np.all(np.isinf(got[(e == 31) & (fr == 0)]))
    nan = (e == 31) & (fr != 0)
    assert np.all(np.isnan(got[nan]))
    assert np.array_equal(got[nan].view(np.uint32) & 0x7FFFFF, fr[nan] << 13)  # payload kept
    npy = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(got[finite].view(np.uint32), npy[finite].view(np.uint32))


# -- binary16 encode ----------------------------------------------------------------

@pytest.mark.parametrize("which,name", [(0, "RNE vs F16C"), (2, "RNE vs f64 search"),
                                        (1, "ties-away vs f64 search")])
def test_f16_encoder_exhaustive(which, name):
    bad, first = ref.selftest_f16(which, 1)
    assert bad == 0, f"{name}: {bad} of 2^32 inputs differ, first 0x{first:08x}"


def test_f16_rne_sweep_matches_numpy():
    x = f16_sweep_bits().view(np.float32)
    got = ref.f32_to_f16(x, 0)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    ok = ~np.isnan(x)
    assert np.array_equal(got[ok], want[ok])
    # NaN: top 10 payload bits kept, forced non-zero (q8_dot.rs:118-121)
    nb = x[~ok].view(np.uint32)
    hf = (nb & 0x7FFFFF) >> 13
    exp_nan = ((nb >> 16) & 0x8000) | 0x7C00 | hf | (hf == 0)
    assert np.array_equal(got[~ok], exp_nan.astype(np.uint16))


def test_f16_ties_away_sweep_matches_ferrum_encoder():
    x = f16_sweep_bits(1).view(np.float32)
    assert np.array_equal(ref.f32_to_f16(x, 1), ferrum_f16_bits_away(x))


def test_rne_and_ties_away_differ_exactly_on_ties():
    x = f16_sweep_bits(2).view(np.float32)
    rne, away = ref.f32_to_f16(x, 0), ref.f32_to_f16(x, 1)
    diff = rne != away
    # every difference is an exact tie: the f32 sits exactly halfway between the two
    lo = np.minimum(ref.f16_to_f32(rne[diff]).astype(np.float64),
                    ref.f16_to_f32(away[diff]).astype(np.float64))
    hi = np.maximum(ref.f16_to_f32(rne[diff]).astype(np.float64),
                    ref.f16_to_f32(away[diff]).astype(np.float64))
    xa = x[diff].astype(np.float64)
    fin = np.isfinite(hi)
    assert np.all(xa[fin] - lo[fin] == hi[fin] - xa[fin])
    assert diff.sum() > 10000  # the sweep hits every even-neighbour tie of the top-19-bit grid


def test_f16_roundtrip_of_every_non_nan_code():
    bits = np.arange(1 << 16, dtype=np.uint16)
    v = ref.f16_to_f32(bits)
    ok = ~np.isnan(v)
    for r in (0, 1):
        assert np.array_equal(ref.f32_to_f16(v[ok], r), bits[ok])


# -- Q8_0 ---------------------------------------------------------------------------------

def test_q8_reference_kat_ones():
    # tests.rs:299-309: x == 1.0 -> every q == 127, scale == f16(1/127)
    for r in (0, 1):
        s, q = ref.q8_quantize_block(np.ones(32, np.float32), r)
        assert np.all(q == 127)
        d = np.float32(1.0) / np.float32(127.0)
        assert s == ferrum_f16_bits_away(np.array([d]))[0] or r == 0
        assert s == ref.f32_to_f16(np.array([d], np.float32), r)[0]


def test_q8_special_blocks():
    s, q = ref.q8_quantize_block(np.zeros(32, np.float32))
    assert s == 0 and np.all(q == 0)  # d = 0 -> id = 0 -> q = 0
    x = np.zeros(32, np.float32)
    x[7] = -5.0
    s, q = ref.q8_quantize_block(x)
    assert q[7] == -127 and np.all(np.delete(q, 7) == 0)
    # exact .5 ties round away from zero (Rust f32::round): amax 127 -> d = 1, id = 1
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:] = np.arange(-15, 16, dtype=np.float32) + np.float32(0.5)
    s, q = ref.q8_quantize_block(x)
    want = np.where(x[1:] > 0, np.floor(x[1:]) + 1, np.ceil(x[1:]) - 1).astype(np.int8)
    assert s == 0x3C00 and np.array_equal(q[1:], want)


def test_q8_invariants_on_random_blocks():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((4096, 32)) * 10.0 ** rng.uniform(-6, 6, (4096, 1))).astype(np.float32)
    rows = ref.q8_quantize_row(x.ravel()).reshape(-1, 34)
    q = rows[:, 2:].view(np.int8).astype(np.int32)
    amax = np.abs(x).max(1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    assert np.all(np.abs(q) <= 127)
    # the amax lane quantises to +-127
    arg = np.abs(x).argmax(1)
    assert np.all(np.abs(q[np.arange(len(q)), arg]) == 127)
    # reconstruction with the pre-f16 d is within d/2 (+ one rounding of v*id)
    err = np.abs(x.astype(np.float64) - q * d[:, None].astype(np.float64))
    assert np.all(err <= d[:, None] * (0.5 + 1e-5) + 1e-30)


def test_q8_dequant_every_code_times_every_scale():
    # kernels_contract.rs:700-744 with all 256 codes (tests.rs:553-566)
    codes = np.arange(256, dtype=np.uint8)
    scales = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    blocks = np.zeros((len(scales), 8, 34), np.uint8)
    blocks[:, :, 0] = (scales & 0xFF)[:, None]
    blocks[:, :, 1] = (scales >> 8)[:, None]
    blocks[:, :, 2:] = codes.reshape(8, 32)[None]
    out = ref.q8_dequant(blocks.ravel(), len(scales) * 256).reshape(len(scales), 256)
    sf = scales.view(np.float16).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        want = sf[:, None] * codes.view(np.int8).astype(np.float32)[None, :]
    assert np.array_equal(out.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.array_equal(np.isnan(out), np.isnan(want))


# -- dot / softmax ------------------------------------------------------------------

def test_dot_and_softmax_kats():
    # tests.rs:178-195
    assert ref.dot([1.0, 2.0, 3.0], [4.0, -1.0, 0.5]) == np.float32(3.5)
    assert ref.softmax([7.5])[0].view(np.uint32) == np.float32(1.0).view(np.uint32)
    for bad in (np.nan, np.inf, -np.inf):
        assert ref.softmax([bad])[0].view(np.uint32) == 0
    # softmax([1,2,3]) bits == expf(x - 3) / serial sum, with the platform expf that
    # the reference's f32::exp also calls (exp-level parity is self-consistent there too)
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.restype, libm.expf.argtypes = ctypes.c_float, [ctypes.c_float]
    got = ref.softmax([1.0, 2.0, 3.0])
    ex = np.array([libm.expf(-2.0), libm.expf(-1.0), libm.expf(0.0)], np.float32)
    s = np.float32(np.float32(ex[0] + ex[1]) + ex[2])
    assert np.array_equal(got.view(np.uint32), (ex / s).astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("value", [0.0, 1.0, -4.0, 12.5, 1.0e-20, -100.0, 50.0])
def test_softmax_of_one_finite_element_is_one(value):
    # kernels_contract.rs:437-446
    assert ref.softmax([value])[0] == 1.0
    assert ref.avx2_softmax([value])[0] == 1.0


@pytest.mark.parametrize("case", [[np.nan], [np.inf], [-np.inf, -np.inf], [np.nan, np.nan],
                                  [1.0, np.inf, -3.0], [-np.inf, np.inf]])
def test_non_finite_softmax_max_writes_zeros(case):
    # kernels_contract.rs:448-467
    assert np.all(ref.softmax(case) == 0.0)
    assert np.all(ref.avx2_softmax(case) == 0.0)


def _lcg_vec(state, n):
    """The test LCG of crates/kernels/src/tests.rs:21-33."""
    out = np.empty(n, np.float32)
    for i in range(n):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(state >> 8) / np.float32(16777216.0)) * np.float32(2.0) - np.float32(1.0)
    return state, out


def test_avx2_dot_is_bit_identical_to_scalar():
    if not ref.avx2_available():
        pytest.skip("host has no AVX2/FMA/F16C")
    st = 0x1234
    for n in [1, 7, 8, 9, 31, 32, 33, 128, 4096, 4097, 5000]:  # tests.rs:616-621
        st, a = _lcg_vec(st, n)
        st, b = _lcg_vec(st, n)
        assert ref.avx2_dot(a, b).view(np.uint32) == ref.dot(a, b).view(np.uint32), n
        # scalar dot is strict left-to-right f32 without FMA
        acc = np.float32(0.0)
        for x, y in zip(a[:64], b[:64]):
            acc = np.float32(acc + np.float32(x * y))
        assert ref.dot(a[:64], b[:64]) == acc


def test_avx2_softmax_within_tolerance_of_scalar():
    if not ref.avx2_available():
        pytest.skip("host has no AVX2/FMA/F16C")
    rng = np.random.default_rng(0)
    for n in (1, 7, 8, 100, 4097):
        x = (rng.standard_normal(n) * 5).astype(np.float32)
        a, s = ref.avx2_softmax(x), ref.softmax(x)
        assert np.allclose(a, s, rtol=1e-6, atol=1e-7)
        assert abs(float(a.astype(np.float64).sum()) - 1.0) < 1e-5

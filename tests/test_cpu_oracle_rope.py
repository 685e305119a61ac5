"""Pins the oracle's RoPE (fo_rope) before it checks the GPU's RoPE decode step.

The reference: Kernels::rope (crates/kernels/src/scalar.rs:77-82) rotates q and k
with rope_tensor (:167-189) at the angle of math.rs:31-34. What pins it here:
- the reference's own known-answer shapes (crates/kernels/src/tests.rs:197-239):
  position 0 is the identity bit for bit, and dims from rope_dim on are untouched;
- the pairing: a unit vector on dim 2i turns within dims (2i, 2i+1)
  (GGML_ROPE_TYPE_NORMAL), not towards dim 2i + rope_dim/2 (NeoX);
- every rotated value against an f64 evaluation of the same f32 angle
  (theta^(2i/rope_dim) rounded to f32, pos / that in f32) with sin and cos in
  f64, to 2 ulps of the larger operand of its pair (a cos - b sin cancels);
- pair norms and rotation angles at position 131,071 (the C5 context).
"""
import numpy as np
import pytest

from oracle import ref


def _angle32(pos, theta, i, rope_dim):
    """The reference's f32 angle, evaluated in f64 and rounded where it rounds."""
    den = np.float32(np.float64(np.float32(theta)) ** (np.float64(np.float32(2 * i) / np.float32(rope_dim))))
    return np.float32(np.float32(pos) / den)


def _expect(x, rope_dim, pos, theta):
    out = np.array(x, np.float32, copy=True)
    for i in range(0, rope_dim, 2):
        f = np.float64(_angle32(pos, theta, i // 2, rope_dim))
        sn, cs = np.float32(np.sin(f)), np.float32(np.cos(f))
        a, b = out[..., i].copy(), out[..., i + 1].copy()
        out[..., i] = a * cs - b * sn
        out[..., i + 1] = a * sn + b * cs
    return out


def test_position_zero_is_identity_bit_for_bit():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 128), dtype=np.float32)
    y = ref.rope(x, 128, 0, 10000.0)
    assert np.array_equal(y.view(np.uint32), x.view(np.uint32))
    # tests.rs:197-212: q = [1, 0, 0, 0], head_dim = rope_dim = 4, pos 0
    e = np.array([1.0, 0.0, 0.0, 0.0], np.float32)
    assert np.array_equal(ref.rope(e, 4, 0, 10000.0).view(np.uint32), e.view(np.uint32))


def test_dims_past_rope_dim_are_untouched_and_pairs_rotate():
    """tests.rs:214-239: head_dim 6, rope_dim 4, pos 1; q[4..] bit-identical and
    q[0..4] the NORMAL-pair rotation."""
    q = np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], np.float32)
    y = ref.rope(q, 4, 1, 10000.0)
    assert np.array_equal(y[4:].view(np.uint32), q[4:].view(np.uint32))
    want = _expect(q, 4, 1, 10000.0)
    assert np.all(np.abs(y[:4] - want[:4]) <= 2 * np.spacing(np.float32(4.0)))


def test_pairs_are_adjacent_dims():
    d, rope_dim, pos, theta = 8, 8, 7, 10000.0
    for i in range(0, rope_dim, 2):
        e = np.zeros(d, np.float32)
        e[i] = 1.0
        y = ref.rope(e, rope_dim, pos, theta)
        f = np.float64(_angle32(pos, theta, i // 2, rope_dim))
        assert abs(y[i] - np.cos(f)) < 1e-6 and abs(y[i + 1] - np.sin(f)) < 1e-6
        others = np.delete(y, [i, i + 1])
        assert np.all(others == 0.0)


@pytest.mark.parametrize("d,rope_dim", [(128, 128), (128, 64), (64, 64), (64, 32)])
@pytest.mark.parametrize("pos", [1, 17, 4095, 131071])
def test_rotation_against_f64(d, rope_dim, pos):
    rng = np.random.default_rng(pos + d)
    x = rng.standard_normal((8, d), dtype=np.float32)
    y = ref.rope(x, rope_dim, pos, 500000.0 if d == 128 else 10000.0)
    want = _expect(x, rope_dim, pos, 500000.0 if d == 128 else 10000.0)
    # a cos - b sin cancels: the error bound is in ulps of the pair's operands
    pair_max = np.repeat(np.maximum(np.abs(x[:, 0:rope_dim:2]), np.abs(x[:, 1:rope_dim:2])), 2, axis=1)
    assert np.all(np.abs(y[:, :rope_dim] - want[:, :rope_dim]) <= 2 * np.spacing(pair_max))
    assert np.array_equal(y[:, rope_dim:].view(np.uint32), x[:, rope_dim:].view(np.uint32))
    n0 = x[:, 0:rope_dim:2].astype(np.float64) ** 2 + x[:, 1:rope_dim:2].astype(np.float64) ** 2
    n1 = y[:, 0:rope_dim:2].astype(np.float64) ** 2 + y[:, 1:rope_dim:2].astype(np.float64) ** 2
    assert np.allclose(n1, n0, rtol=2e-6, atol=1e-9)


def test_rope_dim_zero_or_too_large_changes_nothing():
    """scalar.rs:174-176 returns early; the API rejects these before the kernels."""
    x = np.random.default_rng(1).standard_normal((2, 64), dtype=np.float32)
    for rd in (0, 66):
        assert np.array_equal(ref.rope(x, rd, 9, 10000.0).view(np.uint32), x.view(np.uint32))


def test_rope_step_positions():
    """rope_step rotates sequence s at ctx_lens[s] - 1 (and an empty context at 0)."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((3, 4, 64), dtype=np.float32)
    k = rng.standard_normal((3, 2, 64), dtype=np.float32)
    qr, kr = ref.rope_step(q, k, [0, 1, 40], 64, 10000.0)
    assert np.array_equal(qr[0], q[0]) and np.array_equal(qr[1], q[1])
    assert np.array_equal(qr[2], ref.rope(q[2], 64, 39, 10000.0))
    assert np.array_equal(kr[2], ref.rope(k[2], 64, 39, 10000.0))

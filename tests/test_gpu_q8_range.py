"""GPU parity: Q8_0 decode attention past the binary16 range.

The reference dequantises Q8_0 in f32, f16_to_f32(scale) * (i8 as f32)
(crates/kernels/src/scalar.rs:268-275), exact for every finite scale. Workgroups over a
block that holds a scale of 512 or more (values beyond 512 * 127, where scale x quant
can pass 65504; the store marks the block) run the exact kernel instance: quants as
exact binary16/bf16 operands, scales applied in f32. Checked against the oracle (which dequantises exactly as the
reference) at the attention bar, with no fault raised, for:
- K and V values up to +-1e6 scattered through ordinary N(0,1) rows;
- blocks where one token's scale is ~7,874 and its neighbours' ~0.02, with the big
  token's weight small so the ordinary tokens carry the output;
- the fused step (and the RoPE fused step) appending such a token onto a pool that
  held none: the step's own workgroup marks the token's block and the exact instance
  recomputes that workgroup's outputs;
- fkv_paged_write / fkv_paged_fill putting such scales in place.
A scale past the binary16 range itself (a 32-value run with |x| >= 65520 * 127) is
stored as the reference's encoder stores it (+-inf) and raises FKV_FAULT_VALUE_RANGE.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, slots_for, to_dev

pytestmark = pytest.mark.gpu


def _sprinkle(rng, x, per_row=2, big=1e6):
    """x with `per_row` random elements of every (token, head) row set to +-big."""
    x = x.copy()
    n, h, d = x.shape
    for _ in range(per_row):
        idx = rng.integers(0, d, size=(n, h))
        sign = rng.choice([-1.0, 1.0], size=(n, h)).astype(np.float32)
        np.put_along_axis(x, idx[..., None], (sign * big)[..., None], axis=-1)
    return x


def _table(rng, ctxs, extra=4):
    nb = [max(1, (c + 15) // 16) for c in ctxs]
    nblk = sum(nb) + extra
    perm = rng.permutation(nblk).astype(np.int32)
    tab = np.zeros((len(ctxs), max(nb)), np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = perm[off: off + n]
        off += n
    return nblk, tab


def _attend(pool, layout, q, tab, ctxs):
    import torch
    import ferrum_amd as fa
    from oracle import ref
    ctx = np.array(ctxs, np.int32)
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(ctx), int(ctx.max()))
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    want = ref.attention(layout, pool.read(), 0, q, tab, ctx, fa.default_scale(q.shape[2]))
    return out.cpu().numpy(), want


SHAPES = [(128, 8, 4), (64, 4, 8), (128, 2, 1)]
CTXS = [1, 16, 17, 300, 2100, 5000]


@pytest.mark.parametrize("which", ["k", "v", "both"])
@pytest.mark.parametrize("d,hkv,g", SHAPES)
def test_wide_values_match_the_oracle(d, hkv, g, which):
    rng = np.random.default_rng(d * 7 + g)
    nblk, tab = _table(rng, CTXS)
    pool, layout = make_pools(1, hkv, d, nblk, dtype=8)
    pool.fill(0)
    total = sum(CTXS)
    k = rng.standard_normal((total, hkv, d), dtype=np.float32)
    v = rng.standard_normal((total, hkv, d), dtype=np.float32)
    q = rng.standard_normal((len(CTXS), hkv * g, d), dtype=np.float32)
    if which in ("k", "both"):
        # K up to 1e6 (scale ~7,874: a binary16 operand would be inf); q small enough
        # that the scores stay O(1), so the outputs are well conditioned (under a peaky
        # softmax over +-1e6 values an output that cancels to a small number depends on
        # the last bit of the f32 scores, where any two orders of f32 arithmetic differ)
        k = _sprinkle(rng, k, per_row=2, big=1e6)
        q *= np.float32(2e-6)
    if which in ("v", "both"):
        v = _sprinkle(rng, v, per_row=2, big=1e6)
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(CTXS)])
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    got, want = _attend(pool, layout, q, tab, CTXS)
    assert np.all(np.isfinite(want))
    if which != "k":
        assert np.abs(want).max() > 1e3  # the big values reach the output
    assert_close(got, want)


def test_mixed_scales_in_one_block():
    """Every block holds one token with a V value of 1e6 (scale ~7,874) beside fifteen
    N(0,1) tokens (scales ~0.02); the big token's score is pushed far down, so the
    output is carried by the ordinary tokens of the same blocks."""
    d, hkv, g, ctx = 128, 2, 4, 1024
    rng = np.random.default_rng(5)
    nblk, tab = _table(rng, [ctx])
    pool, layout = make_pools(1, hkv, d, nblk, dtype=8)
    pool.fill(0)
    k = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    v = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    v[::16, :, 7] = 1e6
    k[::16, :, :] = -3.0
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots_for(tab[0], ctx)))
    q = np.abs(rng.standard_normal((1, hkv * g, d), dtype=np.float32))
    got, want = _attend(pool, layout, q, tab, [ctx])
    assert np.abs(want).max() < 1e2  # carried by the ordinary tokens
    assert_close(got, want)


@pytest.mark.parametrize("rope", [False, True])
def test_fused_step_appending_a_wide_token(rope):
    """The pool holds ordinary values; the step's new token of sequence 2 has a V value
    of 1e6. Its workgroup marks the token's block during the call and the exact
    instance launched after recomputes that split's outputs. V and K bytes are the oracle's
    append, bit for bit, with and without RoPE."""
    import torch
    import ferrum_amd as fa
    from oracle import ref
    from tests.test_gpu_append_attention import _setup
    from tests.test_gpu_rope_attention import _check_k
    d, hkv, g, theta = 128, 8, 4, 500000.0
    ctxs = [17, 300, 513, 2100]
    pool, layout, tab, knew, vnew = _setup(8, d, hkv, ctxs, seed=9, layers=1)
    vnew[2, 3, 11] = 1e6
    q = np.random.default_rng(9).standard_normal((len(ctxs), hkv * g, d), dtype=np.float32)
    ctx = np.array(ctxs, np.int32)
    before = pool.read()
    out = torch.full(q.shape, 7.0, dtype=torch.float32, device="cuda")
    if rope:
        pool.rope_append_decode_attention(0, to_dev(knew), to_dev(vnew), to_dev(q), out,
                                          to_dev(tab), to_dev(ctx), int(ctx.max()), d, theta)
    else:
        pool.append_decode_attention(0, to_dev(knew), to_dev(vnew), to_dev(q), out, to_dev(tab),
                                     to_dev(ctx), int(ctx.max()))
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    image = pool.read()
    tail = np.array([slots_for(tab[i], c)[-1] for i, c in enumerate(ctxs)], np.int64)
    qq, kk = ref.rope_step(q, knew, ctx, d, theta) if rope else (q, knew)
    want_image = before.copy()
    ref.append(layout, want_image, 0, kk, vnew, tail)
    got_k, got_v = ref.gather_slots(layout, image, 0, tail, fmt=1)
    want_k, want_v = ref.gather_slots(layout, want_image, 0, tail, fmt=1)
    assert np.array_equal(got_v, want_v)
    if rope:
        gk, _ = ref.gather_slots(layout, image, 0, tail)
        wk, _ = ref.gather_slots(layout, want_image, 0, tail)
        _check_k(8, gk, wk, kk)
    else:
        assert np.array_equal(image, want_image)
    want = ref.attention(layout, image, 0, qq, tab, ctx, fa.default_scale(d))
    assert np.abs(want[2]).max() > 1e2
    assert_close(out.cpu().numpy(), want)


def test_scale_past_binary16_is_stored_as_inf_and_flagged():
    import torch
    import ferrum_amd as fa
    from oracle import ref
    pool, layout = make_pools(1, 1, 64, 2, dtype=8)
    pool.fill(0)
    k = np.ones((2, 1, 64), np.float32)
    v = np.ones((2, 1, 64), np.float32)
    slots = np.array([0, 1], np.int64)
    v[1, 0, 40] = 70000.0  # scale ~551: wide, finite, not a fault
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == 0
    v[1, 0, 40] = 1e7  # 1e7 / 127 > 65504: the scale is +inf
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    torch.cuda.synchronize()
    assert pool.take_fault_flags() == fa.FAULT_VALUE_RANGE
    want = ref.new_pool(layout)
    ref.append(layout, want, 0, k, v, slots)
    assert np.array_equal(pool.read(), want)


@pytest.mark.parametrize("how", ["write", "fill"])
def test_write_and_fill_mark_the_blocks(how):
    """A pool image with a wide scale put in place by fkv_paged_write, or every scale
    made 0x6060 (560) by fkv_paged_fill and then ordinary tokens appended over part of
    it: attention over it meets the bar against the oracle."""
    from oracle import ref
    d, hkv, g, ctx = 128, 2, 4, 700
    rng = np.random.default_rng(11)
    nblk, tab = _table(rng, [ctx], extra=1)
    pool, layout = make_pools(1, hkv, d, nblk, dtype=8)
    slots = slots_for(tab[0], ctx)
    k = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    v = rng.standard_normal((ctx, hkv, d), dtype=np.float32)
    if how == "write":
        v[100, 1, 5] = -3e5
        image = ref.new_pool(layout)
        ref.append(layout, image, 0, k, v, slots)
        pool.write(image)
    else:
        pool.fill(0x60)
        pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    q = rng.standard_normal((1, hkv * g, d), dtype=np.float32)
    got, want = _attend(pool, layout, q, tab, [ctx])
    if how == "write":
        assert np.abs(want).max() > 1e2
    assert_close(got, want)

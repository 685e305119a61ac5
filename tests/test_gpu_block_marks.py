"""GPU parity: per-block marks travel with the blocks' bytes.

A block is marked when a value the fast attention instances cannot take is stored in it
(a Q8_0 scale of 512 or more; an Inf/NaN K or V of an F16 pool). Attention workgroups
whose blocks include a marked one run the exact (Q8_0, f32 dequantisation as
crates/kernels/src/scalar.rs:268-275) or leak-safe (F16 prefill: no query reads a
position past its own, crates/model/src/llama.rs:229-245) instance; the others keep the
fast one. Checked here:
- the count of marked blocks follows appends, whole-block and partial writes, fill;
- swap_out -> fill(0) -> swap_in brings the marks back with the bytes: Q8_0 values to
  +-1e6 through decode and prefill, F16 Inf/NaN V inside a chunk through prefill (exact
  NaN positions), all against the oracle;
- copy_blocks copies a block's mark to its destination (and a clean source clears a
  marked destination);
- workgroups over unmarked blocks stay on the fast instance: their outputs are the same
  bits as before any block was marked, while the marked sequence meets the bar.
"""
import numpy as np
import pytest

from tests.helpers import assert_close, make_pools, slots_for, to_dev
from tests.test_gpu_prefill import _prefill, _want, assert_close_nonfinite
from tests.test_gpu_q8_range import _attend, _sprinkle, _table

pytestmark = pytest.mark.gpu


def _sync():
    import torch
    torch.cuda.synchronize()


def _used_blocks(tab, ctxs):
    return [int(b) for i, c in enumerate(ctxs) for b in tab[i, :(c + 15) // 16]]


@pytest.mark.parametrize("dtype", [8, 1])
def test_marked_count_follows_appends_writes_and_fill(dtype):
    from oracle import ref
    d, hkv = 64, 2
    pool, layout = make_pools(2, hkv, d, 8, dtype=dtype)
    pool.fill(0)
    assert pool.marked_blocks() == 0
    rng = np.random.default_rng(1)
    k = rng.standard_normal((16 * 8, hkv, d), dtype=np.float32)
    v = rng.standard_normal((16 * 8, hkv, d), dtype=np.float32)
    slots = np.arange(16 * 8, dtype=np.int64)
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    assert pool.marked_blocks() == 0  # ordinary values mark nothing
    big = 1e6 if dtype == 8 else np.inf
    kb, vb = k.copy(), v.copy()
    vb[3 * 16 + 5, 1, 7] = big       # block 3
    kb[5 * 16 + 0, 0, 2] = -big      # block 5 (K)
    vb[6 * 16 + 15, 0, 0] = big      # block 6 (layer 1 below)
    pool.append(0, to_dev(kb[:6 * 16]), to_dev(vb[:6 * 16]), to_dev(slots[:6 * 16]))
    pool.append(1, to_dev(kb), to_dev(vb), to_dev(slots))
    assert pool.marked_blocks() == 3
    # a whole-block write without a marking value clears that block's mark, a partial
    # one keeps it, a partial one holding such a value sets it
    img = pool.read()
    bb = pool.block_bytes
    clean = ref.new_pool(layout)
    ref.append(layout, clean, 0, k, v, slots)
    ref.append(layout, clean, 1, k, v, slots)
    pool.write(clean[3 * bb:4 * bb], offset=3 * bb)
    assert pool.marked_blocks() == 2
    pool.write(clean[5 * bb + 8:6 * bb - 8], offset=5 * bb + 8)
    assert pool.marked_blocks() == 2
    pool.write(img[3 * bb + 16:4 * bb - 16], offset=3 * bb + 16)  # the marked bytes again
    assert pool.marked_blocks() == 3
    pool.fill(0)
    assert pool.marked_blocks() == 0
    pool.fill(0x60 if dtype == 8 else 0x7c)  # scales 0x6060 = 560 / every value NaN (0x7c7c)
    assert pool.marked_blocks() == 8
    pool.fill(0x20)
    assert pool.marked_blocks() == 0
    assert pool.take_fault_flags() == 0


def _q8_wide_pool(ctxs, seed, host=False):
    rng = np.random.default_rng(seed)
    d, hkv = 128, 2
    nblk, tab = _table(rng, ctxs)
    pool, layout = make_pools(1, hkv, d, nblk, dtype=8, num_host_blocks=nblk if host else 0)
    pool.fill(0)
    total = sum(ctxs)
    k = _sprinkle(rng, rng.standard_normal((total, hkv, d), dtype=np.float32), per_row=1)
    v = _sprinkle(rng, rng.standard_normal((total, hkv, d), dtype=np.float32), per_row=1)
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    return pool, layout, tab, rng


def _swap_round_trip(pool, used):
    """Every used block out to host block i, the device pool cleared to zeros (which
    marks nothing), then back in."""
    out = np.stack([np.array(used, np.int64), np.arange(len(used), dtype=np.int64)], 1)
    before = pool.read()
    marked = pool.marked_blocks()
    assert marked > 0
    pool.swap_out(out)
    pool.fill(0)
    assert pool.marked_blocks() == 0
    pool.swap_in(out[:, ::-1].copy())
    assert pool.marked_blocks() == marked
    assert np.array_equal(pool.read(), before)


def test_q8_swap_out_fill_swap_in_keeps_the_exact_instance():
    """Q8_0 K and V with +-1e6 values (scales ~7,874: a binary16 operand would be inf)
    swapped out, the device pool filled with zeros, swapped back: decode and chunked
    prefill still match the oracle (f32 dequantisation), not the binary16 path."""
    ctxs = [300, 1100, 2100]
    pool, layout, tab, rng = _q8_wide_pool(ctxs, seed=3, host=True)
    _swap_round_trip(pool, _used_blocks(tab, ctxs))
    d, hkv, g = 128, 2, 4
    q = rng.standard_normal((len(ctxs), hkv * g, d), dtype=np.float32) * np.float32(2e-6)
    got, want = _attend(pool, layout, q, tab, ctxs)
    assert np.all(np.isfinite(want)) and np.abs(want).max() > 1e3
    assert_close(got, want, what="decode after swap")
    qls = [100, 200, 64]
    offs = np.array([0, 100, 300], np.int64)
    qp = rng.standard_normal((364, hkv * g, d), dtype=np.float32) * np.float32(2e-6)
    got = _prefill(pool, 0, qp, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, qp, tab, ctxs, qls, offs, d)
    assert np.all(np.isfinite(want)) and np.abs(want).max() > 1e3
    assert_close(got, want, what="prefill after swap")


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_f16_swap_out_fill_swap_in_keeps_the_leak_safe_instance(bad):
    """An F16 V holding Inf/NaN inside a 40-token chunk, taken through swap_out ->
    fill(0) -> swap_in: queries before it stay finite, later ones are what the oracle
    gives, NaN positions exact."""
    hkv, g, d = 2, 4, 128
    ctxs, qls = [40, 140], [40, 40]
    rng = np.random.default_rng(21)
    nblk, tab = _table(rng, ctxs)
    pool, layout = make_pools(1, hkv, d, nblk, dtype=1, num_host_blocks=nblk)
    pool.fill(0)
    n = sum(ctxs)
    k = rng.standard_normal((n, hkv, d), dtype=np.float32)
    v = rng.standard_normal((n, hkv, d), dtype=np.float32)
    v[9, 1, [3, 70, 127]] = bad
    v[40 + 100 + 3, 0, [0, 64]] = bad
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    pool.append(0, to_dev(k), to_dev(v), to_dev(slots))
    _swap_round_trip(pool, _used_blocks(tab, ctxs))
    offs = np.array([0, 40], np.int64)
    q = rng.standard_normal((80, hkv * g, d), dtype=np.float32)
    got = _prefill(pool, 0, q, tab, ctxs, qls, offs)
    assert pool.take_fault_flags() == 0
    want = _want(pool, layout, q, tab, ctxs, qls, offs, d)
    assert np.all(np.isfinite(want[:9])) and np.all(np.isfinite(want[40:43]))
    assert not np.all(np.isfinite(want[9:40]))
    assert_close_nonfinite(got, want, what="prefill after swap")


def test_copy_blocks_carries_the_mark():
    """A sequence's blocks copied to fresh blocks (copy-on-write): the copies are marked,
    the sources then overwritten whole with clean bytes (clearing their marks), and
    attention through the copies still takes the exact instance. A clean block copied
    over a marked one clears its mark."""
    from oracle import ref
    ctxs = [700]
    pool, layout, tab, rng = _q8_wide_pool(ctxs, seed=5)
    src = _used_blocks(tab, ctxs)
    marked = pool.marked_blocks()
    assert marked == len(src)
    free = np.setdiff1d(np.arange(pool.config.num_blocks), src)
    assert len(free) >= 2
    # copy the first two blocks to the two spare blocks, then point the table at them
    pairs = np.array([[src[0], free[0]], [src[1], free[1]]], np.int64)
    pool.copy_blocks(to_dev(pairs))
    _sync()
    assert pool.marked_blocks() == marked + 2
    bb = pool.block_bytes
    clean = ref.new_pool(layout)
    for b in src[:2]:
        pool.write(clean[b * bb:(b + 1) * bb], offset=b * bb)
    assert pool.marked_blocks() == marked
    tab2 = tab.copy()
    tab2[0, :2] = free[:2]
    d, hkv, g = 128, 2, 4
    q = rng.standard_normal((1, hkv * g, d), dtype=np.float32) * np.float32(2e-6)
    got, want = _attend(pool, layout, q, tab2, ctxs)
    assert np.abs(want).max() > 1e3
    assert_close(got, want, what="decode through copied blocks")
    # a clean block (the zeroed src[0]) copied over a marked one
    pool.copy_blocks(to_dev(np.array([[src[0], free[0]]], np.int64)))
    _sync()
    assert pool.marked_blocks() == marked - 1
    assert pool.take_fault_flags() == 0


@pytest.mark.parametrize("dtype", [8, 1])
def test_unmarked_workgroups_keep_the_fast_instance(dtype):
    """Two layers; sequence 1's blocks get a marking value in layer 1 only. Over layer 0
    (ordinary values everywhere), sequence 0's decode (Q8_0) or prefill (F16) outputs
    are the same bits as before any block was marked, so its workgroups stayed on the
    fast instance; sequence 1's workgroups take the other instance and still meet the
    bar against the oracle."""
    import torch
    import ferrum_amd as fa
    from oracle import ref
    d, hkv, g = 128, 2, 4
    ctxs = [900, 1300]
    rng = np.random.default_rng(17)
    nblk, tab = _table(rng, ctxs)
    pool, layout = make_pools(2, hkv, d, nblk, dtype=dtype)
    pool.fill(0)
    n = sum(ctxs)
    k = rng.standard_normal((n, hkv, d), dtype=np.float32)
    v = rng.standard_normal((n, hkv, d), dtype=np.float32)
    slots = np.concatenate([slots_for(tab[i], c) for i, c in enumerate(ctxs)])
    for layer in (0, 1):
        pool.append(layer, to_dev(k), to_dev(v), to_dev(slots))
    ctx = np.array(ctxs, np.int32)
    q = rng.standard_normal((len(ctxs), hkv * g, d), dtype=np.float32)
    qls = [300, 300]
    offs = np.array([0, 300], np.int64)
    qp = rng.standard_normal((600, hkv * g, d), dtype=np.float32)

    def run():
        if dtype == 8:
            out = torch.zeros(q.shape, dtype=torch.float32, device="cuda")
            pool.decode_attention(0, to_dev(q), out, to_dev(tab), to_dev(ctx), int(ctx.max()))
            _sync()
            return out.cpu().numpy()
        return _prefill(pool, 0, qp, tab, ctxs, qls, offs)

    before = run()
    # every block of sequence 1 gets a marking value at one token of layer 1
    s1 = slots_for(tab[1], ctxs[1])[::16]
    kb = np.zeros((len(s1), hkv, d), np.float32)
    vb = np.zeros((len(s1), hkv, d), np.float32)
    vb[:, 0, 0] = 1e6 if dtype == 8 else np.nan
    pool.append(1, to_dev(kb), to_dev(vb), to_dev(s1))
    _sync()
    assert pool.marked_blocks() == len(s1)
    after = run()
    assert pool.take_fault_flags() == 0
    img = pool.read()
    if dtype == 8:
        assert np.array_equal(after[0], before[0])
        want = ref.attention(layout, img, 0, q, tab, ctx, fa.default_scale(d))
        assert_close(after[1], want[1], what="exact instance beside a fast sequence")
    else:
        assert np.array_equal(after[:300], before[:300])
        want = _want(pool, layout, qp, tab, ctxs, qls, offs, d)
        assert_close(after[300:], want[300:], what="leak-safe instance beside a fast sequence")
